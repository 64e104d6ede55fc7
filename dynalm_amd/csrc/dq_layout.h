// dq_layout.h -- GGUF block sizes and the repacked HBM layout, shared by host and device code.
//
// GGUF blocks (dynacore/include/dynacore/quantization/quant_formats.h:18-39,
// sizes dynacore/src/tensor/dtype.cpp:24-45):
//   Q4_0  {fp16 d; u8 qs[16]}                                  18 B / 32 values
//   Q8_0  {fp16 d; i8 qs[32]}                                  34 B / 32
//   Q4_K  {fp16 d, dmin; u8 scales[12]; u8 qs[128]}           144 B / 256
//   Q6_K  {u8 ql[128]; u8 qh[64]; i8 scales[16]; fp16 d}      210 B / 256
//
// Device layout: rows are taken in groups of 64 (n padded up to a multiple of 64
// with zero rows) and each block is split into planes; inside a plane, for every
// block b and 16-byte chunk c of a row's unit, the chunks of the 64 rows of a
// group are adjacent:
//   unit >= 16:  plane[p][(((G * nblk + b) * (unit / 16) + c) * 64 + r) * 16 + byte]
//   unit <  16:  plane[p][((G * nblk + b) * 64 + r) * unit + byte]
// with G = n / 64, r = n % 64. One wave, lane r <-> row r, then reads 1 KB
// contiguous per 16-byte-per-lane load instruction, and all 64 lanes use the same
// activation values at the same time (so those are wave-uniform scalar loads).
// Planes per type (unit bytes per row and block):
//   Q4_K  0: qs 128          1: header {d, dmin, scales[12]} 16
//   Q6_K  0: ql 128          1: qh 64    2: scales 16    3: d 2
//   Q8_0  0: qs 32           1: d 2
//   Q4_0  0: qs 16           1: d 2
// The bytes of every plane are the block's bytes (a permutation of the GGUF row
// bytes), so the device copy holds exactly the GGUF byte count plus the zero
// padding rows. One transform: in Q4_K's qs plane every byte has bit 7 flipped
// (the high nibble XOR 8), so that `byte & 0xF0` read as int8 is 16 * (q - 8) for
// the high nibble q, which a signed int8 dot product takes directly
// (plane_xor; the unpack flips it back).
#pragma once

#include <stdint.h>

#ifdef __HIPCC__
#define DQ_HD __host__ __device__ __forceinline__
#else
#define DQ_HD inline
#endif

namespace dq {

enum : int { kQ4_0 = 6, kQ8_0 = 10, kQ4_K = 14, kQ6_K = 16 };
enum : int { kActPer32 = 0, kActQ8_0 = 1, kActQ8_K = 2, kActSX = 3, kActQ16 = 4, kActF32 = 5 };

constexpr int kRowGroup = 64;
constexpr int kMaxPlanes = 4;

DQ_HD int block_elems(int t) { return (t == kQ4_K || t == kQ6_K) ? 256 : (t == kQ4_0 || t == kQ8_0) ? 32 : -1; }
DQ_HD int block_bytes(int t) {
  return t == kQ4_0 ? 18 : t == kQ8_0 ? 34 : t == kQ4_K ? 144 : t == kQ6_K ? 210 : -1;
}
DQ_HD int num_planes(int t) { return t == kQ6_K ? 4 : 2; }
// Bytes of plane p per (row, block).
DQ_HD int plane_unit(int t, int p) {
  switch (t) {
    case kQ4_K: return p == 0 ? 128 : 16;
    case kQ6_K: return p == 0 ? 128 : p == 1 ? 64 : p == 2 ? 16 : 2;
    case kQ8_0: return p == 0 ? 32 : 2;
    case kQ4_0: return p == 0 ? 16 : 2;
    default: return 0;
  }
}
// Plane and offset-in-unit of byte i (0 <= i < block_bytes) of a block.
DQ_HD void plane_of_byte(int t, int i, int* p, int* off) {
  switch (t) {
    case kQ4_K:
      if (i < 16) { *p = 1; *off = i; } else { *p = 0; *off = i - 16; }
      break;
    case kQ6_K:
      if (i < 128) { *p = 0; *off = i; }
      else if (i < 192) { *p = 1; *off = i - 128; }
      else if (i < 208) { *p = 2; *off = i - 192; }
      else { *p = 3; *off = i - 208; }
      break;
    default: /* Q8_0, Q4_0: fp16 d first */
      if (i < 2) { *p = 1; *off = i; } else { *p = 0; *off = i - 2; }
      break;
  }
}

// XOR applied to every byte of plane p on upload (and undone on download).
DQ_HD int plane_xor(int t, int p) { return t == kQ4_K && p == 0 ? 0x80 : 0; }

// Offset in plane p of byte `off` of the unit of row n, block b.
DQ_HD int64_t plane_offset(int t, int p, int64_t n, int64_t b, int64_t nblk, int off) {
  const int64_t G = n / kRowGroup, r = n % kRowGroup;
  const int unit = plane_unit(t, p);
  if (unit >= 16) return (((G * nblk + b) * (unit / 16) + off / 16) * kRowGroup + r) * 16 + off % 16;
  return ((G * nblk + b) * kRowGroup + r) * unit + off;
}

DQ_HD int act_block_elems(int f) {
  return (f == kActQ8_K || f == kActSX) ? 256 : (f == kActPer32 || f == kActQ8_0 || f == kActQ16 || f == kActF32) ? 32 : -1;
}
DQ_HD int act_block_bytes(int f) {
  return f == kActPer32 ? 40 : f == kActQ8_0 ? 34 : f == kActQ8_K ? 292 : f == kActSX ? 320 : f == kActQ16 ? 72
         : f == kActF32 ? 128 : -1;
}

}  // namespace dq
