// dq_device.h -- device-side helpers for the gfx950 kernels (buffer loads, DPP
// reductions, fp16, Q4_K scale unpacking).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dq_layout.h"

namespace dq {

typedef uint32_t u32;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef u32 v4u __attribute__((ext_vector_type(4)));
typedef u32 v2u __attribute__((ext_vector_type(2)));

#define DQ_DEV __device__ __forceinline__

// Raw buffer resource over [p, p + bytes): loads past the end return 0 instead of
// faulting (gfx9 buffer descriptor, dword 3 = 0x00020000).
DQ_DEV __amdgpu_buffer_rsrc_t rsrc(const void* p, u32 bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
DQ_DEV v4u ld16(__amdgpu_buffer_rsrc_t r, u32 off) {
  return __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// Streaming loads of weight bytes that a launch reads exactly once: the nt cache
// policy (bit 1 of the buffer instruction's cache-policy operand on gfx950) marks
// the lines non-temporal, so the weight stream does not displace reused data
// (activations, outputs) and is not retained in L2 / MALL after use.
constexpr int kNonTemporal = 2;
DQ_DEV v4u ld16nt(__amdgpu_buffer_rsrc_t r, u32 off) {
  return __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNonTemporal));
}
DQ_DEV u32 ld2nt(__amdgpu_buffer_rsrc_t r, u32 off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, kNonTemporal);
}
DQ_DEV v2u ld8(__amdgpu_buffer_rsrc_t r, u32 off) {
  return __builtin_bit_cast(v2u, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
DQ_DEV u32 ld4(__amdgpu_buffer_rsrc_t r, u32 off) { return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0); }
DQ_DEV u32 ld2(__amdgpu_buffer_rsrc_t r, u32 off) { return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0); }

DQ_DEV float h2f(u32 h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu)); }
DQ_DEV uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
DQ_DEV float as_f(u32 u) { return __builtin_bit_cast(float, u); }
DQ_DEV u32 as_u(float f) { return __builtin_bit_cast(u32, f); }

// Bit-field extracts (v_bfe_u32 / v_bfe_i32).
DQ_DEV u32 bfe(u32 v, int off, int w) { return __builtin_amdgcn_ubfe(v, off, w); }
DQ_DEV int sbfe(u32 v, int off, int w) { return __builtin_amdgcn_sbfe((int)v, off, w); }

// The sum of the pair of int16 values in one dword (two Q8_K bsums: the code sum
// of one 32-value sub-block).
DQ_DEV int bsum_pair(u32 v) { return (int)(int16_t)(v & 0xFFFFu) + (int)(int16_t)(v >> 16); }

DQ_DEV int sdot4(u32 a, u32 b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }
// sum_i a[i] * b[i] over 16 int8 lanes, added to c.
DQ_DEV int sdot16(v4u a, v4u b, int c) {
  c = sdot4(a.x, b.x, c);
  c = sdot4(a.y, b.y, c);
  c = sdot4(a.z, b.z, c);
  return sdot4(a.w, b.w, c);
}

// sum_i a[i] * b[i] over 16 uint8 lanes, added to c (v_dot4_u32_u8).
DQ_DEV u32 udot16(v4u a, v4u b, u32 c) {
  c = __builtin_amdgcn_udot4(a.x, b.x, c, false);
  c = __builtin_amdgcn_udot4(a.y, b.y, c, false);
  c = __builtin_amdgcn_udot4(a.z, b.z, c, false);
  return __builtin_amdgcn_udot4(a.w, b.w, c, false);
}
// The two int16 halves of a, added to c (v_dot2_i32_i16 against (1, 1)).
DQ_DEV int sdot2w(u32 a, int c) {
  typedef short s2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, a), s2{1, 1}, c, false);
}

// DPP lane moves inside rows of 16 lanes.
template <int kCtrl>
DQ_DEV int dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, kCtrl, 0xF, 0xF, false);
}
constexpr int kQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kHalfMirror = 0x141;  // row_half_mirror: lane i <-> 7 - i in each 8
constexpr int kRowRor8 = 0x128;     // row_ror:8: lane i <- lane (i + 8) % 16 of its row of 16

// Exact integer sum over each aligned group of 8 lanes (every lane gets it).
DQ_DEV int red8(int v) {
  v += dpp<kQuadXor1>(v);
  v += dpp<kQuadXor2>(v);
  v += dpp<kHalfMirror>(v);
  return v;
}
DQ_DEV int red2(int v) { return v + dpp<kQuadXor1>(v); }
DQ_DEV float red8f(float v) {
  v += as_f((u32)dpp<kQuadXor1>((int)as_u(v)));
  v += as_f((u32)dpp<kQuadXor2>((int)as_u(v)));
  v += as_f((u32)dpp<kHalfMirror>((int)as_u(v)));
  return v;
}
DQ_DEV float max8f(float v) {
  v = fmaxf(v, as_f((u32)dpp<kQuadXor1>((int)as_u(v))));
  v = fmaxf(v, as_f((u32)dpp<kQuadXor2>((int)as_u(v))));
  v = fmaxf(v, as_f((u32)dpp<kHalfMirror>((int)as_u(v))));
  return v;
}

// Byte i (0..11) of the Q4_K packed scales held in three dwords.
DQ_DEV u32 sbyte(u32 s0, u32 s1, u32 s2, int i) {
  const u32 w = i < 4 ? s0 : (i < 8 ? s1 : s2);
  return (w >> (8 * (i & 3))) & 0xFFu;
}
// 6-bit scale and min of Q4_K sub-block j (dynacore/include/dynacore/quantization/quant_formats.h:62-70).
DQ_DEV void scale_min_k4(int j, u32 s0, u32 s1, u32 s2, int& sc, int& m) {
  if (j < 4) {
    sc = (int)(sbyte(s0, s1, s2, j) & 63u);
    m = (int)(sbyte(s0, s1, s2, j + 4) & 63u);
  } else {
    sc = (int)((sbyte(s0, s1, s2, j + 4) & 15u) | ((sbyte(s0, s1, s2, j - 4) >> 6) << 4));
    m = (int)((sbyte(s0, s1, s2, j + 4) >> 4) | ((sbyte(s0, s1, s2, j) >> 6) << 4));
  }
}

}  // namespace dq
