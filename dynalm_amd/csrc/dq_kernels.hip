// dq_kernels.hip -- gfx950 kernels: activation quantizers, weight repack/unpack,
// decode GEMV (M <= 4 per pass, int8 dot products), integer-partial debug
// kernel, and their host launchers. The MFMA GEMM lives in dq_gemm.hip.
//
// Arithmetic contracts (what "bit-exact" means) follow the reference:
//   quantizers   dynacore/cpu/generic/kernels_generic.cpp:187-207 (per-32),
//                dynacore/src/quantization/quant_formats.cpp:60-74 (GGUF Q8_0),
//                dynacore/cpu/avx2/kernels_avx2.cpp:638-644 (one scale per 256, Q8_K)
//   partials     dynacore/cpu/generic/kernels_generic.cpp:210-310,
//                dynacore/cpu/avx2/kernels_avx2.cpp:976-1058
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "dq_device.h"
#include "dq_internal.h"

namespace dq {

// ===================================================================== quantizers
// One wave per 256 values of a row; lane l holds values 4l .. 4l+3.

// Loads values [v0, v0 + 4) of a row through a buffer resource (zeros past the end).
DQ_DEV void load4f(__amdgpu_buffer_rsrc_t r, u32 off, float v[4]) {
  const v4u u = ld16(r, off);
  v[0] = as_f(u.x);
  v[1] = as_f(u.y);
  v[2] = as_f(u.z);
  v[3] = as_f(u.w);
}

// The comparison clamp of kernels_generic.cpp:199 (NaN goes to -L).
DQ_DEV float clampl(float v, float l) { return v > -l ? (v < l ? v : l) : -l; }

// 4 codes at inverse scale id, round half to even; returns the packed bytes and adds their sum.
DQ_DEV u32 codes4_rne(const float v[4], float id, int& sum) {
  u32 packed = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int c = (int)__builtin_rintf(clampl(v[i] * id, 127.0f));
    c = c < -127 ? -127 : (c > 127 ? 127 : c);
    sum += c;
    packed |= ((u32)c & 0xFFu) << (8 * i);
  }
  return packed;
}

// Q8_K quantization of one 256-value super-block held 4 values per lane (lane l:
// values 4l .. 4l+3): d = amax/127, codes round half to even at 1/d
// (kernels_avx2.cpp:638-644). Returns the lane's 4 packed codes, d, and in every
// lane the sum of the 16 codes of its 4-lane group (bsums[l / 4]).
DQ_DEV u32 q8k_quant(const float v[4], float& d, int& bsum) {
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = max8f(amax);
#pragma unroll
  for (int s = 8; s < 64; s <<= 1) amax = fmaxf(amax, __shfl_xor(amax, s, 64));
  d = amax / 127.0f;
  const float id = d > 0 ? 1.0f / d : 0.0f;
  int sum = 0;
  const u32 packed = codes4_rne(v, id, sum);
  sum += dpp<kQuadXor1>(sum);
  sum += dpp<kQuadXor2>(sum);
  bsum = sum;
  return packed;
}

// Per-32 ActBlockQ8 quantization (kernels_generic.cpp:187-207) of 8 blocks held 4
// values per lane (lanes 8i .. 8i+7 hold block i): returns the lane's packed codes,
// the block's d and (in every lane of the block) the block's code sum.
DQ_DEV u32 per32_quant(const float v[4], float& d, int& sum) {
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = max8f(amax);
  d = amax / 127.0f;
  const float id = d > 0 ? 1.0f / d : 0.0f;
  int s = 0;
  const u32 packed = codes4_rne(v, id, s);
  sum = red8(s);
  return packed;
}

__global__ __launch_bounds__(64) void k_quant_q8k(const float* __restrict__ x, int64_t x_stride, int64_t k,
                                                  uint8_t* __restrict__ out, int64_t orb) {
  const int l = threadIdx.x;
  const int64_t sb = blockIdx.x, row = blockIdx.y;
  const auto rx = rsrc(x + row * x_stride, (u32)(k * 4));
  float v[4];
  load4f(rx, (u32)((sb * 256 + 4 * l) * 4), v);
  float d;
  int bsum;
  const u32 packed = q8k_quant(v, d, bsum);
  uint8_t* o = out + row * orb + sb * 292;
  *reinterpret_cast<u32*>(o + 4 + 4 * l) = packed;
  if ((l & 3) == 0) *reinterpret_cast<int16_t*>(o + 260 + 2 * (l >> 2)) = (int16_t)bsum;
  if (l == 0) *reinterpret_cast<float*>(o) = d;
}

// Per-32 blocks (ActBlockQ8 40 B or GGUF Q8_0 34 B): 8 lanes per block.
template <int AF>
__global__ __launch_bounds__(64) void k_quant_b32(const float* __restrict__ x, int64_t x_stride, int64_t k,
                                                  uint8_t* __restrict__ out, int64_t orb) {
  const int l = threadIdx.x;
  const int64_t row = blockIdx.y;
  const int64_t blk = blockIdx.x * 8 + (l >> 3);  // 32-value block of this lane
  const auto rx = rsrc(x + row * x_stride, (u32)(k * 4));
  float v[4];
  load4f(rx, (u32)((blockIdx.x * 256 + 4 * l) * 4), v);
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = max8f(amax);
  const float d = amax / 127.0f;
  const bool valid = blk * 32 < k;
  if (AF == kActPer32) {
    float dd;
    int sum;
    const u32 packed = per32_quant(v, dd, sum);
    if (valid) {
      uint8_t* o = out + row * orb + blk * 40;
      *reinterpret_cast<u32*>(o + 8 + 4 * (l & 7)) = packed;
      if ((l & 7) == 0) {
        *reinterpret_cast<float*>(o) = dd;
        *reinterpret_cast<int32_t*>(o + 4) = sum;
      }
    }
  } else {
    // GGUF Q8_0: codes round half away from zero at the fp32 d, fp16 d stored.
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    u32 packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = (int)__builtin_roundf(clampl(v[i] * id, 127.0f));
      packed |= ((u32)c & 0xFFu) << (8 * i);
    }
    if (valid) {
      uint8_t* o = out + row * orb + blk * 34;
      uint16_t* oc = reinterpret_cast<uint16_t*>(o + 2 + 4 * (l & 7));
      oc[0] = (uint16_t)(packed & 0xFFFFu);
      oc[1] = (uint16_t)(packed >> 16);
      if ((l & 7) == 0) *reinterpret_cast<uint16_t*>(o) = f2h(d);
    }
  }
}

// ============================================================ repack / unpack
// One thread per GGUF byte: row n, byte o of the row -> plane p, offset.

struct Planes {
  uint8_t* p[kMaxPlanes];
};

template <bool kPack>
__global__ __launch_bounds__(256) void k_repack(int t, const uint8_t* __restrict__ src, uint8_t* __restrict__ dst_rows,
                                                int64_t row_stride, int64_t n, int64_t nblk, Planes planes) {
  const int bb = block_bytes(t);
  const int64_t row_bytes = nblk * bb;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * row_bytes) return;
  const int64_t row = idx / row_bytes, o = idx % row_bytes;
  const int64_t blk = o / bb;
  int p, off;
  plane_of_byte(t, (int)(o % bb), &p, &off);
  const int64_t at = plane_offset(t, p, row, blk, nblk, off);
  if (kPack) {
    planes.p[p][at] = src[row * row_stride + o];
  } else {
    dst_rows[row * row_stride + o] = planes.p[p][at];
  }
}

// ===================================================================== GEMV
// Lane r of every wave owns weight row 64*G + r of the workgroup's row group G
// (the 64-row layout of dq_layout.h), so at each step all lanes multiply their
// own weight bytes with the same activation values: those are wave-uniform and
// come through scalar loads, the weights through 1 KB-contiguous vector loads,
// and a row's sums need no cross-lane reduction. The W waves of a workgroup
// split the row's blocks into W contiguous slices (W times more bytes in flight
// per row group).
//
// fp32 order. K-quants x Q8_K: each lane computes its super-blocks' exact S, Mn
// and t = fma(-dmin, (float)Mn, d*(float)S) and writes t to LDS; after a barrier
// lane r of wave 0 runs acc = fma(da, t, acc) over all super-blocks in order --
// the canonical order of the CPU oracle, so outputs are bit-identical to it.
// Per-32 activations: each wave accumulates its slice in the reference's generic
// per-block order; the W slice sums are then added in slice order.

typedef u32 v4ua __attribute__((ext_vector_type(4), aligned(4)));

// Wave-uniform loads (scalar loads when base and offset are uniform).
DQ_DEV u32 uld(const uint8_t* __restrict__ p, u32 off) { return *reinterpret_cast<const u32*>(p + off); }
DQ_DEV v4u uld16(const uint8_t* __restrict__ p, u32 off) {
  const v4ua v = *reinterpret_cast<const v4ua*>(p + off);
  return v4u{v.x, v.y, v.z, v.w};
}
DQ_DEV u32 bfe(u32 v, int off, int w) { return __builtin_amdgcn_ubfe(v, off, w); }
DQ_DEV int sbfe(u32 v, int off, int w) { return __builtin_amdgcn_sbfe((int)v, off, w); }
DQ_DEV int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Activation codes 16c .. 16c+15 of a 32-value per-32 / GGUF-Q8_0 block at base (uniform).
template <int AF>
DQ_DEV void act_codes32(const uint8_t* __restrict__ a, u32 base, v4u& x0, v4u& x1) {
  if (AF == kActPer32) {
    x0 = uld16(a, base + 8);
    x1 = uld16(a, base + 24);
  } else {  // GGUF Q8_0: codes at byte 2 of the 34-byte block
    const u32 off = base + 2, al = off & ~3u;
    const v4u y0 = uld16(a, al), y1 = uld16(a, al + 16);
    const u32 y2 = uld(a, al + 32);
    if ((off & 3u) == 0) {
      x0 = y0;
      x1 = y1;
    } else {
      x0 = v4u{__builtin_amdgcn_alignbyte(y0.y, y0.x, 2), __builtin_amdgcn_alignbyte(y0.z, y0.y, 2),
               __builtin_amdgcn_alignbyte(y0.w, y0.z, 2), __builtin_amdgcn_alignbyte(y1.x, y0.w, 2)};
      x1 = v4u{__builtin_amdgcn_alignbyte(y1.y, y1.x, 2), __builtin_amdgcn_alignbyte(y1.z, y1.y, 2),
               __builtin_amdgcn_alignbyte(y1.w, y1.z, 2), __builtin_amdgcn_alignbyte(y2, y1.w, 2)};
    }
  }
}

// ---- per-format weight chunks: the vector loads of U consecutive blocks of the
// lane's row (blocks past the wave's slice read as zeros and are not used).
struct Rsrcs {
  __amdgpu_buffer_rsrc_t r0, r1, r2, r3;
};

template <int WT, int U>
struct Chunk;

template <int U>
struct Chunk<kQ4_K, U> {
  v4u q[U][8], hd[U];
  DQ_DEV void load(const Rsrcs& rs, int bb, int b1, int nblk, int r) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = bb + u < b1 ? bb + u : nblk;
#pragma unroll
      for (int c = 0; c < 8; ++c) q[u][c] = ld16(rs.r0, (u32)(((b * 8 + c) * 64 + r) * 16));
      hd[u] = ld16(rs.r1, (u32)((b * 64 + r) * 16));
    }
  }
};

template <int U>
struct Chunk<kQ6_K, U> {
  v4u L[U][8], H[U][4], SC[U];
  u32 DW[U];
  DQ_DEV void load(const Rsrcs& rs, int bb, int b1, int nblk, int r) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = bb + u < b1 ? bb + u : nblk;
#pragma unroll
      for (int c = 0; c < 8; ++c) L[u][c] = ld16(rs.r0, (u32)(((b * 8 + c) * 64 + r) * 16));
#pragma unroll
      for (int c = 0; c < 4; ++c) H[u][c] = ld16(rs.r1, (u32)(((b * 4 + c) * 64 + r) * 16));
      SC[u] = ld16(rs.r2, (u32)((b * 64 + r) * 16));
      DW[u] = ld2(rs.r3, (u32)((b * 64 + r) * 2));
    }
  }
};

template <int WT, int U>
struct Chunk32 {  // Q8_0 (2 chunks of 16 B per block) and Q4_0 (1)
  static constexpr int kC = WT == kQ8_0 ? 2 : 1;
  v4u q[U][kC];
  u32 DW[U];
  DQ_DEV void load(const Rsrcs& rs, int bb, int b1, int nblk, int r) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = bb + u < b1 ? bb + u : nblk;
#pragma unroll
      for (int c = 0; c < kC; ++c) q[u][c] = ld16(rs.r0, (u32)(((b * kC + c) * 64 + r) * 16));
      DW[u] = ld2(rs.r1, (u32)((b * 64 + r) * 2));
    }
  }
};
template <int U>
struct Chunk<kQ8_0, U> : Chunk32<kQ8_0, U> {};
template <int U>
struct Chunk<kQ4_0, U> : Chunk32<kQ4_0, U> {};

// Activations staged in LDS (both the plain and the fused path), 16-byte aligned
// so that compute reads them with broadcast ds_read_b128 at wave-uniform addresses:
//   Q8_K super-block (320 B):  d float @0, codes int8[256] @16, bsums int16[16] @272
//   32-value block   (48 B):   d float @0, code sum int32 @4, codes int8[32] @16
// (per-32 ActBlockQ8 and GGUF Q8_0 activations both stage as the latter; the GGUF
// fp16 d converts exactly to float).
constexpr int kStageQ8K = 320;
constexpr int kStage32 = 48;

DQ_DEV v4u lds16(const uint8_t* p) { return *reinterpret_cast<const v4u*>(p); }
DQ_DEV u32 lds4(const uint8_t* p) { return *reinterpret_cast<const u32*>(p); }

// Per-lane state the compute steps write: Q8_K t-terms and da go to LDS (rec,
// dav); per-32 sums accumulate in acc.
template <int M>
struct Out {
  float* rec;
  float* dav;
  float acc[M];
  int32_t* dbg;
  int64_t dbg_n, n;
  int nblk, r;
};

template <int AF, int M, int U>
DQ_DEV void compute(const Chunk<kQ4_K, U>& ch, int bb, const uint8_t* st, Out<M>& o) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int b = bb + u;
    // the 8 6-bit scales and mins as bytes (get_scale_min_k4, quant_formats.h:62-70)
    const u32 s0 = ch.hd[u].y, s1 = ch.hd[u].z, s2 = ch.hd[u].w;
    const u32 sc_lo = s0 & 0x3F3F3F3Fu, mn_lo = s1 & 0x3F3F3F3Fu;
    const u32 sc_hi = (s2 & 0x0F0F0F0Fu) | (((s0 >> 6) & 0x03030303u) << 4);
    const u32 mn_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | (((s1 >> 6) & 0x03030303u) << 4);
    const float d = h2f(ch.hd[u].x), dmin = h2f(ch.hd[u].x >> 16);
#pragma unroll
    for (int mm = 0; mm < M; ++mm) {
      if (AF == kActQ8_K) {
        const uint8_t* ab = st + (mm * o.nblk + b) * kStageQ8K;
        int S = 0, Mn = 0;
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) {
          const v4u c0 = ch.q[u][2 * jp], c1 = ch.q[u][2 * jp + 1];
          const uint8_t* cp = ab + 16 + 64 * jp;
          const int pe = sdot16(c1 & 0x0F0F0F0Fu, lds16(cp + 16), sdot16(c0 & 0x0F0F0F0Fu, lds16(cp), 0));
          const int po = sdot16((c1 >> 4) & 0x0F0F0F0Fu, lds16(cp + 48), sdot16((c0 >> 4) & 0x0F0F0F0Fu, lds16(cp + 32), 0));
          const u32 scw = jp < 2 ? sc_lo : sc_hi, mnw = jp < 2 ? mn_lo : mn_hi;
          const int e = 16 * (jp & 1);
          S += (int)bfe(scw, e, 8) * pe + (int)bfe(scw, e + 8, 8) * po;
          const u32 bsw = lds4(ab + 272 + 8 * jp), bsw2 = lds4(ab + 276 + 8 * jp);  // bsums 4jp .. 4jp+3
          const int bse = (int)(int16_t)(bsw & 0xFFFFu) + (int)(int16_t)(bsw >> 16);
          const int bso = (int)(int16_t)(bsw2 & 0xFFFFu) + (int)(int16_t)(bsw2 >> 16);
          Mn += (int)bfe(mnw, e, 8) * bse + (int)bfe(mnw, e + 8, 8) * bso;
        }
        float t = d * (float)S;
        t = fmaf(-dmin, (float)Mn, t);
        o.rec[(mm * o.nblk + b) * 64 + o.r] = t;
        if (o.r == 0) o.dav[mm * o.nblk + b] = as_f(lds4(ab));
        if (o.dbg != nullptr && o.n < o.dbg_n) {
          int32_t* p = o.dbg + (((int64_t)mm * o.dbg_n + o.n) * o.nblk + b) * 2;
          p[0] = S;
          p[1] = Mn;
        }
      } else {
        // per-32 activations, sub-block order j = 0..7 (kernels_generic.cpp:267-275)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int jp = j >> 1;
          const uint8_t* ab = st + (mm * o.nblk * 8 + b * 8 + j) * kStage32;
          const v4u c0 = ch.q[u][2 * jp], c1 = ch.q[u][2 * jp + 1];
          const v4u w0 = (j & 1) ? ((c0 >> 4) & 0x0F0F0F0Fu) : (c0 & 0x0F0F0F0Fu);
          const v4u w1 = (j & 1) ? ((c1 >> 4) & 0x0F0F0F0Fu) : (c1 & 0x0F0F0F0Fu);
          const int P = sdot16(w1, lds16(ab + 32), sdot16(w0, lds16(ab + 16), 0));
          const u32 scw = j < 4 ? sc_lo : sc_hi, mnw = j < 4 ? mn_lo : mn_hi;
          const int sc = (int)bfe(scw, 8 * (j & 3), 8), mn = (int)bfe(mnw, 8 * (j & 3), 8);
          const float ad = as_f(lds4(ab));
          const int sum = (int)lds4(ab + 4);
          const float t = (d * (float)sc) * (float)P - (dmin * (float)mn) * (float)sum;
          o.acc[mm] = o.acc[mm] + ad * t;
        }
      }
    }
  }
}

template <int AF, int M, int U>
DQ_DEV void compute(const Chunk<kQ6_K, U>& ch, int bb, const uint8_t* st, Out<M>& o) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int b = bb + u;
    const float d = h2f(ch.DW[u]);
    // ql chunk c: half p = c/4, values 128p + 16(c%4) + i (low nibbles) and + 64
    // (high); their top bits are qh chunk 2p + c%2 at bit pairs s and s+2,
    // s = (c%4)/2 (quant_formats.cpp:192-216). Units u_lo = 8p + c%4, u_hi = u_lo + 4.
    v4u qlo[8], qhi[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int p = c >> 2, cc = c & 3, s = cc >> 1;
      const v4u hb = ch.H[u][2 * p + (c & 1)];
      qlo[c] = (ch.L[u][c] & 0x0F0F0F0Fu) | (((hb >> (2 * s)) & 0x03030303u) << 4);
      qhi[c] = ((ch.L[u][c] >> 4) & 0x0F0F0F0Fu) | (((hb >> (2 * s + 4)) & 0x03030303u) << 4);
    }
#pragma unroll
    for (int mm = 0; mm < M; ++mm) {
      if (AF == kActQ8_K) {
        const uint8_t* ab = st + (mm * o.nblk + b) * kStageQ8K;
        int S = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const int ulo = 8 * (c >> 2) + (c & 3), uhi = ulo + 4;
          const u32 bsl = lds4(ab + 272 + 4 * (ulo >> 1)), bsh = lds4(ab + 272 + 4 * (uhi >> 1));
          const int sl = (int)(int16_t)(bsl >> (16 * (ulo & 1))), sh = (int)(int16_t)(bsh >> (16 * (uhi & 1)));
          const int plo = sdot16(qlo[c], lds16(ab + 16 + 16 * ulo), 0) - 32 * sl;
          const int phi = sdot16(qhi[c], lds16(ab + 16 + 16 * uhi), 0) - 32 * sh;
          const u32 wl = ulo < 4 ? ch.SC[u].x : ulo < 8 ? ch.SC[u].y : ulo < 12 ? ch.SC[u].z : ch.SC[u].w;
          const u32 wh = uhi < 4 ? ch.SC[u].x : uhi < 8 ? ch.SC[u].y : uhi < 12 ? ch.SC[u].z : ch.SC[u].w;
          S += sbfe(wl, 8 * (ulo & 3), 8) * plo + sbfe(wh, 8 * (uhi & 3), 8) * phi;
        }
        o.rec[(mm * o.nblk + b) * 64 + o.r] = d * (float)S;
        if (o.r == 0) o.dav[mm * o.nblk + b] = as_f(lds4(ab));
        if (o.dbg != nullptr && o.n < o.dbg_n) {
          int32_t* p = o.dbg + (((int64_t)mm * o.dbg_n + o.n) * o.nblk + b) * 2;
          p[0] = S;
          p[1] = 0;
        }
      } else {
        // per-32 activations, units of 16 in order (kernels_generic.cpp:299-306)
        const v4u ones = {0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};
#pragma unroll
        for (int uu = 0; uu < 16; ++uu) {
          const int p = uu >> 3, cc = uu & 3, c = 4 * p + cc;  // unit uu lives in chunk c
          const v4u qv = (uu & 4) ? qhi[c] : qlo[c];
          const uint8_t* ab = st + (mm * o.nblk * 8 + b * 8 + uu / 2) * kStage32;
          const v4u av = lds16(ab + 16 + 16 * (uu & 1));
          const int P = sdot16(qv, av, 0) - 32 * sdot16(ones, av, 0);
          const u32 sw = uu < 4 ? ch.SC[u].x : uu < 8 ? ch.SC[u].y : uu < 12 ? ch.SC[u].z : ch.SC[u].w;
          o.acc[mm] = o.acc[mm] + ((as_f(lds4(ab)) * d) * (float)sbfe(sw, 8 * (uu & 3), 8)) * (float)P;
        }
      }
    }
  }
}

template <int WT, int AF, int M, int U>
DQ_DEV void compute32(const Chunk32<WT, U>& ch, int bb, const uint8_t* st, Out<M>& o) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int b = bb + u;
    const float dw = h2f(ch.DW[u]);
#pragma unroll
    for (int mm = 0; mm < M; ++mm) {
      const uint8_t* ab = st + (mm * o.nblk + b) * kStage32;
      const v4u x0 = lds16(ab + 16), x1 = lds16(ab + 32);
      int P;
      if (WT == kQ8_0) {
        P = sdot16(ch.q[u][Chunk32<WT, U>::kC - 1], x1, sdot16(ch.q[u][0], x0, 0));
      } else {
        // low nibbles are values 0..15, high nibbles 16..31; code = nibble - 8
        P = sdot16((ch.q[u][0] >> 4) & 0x0F0F0F0Fu, x1, sdot16(ch.q[u][0] & 0x0F0F0F0Fu, x0, 0)) -
            8 * (int)lds4(ab + 4);
      }
      // generic order: acc += (dw * da) * (float)P (kernels_generic.cpp:220,235)
      o.acc[mm] = o.acc[mm] + (dw * as_f(lds4(ab))) * (float)P;
    }
  }
}
template <int AF, int M, int U>
DQ_DEV void compute(const Chunk<kQ8_0, U>& ch, int bb, const uint8_t* st, Out<M>& o) {
  compute32<kQ8_0, AF, M, U>(ch, bb, st, o);
}
template <int AF, int M, int U>
DQ_DEV void compute(const Chunk<kQ4_0, U>& ch, int bb, const uint8_t* st, Out<M>& o) {
  compute32<kQ4_0, AF, M, U>(ch, bb, st, o);
}

// ---- staging a wave's slice of activations into LDS. Loads are issued first
// (issue), the weight loads after them, then commit() waits for the activation
// loads only (vector loads complete in order) and writes the staged layout.

// Copies this wave's slice (weight blocks [b0, b1); bpu 32-value activation blocks
// per weight block for per-32 formats) of M pre-quantized rows into the staged
// LDS layout.
template <int AF, int M>
DQ_DEV void stage_acts(const uint8_t* __restrict__ acts, int64_t arb, int nblk, int b0, int b1, int bpu, int r,
                       uint8_t* st) {
  const auto ra = rsrc(acts, (u32)(M * arb));
  for (int mm = 0; mm < M; ++mm) {
    if (AF == kActQ8_K) {
      for (int b = b0; b < b1; ++b) {
        const u32 base = (u32)(mm * arb + (int64_t)b * 292);
        uint8_t* o = st + (mm * nblk + b) * kStageQ8K;
        for (int i = r; i < 73; i += 64) {
          const u32 v = ld4(ra, base + 4 * i);
          const int at = i == 0 ? 0 : (i <= 64 ? 16 + 4 * (i - 1) : 272 + 4 * (i - 65));
          *reinterpret_cast<u32*>(o + at) = v;
        }
      }
    } else {
      for (int blk = b0 * bpu + r; blk < b1 * bpu; blk += 64) {
        uint8_t* o = st + (mm * nblk * bpu + blk) * kStage32;
        if (AF == kActPer32) {
          const u32 base = (u32)(mm * arb + (int64_t)blk * 40);
          const v2u ds = ld8(ra, base);
          const v4u c0 = ld16(ra, base + 8), c1 = ld16(ra, base + 24);
          *reinterpret_cast<v2u*>(o) = ds;
          *reinterpret_cast<v4u*>(o + 16) = c0;
          *reinterpret_cast<v4u*>(o + 32) = c1;
        } else {  // GGUF Q8_0: fp16 d at 0, codes at 2 (the block is 2-byte aligned)
          const u32 base = (u32)(mm * arb + (int64_t)blk * 34);
          const u32 al = base & ~3u, sh = base & 3u;  // sh is 0 or 2
          u32 w[10];
#pragma unroll
          for (int i = 0; i < 10; ++i) w[i] = ld4(ra, al + 4 * i);
          u32 cw[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            // codes start at byte sh + 2 of w[]
            cw[i] = sh == 0 ? __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2) : w[i + 1];
          }
          const float d = h2f(sh == 0 ? w[0] : (w[0] >> 16));
          const v4u ones = {0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};
          const v4u c0 = {cw[0], cw[1], cw[2], cw[3]}, c1 = {cw[4], cw[5], cw[6], cw[7]};
          const int sum = sdot16(ones, c1, sdot16(ones, c0, 0));
          *reinterpret_cast<v2u*>(o) = v2u{as_u(d), (u32)sum};
          *reinterpret_cast<v4u*>(o + 16) = c0;
          *reinterpret_cast<v4u*>(o + 32) = c1;
        }
      }
    }
  }
}

// Activation loads of a wave's slice (one activation row) held in registers
// between issue() and commit(), so they go out before the weight loads: vector
// loads retire in order, so commit() waits for these loads only. Loops are
// unrolled over at most 8 super-blocks / one block per lane, with predication.
template <int AF>
struct ActRegs {
  u32 v[16];
  DQ_DEV static bool fits(int nslice, int bpu) { return AF == kActQ8_K ? nslice <= 8 : nslice * bpu <= 64; }
  // Q8_K: super-block b0 + i, dword j (0..72) -> lane j % 64, register 2i + j / 64.
  // 32-value blocks: one block per lane (lane = block index in the slice).
  DQ_DEV void issue(const uint8_t* __restrict__ acts, int64_t arb, int b0, int b1, int bpu, int r) {
    const auto ra = rsrc(acts, (u32)arb);
    if (AF == kActQ8_K) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const u32 base = (u32)((int64_t)(b0 + i < b1 ? b0 + i : b1) * 292);
        v[2 * i] = b0 + i < b1 ? ld4(ra, base + 4 * r) : 0u;
        v[2 * i + 1] = b0 + i < b1 && r < 9 ? ld4(ra, base + 4 * (64 + r)) : 0u;
      }
    } else {
      const int nsl = (b1 - b0) * bpu;
      const int blk = b0 * bpu + (r < nsl ? r : 0);
      const u32 base = AF == kActPer32 ? (u32)((int64_t)blk * 40) : ((u32)((int64_t)blk * 34) & ~3u);
#pragma unroll
      for (int i = 0; i < 10; ++i) v[i] = ld4(ra, base + 4 * i);
    }
  }
  DQ_DEV void commit(int64_t arb, int nblk, int b0, int b1, int bpu, int r, uint8_t* st) {
    if (AF == kActQ8_K) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (b0 + i >= b1) break;
        uint8_t* o = st + (b0 + i) * kStageQ8K;
        // dword j of the block: 0 -> d @0, 1..64 -> codes @16, 65..72 -> bsums @272
        *reinterpret_cast<u32*>(o + (r == 0 ? 0 : 16 + 4 * (r - 1))) = v[2 * i];
        if (r < 9) *reinterpret_cast<u32*>(o + (r == 0 ? 16 + 4 * 63 : 272 + 4 * (r - 1))) = v[2 * i + 1];
      }
    } else {
      const int nsl = (b1 - b0) * bpu;
      if (r >= nsl) return;
      const int blk = b0 * bpu + r;
      uint8_t* o = st + blk * kStage32;
      if (AF == kActPer32) {
        *reinterpret_cast<v2u*>(o) = v2u{v[0], v[1]};
        *reinterpret_cast<v4u*>(o + 16) = v4u{v[2], v[3], v[4], v[5]};
        *reinterpret_cast<v4u*>(o + 32) = v4u{v[6], v[7], v[8], v[9]};
      } else {  // GGUF Q8_0: fp16 d at byte 0, codes at byte 2 of the 2-byte-aligned block
        const bool sh = (((int64_t)blk * 34) & 3) != 0;  // the block starts at byte 2 of v[0]
        u32 cw[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) cw[i] = sh ? v[i + 1] : __builtin_amdgcn_alignbyte(v[i + 1], v[i], 2);
        const float d = h2f(sh ? (v[0] >> 16) : v[0]);
        const v4u ones = {0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};
        const v4u c0 = {cw[0], cw[1], cw[2], cw[3]}, c1 = {cw[4], cw[5], cw[6], cw[7]};
        const int sum = sdot16(ones, c1, sdot16(ones, c0, 0));
        *reinterpret_cast<v2u*>(o) = v2u{as_u(d), (u32)sum};
        *reinterpret_cast<v4u*>(o + 16) = c0;
        *reinterpret_cast<v4u*>(o + 32) = c1;
      }
    }
  }
};

// Makes this wave's LDS writes visible to its own later LDS reads (each wave
// stages and reads only its own slice, so no workgroup barrier is needed).
DQ_DEV void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Quantize this wave's blocks [b0, b1) of M fp32 rows into the staged LDS layout
// (the fused decode path), with the standalone quantizers' device functions.
template <int AF, int M>
DQ_DEV void quantize_slice(const float* __restrict__ x, int64_t xs, int nblk, int b0, int b1, int r, uint8_t* st) {
  constexpr bool kSb = AF == kActQ8_K;
  for (int mm = 0; mm < M; ++mm) {
    const int64_t kk = (int64_t)nblk * (kSb ? 256 : 32);
    const auto rx = rsrc(x + mm * xs, (u32)(kk * 4));
    if (kSb) {
      for (int b = b0; b < b1; ++b) {
        float v[4];
        load4f(rx, (u32)((b * 256 + 4 * r) * 4), v);
        float d;
        int bsum;
        const u32 packed = q8k_quant(v, d, bsum);
        uint8_t* o = st + (mm * nblk + b) * kStageQ8K;
        *reinterpret_cast<u32*>(o + 16 + 4 * r) = packed;
        if ((r & 3) == 0) *reinterpret_cast<int16_t*>(o + 272 + 2 * (r >> 2)) = (int16_t)bsum;
        if (r == 0) *reinterpret_cast<float*>(o) = d;
      }
    } else {
      for (int bb = b0; bb < b1; bb += 8) {
        const int blk = bb + (r >> 3);
        float v[4];
        load4f(rx, (u32)((blk * 32 + 4 * (r & 7)) * 4), v);
        float d;
        int sum;
        const u32 packed = per32_quant(v, d, sum);
        if (blk < b1) {
          uint8_t* o = st + (mm * nblk + blk) * kStage32;
          *reinterpret_cast<u32*>(o + 16 + 4 * (r & 7)) = packed;
          if ((r & 7) == 0) {
            *reinterpret_cast<float*>(o) = d;
            *reinterpret_cast<int32_t*>(o + 4) = sum;
          }
        }
      }
    }
  }
}

// kFuse: the activations arrive as fp32 rows (x, row stride xs floats) and each
// wave quantizes its own slice into LDS with the standalone quantizers' device
// functions (q8k_quant / per32_quant), so the codes are the same bytes.
template <int WT, int AF, int M, int W, int U, bool kFuse>
__global__ __launch_bounds__(W * 64) void k_gemv(const uint8_t* __restrict__ p0, const uint8_t* __restrict__ p1,
                                                 const uint8_t* __restrict__ p2, const uint8_t* __restrict__ p3,
                                                 int nblk, int64_t g0, int64_t n0, int64_t n1,
                                                 const uint8_t* __restrict__ acts, int64_t arb,
                                                 const float* __restrict__ x, int64_t xs,
                                                 float* __restrict__ y, int64_t ys, const float* __restrict__ bias,
                                                 int32_t* __restrict__ dbg, int64_t dbg_n) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr bool kSb = AF == kActQ8_K;
  // LDS: Q8_K t-terms [M][nblk][64] + da [M][nblk]  |  per-32 slice sums [W][M][64];
  // then the staged activation rows [M][nblk (blocks of 32 for per-32)][stage bytes]
  const int r = threadIdx.x & 63, wave = wave_id();
  const int64_t G = g0 + blockIdx.x;
  Out<M> o;
  o.rec = reinterpret_cast<float*>(smem);
  o.dav = o.rec + M * nblk * 64;
  o.dbg = dbg;
  o.dbg_n = dbg_n;
  o.n = G * kRowGroup + r;
  o.nblk = nblk;
  o.r = r;
#pragma unroll
  for (int mm = 0; mm < M; ++mm) o.acc[mm] = 0.0f;
  const int b0 = wave * nblk / W, b1 = (wave + 1) * nblk / W;  // this wave's blocks
  uint8_t* st = smem + (kSb ? ((size_t)M * nblk * 65 * 4 + 15) / 16 * 16 : (size_t)W * M * 64 * 4);

  // plane buffer resources of this row group (64 rows x nblk blocks)
  const int u0 = plane_unit(WT, 0), u1 = plane_unit(WT, 1);
  Rsrcs rs;
  rs.r0 = rsrc(p0 + G * nblk * 64 * u0, (u32)(nblk * 64 * u0));
  rs.r1 = rsrc(p1 + G * nblk * 64 * u1, (u32)(nblk * 64 * u1));
  rs.r2 = rs.r0;
  rs.r3 = rs.r0;
  if (WT == kQ6_K) {
    rs.r2 = rsrc(p2 + G * nblk * 64 * 16, (u32)(nblk * 64 * 16));
    rs.r3 = rsrc(p3 + G * nblk * 64 * 2, (u32)(nblk * 64 * 2));
  }

  // activations for this slice: their loads go out first, so their latency hides
  // behind the weight loads issued next; each wave stages only its own slice
  const int bpu = (WT == kQ4_K || WT == kQ6_K) && !kSb ? 8 : 1;
  float xv[2][4];
  const bool pre = kFuse && kSb && M == 1 && b1 - b0 <= 2;
  const bool held = !kFuse && M == 1 && ActRegs<AF>::fits(b1 - b0, bpu);
  ActRegs<AF> ar;
  if (pre) {
    const auto rx = rsrc(x, (u32)(nblk * 256 * 4));
#pragma unroll
    for (int i = 0; i < 2; ++i) load4f(rx, (u32)(((b0 + i) * 256 + 4 * r) * 4), xv[i]);
  } else if (held) {
    ar.issue(acts, arb, b0, b1, bpu, r);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weight loads
  Chunk<WT, U> c0;
  const bool full0 = b0 + U <= b1;
  if (full0) c0.load(rs, b0, b1, nblk, r);
  __builtin_amdgcn_sched_barrier(0);
  if (pre) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (b0 + i < b1) {
        float d;
        int bsum;
        const u32 packed = q8k_quant(xv[i], d, bsum);
        uint8_t* ob = st + (b0 + i) * kStageQ8K;
        *reinterpret_cast<u32*>(ob + 16 + 4 * r) = packed;
        if ((r & 3) == 0) *reinterpret_cast<int16_t*>(ob + 272 + 2 * (r >> 2)) = (int16_t)bsum;
        if (r == 0) *reinterpret_cast<float*>(ob) = d;
      }
    }
  } else if (held) {
    ar.commit(arb, nblk, b0, b1, bpu, r, st);
  } else if (kFuse) {
    quantize_slice<AF, M>(x, xs, nblk, b0, b1, r, st);
  } else {
    stage_acts<AF, M>(acts, arb, nblk, b0, b1, bpu, r, st);
  }
  wave_lds_sync();

  int bb = b0;
  if (full0) {
    compute<AF, M, U>(c0, bb, st, o);
    bb += U;
  }
  for (; bb + U <= b1; bb += U) {
    Chunk<WT, U> c;
    c.load(rs, bb, b1, nblk, r);
    compute<AF, M, U>(c, bb, st, o);
  }
  for (; bb < b1; ++bb) {
    Chunk<WT, 1> c;
    c.load(rs, bb, b1, nblk, r);
    compute<AF, M, 1>(c, bb, st, o);
  }

  if (!kSb) {
#pragma unroll
    for (int mm = 0; mm < M; ++mm) o.rec[(wave * M + mm) * 64 + r] = o.acc[mm];
  }
  __syncthreads();
  if (wave != 0) return;
  const int64_t n = o.n;
#pragma unroll
  for (int mm = 0; mm < M; ++mm) {
    float v = 0.0f;
    if (kSb) {
      const float* tp = o.rec + mm * nblk * 64 + r;
      const float* dp = o.dav + mm * nblk;
      int b = 0;
      for (; b + 4 <= nblk; b += 4) {
        const float t0 = tp[b * 64], t1 = tp[(b + 1) * 64], t2 = tp[(b + 2) * 64], t3 = tp[(b + 3) * 64];
        const float d0 = dp[b], d1 = dp[b + 1], d2 = dp[b + 2], d3 = dp[b + 3];
        v = fmaf(d0, t0, v);
        v = fmaf(d1, t1, v);
        v = fmaf(d2, t2, v);
        v = fmaf(d3, t3, v);
      }
      for (; b < nblk; ++b) v = fmaf(dp[b], tp[b * 64], v);
    } else {
#pragma unroll
      for (int w = 0; w < W; ++w) v = v + o.rec[(w * M + mm) * 64 + r];
    }
    if (n >= n0 && n < n1) y[mm * ys + n] = bias ? v + bias[n] : v;
  }
}

// ========================================================== integer partials
// One thread per (activation row, weight row, scale unit): the exact integer dot
// of the unit, decoded from the device layout with plain byte arithmetic.

DQ_DEV int act_code(int af, const uint8_t* a, int64_t i) {
  switch (af) {
    case kActPer32: return (int8_t)a[(i / 32) * 40 + 8 + i % 32];
    case kActQ8_0: return (int8_t)a[(i / 32) * 34 + 2 + i % 32];
    default: return (int8_t)a[(i / 256) * 292 + 4 + i % 256];
  }
}

__global__ __launch_bounds__(256) void k_units(int t, int af, const uint8_t* p0, const uint8_t* p1, int64_t nblk,
                                               int64_t n, int64_t k, int64_t m, const uint8_t* __restrict__ acts,
                                               int64_t arb, int32_t* __restrict__ units, int64_t nu) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= m * n * nu) return;
  const int64_t u = idx % nu, row = (idx / nu) % n, mm = idx / (nu * n);
  const uint8_t* a = acts + mm * arb;
  int s = 0;
  if (t == kQ8_0 || t == kQ4_0) {
    for (int i = 0; i < 32; ++i) {
      int w;
      if (t == kQ8_0) {
        w = (int)(int8_t)p0[plane_offset(t, 0, row, u, nblk, i)];
      } else {
        const uint8_t q = p0[plane_offset(t, 0, row, u, nblk, i % 16)];
        w = (int)(i < 16 ? (q & 15) : (q >> 4)) - 8;
      }
      s += w * act_code(af, a, u * 32 + i);
    }
  } else if (t == kQ4_K) {
    const int64_t b = u / 8;
    const int j = (int)(u % 8);
    for (int i = 0; i < 32; ++i) {
      const uint8_t q = p0[plane_offset(t, 0, row, b, nblk, 32 * (j / 2) + i)];
      const int w = (j & 1) ? (q >> 4) : (q & 15);
      s += w * act_code(af, a, b * 256 + 32 * j + i);
    }
  } else {  // Q6_K: unit = 16 values 16*uu .. of super-block b
    const int64_t b = u / 16;
    const int uu = (int)(u % 16);
    for (int i = 0; i < 16; ++i) {
      const int v = 16 * uu + i;  // value index in the super-block
      const int half = v / 128, w = v % 128, quarter = w / 32, l = w % 32;
      const int lb = p0[plane_offset(t, 0, row, b, nblk, 64 * half + l + (quarter & 1) * 32)];
      const int nib = quarter < 2 ? (lb & 15) : (lb >> 4);
      const int hb = (p1[plane_offset(t, 1, row, b, nblk, 32 * half + l)] >> (2 * quarter)) & 3;
      s += ((nib | (hb << 4)) - 32) * act_code(af, a, b * 256 + v);
    }
  }
  units[idx] = s;
}

// ================================================================ launchers

static inline dim3 grid1(int64_t total, int block) { return dim3((unsigned)((total + block - 1) / block)); }

hipError_t launch_quantize(int af, const float* x, int64_t m, int64_t k, int64_t x_stride, uint8_t* out,
                           int64_t orb, hipStream_t s) {
  if (m == 0 || k == 0) return hipSuccess;
  if (af == kActQ8_K) {
    hipLaunchKernelGGL(k_quant_q8k, dim3((unsigned)(k / 256), (unsigned)m), dim3(64), 0, s, x, x_stride, k, out, orb);
  } else if (af == kActPer32) {
    hipLaunchKernelGGL(k_quant_b32<kActPer32>, dim3((unsigned)((k + 255) / 256), (unsigned)m), dim3(64), 0, s, x,
                       x_stride, k, out, orb);
  } else {
    hipLaunchKernelGGL(k_quant_b32<kActQ8_0>, dim3((unsigned)((k + 255) / 256), (unsigned)m), dim3(64), 0, s, x,
                       x_stride, k, out, orb);
  }
  return hipGetLastError();
}

hipError_t launch_repack(int t, const uint8_t* src, int64_t row_stride, int64_t n, int64_t nblk, uint8_t* const* planes,
                         hipStream_t s) {
  Planes pl{};
  for (int i = 0; i < num_planes(t); ++i) pl.p[i] = planes[i];
  const int64_t total = n * nblk * block_bytes(t);
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(k_repack<true>, grid1(total, 256), dim3(256), 0, s, t, src, nullptr, row_stride, n, nblk, pl);
  return hipGetLastError();
}

hipError_t launch_unpack(int t, uint8_t* dst, int64_t row_stride, int64_t n, int64_t nblk, uint8_t* const* planes,
                         hipStream_t s) {
  Planes pl{};
  for (int i = 0; i < num_planes(t); ++i) pl.p[i] = planes[i];
  const int64_t total = n * nblk * block_bytes(t);
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(k_repack<false>, grid1(total, 256), dim3(256), 0, s, t, nullptr, dst, row_stride, n, nblk, pl);
  return hipGetLastError();
}

constexpr int kGemvWaves = 8;

template <int WT, int AF, int M, bool kFuse>
static hipError_t gemv_launch(const WeightDev& w, const uint8_t* acts, int64_t arb, const float* x, int64_t xs,
                              int64_t n0, int64_t n1, float* y, int64_t ys, const float* bias, int32_t* dbg,
                              hipStream_t s) {
  constexpr int U = (WT == kQ8_0 || WT == kQ4_0) ? 8 : 2;
  const int64_t g0 = n0 / kRowGroup, g1 = (n1 + kRowGroup - 1) / kRowGroup;
  size_t lds = AF == kActQ8_K ? ((size_t)M * w.nblk * 65 * sizeof(float) + 15) / 16 * 16
                              : (size_t)kGemvWaves * M * 64 * sizeof(float);
  // staged activations: Q8_K super-blocks of 320 B, or 32-value blocks of 48 B
  lds += AF == kActQ8_K ? (size_t)M * w.nblk * 320
                        : (size_t)M * w.nblk * (WT == kQ4_K || WT == kQ6_K ? 8 : 1) * 48;
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  const void* fn = reinterpret_cast<const void*>(&k_gemv<WT, AF, M, kGemvWaves, U, kFuse>);
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((k_gemv<WT, AF, M, kGemvWaves, U, kFuse>), dim3((unsigned)(g1 - g0)), dim3(64 * kGemvWaves), lds,
                     s, w.plane[0], w.plane[1], w.plane[2], w.plane[3], (int)w.nblk, g0, n0, n1, acts, arb, x, xs, y,
                     ys, bias, dbg, w.n);
  return hipGetLastError();
}

// M rows (1..4) of one pass; x != nullptr: fused quantization of fp32 rows.
template <int M>
static hipError_t gemv_pass(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, const float* x, int64_t xs,
                            int64_t n0, int64_t n1, float* y, int64_t ys, const float* bias, int32_t* dbg,
                            hipStream_t s) {
  if (x != nullptr) {
    switch (w.dtype) {
      case kQ4_K: return gemv_launch<kQ4_K, kActQ8_K, M, true>(w, nullptr, 0, x, xs, n0, n1, y, ys, bias, dbg, s);
      case kQ6_K: return gemv_launch<kQ6_K, kActQ8_K, M, true>(w, nullptr, 0, x, xs, n0, n1, y, ys, bias, dbg, s);
      case kQ8_0: return gemv_launch<kQ8_0, kActPer32, M, true>(w, nullptr, 0, x, xs, n0, n1, y, ys, bias, dbg, s);
      default: return gemv_launch<kQ4_0, kActPer32, M, true>(w, nullptr, 0, x, xs, n0, n1, y, ys, bias, dbg, s);
    }
  }
  switch (w.dtype) {
    case kQ4_K:
      return af == kActQ8_K ? gemv_launch<kQ4_K, kActQ8_K, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, s)
                            : gemv_launch<kQ4_K, kActPer32, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, s);
    case kQ6_K:
      return af == kActQ8_K ? gemv_launch<kQ6_K, kActQ8_K, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, s)
                            : gemv_launch<kQ6_K, kActPer32, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, s);
    case kQ8_0:
      return af == kActPer32 ? gemv_launch<kQ8_0, kActPer32, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, s)
                             : gemv_launch<kQ8_0, kActQ8_0, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, s);
    default:
      return af == kActPer32 ? gemv_launch<kQ4_0, kActPer32, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, s)
                             : gemv_launch<kQ4_0, kActQ8_0, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, s);
  }
}

static hipError_t gemv_rows(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, const float* x, int64_t xs,
                            int64_t m, int64_t n0, int64_t n1, float* y, int64_t ys, const float* bias, int32_t* dbg,
                            hipStream_t s) {
  for (int64_t r0 = 0; r0 < m; r0 += 4) {
    const int rows = (int)(m - r0 < 4 ? m - r0 : 4);
    const uint8_t* a = acts ? acts + r0 * arb : nullptr;
    const float* xx = x ? x + r0 * xs : nullptr;
    float* yy = y + r0 * ys;
    int32_t* dd = dbg ? dbg + r0 * w.n * w.nblk * 2 : nullptr;
    hipError_t e;
    switch (rows) {
      case 1: e = gemv_pass<1>(w, af, a, arb, xx, xs, n0, n1, yy, ys, bias, dd, s); break;
      case 2: e = gemv_pass<2>(w, af, a, arb, xx, xs, n0, n1, yy, ys, bias, dd, s); break;
      case 3: e = gemv_pass<3>(w, af, a, arb, xx, xs, n0, n1, yy, ys, bias, dd, s); break;
      default: e = gemv_pass<4>(w, af, a, arb, xx, xs, n0, n1, yy, ys, bias, dd, s); break;
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_gemv(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0, int64_t n1,
                       float* y, int64_t ys, const float* bias, int32_t* dbg, hipStream_t s) {
  return gemv_rows(w, af, acts, arb, nullptr, 0, m, n0, n1, y, ys, bias, dbg, s);
}

hipError_t launch_gemv_fused(const WeightDev& w, const float* x, int64_t xs, int64_t m, float* y, int64_t ys,
                             const float* bias, hipStream_t s) {
  return gemv_rows(w, -1, nullptr, 0, x, xs, m, 0, w.n, y, ys, bias, nullptr, s);
}

hipError_t launch_units(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int32_t* units,
                        int64_t nu, hipStream_t s) {
  const int64_t total = m * w.n * nu;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(k_units, grid1(total, 256), dim3(256), 0, s, w.dtype, af, w.plane[0], w.plane[1], w.nblk, w.n,
                     w.k, m, acts, arb, units, nu);
  return hipGetLastError();
}

}  // namespace dq
