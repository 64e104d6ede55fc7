// dq_kernels.hip -- gfx950 kernels: activation quantizers, weight repack/unpack,
// the integer-partial debug kernel, and their host launchers. The GEMV lives in
// dq_gemv.hip, the MFMA GEMM in dq_gemm.hip.
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

#include "dq_act.h"
#include "dq_device.h"
#include "dq_internal.h"
#include "dq_quant.h"

namespace dq {

// ===================================================================== quantizers
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

// Sub-scaled ActSuperQ8 (320 B per 256 values: codes @0, u @256, m int16[8] @260,
// ms float[8] @276 with ms = (u m) sum, 12 zero bytes), one wave per super-block.
__global__ __launch_bounds__(64) void k_quant_sx(const float* __restrict__ x, int64_t x_stride, int64_t k,
                                                 uint8_t* __restrict__ out, int64_t orb) {
  const int l = threadIdx.x;
  const int64_t sb = blockIdx.x, row = blockIdx.y;
  const auto rx = rsrc(x + row * x_stride, (u32)(k * 4));
  float v[4];
  load4f(rx, (u32)((sb * 256 + 4 * l) * 4), v);
  float u;
  int m, sum;
  const u32 packed = sx_quant(v, u, m, sum);
  uint8_t* o = out + row * orb + sb * 320;
  *reinterpret_cast<u32*>(o + 4 * l) = packed;
  if ((l & 7) == 0) {
    const int b = l >> 3;
    *reinterpret_cast<int16_t*>(o + 260 + 2 * b) = (int16_t)m;
    *reinterpret_cast<float*>(o + 276 + 4 * b) = (u * (float)m) * (float)sum;
  }
  if (l == 0) *reinterpret_cast<float*>(o + 256) = u;
  if (l >= 1 && l <= 3) *reinterpret_cast<u32*>(o + 304 + 4 * l) = 0u;
}

// Per-32 blocks (ActBlockQ8 40 B, GGUF Q8_0 34 B or ActBlockQ16 72 B): 8 lanes per block.
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
  if (AF == kActQ16) {
    float dd;
    int sum;
    const v2u codes = q16_quant(v, dd, sum);
    if (valid) {
      uint8_t* o = out + row * orb + blk * 72;
      u32* oc = reinterpret_cast<u32*>(o + 8 + 8 * (l & 7));  // rows are only 4-byte aligned
      oc[0] = codes.x;
      oc[1] = codes.y;
      if ((l & 7) == 0) {
        *reinterpret_cast<float*>(o) = dd;
        *reinterpret_cast<int32_t*>(o + 4) = sum;
      }
    }
  } else if (AF == kActPer32) {
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
  const uint8_t x = (uint8_t)plane_xor(t, p);
  if (kPack) {
    planes.p[p][at] = src[row * row_stride + o] ^ x;
  } else {
    dst_rows[row * row_stride + o] = planes.p[p][at] ^ x;
  }
}

// ========================================================== integer partials
// One thread per (activation row, weight row, scale unit): the exact integer dot
// of the unit, decoded from the device layout with plain byte arithmetic.

DQ_DEV int act_code(int af, const uint8_t* a, int64_t i) {
  switch (af) {
    case kActPer32: return (int8_t)a[(i / 32) * 40 + 8 + i % 32];
    case kActQ8_0: return (int8_t)a[(i / 32) * 34 + 2 + i % 32];
    case kActSX: return (int8_t)a[(i / 256) * 320 + i % 256];
    case kActQ16: return (int)*reinterpret_cast<const int16_t*>(a + (i / 32) * 72 + 8 + 2 * (i % 32));
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
      const int w = (j & 1) ? ((q >> 4) ^ 8) : (q & 15);  // high nibbles are stored XOR 8
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

// ===================================================================== act_mul
// out[r, c] = act(g[r, c]) * u[r, c] (dynacore/cpu/cpu_device.cpp:1912-1930): the
// unfused tail of the gated projection. Thread t of a 256-thread block handles 4
// columns of one row (one 16-byte load of each input when kVec), rows in the grid's
// y dimension and then in steps of gridDim.y.
// (no __restrict__: out may alias an input; each element is read before it is written)
template <bool kVec>
__global__ __launch_bounds__(256) void k_act_mul(int act, const float* g, int64_t gs, const float* u, int64_t us,
                                                 int64_t m, int64_t n, float* o, int64_t os) {
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (c >= n) return;
  for (int64_t r = blockIdx.y; r < m; r += gridDim.y) {
    const float* gr = g + r * gs + c;
    const float* ur = u + r * us + c;
    float* orow = o + r * os + c;
    if (kVec) {
      const float4 gv = *reinterpret_cast<const float4*>(gr);
      const float4 uv = *reinterpret_cast<const float4*>(ur);
      float4 ov;
      ov.x = act_apply(act, gv.x) * uv.x;
      ov.y = act_apply(act, gv.y) * uv.y;
      ov.z = act_apply(act, gv.z) * uv.z;
      ov.w = act_apply(act, gv.w) * uv.w;
      *reinterpret_cast<float4*>(orow) = ov;
    } else {
      const int64_t e = n - c < 4 ? n - c : 4;
      for (int64_t i = 0; i < e; ++i) orow[i] = act_apply(act, gr[i]) * ur[i];
    }
  }
}

// ================================================================ launchers

static inline dim3 grid1(int64_t total, int block) { return dim3((unsigned)((total + block - 1) / block)); }

hipError_t launch_quantize(int af, const float* x, int64_t m, int64_t k, int64_t x_stride, uint8_t* out,
                           int64_t orb, hipStream_t s) {
  if (m == 0 || k == 0) return hipSuccess;
  if (af == kActQ8_K) {
    hipLaunchKernelGGL(k_quant_q8k, dim3((unsigned)(k / 256), (unsigned)m), dim3(64), 0, s, x, x_stride, k, out, orb);
  } else if (af == kActSX) {
    hipLaunchKernelGGL(k_quant_sx, dim3((unsigned)(k / 256), (unsigned)m), dim3(64), 0, s, x, x_stride, k, out, orb);
  } else if (af == kActQ16) {
    hipLaunchKernelGGL(k_quant_b32<kActQ16>, dim3((unsigned)((k + 255) / 256), (unsigned)m), dim3(64), 0, s, x,
                       x_stride, k, out, orb);
  } else if (af == kActPer32) {
    hipLaunchKernelGGL(k_quant_b32<kActPer32>, dim3((unsigned)((k + 255) / 256), (unsigned)m), dim3(64), 0, s, x,
                       x_stride, k, out, orb);
  } else {
    hipLaunchKernelGGL(k_quant_b32<kActQ8_0>, dim3((unsigned)((k + 255) / 256), (unsigned)m), dim3(64), 0, s, x,
                       x_stride, k, out, orb);
  }
  return hipGetLastError();
}

// qmm's activation buffer (dynacore/include/dynacore/cpu/qmm.h:57-86), written by
// quantize_row_ref (dynacore/cpu/qmm/qmm_reference.cpp:25-51) as ActBuffer::quantize_rows
// lays it out (qmm_reference.cpp:472-488): per 32-value block d = amax / qmax
// (qmax 127, or 32767 for the int16 mode), codes RNE of the clamped x * (1 / d), and
// c = d * (float)(code sum). Code i of a block goes to chunk 4 b + i / 8, byte i % 8,
// chunks cs bytes apart (row layout: 8, row r at hi + r k; pair layout: 16, row r at
// hi + (r / 2) 2 k + 8 (r & 1)); scales ds floats apart (1, or 2 interleaving a pair).
// The int16 mode stores q = 256 hi + lo (hi the arithmetic shift, lo the low byte).
// Thread (row, block, quad): four values, the block's amax and sum across its 8 lanes.
template <bool kI16>
__global__ __launch_bounds__(256) void k_qmm_quant(const float* __restrict__ x, int64_t x_stride, int64_t r0,
                                                   int64_t rows, int64_t k, int paired, int8_t* __restrict__ hi,
                                                   uint8_t* __restrict__ lo, float* __restrict__ d,
                                                   float* __restrict__ c) {
  const int64_t kb = k / 32;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const bool live = t < rows * kb * 8;  // dead lanes still take part in the shuffles
  const int64_t tt = live ? t : 0;
  const int64_t r = r0 + tt / (kb * 8);
  const int64_t b = (tt / 8) % kb;
  const int q4 = (int)(tt & 7);
  const float* xp = x + r * x_stride + b * 32 + 4 * q4;
  const float v[4] = {xp[0], xp[1], xp[2], xp[3]};
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  amax = fmaxf(amax, __shfl_xor(amax, 2));
  amax = fmaxf(amax, __shfl_xor(amax, 4));
  constexpr float qmax = kI16 ? 32767.0f : 127.0f;
  const float db = amax / qmax;
  const float id = db > 0 ? 1.0f / db : 0.0f;
  int sum = 0;
  u32 whi = 0, wlo = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float s = v[e] * id;
    s = s > -qmax ? (s < qmax ? s : qmax) : -qmax;  // NaN -> -qmax, as the reference's clamp
    const int q = (int)__builtin_rintf(s);
    sum += q;
    if (kI16) {
      whi |= ((u32)(q >> 8) & 0xFFu) << (8 * e);
      wlo |= ((u32)q & 0xFFu) << (8 * e);
    } else {
      whi |= ((u32)q & 0xFFu) << (8 * e);
    }
  }
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  sum += __shfl_xor(sum, 4);
  if (!live) return;
  const int64_t rowoff = paired ? (r / 2) * 2 * k + 8 * (r & 1) : r * k;
  const int64_t cs = paired ? 16 : 8;
  const int64_t at = rowoff + (4 * b + q4 / 2) * cs + 4 * (q4 & 1);
  *reinterpret_cast<u32*>(hi + at) = whi;
  if (kI16) *reinterpret_cast<u32*>(lo + at) = wlo;
  if (q4 == 0) {
    const int64_t so = paired ? ((r / 2) * kb + b) * 2 + (r & 1) : r * kb + b;
    d[so] = db;
    c[so] = db * (float)sum;
  }
}

// The pad row of a paired buffer with odd m (row m of the last pair): zero codes and
// scales, as ActBuffer::prepare writes them (qmm_reference.cpp:455-469).
__global__ __launch_bounds__(256) void k_qmm_pad(int64_t m, int64_t k, int8_t* __restrict__ hi,
                                                 uint8_t* __restrict__ lo, float* __restrict__ d,
                                                 float* __restrict__ c) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t kb = k / 32, base = (m / 2) * 2 * k;
  if (t < k / 8) {
    *reinterpret_cast<uint2*>(hi + base + t * 16 + 8) = uint2{0u, 0u};
    if (lo) *reinterpret_cast<uint2*>(lo + base + t * 16 + 8) = uint2{0u, 0u};
  }
  if (t < kb) {
    const int64_t so = ((m / 2) * kb + t) * 2 + 1;
    d[so] = 0.0f;
    c[so] = 0.0f;
  }
}

hipError_t launch_qmm_quantize(const float* x, int64_t x_stride, int64_t r0, int64_t r1, int64_t k, bool i16,
                               bool paired, int8_t* hi, uint8_t* lo, float* d, float* c, hipStream_t s) {
  const int64_t rows = r1 - r0;
  if (rows <= 0 || k <= 0) return hipSuccess;
  const dim3 g = grid1(rows * (k / 32) * 8, 256);
  if (i16) {
    hipLaunchKernelGGL(k_qmm_quant<true>, g, dim3(256), 0, s, x, x_stride, r0, rows, k, paired ? 1 : 0, hi, lo, d, c);
  } else {
    hipLaunchKernelGGL(k_qmm_quant<false>, g, dim3(256), 0, s, x, x_stride, r0, rows, k, paired ? 1 : 0, hi, lo, d, c);
  }
  return hipGetLastError();
}

hipError_t launch_qmm_pad(int64_t m, int64_t k, int8_t* hi, uint8_t* lo, float* d, float* c, hipStream_t s) {
  hipLaunchKernelGGL(k_qmm_pad, grid1(k / 8, 256), dim3(256), 0, s, m, k, hi, lo, d, c);
  return hipGetLastError();
}

// Rows [r0, r0 + rows) of a qmm activation buffer as the library's per-32 activation
// blocks, for qmm's gemv / gemm tables: ActBlockQ8 {d, sum, q[32]} (int8 mode) or
// ActBlockQ16 {d, sum, int16 q[32]} (int16 mode, q = 256 hi + lo;
// dynacore/include/dynacore/cpu/cpu_kernels.h:31-36,77-82). Both quantizers have the
// same arithmetic (d = amax / qmax, RNE, clamp), so the codes and d carry over and sum
// is the exact code sum (c = d * sum is not needed). Thread (row, block, quad).
template <bool kI16>
__global__ __launch_bounds__(256) void k_qmm_to_blocks(const int8_t* __restrict__ hi, const uint8_t* __restrict__ lo,
                                                       const float* __restrict__ d, int64_t k, int paired, int64_t r0,
                                                       int64_t rows, uint8_t* __restrict__ out, int64_t orb) {
  const int64_t kb = k / 32;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const bool live = t < rows * kb * 8;
  const int64_t tt = live ? t : 0;
  const int64_t rr = tt / (kb * 8), r = r0 + rr;
  const int64_t b = (tt / 8) % kb;
  const int q4 = (int)(tt & 7);
  const int64_t rowoff = paired ? (r / 2) * 2 * k + 8 * (r & 1) : r * k;
  const int64_t at = rowoff + (4 * b + q4 / 2) * (paired ? 16 : 8) + 4 * (q4 & 1);
  const u32 wh = *reinterpret_cast<const u32*>(hi + at);
  const u32 wl = kI16 ? *reinterpret_cast<const u32*>(lo + at) : 0u;
  int q[4], sum = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int h = (int)(int8_t)(wh >> (8 * e));
    q[e] = kI16 ? 256 * h + (int)((wl >> (8 * e)) & 0xFFu) : h;
    sum += q[e];
  }
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  sum += __shfl_xor(sum, 4);
  if (!live) return;
  uint8_t* blk = out + rr * orb + b * (kI16 ? 72 : 40);
  if (kI16) {
    *reinterpret_cast<uint2*>(blk + 8 + 8 * q4) =
        uint2{((u32)q[0] & 0xFFFFu) | ((u32)q[1] << 16), ((u32)q[2] & 0xFFFFu) | ((u32)q[3] << 16)};
  } else {
    *reinterpret_cast<u32*>(blk + 8 + 4 * q4) = wh;
  }
  if (q4 == 0) {
    const int64_t so = paired ? ((r / 2) * kb + b) * 2 + (r & 1) : r * kb + b;
    *reinterpret_cast<float*>(blk) = d[so];
    *reinterpret_cast<int*>(blk + 4) = sum;
  }
}

hipError_t launch_qmm_to_blocks(const int8_t* hi, const uint8_t* lo, const float* d, int64_t k, bool i16, bool paired,
                                int64_t r0, int64_t rows, uint8_t* out, int64_t orb, hipStream_t s) {
  if (rows <= 0 || k <= 0) return hipSuccess;
  const dim3 g = grid1(rows * (k / 32) * 8, 256);
  if (i16) {
    hipLaunchKernelGGL(k_qmm_to_blocks<true>, g, dim3(256), 0, s, hi, lo, d, k, paired ? 1 : 0, r0, rows, out, orb);
  } else {
    hipLaunchKernelGGL(k_qmm_to_blocks<false>, g, dim3(256), 0, s, hi, lo, d, k, paired ? 1 : 0, r0, rows, out, orb);
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

hipError_t launch_act_mul(int act, const float* g, int64_t gs, const float* u, int64_t us, int64_t m, int64_t n,
                          float* out, int64_t os, hipStream_t s) {
  if (m == 0 || n == 0) return hipSuccess;
  if (!act_ok(act)) return hipErrorInvalidValue;
  const auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  const bool vec = n % 4 == 0 && (m == 1 || (gs % 4 == 0 && us % 4 == 0 && os % 4 == 0)) && al16(g) && al16(u) &&
                   al16(out);
  const dim3 grid((unsigned)((n + 1023) / 1024), (unsigned)(m < 65535 ? m : 65535));
  if (vec) {
    hipLaunchKernelGGL(k_act_mul<true>, grid, dim3(256), 0, s, act, g, gs, u, us, m, n, out, os);
  } else {
    hipLaunchKernelGGL(k_act_mul<false>, grid, dim3(256), 0, s, act, g, gs, u, us, m, n, out, os);
  }
  return hipGetLastError();
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
