// dq_gemm_f32.hip -- the fp32-activation prefill GEMM on the matrix cores (the
// "expand + GEMM" accuracy class, dynacore's kF32ExpandGemm:
// dynacore/cpu/cpu_device.cpp:1114-1152 with gemm_panel, kernels_avx2.cpp:146-230).
//
// The reference expands panels of weight rows to fp32 once and multiplies them with
// every activation row in fp32. Here a workgroup expands a 128-row weight tile one
// 64-value K slice at a time into LDS, stages the matching slice of 128 fp32
// activation rows beside it, and contracts both on v_mfma_f32_32x32x2_f32: the
// weights are expanded once per workgroup and slice, never per activation row.
//
// Expanded values are the reference's x86 expansion (kernels_avx2.cpp:370-466,
// store_scaled = fma(q, scale, offset)):
//   Q4_K  fma((float)q, d * sc_j, -(dmin * m_j))        q in 0..15
//   Q6_K  (float)q * (d * sc_g)                          q in -32..31
//   Q8_0  (float)q * d,  Q4_0  (float)(nibble - 8) * d
// The products are then summed by the matrix cores in their own order, so results
// match the reference's fp32 paths to rounding: within 1e-5 of the sum of |terms|
// (the tolerance of the class; the tests check it against the oracle's vec_dot order
// and against an exact fp64 product).
//
// MFMA lane layout (v_mfma_f32_32x32x2_f32): A lane l holds row l % 32, K index l / 32;
// B lane l holds column l % 32, K index l / 32; result register r of lane l is row
// 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32. In LDS every 8-value group of a row's
// slice is stored as its even then its odd K values, so one ds_read_b128 gives a lane
// the operands of four consecutive MFMA steps.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dq_device.h"
#include "dq_internal.h"

namespace dq {

namespace {

typedef float v16f_t __attribute__((ext_vector_type(16)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

constexpr int kFM = 128, kFN = 128;  // activation rows x weight rows per workgroup
constexpr int kKc = 64;              // K values per slice
constexpr int kStride = kKc + 4;     // floats per LDS row (16 B pad: conflict-free b128 reads)
constexpr int kThreadsF = 256;       // 4 waves, each 64 x 64 outputs
constexpr int kLdsF = 2 * kFM * kStride * 4;

// Stores 16 consecutive K values (k0 % 8 == 0) of one LDS row in the permuted order:
// value k of the slice at float (k & ~7) | ((k & 1) << 2) | ((k >> 1) & 3).
DQ_DEV void put16(float* row, int k0, const float* v) {
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const float* u = v + 8 * g;
    *reinterpret_cast<v4f_t*>(row + k0 + 8 * g) = v4f_t{u[0], u[2], u[4], u[6]};
    *reinterpret_cast<v4f_t*>(row + k0 + 8 * g + 4) = v4f_t{u[1], u[3], u[5], u[7]};
  }
}

DQ_DEV float fcvt(int q) { return (float)q; }

// The raw bytes one thread expands per slice: weight row r of group G, half h of the
// slice (32 K values), slice c.
template <int WT>
struct Raw;

// Q4_K: slice c = super-block c / 4, 64-value group q = c % 4 = sub-blocks 2q (low
// nibbles of qs bytes 32q ..) and 2q + 1 (high nibbles); half h takes qs chunk 2q + h:
// values 16h + t (low) and 32 + 16h + t (high), t = 0..15.
template <>
struct Raw<kQ4_K> {
  v4u qs, hd;
  DQ_DEV void load(const __amdgpu_buffer_rsrc_t* rs, int c, int h, int r) {
    const int b = c >> 2, q = c & 3;
    qs = ld16nt(rs[0], (u32)(((b * 8 + 2 * q + h) * 64 + r) * 16));
    hd = ld16(rs[1], (u32)((b * 64 + r) * 16));
  }
  DQ_DEV void expand(int c, int h, float* row) const {
    const int q = c & 3;
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    // get_scale_min_k4 (quant_formats.h:62-70) for j = 2q, 2q + 1 from the scale bytes
    // s[0..3] = hd.y, s[4..7] = hd.z, s[8..11] = hd.w
    int sc[2], mn[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int j = 2 * q + i, sh = 8 * (j & 3);
      const u32 a = hd.y >> sh, bq = hd.z >> sh, cq = hd.w >> sh;
      if (j < 4) {
        sc[i] = (int)(a & 63u);
        mn[i] = (int)(bq & 63u);
      } else {
        sc[i] = (int)((cq & 15u) | (((a >> 6) & 3u) << 4));
        mn[i] = (int)(((cq >> 4) & 15u) | (((bq >> 6) & 3u) << 4));
      }
    }
    const float d0 = d * (float)sc[0], m0 = -(dmin * (float)mn[0]);
    const float d1 = d * (float)sc[1], m1 = -(dmin * (float)mn[1]);
    float lo[16], hi[16];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const u32 v = qs[w];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const u32 byte = (v >> (8 * e)) & 0xFFu;
        lo[4 * w + e] = fmaf(fcvt((int)(byte & 15u)), d0, m0);
        hi[4 * w + e] = fmaf(fcvt((int)((byte >> 4) ^ 8u)), d1, m1);  // the plane stores the high nibble XOR 8
      }
    }
    put16(row, 16 * h, lo);
    put16(row, 32 + 16 * h, hi);
  }
};

// Q6_K: slice c = super-block c / 4, group q = c % 4 (p = q / 2, part = q % 2): values
// 128 p + 64 part + i (quant_formats.cpp:192-216). Half h takes i = 32 h .. 32 h + 31:
// ql bytes 64 p + 32 h + (0..31) (nibble `part`), qh bytes 32 p + (0..31) (bits
// 2 h + 4 part), scales 8 p + 4 part + 2 h + (0, 1).
template <>
struct Raw<kQ6_K> {
  v4u l0, l1, h0, h1, sc;
  u32 dw;
  DQ_DEV void load(const __amdgpu_buffer_rsrc_t* rs, int c, int h, int r) {
    const int b = c >> 2, p = (c & 3) >> 1;
    l0 = ld16nt(rs[0], (u32)(((b * 8 + 4 * p + 2 * h) * 64 + r) * 16));
    l1 = ld16nt(rs[0], (u32)(((b * 8 + 4 * p + 2 * h + 1) * 64 + r) * 16));
    h0 = ld16nt(rs[1], (u32)(((b * 4 + 2 * p) * 64 + r) * 16));
    h1 = ld16nt(rs[1], (u32)(((b * 4 + 2 * p + 1) * 64 + r) * 16));
    sc = ld16(rs[2], (u32)((b * 64 + r) * 16));
    dw = ld2nt(rs[3], (u32)((b * 64 + r) * 2));
  }
  DQ_DEV void expand(int c, int h, float* row) const {
    const int q = c & 3, p = q >> 1, part = q & 1;
    const float d = h2f(dw);
    // scales 8 p + 4 part + 2 h and + 1: bytes 2 h, 2 h + 1 of word 2 p + part
    const int wi = 2 * p + part;
    const u32 sw = wi == 0 ? sc.x : wi == 1 ? sc.y : wi == 2 ? sc.z : sc.w;
    const float dsc0 = d * (float)(int8_t)((sw >> (16 * h)) & 0xFFu);
    const float dsc1 = d * (float)(int8_t)((sw >> (16 * h + 8)) & 0xFFu);
    const int shift = 2 * h + 4 * part;
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const u32 lw = i < 16 ? l0[i >> 2] : l1[(i - 16) >> 2];
      const u32 hw = i < 16 ? h0[i >> 2] : h1[(i - 16) >> 2];
      const u32 lb = (lw >> (8 * (i & 3))) & 0xFFu, hb = (hw >> (8 * (i & 3))) & 0xFFu;
      const int qv = (int)(((part ? lb >> 4 : lb & 15u)) | (((hb >> shift) & 3u) << 4)) - 32;
      v[i] = fcvt(qv) * (i < 16 ? dsc0 : dsc1);
    }
    put16(row, 32 * h, v);
    put16(row, 32 * h + 16, v + 16);
  }
};

// Q8_0 / Q4_0: slice c = 32-value blocks 2c, 2c + 1; half h takes block 2c + h (past
// the row's last block the buffer reads give zeros, so that half expands to 0).
template <>
struct Raw<kQ8_0> {
  v4u q0, q1;
  u32 dw;
  DQ_DEV void load(const __amdgpu_buffer_rsrc_t* rs, int c, int h, int r) {
    const int b = 2 * c + h;
    q0 = ld16nt(rs[0], (u32)(((b * 2) * 64 + r) * 16));
    q1 = ld16nt(rs[0], (u32)(((b * 2 + 1) * 64 + r) * 16));
    dw = ld2nt(rs[1], (u32)((b * 64 + r) * 2));
  }
  DQ_DEV void expand(int, int h, float* row) const {
    const float d = h2f(dw);
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const u32 w = i < 16 ? q0[i >> 2] : q1[(i - 16) >> 2];
      v[i] = fcvt((int)(int8_t)((w >> (8 * (i & 3))) & 0xFFu)) * d;
    }
    put16(row, 32 * h, v);
    put16(row, 32 * h + 16, v + 16);
  }
};

template <>
struct Raw<kQ4_0> {
  v4u qs;
  u32 dw;
  DQ_DEV void load(const __amdgpu_buffer_rsrc_t* rs, int c, int h, int r) {
    const int b = 2 * c + h;
    qs = ld16nt(rs[0], (u32)((b * 64 + r) * 16));
    dw = ld2nt(rs[1], (u32)((b * 64 + r) * 2));
  }
  DQ_DEV void expand(int, int h, float* row) const {
    const float d = h2f(dw);
    float v[32];
#pragma unroll
    for (int i = 0; i < 16; ++i) {  // quant_formats.cpp:12-20: low nibbles values 0..15, high 16..31
      const u32 byte = (qs[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      v[i] = fcvt((int)(byte & 15u) - 8) * d;
      v[i + 16] = fcvt((int)(byte >> 4) - 8) * d;
    }
    put16(row, 32 * h, v);
    put16(row, 32 * h + 16, v + 16);
  }
};

}  // namespace

// One workgroup: activation rows [mbase, mbase + 128) x the weight rows of the 64-row
// groups g_first + 2 tn, + 1. x: fp32 rows of stride xs floats; nslices K slices of 64.
template <int WT>
__global__ __launch_bounds__(kThreadsF) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm_f32(const uint8_t* __restrict__ p0, const uint8_t* __restrict__ p1,
                                                         const uint8_t* __restrict__ p2, const uint8_t* __restrict__ p3,
                                                         int nblk, int k, int nslices, int64_t g_first, int64_t n_groups,
                                                         int64_t n0, int64_t n1, const float* __restrict__ x, int64_t xs,
                                                         int64_t m, float* __restrict__ y, int64_t ys,
                                                         const float* __restrict__ bias, int tiles_m) {
  extern __shared__ __align__(16) uint8_t smem[];
  float* As = reinterpret_cast<float*>(smem);
  float* Bs = As + kFM * kStride;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int li = lane & 31, lg = lane >> 5;

  // consecutive workgroups (one per XCD in turn) take the activation tiles of one
  // weight tile first, so the weight tile is fetched into one L2 at a time
  const int L = blockIdx.x;
  const int tn = __builtin_amdgcn_readfirstlane(L / tiles_m);
  const int tm = __builtin_amdgcn_readfirstlane(L - tn * tiles_m);
  const int64_t G0 = g_first + 2 * (int64_t)tn;
  const int64_t mbase = (int64_t)tm * kFM;
  const int64_t mrows = m - mbase < kFM ? m - mbase : kFM;

  // ---- weight expansion role: row group G0 + (t >> 7), row r = t & 63, half h
  const int eg = t >> 7, eh = (t >> 6) & 1, er = t & 63;
  const int64_t G = G0 + eg;
  const bool g_ok = G - g_first < n_groups;
  __amdgpu_buffer_rsrc_t rs[4];
  {
    const uint8_t* pl[4] = {p0, p1, p2, p3};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int unit = plane_unit(WT, p);
      rs[p] = unit > 0 && g_ok ? rsrc(pl[p] + G * nblk * 64 * unit, (u32)(nblk * 64 * unit)) : rsrc(p0, 0u);
    }
  }
  float* erow = Bs + (64 * eg + er) * kStride;

  // ---- activation staging role: row t >> 1, K values 32 (t & 1) .. + 31 of the slice
  const int ar = t >> 1, ah = t & 1;
  const bool a_ok = ar < mrows;
  const auto rx = rsrc(x + mbase * xs, (u32)(mrows > 0 ? ((mrows - 1) * xs + k) * 4 : 0));
  float* arow = As + ar * kStride;

  Raw<WT> raw;
  v4u av[8];
  auto load = [&](int c) {
    raw.load(rs, c, eh, er);
    const int k0 = c * kKc + 32 * ah;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // whole 8-value groups lie inside or outside the row (k % 32 == 0)
      const bool in = a_ok && k0 + 4 * j < k;
      av[j] = in ? ld16(rx, (u32)((ar * xs + k0 + 4 * j) * 4)) : v4u{0u, 0u, 0u, 0u};
    }
  };
  auto put = [&](int c) {
    raw.expand(c, eh, erow);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const v4u a = av[2 * j], b = av[2 * j + 1];
      float* dst = arow + 32 * ah + 8 * j;
      *reinterpret_cast<v4u*>(dst) = v4u{a.x, a.z, b.x, b.z};
      *reinterpret_cast<v4u*>(dst + 4) = v4u{a.y, a.w, b.y, b.w};
    }
  };

  v16f_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v16f_t{};

  const float* ard[2] = {As + (64 * wm + li) * kStride + 4 * lg, As + (64 * wm + 32 + li) * kStride + 4 * lg};
  const float* brd[2] = {Bs + (64 * wn + li) * kStride + 4 * lg, Bs + (64 * wn + 32 + li) * kStride + 4 * lg};

  load(0);
#pragma unroll 1
  for (int c = 0; c < nslices; ++c) {
    __syncthreads();  // the previous slice's operands have been read
    put(c);
    __syncthreads();
    if (c + 1 < nslices) load(c + 1);  // lands while the matrix cores work on slice c
#pragma unroll
    for (int q = 0; q < kKc / 8; ++q) {
      const v4f_t a0 = *reinterpret_cast<const v4f_t*>(ard[0] + 8 * q);
      const v4f_t a1 = *reinterpret_cast<const v4f_t*>(ard[1] + 8 * q);
      const v4f_t b0 = *reinterpret_cast<const v4f_t*>(brd[0] + 8 * q);
      const v4f_t b1 = *reinterpret_cast<const v4f_t*>(brd[1] + 8 * q);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[s], b0[s], acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[s], b1[s], acc[0][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[s], b0[s], acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[s], b1[s], acc[1][1], 0, 0, 0);
      }
    }
  }

  // ---- outputs (+ bias): rows 64 wm + 32 mt + 8 (r / 4) + 4 lg + r % 4, weight rows
  // 64 wn + 32 nt + li of the tile
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int64_t n = G0 * kRowGroup + 64 * wn + 32 * nt + li;
    if (n < n0 || n >= n1) continue;
    const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 64 * wm + 32 * mt + 8 * (r >> 2) + 4 * lg + (r & 3);
        if (row < mrows) {
          const float v = acc[mt][nt][r];
          y[(mbase + row) * ys + n] = bias ? v + bv : v;
        }
      }
  }
}

hipError_t launch_gemm_f32(const WeightDev& w, const float* x, int64_t xs, int64_t m, int64_t n0, int64_t n1, float* y,
                           int64_t ys, const float* bias, hipStream_t s) {
  if (m == 0 || n1 <= n0) return hipSuccess;
  const int64_t g_first = n0 / kRowGroup;
  const int64_t n_groups = (n1 + kRowGroup - 1) / kRowGroup - g_first;
  constexpr int64_t gpt = kFN / kRowGroup;  // row groups per tile
  const int64_t tiles_n = (n_groups + gpt - 1) / gpt;
  const int64_t tiles_m = (m + kFM - 1) / kFM;
  const int nslices = (int)((w.k + kKc - 1) / kKc);
  // 32-bit buffer offsets: one row group's planes and one tile's activation rows
  int64_t plane_bytes = 0;
  for (int p = 0; p < num_planes(w.dtype); ++p) {
    const int64_t b = (int64_t)w.nblk * kRowGroup * plane_unit(w.dtype, p);
    plane_bytes = b > plane_bytes ? b : plane_bytes;
  }
  if (plane_bytes >= (1ll << 32) || ((kFM - 1) * xs + w.k) * 4 >= (1ll << 32) || tiles_n * tiles_m >= (1ll << 31)) {
    return hipErrorInvalidValue;
  }
  const void* fn = nullptr;
  switch (w.dtype) {
    case kQ4_K: fn = reinterpret_cast<const void*>(&k_gemm_f32<kQ4_K>); break;
    case kQ6_K: fn = reinterpret_cast<const void*>(&k_gemm_f32<kQ6_K>); break;
    case kQ8_0: fn = reinterpret_cast<const void*>(&k_gemm_f32<kQ8_0>); break;
    case kQ4_0: fn = reinterpret_cast<const void*>(&k_gemm_f32<kQ4_0>); break;
    default: return hipErrorInvalidValue;
  }
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsF);
  if (e != hipSuccess) return e;
  const dim3 grid((unsigned)(tiles_n * tiles_m)), block(kThreadsF);
#define DQ_F32_LAUNCH(T)                                                                                             \
  hipLaunchKernelGGL(k_gemm_f32<T>, grid, block, kLdsF, s, w.plane[0], w.plane[1], w.plane[2], w.plane[3],           \
                     (int)w.nblk, (int)w.k, nslices, g_first, n_groups, n0, n1, x, xs, m, y, ys, bias, (int)tiles_m)
  switch (w.dtype) {
    case kQ4_K: DQ_F32_LAUNCH(kQ4_K); break;
    case kQ6_K: DQ_F32_LAUNCH(kQ6_K); break;
    case kQ8_0: DQ_F32_LAUNCH(kQ8_0); break;
    default: DQ_F32_LAUNCH(kQ4_0); break;
  }
#undef DQ_F32_LAUNCH
  return hipGetLastError();
}

}  // namespace dq
