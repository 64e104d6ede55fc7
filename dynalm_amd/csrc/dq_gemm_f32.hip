// dq_gemm_f32.hip -- the fp32-activation prefill GEMM on the matrix cores (the
// "expand + GEMM" accuracy class, dynacore's kF32ExpandGemm:
// dynacore/cpu/cpu_device.cpp:1114-1152 with gemm_panel, kernels_avx2.cpp:146-230).
//
// The reference expands panels of weight rows to fp32 once and multiplies them with
// every activation row in fp32. Here a workgroup expands its weight tile one 32-value
// K slice at a time into LDS, stages the matching slice of 128 fp32 activation rows
// beside it, and contracts both on v_mfma_f32_32x32x2_f32: the weights are expanded
// once per workgroup and slice, never per activation row. Two LDS buffers: the
// expansion of slice c + 1 is issued between the MFMAs of slice c, and one barrier per
// slice separates them.
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

constexpr int kFM = 128;             // activation rows per workgroup (4 waves x 32)
constexpr int kKc = 32;              // K values per slice: one block (Q8_0, Q4_0) or sub-block (K-quants)
constexpr int kStride = kKc + 4;     // floats per LDS row (16 B pad: conflict-free b128 reads and writes)
constexpr int kThreadsF = 256;
constexpr u32 kNoLoad = 0xFFFFFFF0u;  // a buffer offset past every resource: the load returns zeros

// A workgroup's weight rows: NT 32-row MFMA tiles. NT = 4 (128 rows, 72 KB of LDS, two
// workgroups per CU) or NT = 7 (224 rows, 108 KB, one per CU): the host picks the width
// whose grid fills the CUs best (at N = 14336, 224-row tiles make exactly 256
// workgroups for M = 512 where 128-row tiles make 448 in 512 slots). The expansion
// works on whole 64-row blocks; rows past the tile (NT = 7: 224..255) go to LDS rows
// that the MFMAs never read.
template <int NT>
struct F32Tile {
  static constexpr int kBN = 32 * NT;
  static constexpr int kRows = 64 * ((kBN + 63) / 64);         // expansion rows
  static constexpr int kBuf = (kFM + kRows) * kStride;         // floats per buffer
  static constexpr int kLds = 2 * kBuf * 4;
  static constexpr int kPasses = 2 * kRows / kThreadsF;        // (row, half) items per thread
  static_assert(2 * kRows % kThreadsF == 0, "whole passes");
  static_assert(kLds <= 160 * 1024, "LDS");
};

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
DQ_DEV u32 byte_of(v4u v, int i) { return (v[i >> 2] >> (8 * (i & 3))) & 0xFFu; }

// The raw bytes one thread expands per slice: weight row r of its 64-row group, whose
// blocks start at block index gb of the plane (G * nblk), half h of the slice (K values
// 16 h .. 16 h + 15), slice c. The resources span whole planes; rows past the
// weight's padded rows read zeros.
template <int WT>
struct Raw;

// Q4_K: slice c = sub-block j = c % 8 of super-block c / 8: the low (j even) or high
// (j odd) nibbles of qs bytes 32 (j / 2) .. + 31; half h is qs chunk 2 (j / 2) + h.
template <>
struct Raw<kQ4_K> {
  v4u qs, hd;
  DQ_DEV void load(const __amdgpu_buffer_rsrc_t* rs, u32 gb, int c, int h, int r) {
    const u32 b = gb + (u32)(c >> 3), j = (u32)(c & 7);
    qs = ld16nt(rs[0], ((b * 8 + 2 * (j >> 1) + (u32)h) * 64 + (u32)r) * 16);
    hd = ld16(rs[1], (b * 64 + (u32)r) * 16);
  }
  DQ_DEV void expand(int c, int h, float* row) const {
    const int j = c & 7;
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    // get_scale_min_k4 (quant_formats.h:62-70) for sub-block j from the scale bytes
    // s[0..3] = hd.y, s[4..7] = hd.z, s[8..11] = hd.w
    const int sh = 8 * (j & 3);
    const u32 a = hd.y >> sh, bq = hd.z >> sh, cq = hd.w >> sh;
    const int sc = j < 4 ? (int)(a & 63u) : (int)((cq & 15u) | (((a >> 6) & 3u) << 4));
    const int mn = j < 4 ? (int)(bq & 63u) : (int)(((cq >> 4) & 15u) | (((bq >> 6) & 3u) << 4));
    const float d1 = d * (float)sc, m1 = -(dmin * (float)mn);
    const u32 shift = (j & 1) ? 4u : 0u, flip = (j & 1) ? 8u : 0u;  // the plane stores the high nibble XOR 8
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = fmaf(fcvt((int)(((byte_of(qs, i) >> shift) & 15u) ^ flip)), d1, m1);
    put16(row, 16 * h, v);
  }
};

// Q6_K: slice c = values 32 u .. 32 u + 31 of super-block c / 8 (u = c % 8; p = u / 4,
// s = u % 4; quant_formats.cpp:192-216): value 32 u + l has its low four bits in ql byte
// 64 p + 32 (s & 1) + l (nibble s / 2) and its top two in qh byte 32 p + l (bits 2 s);
// half h takes l = 16 h .. 16 h + 15 and scale 2 u + h.
template <>
struct Raw<kQ6_K> {
  v4u ql, qh, sc;
  u32 dw;
  DQ_DEV void load(const __amdgpu_buffer_rsrc_t* rs, u32 gb, int c, int h, int r) {
    const u32 b = gb + (u32)(c >> 3), u = (u32)(c & 7), p = u >> 2, s = u & 3, hh = (u32)h, rr = (u32)r;
    ql = ld16nt(rs[0], ((b * 8 + 4 * p + 2 * (s & 1) + hh) * 64 + rr) * 16);
    qh = ld16nt(rs[1], ((b * 4 + 2 * p + hh) * 64 + rr) * 16);
    sc = ld16(rs[2], (b * 64 + rr) * 16);
    dw = ld2nt(rs[3], (b * 64 + rr) * 2);
  }
  DQ_DEV void expand(int c, int h, float* row) const {
    const int u = c & 7, s = u & 3;
    const int si = 2 * u + h;  // scale index
    const u32 sw = (si >> 2) == 0 ? sc.x : (si >> 2) == 1 ? sc.y : (si >> 2) == 2 ? sc.z : sc.w;
    const float d1 = h2f(dw) * (float)(int8_t)((sw >> (8 * (si & 3))) & 0xFFu);
    const u32 ls = (s >> 1) ? 4u : 0u, hs = 2u * (u32)s;
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int q = (int)(((byte_of(ql, i) >> ls) & 15u) | (((byte_of(qh, i) >> hs) & 3u) << 4)) - 32;
      v[i] = fcvt(q) * d1;
    }
    put16(row, 16 * h, v);
  }
};

// Q8_0: slice c = block c; half h is qs chunk 2 c + h.
template <>
struct Raw<kQ8_0> {
  v4u qs;
  u32 dw;
  DQ_DEV void load(const __amdgpu_buffer_rsrc_t* rs, u32 gb, int c, int h, int r) {
    const u32 b = gb + (u32)c, rr = (u32)r;
    qs = ld16nt(rs[0], ((b * 2 + (u32)h) * 64 + rr) * 16);
    dw = ld2nt(rs[1], (b * 64 + rr) * 2);
  }
  DQ_DEV void expand(int, int h, float* row) const {
    const float d = h2f(dw);
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = fcvt((int)(int8_t)byte_of(qs, i)) * d;
    put16(row, 16 * h, v);
  }
};

// Q4_0: slice c = block c; half 0 takes the low nibbles (values 0..15), half 1 the high
// ones (16..31) of the block's 16 bytes (quant_formats.cpp:12-20).
template <>
struct Raw<kQ4_0> {
  v4u qs;
  u32 dw;
  DQ_DEV void load(const __amdgpu_buffer_rsrc_t* rs, u32 gb, int c, int, int r) {
    const u32 b = gb + (u32)c, rr = (u32)r;
    qs = ld16nt(rs[0], (b * 64 + rr) * 16);
    dw = ld2nt(rs[1], (b * 64 + rr) * 2);
  }
  DQ_DEV void expand(int, int h, float* row) const {
    const float d = h2f(dw);
    const u32 shift = h ? 4u : 0u;
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = fcvt((int)((byte_of(qs, i) >> shift) & 15u) - 8) * d;
    put16(row, 16 * h, v);
  }
};

}  // namespace

// One workgroup: activation rows [mbase, mbase + 128) x weight rows
// [nbase0 + 32 NT tn, + 32 NT). x: fp32 rows of stride xs floats; nslices = K / 32.
// Wave w owns activation rows 32 w .. + 31 against all NT weight tiles.
template <int WT, int NT>
__global__ __launch_bounds__(kThreadsF) __attribute__((amdgpu_waves_per_eu(NT <= 4 ? 2 : 1))) void k_gemm_f32(
    const uint8_t* __restrict__ p0, const uint8_t* __restrict__ p1, const uint8_t* __restrict__ p2,
    const uint8_t* __restrict__ p3, int nblk, int k, int nslices, int64_t nbase0, int64_t n_pad, int64_t n0, int64_t n1,
    const float* __restrict__ x, int64_t xs, int64_t m, float* __restrict__ y, int64_t ys,
    const float* __restrict__ bias, int tiles_m) {
  using T = F32Tile<NT>;
  extern __shared__ __align__(16) uint8_t smem[];
  float* buf0 = reinterpret_cast<float*>(smem);
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int li = lane & 31, lg = lane >> 5;

  // consecutive workgroups take the activation tiles of one weight tile
  const int L = blockIdx.x;
  const int tn = __builtin_amdgcn_readfirstlane(L / tiles_m);
  const int tm = __builtin_amdgcn_readfirstlane(L - tn * tiles_m);
  const int64_t nbase = nbase0 + (int64_t)T::kBN * tn;
  const int64_t mbase = (int64_t)tm * kFM;
  const int64_t mrows = m - mbase < kFM ? m - mbase : kFM;

  // ---- weight expansion role. Item i = 256 p + t of pass p: 64-row block i >> 7, half
  // (i >> 6) & 1, row (i & 63) of the block; a wave's 64 lanes take 64 consecutive rows.
  __amdgpu_buffer_rsrc_t rs[4];
  {
    const uint8_t* pl[4] = {p0, p1, p2, p3};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int unit = plane_unit(WT, p);
      rs[p] = unit > 0 ? rsrc(pl[p], (u32)(n_pad * nblk * unit)) : rsrc(p0, 0u);
    }
  }
  int erow[T::kPasses], eh[T::kPasses], er[T::kPasses];
  u32 egb[T::kPasses];
#pragma unroll
  for (int p = 0; p < T::kPasses; ++p) {
    const int i = kThreadsF * p + t;
    erow[p] = 64 * (i >> 7) + (i & 63);
    eh[p] = (i >> 6) & 1;
    const int64_t n = nbase + erow[p];
    er[p] = (int)(n & 63);
    egb[p] = (u32)((n >> 6) * nblk);
  }

  // ---- activation staging role: row t >> 1, K values 16 (t & 1) .. + 15 of the slice;
  // rows past m load as zeros (an offset outside the resource)
  const int ar = t >> 1, ah = t & 1;
  const auto rx = rsrc(x + mbase * xs, (u32)(mrows > 0 ? ((mrows - 1) * xs + k) * 4 : 0));
  const bool a_ok = ar < mrows;
  const u32 a_off = (u32)((ar * xs + 16 * ah) * 4);

  Raw<WT> raw[T::kPasses];
  v4u av[4];
  auto load = [&](int c) {
#pragma unroll
    for (int p = 0; p < T::kPasses; ++p) raw[p].load(rs, egb[p], c, eh[p], er[p]);
    const u32 o = a_off + (u32)(c * kKc * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) av[j] = ld16(rx, a_ok ? o + 16 * j : kNoLoad);
  };
  auto put_b = [&](int c, float* bufw, int p) { raw[p].expand(c, eh[p], bufw + (kFM + erow[p]) * kStride); };
  auto put_a = [&](float* bufw) {
    float* dst = bufw + ar * kStride + 16 * ah;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const v4u a = av[2 * j], b = av[2 * j + 1];
      *reinterpret_cast<v4u*>(dst + 8 * j) = v4u{a.x, a.z, b.x, b.z};
      *reinterpret_cast<v4u*>(dst + 8 * j + 4) = v4u{a.y, a.w, b.y, b.w};
    }
  };

  v16f_t acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = v16f_t{};
  const int a_rd = (32 * wave + li) * kStride + 4 * lg, b_rd = (kFM + li) * kStride + 4 * lg;

  // slice 0 into buffer 0; slice 1's loads in flight
  load(0);
#pragma unroll
  for (int p = 0; p < T::kPasses; ++p) put_b(0, buf0, p);
  put_a(buf0);
  load(nslices > 1 ? 1 : 0);
  __syncthreads();
#pragma unroll 1
  for (int c = 0; c < nslices; ++c) {
    const float* cur = buf0 + (c & 1) * T::kBuf;
    float* nxt = buf0 + ((c + 1) & 1) * T::kBuf;
    // slice c + 1 (clamped: the last iteration redoes the last slice into the buffer
    // no one reads again) is expanded between the MFMA groups of slice c
    const int cn = c + 1 < nslices ? c + 1 : c;
#pragma unroll
    for (int q = 0; q < kKc / 8; ++q) {
      const v4f_t a = *reinterpret_cast<const v4f_t*>(cur + a_rd + 8 * q);
      v4f_t b[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) b[nt] = *reinterpret_cast<const v4f_t*>(cur + b_rd + 32 * nt * kStride + 8 * q);
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[st], b[nt][st], acc[nt], 0, 0, 0);
      if (q < T::kPasses) put_b(cn, nxt, q);
      if (q == kKc / 8 - 1) put_a(nxt);
    }
    load(c + 2 < nslices ? c + 2 : cn);  // lands during the next slice's MFMAs
    __syncthreads();
  }

  // ---- outputs (+ bias): rows 32 w + 8 (r / 4) + 4 lg + r % 4, weight rows 32 nt + li
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int64_t n = nbase + 32 * nt + li;
    if (n < n0 || n >= n1) continue;
    const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 32 * wave + 8 * (r >> 2) + 4 * lg + (r & 3);
      if (row < mrows) {
        const float v = acc[nt][r];
        y[(mbase + row) * ys + n] = bias ? v + bv : v;
      }
    }
  }
}

namespace {

template <int WT, int NT>
hipError_t launch_f32(const WeightDev& w, const float* x, int64_t xs, int64_t m, int64_t n0, int64_t n1, float* y,
                      int64_t ys, const float* bias, hipStream_t s) {
  using T = F32Tile<NT>;
  const int64_t nbase0 = n0 / kRowGroup * kRowGroup;
  const int64_t tiles_n = (n1 - nbase0 + T::kBN - 1) / T::kBN;
  const int64_t tiles_m = (m + kFM - 1) / kFM;
  const int nslices = (int)(w.k / kKc);
  const void* fn = reinterpret_cast<const void*>(&k_gemm_f32<WT, NT>);
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, T::kLds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_gemm_f32<WT, NT>), dim3((unsigned)(tiles_n * tiles_m)), dim3(kThreadsF), T::kLds, s,
                     w.plane[0], w.plane[1], w.plane[2], w.plane[3], (int)w.nblk, (int)w.k, nslices, nbase0, w.n_pad, n0,
                     n1, x, xs, m, y, ys, bias, (int)tiles_m);
  return hipGetLastError();
}

template <int WT>
hipError_t launch_f32_type(const WeightDev& w, const float* x, int64_t xs, int64_t m, int64_t n0, int64_t n1, float* y,
                           int64_t ys, const float* bias, hipStream_t s) {
  // Tile width by a rounds-over-CUs cost: the workgroups each CU runs in turn times
  // their width (two 128-row workgroups share a CU's matrix cores as one 224-row one
  // uses them alone).
  const int64_t cus = w.cus > 0 ? w.cus : 256;
  const int64_t nbase0 = n0 / kRowGroup * kRowGroup, tiles_m = (m + kFM - 1) / kFM;
  auto cost = [&](int nt) {
    const int64_t tiles = (n1 - nbase0 + 32 * nt - 1) / (32 * nt) * tiles_m;
    return (tiles + cus - 1) / cus * nt;
  };
  if (cost(7) < cost(4)) return launch_f32<WT, 7>(w, x, xs, m, n0, n1, y, ys, bias, s);
  return launch_f32<WT, 4>(w, x, xs, m, n0, n1, y, ys, bias, s);
}

}  // namespace

hipError_t launch_gemm_f32(const WeightDev& w, const float* x, int64_t xs, int64_t m, int64_t n0, int64_t n1, float* y,
                           int64_t ys, const float* bias, hipStream_t s) {
  if (m == 0 || n1 <= n0) return hipSuccess;
  // 32-bit buffer offsets: each plane of the whole weight (below kNoLoad) and one tile's
  // activation rows
  for (int p = 0; p < num_planes(w.dtype); ++p) {
    if (w.n_pad * w.nblk * plane_unit(w.dtype, p) >= (int64_t)kNoLoad) return hipErrorInvalidValue;
  }
  if (((kFM - 1) * xs + w.k) * 4 >= (int64_t)kNoLoad || w.k % kKc != 0 ||
      (m + kFM - 1) / kFM * ((n1 - n0) / 128 + 2) >= (1ll << 31)) {
    return hipErrorInvalidValue;
  }
  switch (w.dtype) {
    case kQ4_K: return launch_f32_type<kQ4_K>(w, x, xs, m, n0, n1, y, ys, bias, s);
    case kQ6_K: return launch_f32_type<kQ6_K>(w, x, xs, m, n0, n1, y, ys, bias, s);
    case kQ8_0: return launch_f32_type<kQ8_0>(w, x, xs, m, n0, n1, y, ys, bias, s);
    case kQ4_0: return launch_f32_type<kQ4_0>(w, x, xs, m, n0, n1, y, ys, bias, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dq
