// dq_gemm.hip -- prefill GEMM for Q4_K weights x Q8_K activations on gfx950 int8
// MFMA (v_mfma_i32_16x16x64_i8).
//
// Per super-block b (256 values) and output (m, n), the arithmetic contract is
// the exact integer pair of the reference's super-block kernel
// (dynacore/cpu/avx2/kernels_avx2.cpp:976-1014):
//   S  = sum_j sc_j * P_j
//   Mn = sum_j m_j * (sum of the activation codes of sub-block j)
// combined in fp32 once per super-block in this library's canonical order
//   u = d * (float)S;  u = fma(-dmin, (float)Mn, u);  acc = fma(da, u, acc)
// (the same order as the GEMV kernels and the CPU oracle).
//
// The effective integer weight sc*q (0..945) does not fit int8, so each weight
// tile is dequantized in LDS into two int8 planes sc*q = 32*H + L (L in 0..31,
// H in 0..29) and a third plane holding m_j at every position of sub-block j,
// whose MFMA sum is exactly Mn. Three int8 MFMA accumulations per output give
// S = L + 32*H and Mn exactly in int32.
//
// Tiling: a workgroup of 4 waves computes 256 activation rows x 64 weight rows;
// wave w owns activation rows 64w .. 64w+63 (4 x 4 MFMA tiles of 16 x 16). Per
// super-block the 256 x 256 activation codes (64 KB) and the three 64 x 256
// weight planes (48 KB) are staged in LDS; the next super-block's global loads
// are issued before the MFMA phase so they overlap it.
//
// MFMA operand layout (16x16x64 i8): lane l supplies row (A) / column (B) l%16
// and 16 K-values of lane group l/16; the result lane l holds column l%16, rows
// 4*(l/16) .. 4*(l/16)+3. K-step s of a super-block covers values 64s .. 64s+63,
// lane group g the 16 values 64s + 16g ..: for Q4_K these are the low nibbles of
// qs[32s + 16g ..] (g < 2, sub-block 2s) or the high nibbles of qs[32s + 16(g-2) ..]
// (g >= 2, sub-block 2s+1) (dynacore/src/quantization/quant_formats.cpp:150-167).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dq_device.h"
#include "dq_internal.h"

namespace dq {

namespace {

constexpr int kBM = 256;       // activation rows per workgroup
constexpr int kBN = 64;        // weight rows per workgroup
constexpr int kThreads = 256;  // 4 waves
constexpr int kPlanes = 3;     // H, L, M

// LDS layout (bytes)
constexpr int kLdsA = 0;                                 // [4 steps][256 rows][64 B]
constexpr int kLdsB = kLdsA + 4 * kBM * 64;              // [4 steps][3 planes][64 rows][64 B]
constexpr int kLdsDW = kLdsB + 4 * kPlanes * kBN * 64;   // [64 rows] {d, dmin} float
constexpr int kLdsDA = kLdsDW + kBN * 8;                 // [256 rows] float
constexpr int kLdsBytes = kLdsDA + kBM * 4;              // 115200

typedef int v4i_t __attribute__((ext_vector_type(4)));

DQ_DEV v4i_t mfma(v4u a, v4u b, v4i_t c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i_t, a), __builtin_bit_cast(v4i_t, b), c, 0, 0,
                                               0);
}

DQ_DEV u32 pack_even_odd(u32 even, u32 odd) { return (even & 0x00FF00FFu) | ((odd & 0x00FF00FFu) << 8); }

// 4 codes (bytes, 0..15) times sc -> the L (split_lo) and H (split_hi) bytes of
// sc*q = 32*H + L.
DQ_DEV u32 split_lo(u32 q, u32 sc) {
  const u32 pe = (q & 0x00FF00FFu) * sc, po = ((q >> 8) & 0x00FF00FFu) * sc;  // 16-bit lanes, <= 945
  return pack_even_odd(pe & 0x001F001Fu, po & 0x001F001Fu);
}
DQ_DEV u32 split_hi(u32 q, u32 sc) {
  const u32 pe = (q & 0x00FF00FFu) * sc, po = ((q >> 8) & 0x00FF00FFu) * sc;
  return pack_even_odd((pe >> 5) & 0x001F001Fu, (po >> 5) & 0x001F001Fu);
}

DQ_DEV void lds_st16(uint8_t* lds, int off, v4u v) { *reinterpret_cast<v4u*>(lds + off) = v; }
DQ_DEV v4u lds_ld16(const uint8_t* lds, int off) { return *reinterpret_cast<const v4u*>(lds + off); }

}  // namespace

__global__ __launch_bounds__(kThreads) void k_gemm_q4k(const uint8_t* __restrict__ qs_plane,
                                                       const uint8_t* __restrict__ hdr_plane, int nb, int64_t n_pad,
                                                       int64_t nt0, int64_t n0, int64_t n1,
                                                       const uint8_t* __restrict__ acts, int64_t arb, int64_t m,
                                                       float* __restrict__ y, int64_t ys,
                                                       const float* __restrict__ bias) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int64_t nbase = nt0 + (int64_t)blockIdx.x * kBN;  // first weight row of the tile (multiple of 8)
  const int64_t mbase = (int64_t)blockIdx.y * kBM;
  const int64_t mrows = m - mbase < kBM ? m - mbase : kBM;

  // ---- global sources
  const auto ra = rsrc(acts + mbase * arb, (u32)(mrows * arb));
  const int bn = t >> 2, bs = t & 3;  // B staging: weight row nbase + bn, K-step bs
  const int64_t wn = nbase + bn;
  const bool wn_ok = wn < n_pad;
  const int64_t G = wn_ok ? wn / kRowGroup : 0, r8 = wn % kRowGroup;
  const auto rq = rsrc(qs_plane + G * nb * 1024, wn_ok ? (u32)(nb * 1024) : 0u);
  const auto rh = rsrc(hdr_plane + G * nb * 128, wn_ok ? (u32)(nb * 128) : 0u);

  // ---- prefetch registers for one super-block
  v4u ga[16];
  u32 gda;
  v4u gq0, gq1, ghd;
  auto prefetch = [&](int b) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = (t >> 4) + 16 * i, col = t & 15;
      ga[i] = ld16(ra, (u32)(row * arb + (int64_t)b * 292 + 4 + 16 * col));
    }
    gda = ld4(ra, (u32)(t * arb + (int64_t)b * 292));
    const u32 o = (u32)((b * 8 + r8) * 128 + 32 * bs);
    gq0 = ld16(rq, o);
    gq1 = ld16(rq, o + 16);
    ghd = ld16(rh, (u32)((b * 8 + r8) * 16));
  };

  v4i_t acc[kPlanes][4][4];
  float accf[4][4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
#pragma unroll
      for (int p = 0; p < kPlanes; ++p) acc[p][mt][nt] = v4i_t{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; ++e) accf[mt][nt][e] = 0.0f;
    }

  prefetch(0);
  for (int b = 0; b < nb; ++b) {
    __syncthreads();  // the previous super-block's LDS reads are done
    // ---- stage activations
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = (t >> 4) + 16 * i, col = t & 15;
      lds_st16(lds, kLdsA + (((col >> 2) * kBM + row) * 64 + 16 * (col & 3)), ga[i]);
    }
    reinterpret_cast<float*>(lds + kLdsDA)[t] = as_f(gda);
    // ---- dequantize the weight tile: row bn, K-step bs
    {
      int sca, mna, scb, mnb;
      scale_min_k4(2 * bs, ghd.y, ghd.z, ghd.w, sca, mna);
      scale_min_k4(2 * bs + 1, ghd.y, ghd.z, ghd.w, scb, mnb);
      if (bs == 0) {
        float* dw = reinterpret_cast<float*>(lds + kLdsDW);
        dw[2 * bn] = h2f(ghd.x);
        dw[2 * bn + 1] = h2f(ghd.x >> 16);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const v4u raw = (g & 1) ? gq1 : gq0;
        const v4u q = g < 2 ? (raw & 0x0F0F0F0Fu) : ((raw >> 4) & 0x0F0F0F0Fu);
        const u32 sc = (u32)(g < 2 ? sca : scb);
        const u32 mn = (u32)(g < 2 ? mna : mnb) * 0x01010101u;
        const v4u H = {split_hi(q.x, sc), split_hi(q.y, sc), split_hi(q.z, sc), split_hi(q.w, sc)};
        const v4u L = {split_lo(q.x, sc), split_lo(q.y, sc), split_lo(q.z, sc), split_lo(q.w, sc)};
        const v4u M = {mn, mn, mn, mn};
        lds_st16(lds, kLdsB + (((bs * kPlanes + 0) * kBN + bn) * 64 + 16 * g), H);
        lds_st16(lds, kLdsB + (((bs * kPlanes + 1) * kBN + bn) * 64 + 16 * g), L);
        lds_st16(lds, kLdsB + (((bs * kPlanes + 2) * kBN + bn) * 64 + 16 * g), M);
      }
    }
    __syncthreads();
    if (b + 1 < nb) prefetch(b + 1);

    // ---- MFMA phase: 4 K-steps of 64
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      v4u a[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        a[mt] = lds_ld16(lds, kLdsA + ((s * kBM + 64 * wave + 16 * mt + li) * 64 + 16 * lg));
      }
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
#pragma unroll
        for (int p = 0; p < kPlanes; ++p) {
          const v4u bf = lds_ld16(lds, kLdsB + (((s * kPlanes + p) * kBN + 16 * nt + li) * 64 + 16 * lg));
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) acc[p][mt][nt] = mfma(a[mt], bf, acc[p][mt][nt]);
        }
      }
    }

    // ---- epilogue of this super-block: exact S, Mn -> fp32
    const float* dw = reinterpret_cast<const float*>(lds + kLdsDW);
    const float* da = reinterpret_cast<const float*>(lds + kLdsDA);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const float d = dw[2 * (16 * nt + li)], dmin = dw[2 * (16 * nt + li) + 1];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int S = acc[1][mt][nt][e] + (acc[0][mt][nt][e] << 5);
          const int Mn = acc[2][mt][nt][e];
          float u = d * (float)S;
          u = fmaf(-dmin, (float)Mn, u);
          accf[mt][nt][e] = fmaf(da[64 * wave + 16 * mt + 4 * lg + e], u, accf[mt][nt][e]);
        }
#pragma unroll
        for (int p = 0; p < kPlanes; ++p) acc[p][mt][nt] = v4i_t{0, 0, 0, 0};
      }
    }
  }

  // ---- store
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int64_t n = nbase + 16 * nt + li;
    if (n < n0 || n >= n1) continue;
    const float bn_ = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t mm = mbase + 64 * wave + 16 * mt + 4 * lg + e;
        if (mm < m) y[mm * ys + n] = bias ? accf[mt][nt][e] + bn_ : accf[mt][nt][e];
      }
    }
  }
}

bool gemm_supported(int dtype, int af) { return dtype == kQ4_K && af == kActQ8_K; }

hipError_t launch_gemm(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0, int64_t n1,
                       float* y, int64_t ys, const float* bias, hipStream_t s) {
  if (!gemm_supported(w.dtype, af)) return hipErrorInvalidValue;
  if (m == 0 || n1 <= n0) return hipSuccess;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm_q4k),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int64_t nt0 = (n0 / kRowGroup) * kRowGroup;
  const int64_t ntiles = (n1 - nt0 + kBN - 1) / kBN;
  const int64_t mtiles = (m + kBM - 1) / kBM;
  hipLaunchKernelGGL(k_gemm_q4k, dim3((unsigned)ntiles, (unsigned)mtiles), dim3(kThreads), kLdsBytes, s, w.plane[0],
                     w.plane[1], (int)w.nblk, w.n_pad, nt0, n0, n1, acts, arb, m, y, ys, bias);
  return hipGetLastError();
}

}  // namespace dq
