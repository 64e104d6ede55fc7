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
// Tiling: a workgroup of 8 waves (two per SIMD, so one wave's MFMAs overlap
// another's dequantization and epilogue) computes 256 activation rows x 64
// weight rows; wave w owns 64 activation rows x 32 weight rows (4 x 2 MFMA tiles
// of 16 x 16). Per
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
constexpr int kThreads = 512;  // 8 waves: 4 along M (64 rows each) x 2 along N (32 rows each)
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

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_q4k(
    const uint8_t* __restrict__ qs_plane, const uint8_t* __restrict__ hdr_plane, int nb, int64_t n_pad, int64_t nt0,
    int64_t n0, int64_t n1, const uint8_t* __restrict__ acts, int64_t arb, int64_t m, float* __restrict__ y, int64_t ys,
    const float* __restrict__ bias) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave & 3, wn = wave >> 2;  // this wave's 64 activation rows and 32 weight rows
  const int li = lane & 15, lg = lane >> 4;
  const int64_t nbase = nt0 + (int64_t)blockIdx.x * kBN;  // first weight row of the tile (multiple of 8)
  const int64_t mbase = (int64_t)blockIdx.y * kBM;
  const int64_t mrows = m - mbase < kBM ? m - mbase : kBM;

  // ---- global sources
  const auto ra = rsrc(acts + mbase * arb, (u32)(mrows * arb));
  // B staging: weight row nbase + bn, K-step bs, half hh (qs bytes 32bs + 16hh .. +16)
  const int bn = t >> 3, bs = (t >> 1) & 3, hh = t & 1;
  const int64_t wn_row = nbase + bn;
  const bool wn_ok = wn_row < n_pad;
  // 64-row layout (dq_layout.h): qs chunk c of row r, super-block b at ((b*8 + c)*64 + r)*16
  // of its row group; the header at (b*64 + r)*16.
  const int64_t G = wn_ok ? wn_row / kRowGroup : 0, rr = wn_row % kRowGroup;
  const auto rq = rsrc(qs_plane + G * nb * 8192, wn_ok ? (u32)(nb * 8192) : 0u);
  const auto rh = rsrc(hdr_plane + G * nb * 1024, wn_ok ? (u32)(nb * 1024) : 0u);

  // ---- prefetch registers for one super-block
  v4u ga[8];
  u32 gda;
  v4u gq, ghd;
  auto prefetch = [&](int b) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = (t >> 4) + 32 * i, col = t & 15;
      ga[i] = ld16(ra, (u32)(row * arb + (int64_t)b * 292 + 4 + 16 * col));
    }
    gda = ld4(ra, (u32)((t & 255) * arb + (int64_t)b * 292));
    gq = ld16(rq, (u32)(((b * 8 + 2 * bs + hh) * 64 + rr) * 16));
    ghd = ld16(rh, (u32)((b * 64 + rr) * 16));
  };

  v4i_t acc[kPlanes][4][2];
  float accf[4][2][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
      for (int p = 0; p < kPlanes; ++p) acc[p][mt][nt] = v4i_t{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; ++e) accf[mt][nt][e] = 0.0f;
    }

  prefetch(0);
  for (int b = 0; b < nb; ++b) {
    __syncthreads();  // the previous super-block's LDS reads are done
    // ---- stage activations (values 64s .. 64s+63 of row `row` at [s][row])
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = (t >> 4) + 32 * i, col = t & 15;
      lds_st16(lds, kLdsA + (((col >> 2) * kBM + row) * 64 + 16 * (col & 3)), ga[i]);
    }
    if (t < kBM) reinterpret_cast<float*>(lds + kLdsDA)[t] = as_f(gda);
    // ---- dequantize: low nibbles -> lane group hh (sub-block 2bs), high -> 2 + hh (2bs+1)
    {
      int sca, mna, scb, mnb;
      scale_min_k4(2 * bs, ghd.y, ghd.z, ghd.w, sca, mna);
      scale_min_k4(2 * bs + 1, ghd.y, ghd.z, ghd.w, scb, mnb);
      if (bs == 0 && hh == 0) {
        float* dw = reinterpret_cast<float*>(lds + kLdsDW);
        dw[2 * bn] = h2f(ghd.x);
        dw[2 * bn + 1] = h2f(ghd.x >> 16);
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        // high nibbles are stored XOR 8 (dq_layout.h)
        const v4u q = half == 0 ? (gq & 0x0F0F0F0Fu) : (((gq >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u);
        const int g = 2 * half + hh;
        const u32 sc = (u32)(half == 0 ? sca : scb);
        const u32 mn = (u32)(half == 0 ? mna : mnb) * 0x01010101u;
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

    // ---- MFMA phase: 4 K-steps of 64 (not unrolled: keeps one step's fragments live)
#pragma unroll 1
    for (int s = 0; s < 4; ++s) {
      v4u a[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        a[mt] = lds_ld16(lds, kLdsA + ((s * kBM + 64 * wm + 16 * mt + li) * 64 + 16 * lg));
      }
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
        for (int p = 0; p < kPlanes; ++p) {
          const v4u bf = lds_ld16(lds, kLdsB + (((s * kPlanes + p) * kBN + 32 * wn + 16 * nt + li) * 64 + 16 * lg));
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) acc[p][mt][nt] = mfma(a[mt], bf, acc[p][mt][nt]);
        }
      }
    }

    // ---- epilogue of this super-block: exact S, Mn -> fp32 (canonical order)
    const float* dw = reinterpret_cast<const float*>(lds + kLdsDW);
    const float* da = reinterpret_cast<const float*>(lds + kLdsDA);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int nl = 32 * wn + 16 * nt + li;
      const float d = dw[2 * nl], dmin = dw[2 * nl + 1];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int S = acc[1][mt][nt][e] + (acc[0][mt][nt][e] << 5);
          const int Mn = acc[2][mt][nt][e];
          float u = d * (float)S;
          u = fmaf(-dmin, (float)Mn, u);
          accf[mt][nt][e] = fmaf(da[64 * wm + 16 * mt + 4 * lg + e], u, accf[mt][nt][e]);
        }
#pragma unroll
        for (int p = 0; p < kPlanes; ++p) acc[p][mt][nt] = v4i_t{0, 0, 0, 0};
      }
    }
  }

  // ---- store
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int64_t n = nbase + 32 * wn + 16 * nt + li;
    if (n < n0 || n >= n1) continue;
    const float bn_ = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t mm = mbase + 64 * wm + 16 * mt + 4 * lg + e;
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
