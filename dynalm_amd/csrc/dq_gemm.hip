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
// The effective integer weight sc*q (0..945) does not fit int8. With
// sc = 8*sh + sl (sh, sl in 0..7), sh*q and sl*q are at most 105, so each fits a
// byte and a packed 16-bit multiply of four nibble bytes by sh (or sl) makes four
// of them at once without carries. Three int8 MFMA accumulations per output give
//   S = 8 * sum(sh*q*a) + sum(sl*q*a)   and   Mn = sum(m_j * a)
// exactly in int32 (the third operand holds m_j at every position of sub-block j).
//
// Tiling: a workgroup of 8 waves (two per SIMD, so one wave's MFMAs overlap the
// other's dequantization and epilogue) computes 128 activation rows x 128 weight
// rows; wave (wm, wn) owns 64 activation rows x 32 weight rows (4 x 2 MFMA tiles
// of 16 x 16). Per super-block the activation codes (32 KB) and the weight
// nibbles as clean bytes (32 KB) are staged in LDS, double-buffered: while the
// waves multiply super-block b, the global loads of b + 2 are in flight and the
// registers holding b + 1 are written to the other buffer, with one barrier per
// super-block. 16-byte chunks are XOR-swizzled so that the MFMA operand reads hit
// distinct LDS banks.
//
// MFMA operand layout (16x16x64 i8): lane l supplies row (A) / column (B) l%16
// and 16 K-values of lane group l/16; the result lane l holds column l%16, rows
// 4*(l/16) .. 4*(l/16)+3. K-step s of a super-block covers values 64s .. 64s+63,
// lane group g the 16 values 64s + 16g .., which are values 16(g&1) .. of
// sub-block 2s + g/2 (dynacore/src/quantization/quant_formats.cpp:150-167).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "dq_device.h"
#include "dq_internal.h"
#include "dq_mfma.h"

namespace dq {

namespace {

constexpr int kBM = 128;       // activation rows per workgroup
constexpr int kBN = 128;       // weight rows per workgroup (two 64-row groups)
constexpr int kThreads = 512;  // 8 waves: 2 along M (64 rows each) x 4 along N (32 rows each)

// LDS layout (bytes). Operands of one super-block, two buffers:
constexpr int kLdsA = 0;                       // [4 K-steps][128 rows][4 chunks of 16 B] activation codes
constexpr int kLdsQ = kLdsA + 4 * kBM * 64;    // [128 rows][16 chunks of 16 B] nibbles as bytes, value order
constexpr int kBuf = kLdsQ + kBN * 256;        // 65536
// Scales of one super-block, a ring of three (the delayed epilogue reads b - 1
// while b + 1 is being written):
constexpr int kLdsH = 0;                       // [128 rows] Q4_K header {d, dmin, scales[12]}
constexpr int kLdsDA = kLdsH + kBN * 16;       // [128 rows] activation scale d (float)
constexpr int kRing = kLdsDA + kBM * 4;        // 2560
constexpr int kLdsBytes = 2 * kBuf + 3 * kRing;  // 138752

DQ_DEV void lds_st16(uint8_t* lds, int off, v4u v) { *reinterpret_cast<v4u*>(lds + off) = v; }
DQ_DEV v4u lds_ld16(const uint8_t* lds, int off) { return *reinterpret_cast<const v4u*>(lds + off); }

// Swizzled byte offsets of the 16-byte chunks.
DQ_DEV int a_off(int s, int row, int g) { return ((s * kBM + row) * 4 + (g ^ ((row >> 2) & 3))) * 16; }
DQ_DEV int q_off(int row, int k) { return (row * 16 + (k ^ (row & 15))) * 16; }

// Global loads of one super-block held in registers until they are written to LDS
// (the activation codes go to LDS directly).
struct Stage {
  v4u q[2];  // qs chunk (t >> 6) & 7 of row t & 63 of the tile's row group i
};

}  // namespace

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_q4k(
    const uint8_t* __restrict__ qs_plane, const uint8_t* __restrict__ hdr_plane, int nb, int64_t n_pad, int64_t nt0,
    int64_t n0, int64_t n1, const uint8_t* __restrict__ acts, int64_t arb, int64_t m, float* __restrict__ y, int64_t ys,
    const float* __restrict__ bias) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave & 1, wn = wave >> 1;  // this wave's 64 activation rows and 32 weight rows
  const int li = lane & 15, lg = lane >> 4;
  const int64_t nbase = nt0 + (int64_t)blockIdx.x * kBN;  // first weight row of the tile (multiple of 64)
  const int64_t mbase = (int64_t)blockIdx.y * kBM;
  const int64_t mrows = m - mbase < kBM ? m - mbase : kBM;

  // ---- global sources (buffer resources: reads past the end return zeros)
  const auto ra = rsrc(acts + mbase * arb, (u32)(mrows * arb));
  // the tile's two 64-row groups of the weight layout (dq_layout.h)
  const int64_t G0 = nbase / kRowGroup;
  const bool g0ok = nbase < n_pad, g1ok = nbase + kRowGroup < n_pad;
  const auto rq0 = rsrc(qs_plane + G0 * nb * 8192, g0ok ? (u32)(nb * 8192) : 0u);
  const auto rq1 = rsrc(qs_plane + (G0 + 1) * nb * 8192, g1ok ? (u32)(nb * 8192) : 0u);
  const auto rh0 = rsrc(hdr_plane + G0 * nb * 1024, g0ok ? (u32)(nb * 1024) : 0u);
  const auto rh1 = rsrc(hdr_plane + (G0 + 1) * nb * 1024, g1ok ? (u32)(nb * 1024) : 0u);

  // Activation codes straight to LDS: instruction i of wave w fills the 1 KB
  // [K-step s = i][rows 16 w .. 16 w + 15] of the buffer, lane l the 16-byte slot
  // l, which holds row 16 w + l / 4, chunk (l & 3) ^ ((row >> 2) & 3) (a_off).
  const int arow = 16 * wave + (lane >> 2);
  const int achunk = (lane & 3) ^ ((arow >> 2) & 3);
  auto load_a = [&](int b, auto par) {
    uint8_t* L = lds + decltype(par)::value * kBuf;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ra, (__attribute__((address_space(3))) void*)(L + kLdsA + (s * kBM + 16 * wave) * 64), 16,
          (u32)(arow * arb + (int64_t)b * 292 + 4 + 64 * s + 16 * achunk), 0, 0, 0);
    }
    // headers (waves 0, 1: one 64-row group each, 1 KB contiguous in the weight
    // layout) and activation scales (waves 2, 3: 64 rows each) into ring slot b % 3
    uint8_t* R = lds + 2 * kBuf + (b % 3) * kRing;
    if (wave < 2) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wave == 0 ? rh0 : rh1,
                                               (__attribute__((address_space(3))) void*)(R + kLdsH + 1024 * wave),
                                               16, (u32)((b * 64 + lane) * 16), 0, 0, 0);
    } else if (wave < 4) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ra, (__attribute__((address_space(3))) void*)(R + kLdsDA + 256 * (wave - 2)), 4,
          (u32)((64 * (wave - 2) + lane) * arb + (int64_t)b * 292), 0, 0, 0);
    }
  };
  // staging roles of thread t for the weight bytes
  const int qc = (t >> 6) & 7, qr = t & 63;  // qs chunk qc of row qr of row group i (i = 0, 1)
  Stage st;
  auto load = [&](int b) {
    st.q[0] = ld16(rq0, (u32)(((b * 8 + qc) * 64 + qr) * 16));
    st.q[1] = ld16(rq1, (u32)(((b * 8 + qc) * 64 + qr) * 16));
  };
  auto store = [&](int b, auto par) {
    uint8_t* L = lds + decltype(par)::value * kBuf;
    // qs chunk qc holds values 64(qc/2) + 16(qc&1) + i (low nibbles, sub-block qc & ~1)
    // and the same + 32 (high nibbles, stored XOR 8, dq_layout.h)
    const int klo = 4 * (qc >> 1) + (qc & 1);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = 64 * i + qr;
      lds_st16(L, kLdsQ + q_off(row, klo), st.q[i] & 0x0F0F0F0Fu);
      lds_st16(L, kLdsQ + q_off(row, klo + 2), ((st.q[i] >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u);
    }
  };

  v4i_t acc[3][4][2];  // [sh plane, sl plane, m plane][m tile][n tile]
  float accf[4][2][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
      for (int e = 0; e < 4; ++e) accf[mt][nt][e] = 0.0f;
    }

  // Epilogue of super-block b: exact S, Mn -> fp32 (canonical order).
  auto epilogue = [&](int b) {
    const uint8_t* R = lds + 2 * kBuf + (b % 3) * kRing;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const u32 h = *reinterpret_cast<const u32*>(R + kLdsH + 16 * (32 * wn + 16 * nt + li));
      const float d = h2f(h), dmin = h2f(h >> 16);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const v4u dav = lds_ld16(R, kLdsDA + 4 * (64 * wm + 16 * mt + 4 * lg));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int S = acc[1][mt][nt][e] + (acc[0][mt][nt][e] << 3);
          const int Mn = acc[2][mt][nt][e];
          float u = d * (float)S;
          u = fmaf(-dmin, (float)Mn, u);
          accf[mt][nt][e] = fmaf(as_f(dav[e]), u, accf[mt][nt][e]);
        }
      }
    }
  };

  // K-step s of the super-block in buffer L: 24 MFMAs; the first step starts the
  // accumulators from zero.
  const int hi = lg >> 1;  // this lane group's sub-blocks are 2s + hi
  u32 KH[2], KL[2], MN[2];  // per weight row: bytes s = sh, sl, m of sub-block 2s + hi
  auto kstep = [&](const uint8_t* L, int s, bool first) {
    v4u a[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) a[mt] = lds_ld16(L, kLdsA + a_off(s, 64 * wm + 16 * mt + li, lg));
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const v4u q = lds_ld16(L, kLdsQ + q_off(32 * wn + 16 * nt + li, 4 * s + lg));
      const u32 kh = __builtin_amdgcn_perm(0u, KH[nt], sel_u16x2(s));
      const u32 kl = __builtin_amdgcn_perm(0u, KL[nt], sel_u16x2(s));
      const u32 mm4 = __builtin_amdgcn_perm(0u, MN[nt], sel_x4(s));
      const v4u H = {mul_bytes(q.x, kh), mul_bytes(q.y, kh), mul_bytes(q.z, kh), mul_bytes(q.w, kh)};
      const v4u Lo = {mul_bytes(q.x, kl), mul_bytes(q.y, kl), mul_bytes(q.z, kl), mul_bytes(q.w, kl)};
      const v4u Mp = {mm4, mm4, mm4, mm4};
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const v4i_t z = {0, 0, 0, 0};
        acc[0][mt][nt] = mfma(a[mt], H, first ? z : acc[0][mt][nt]);
        acc[1][mt][nt] = mfma(a[mt], Lo, first ? z : acc[1][mt][nt]);
        acc[2][mt][nt] = mfma(a[mt], Mp, first ? z : acc[2][mt][nt]);
      }
    }
  };

  load_a(0, std::integral_constant<int, 0>{});
  load(0);
  store(0, std::integral_constant<int, 0>{});
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // Waves 4..7 (one per SIMD, beside one of waves 0..3) run each super-block's
  // epilogue at the start of the next one, so that on every SIMD one wave's
  // epilogue overlaps the other wave's MFMAs.
  // Waves 4..7 (one per SIMD, beside one of waves 0..3) run each super-block's
  // epilogue at the start of the next one, so that on every SIMD one wave's
  // epilogue overlaps the other wave's MFMAs.
  const bool late = wave >= 4;
  // One super-block; P = b & 1 is a compile-time constant so that every LDS
  // address is a per-lane base plus an immediate offset.
  auto iter = [&](int b, auto par) {
    constexpr int P = decltype(par)::value;
    const uint8_t* L = lds + P * kBuf;
    const uint8_t* R = lds + 2 * kBuf + (b % 3) * kRing;
    if (late && b > 0) epilogue(b - 1);
    // next super-block's loads: activation codes into the other LDS buffer, the
    // rest into registers (written at the end of this iteration)
    if (b + 1 < nb) {
      load_a(b + 1, std::integral_constant<int, 1 - P>{});
      load(b + 1);
    }

    // the scales and mins of this lane's two weight rows (get_scale_min_k4,
    // quant_formats.h:62-70) for its sub-blocks 2s + hi, as bytes s
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const v4u hd = lds_ld16(R, kLdsH + 16 * (32 * wn + 16 * nt + li));
      const u32 sc_lo = hd.y & 0x3F3F3F3Fu, mn_lo = hd.z & 0x3F3F3F3Fu;
      const u32 sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
      const u32 mn_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
      const u32 sc = __builtin_amdgcn_perm(sc_hi, sc_lo, sel_subblocks(hi));
      KH[nt] = (sc >> 3) & 0x07070707u;
      KL[nt] = sc & 0x07070707u;
      MN[nt] = __builtin_amdgcn_perm(mn_hi, mn_lo, sel_subblocks(hi));
    }

    kstep(L, 0, true);
#pragma unroll 1
    for (int s = 1; s < 4; ++s) kstep(L, s, false);
    if (!late) epilogue(b);

    // ---- stage super-block b + 1 (its activation codes are already on their way)
    if (b + 1 < nb) store(b + 1, std::integral_constant<int, 1 - P>{});
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };
  int b = 0;
  for (; b + 1 < nb; b += 2) {
    iter(b, std::integral_constant<int, 0>{});
    iter(b + 1, std::integral_constant<int, 1>{});
  }
  if (b < nb) iter(b, std::integral_constant<int, 0>{});
  if (late) epilogue(nb - 1);

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
