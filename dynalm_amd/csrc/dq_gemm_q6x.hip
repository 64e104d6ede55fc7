// dq_gemm_q6x.hip -- prefill GEMM for Q6_K weights x per-32 activations (qmm's int8
// contract) and x int16 activations (ActBlockQ16, qmm's int16 mode) on the f16 matrix
// cores. The FFN down projection of a Q4_K_M model is Q6_K, and under the engine's plan
// its prefill takes these contracts.
//
// Arithmetic. Per 32-value block j the contract sums
//   acc += d da_j sum_u sc_u sum_t (q_t - 32) a_t       (qmm_reference.cpp:68-93 with
// Fmt<kQ6_K>, qmm_unpack.h; the int16 row kernel, kernels_avx2.cpp:1661-1765), u the two
// 16-value units of the block, sc_u their int8 scales (quant_formats.cpp:192-216). The
// effective weight w = sc_u (q - 32) lies in [-4064, 4096]: too wide for f16, so it
// splits exactly as w = 64 wh + wl, wh = floor(w / 64) in [-64, 64], wl in [0, 63], and
// both 64 wh and wl are f16 integers. They are the A operand of two v_mfma_f32_32x32x16_f16 per K-step
// into one accumulator, the activation codes the B operand (per-32: the int8 codes;
// int16: lo and 256 hi, two more MFMAs): every product is exact, and a block's sum
// |sum w a| <= 32 * 4096 * 127 < 2^24 is exact (int16: rounded to fp32 where the running
// sum passes 2^24). Then, as the per-32 GEMM (dq_gemm_p32.hip) does,
//   per block:        T = fma(da_j, S_j, T)
//   per super-block:  acc = fma(d, T, acc)
// The order is not the reference's: the outputs agree within the fp32 tolerance of a
// K-term dot product, not bit for bit.
//
// Work split. A workgroup owns 64 activation rows x 128 weight rows with 4 waves; wave w
// owns weight rows 32 w .. 32 w + 31 (lane l builds row l % 32's operands for lane half
// hh = l / 32 from the Q6_K planes it loads itself) against the two 32-row activation
// tiles. 256 workgroups at config 3's down shape (M = 512, N = 4096). A super-block's
// activation operands (32 KB per-32, 64 KB int16) and scales (2 KB) go to LDS one interval
// ahead by direct-to-LDS loads spread over the K-steps, into a ring of two.
//
// Activation layouts: per-32 rows as "act32" (k_act32_from_p32, dq_gemm_p32.hip), int16
// rows as "act16i" (k_act16i_from_q16, dq_gemm_q16.hip), both with the K order in which
// K-step k = 2 j + h of lane half hh holds values 32 j + 16 hh + 8 h + {0, 2, 1, 3, 4, 6,
// 5, 7}; the weight operand is built in that order. Values 32 j + 16 hh + 8 h + t of a
// super-block are, in its half n = j / 4 and quarter qd = j % 4, ql byte n 64 + 32 (qd & 1)
// + 16 hh + 8 h + t (the low nibble for qd < 2, else the high one: ql chunk 4 n + 2 (qd & 1)
// + hh, dwords 2 h, 2 h + 1) with qh bits 2 qd, 2 qd + 1 of qh byte n 32 + 16 hh + 8 h + t
// (qh chunk 2 n + hh), scale sc of unit 2 j + hh.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dq_device.h"
#include "dq_f16mma.h"
#include "dq_internal.h"
#include "dq_mfma.h"

namespace dq {

namespace {

constexpr int kXM = 64, kXN = 128;  // activation rows x weight rows per workgroup
constexpr int kXThreads = 256;      // 4 waves, one per SIMD

// Super-block buffer: activation operands [k (16)][t (2)][p (planes)][lane (64)][16 B],
// then the activation scales [t (2)][j (8)][row (32)].
template <bool kI16>
struct XLds {
  static constexpr int kPlanes = kI16 ? 2 : 1;
  static constexpr int kCodes = 16 * 2 * kPlanes * 1024;
  static constexpr int kDa = kCodes;
  static constexpr int kBuf = kDa + 2048;
  static constexpr int kTotal = 2 * kBuf;
};
static_assert(XLds<true>::kTotal <= 160 * 1024, "LDS");

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef short s2_t __attribute__((ext_vector_type(2)));

// Two codes q (bytes 0 and 2 of the dword p, or 1 and 3) of one unit with scale sc as the
// f16 pairs (64 wh, wl) of w = sc (q - 32) = 64 wh + wl.
DQ_DEV void q6_pair_f16(u32 p, int sc, u32& hi, u32& lo) {
  const s2_t q = __builtin_bit_cast(s2_t, p);
  const s2_t k = {(short)sc, (short)sc}, c = {(short)(-32 * sc), (short)(-32 * sc)};
  const s2_t w = q * k + c;
  const s2_t wh = (w >> (short)6) + (short)64;  // 0 .. 128
  const s2_t m63 = {63, 63};
  const s2_t wl = w & m63;
  // an integer v < 1024 in the mantissa of 1024's f16 (bits 0x6400 | v) is 1024 + v exactly
  const h2_t fl = __builtin_bit_cast(h2_t, __builtin_bit_cast(u32, wl) | 0x64006400u) - h2_t{1024.0f16, 1024.0f16};
  const h2_t fh = (__builtin_bit_cast(h2_t, __builtin_bit_cast(u32, wh) | 0x64006400u) - h2_t{1088.0f16, 1088.0f16}) *
                  h2_t{64.0f16, 64.0f16};
  lo = __builtin_bit_cast(u32, fl);
  hi = __builtin_bit_cast(u32, fh);
}

}  // namespace

// One workgroup: activation rows [64 tm, + 64) x weight rows [nbase0 + 128 tn, + 128), all
// super-blocks. Arguments as launch_gemm_q6x.
template <bool kI16>
__global__ __launch_bounds__(kXThreads) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_gemm_q6k_x(
    const uint8_t* __restrict__ ql_plane, const uint8_t* __restrict__ qh_plane, const uint8_t* __restrict__ sc_plane,
    const uint8_t* __restrict__ d_plane, int nb, int64_t nbase0, int64_t n_pad, int64_t n0, int64_t n1,
    const uint8_t* __restrict__ act, int64_t m_pad, int64_t m, float* __restrict__ y, int64_t ys,
    const float* __restrict__ bias, int tiles_m) {
  using X = XLds<kI16>;
  extern __shared__ __align__(16) uint8_t lds[];
  const int t = threadIdx.x, lane = t & 63;
  const int li = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int L = blockIdx.x;
  const int tn = __builtin_amdgcn_readfirstlane(L / tiles_m), tm = __builtin_amdgcn_readfirstlane(L - (L / tiles_m) * tiles_m);
  const int64_t nbase = nbase0 + (int64_t)kXN * tn;
  const int64_t mbase = (int64_t)tm * kXM;

  // activation layout: codes (bytes per 32-row tile and super-block: 16 K-steps x planes x
  // 1 KB), then da, (then c, unused here)
  const int64_t codes_bytes = m_pad * nb * 512 * X::kPlanes, da_bytes = m_pad / 32 * nb * 1024;
  const auto ra = rsrc(act, (u32)(codes_bytes + da_bytes));
  const auto rl = rsrc(ql_plane, (u32)(n_pad * nb * 128));
  const auto rhq = rsrc(qh_plane, (u32)(n_pad * nb * 64));
  const auto rs = rsrc(sc_plane, (u32)(n_pad * nb * 16));
  const auto rd = rsrc(d_plane, (u32)(n_pad * nb * 2));

  // ---- this wave's loads. Operands of super-block s: blocks jb = 8 wave + i (i < 8, and
  // 16 per wave with two planes) of the buffer; with piece 0 the activation scales of tile
  // wave (waves 0, 1). The wave's weight row: group g0 + wave / 2, row 32 (wave & 1) + li.
  const u32 g0 = (u32)(nbase >> 6);
  const u32 G = g0 + (u32)(wave >> 1), r64 = (u32)(32 * (wave & 1) + li);
  constexpr int kPieces = 8 * X::kPlanes;  // 1 KB pieces per wave and super-block
  auto issue_piece = [&](int s, int i) {
    uint8_t* P = lds + (s & 1) * X::kBuf;
    const int jb = kPieces * wave + i;  // = (k * 2 + tt) * planes + p
    const int p = kI16 ? (jb & 1) : 0, kt = kI16 ? (jb >> 1) : jb;
    const int64_t T = 2 * (int64_t)tm + (kt & 1);
    const int k = kt >> 1;
    dma16(ra, P + jb * 1024, (u32)(lane * 16), (u32)((((T * nb + s) * 16 + k) * X::kPlanes + p) * 1024));
    if (i == 0 && wave < 2) {
      const int64_t Tb = 2 * (int64_t)tm + wave;
      dma16(ra, P + X::kDa + wave * 1024, (u32)(lane * 16), (u32)(codes_bytes + (Tb * nb + s) * 1024));
    }
  };
  // the weight row's planes of super-block s (past the end: the last one again)
  struct W6 {
    v4u ql[4], qh[2], sc;
    u32 d;
  };
  auto ld_w = [&](int s, W6& w) {
    const u32 b = (u32)(s < nb ? s : nb - 1);
    const u32 gb = G * (u32)nb + b;
#pragma unroll
    for (int i = 0; i < 4; ++i) w.ql[i] = ld16(rl, ((gb * 8u + 2u * (u32)i + (u32)hh) * 64u + r64) * 16u);
#pragma unroll
    for (int i = 0; i < 2; ++i) w.qh[i] = ld16(rhq, ((gb * 4u + 2u * (u32)i + (u32)hh) * 64u + r64) * 16u);
    w.sc = ld16(rs, (gb * 64u + r64) * 16u);
    w.d = ld2(rd, (gb * 64u + r64) * 2u);
  };

  v16f_t acc[2], S[2], T[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    acc[mt] = v16f_t{};
    S[mt] = v16f_t{};
  }
  W6 cur, nxt;

  auto run_sb = [&](int s) {
    const bool next = s + 1 < nb;
    ld_w(s + 1, nxt);
    const uint8_t* P = lds + __builtin_amdgcn_readfirstlane((s & 1) * X::kBuf);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) T[tt] = v16f_t{};
    // the A operands (64 wh, wl) of K-step k = 2 j + h for this lane's row
    auto build = [&](int k, v4u& ah, v4u& al) {
      const int j = k >> 1, h = k & 1, n = j >> 2, qd = j & 3;
      // scale of unit 2 j + hh: byte 2 (j & 1) + hh of dword j / 2
      const int sc = (int)(int8_t)((u32)cur.sc[j >> 1] >> (8 * (2 * (j & 1) + hh)));
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        u32 x = cur.ql[2 * n + (qd & 1)][2 * h + e], yq = cur.qh[n][2 * h + e];
        asm volatile("" : "+v"(x), "+v"(yq));  // keeps this K-step's operand build here
        const u32 q = ((qd < 2 ? x : x >> 4) & 0x0F0F0F0Fu) | (((yq >> (2 * qd)) & 0x03030303u) << 4);
        u32 h0, l0, h1, l1;
        q6_pair_f16(__builtin_amdgcn_perm(0u, q, 0x0C020C00u), sc, h0, l0);  // values 4 e + 0, + 2
        q6_pair_f16(__builtin_amdgcn_perm(0u, q, 0x0C030C01u), sc, h1, l1);  // values 4 e + 1, + 3
        ah[2 * e] = h0;
        ah[2 * e + 1] = h1;
        al[2 * e] = l0;
        al[2 * e + 1] = l1;
      }
    };
    auto ld_da = [&](int tt, int j) { return as_f(lds4v(P + X::kDa + ((tt * 8 + j) * 32 + li) * 4)); };
    float da[2];
    v4u ah, al;
    build(0, ah, al);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      __builtin_amdgcn_s_setprio(2);
      if ((k & 1) == 0) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) da[tt] = ld_da(tt, k >> 1);
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
        for (int p = 0; p < X::kPlanes; ++p) {
          const v4u a = lds16(P + (((2 * k + tt) * X::kPlanes + p) * 64 + lane) * 16);
          S[tt] = mfma_h(ah, a, (k & 1) == 0 && p == 0 ? v16f_t{} : S[tt]);
          S[tt] = mfma_h(al, a, S[tt]);
        }
      }
      if (k < 15) build(k + 1, ah, al);
      if (next) {
        // the next super-block's pieces, spread over the K-steps
        if (kPieces == 8 ? (k & 1) == 0 : true) issue_piece(s + 1, kPieces == 8 ? (k >> 1) : k);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (k & 1) {
        // block j = k / 2 done: T += da_j S_j over the two tiles
        __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
          for (int r = 0; r < 16; ++r) T[tt][r] = fmaf(da[tt], S[tt][r], T[tt][r]);
          asm volatile("" : "+v"(T[tt]));  // the block's results exist here, not after later MFMAs
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // acc += d T: d of the lane's 16 result rows 8 (r / 4) + 4 hh + r % 4, which lanes 0-31
    // hold (one weight row each)
    const float dself = h2f(cur.d);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int src = 8 * (r >> 2) + 4 * hh + (r & 3);
      const float dr = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * src, __builtin_bit_cast(int, dself)));
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) acc[tt][r] = fmaf(dr, T[tt][r], acc[tt][r]);
    }
  };

  // prologue: the first super-block's operands and weights
#pragma unroll
  for (int i = 0; i < kPieces; ++i) issue_piece(0, i);
  ld_w(0, cur);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  lds_barrier();
#pragma unroll 1
  for (int s = 0; s < nb; ++s) {
    run_sb(s);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    cur = nxt;
  }

  // ---- outputs (+ bias): activation row 32 mt + li, weight rows nbase + 32 wave +
  // 8 (r / 4) + 4 hh + r % 4
  const int64_t mrows = m - mbase < kXM ? m - mbase : kXM;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int row = 32 * mt + li;
    if (row >= mrows) continue;
    float* yr = y + (mbase + row) * ys;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t nq = nbase + 32 * wave + 8 * q + 4 * hh;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t n = nq + e;
        if (n >= n0 && n < n1) {
          const float v = acc[mt][4 * q + e];
          yr[n] = bias ? v + bias[n] : v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------- host

bool gemm_q6x_ok(const WeightDev& w, int af, int64_t m, int64_t n0, int64_t n1) {
  if (w.dtype != kQ6_K || (af != kActPer32 && af != kActQ16) || m <= 0 || n1 <= n0 || w.nblk <= 0) return false;
  // 32-bit buffer offsets: the ql plane plus one tile's rows past its end, and the layout
  if ((w.n_pad + 2 * kRowGroup) * w.nblk * 128 >= (1ll << 32)) return false;
  // the layout writers' grids have one row of workgroups per 32 padded rows
  const bool i16 = af == kActQ16;
  const int64_t bytes = i16 ? act16i_bytes(m, w.k) : act32_bytes(m, w.k);
  const int64_t rows = i16 ? act16i_rows(m) : act32_rows(m);
  if (bytes >= (1ll << 32) || rows / 32 > 65535) return false;
  // one workgroup per (64 activation rows, 128 weight rows)
  return (rows / kXM) * ((n1 - n0 / kRowGroup * kRowGroup + kXN - 1) / kXN) < (1ll << 31);
}

hipError_t launch_gemm_q6x(const WeightDev& w, int af, const uint8_t* act, int64_t m_pad, int64_t m, int64_t n0,
                           int64_t n1, float* y, int64_t ys, const float* bias, hipStream_t s) {
  if (!gemm_q6x_ok(w, af, m, n0, n1) || m_pad % kXM != 0 || m_pad < m) return hipErrorInvalidValue;
  const int64_t nbase0 = n0 / kRowGroup * kRowGroup;
  const int64_t tiles_n = (n1 - nbase0 + kXN - 1) / kXN;
  const int64_t tiles_m = (m + kXM - 1) / kXM;
  const bool i16 = af == kActQ16;
  const void* fn = i16 ? reinterpret_cast<const void*>(&k_gemm_q6k_x<true>)
                       : reinterpret_cast<const void*>(&k_gemm_q6k_x<false>);
  const int lds = i16 ? XLds<true>::kTotal : XLds<false>::kTotal;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  if (i16) {
    hipLaunchKernelGGL(k_gemm_q6k_x<true>, dim3((unsigned)(tiles_n * tiles_m)), dim3(kXThreads), lds, s, w.plane[0],
                       w.plane[1], w.plane[2], w.plane[3], (int)w.nblk, nbase0, w.n_pad, n0, n1, act, m_pad, m, y, ys,
                       bias, (int)tiles_m);
  } else {
    hipLaunchKernelGGL(k_gemm_q6k_x<false>, dim3((unsigned)(tiles_n * tiles_m)), dim3(kXThreads), lds, s, w.plane[0],
                       w.plane[1], w.plane[2], w.plane[3], (int)w.nblk, nbase0, w.n_pad, n0, n1, act, m_pad, m, y, ys,
                       bias, (int)tiles_m);
  }
  return hipGetLastError();
}

}  // namespace dq
