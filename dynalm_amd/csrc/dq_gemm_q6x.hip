// dq_gemm_q6x.hip -- prefill GEMM for Q6_K weights x per-32 activations (qmm's int8
// contract) and x int16 activations (ActBlockQ16, qmm's int16 mode) on the f16 matrix
// cores. The FFN down projection of a Q4_K_M model is Q6_K, and under the engine's plan
// its prefill takes these contracts.
//
// Arithmetic. Per 32-value block j the contract sums
//   acc += d da_j sum_u sc_u sum_t (q_t - 32) a_t       (qmm_reference.cpp:68-93 with
// Fmt<kQ6_K>, qmm_unpack.h; the int16 row kernel, kernels_avx2.cpp:1661-1765), u the two
// 16-value units of the block, sc_u their int8 scales (quant_formats.cpp:192-216). The
// effective weight w = sc_u (q - 32) lies in [-4064, 4096]: too wide for f16, so the
// scale splits as sc = fh + fl, fh = 16 (sc >> 4) in [-128, 112], fl = sc & 15, and
// w = fh (q - 32) + fl (q - 32), two f16 integers (at most 4096 = 16 * 8 * 32 and 480 in
// magnitude). Each is built, scaled by 2^-24, by one packed fma from q as raw f16 bits
// (the subnormal q 2^-24): fma(q 2^-24, f, -32 f 2^-24), exact because its result is
// representable. They are the A operand of two v_mfma_f32_32x32x16_f16 per K-step into
// one accumulator, the activation codes the B operand (per-32: the int8 codes; int16: lo
// and 256 hi, two more MFMAs): every product is exact, and a block's sum
// |sum w a| <= 32 * 4096 * 127 < 2^24 (in units of 2^-24) is exact (int16: rounded to fp32
// where the running sum passes 2^24). Then, as the per-32 GEMM (dq_gemm_p32.hip) does,
//   per block:        T = fma(da_j, S_j, T)
//   per super-block:  acc = fma(d 2^24, T, acc)
// The order is not the reference's: the outputs agree within the fp32 tolerance of a
// K-term dot product, not bit for bit.
//
// Work split. A workgroup owns 64 activation rows x 128 weight rows with 4 waves; wave w
// owns weight rows 32 w .. 32 w + 31 (lane l builds row l % 32's operands for lane half
// hh = l / 32 from the Q6_K planes it loads itself) against the two 32-row activation
// tiles. 256 workgroups at config 3's down shape (M = 512, N = 4096): one wave per SIMD,
// so a wave overlaps its own work. Per block, tile 0's MFMA chain runs beside the fold of
// tile 1's previous block and half of the next block's operand build, then tile 1's
// chain beside the fold of tile 0's block and the other half. A super-block's activation
// operands (32 KB per-32, 64 KB int16) and scales (2 KB) go to LDS one interval ahead by
// direct-to-LDS loads spread over the blocks, into a ring of two; each weight plane chunk
// is reloaded for the next super-block right after its last read. Each CU streams ~3.3 MB
// (per-32) or ~5.2 MB (int16) at M = 512, N = 4096, K = 14336, so the per-CU read rate
// (~22 KB/us) bounds the kernel near 150 (235) us.
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

}  // namespace

// One workgroup: activation rows [64 tm, + 64) x weight rows [nbase0 + 128 tn, + 128), all
// super-blocks. Arguments as launch_gemm_q6x.
template <bool kI16>
__global__ __launch_bounds__(kXThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_q6k_x(
    const uint8_t* __restrict__ ql_plane, const uint8_t* __restrict__ qh_plane, const uint8_t* __restrict__ sc_plane,
    const uint8_t* __restrict__ d_plane, int nb, int64_t nbase0, int64_t n_pad, int64_t n0, int64_t n1,
    const uint8_t* __restrict__ act, int64_t m_pad, int64_t m, float* __restrict__ y, int64_t ys,
    const float* __restrict__ bias, int tiles_m) {
  using X = XLds<kI16>;
  constexpr int kP = X::kPlanes;
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
  const int64_t codes_bytes = m_pad * nb * 512 * kP, da_bytes = m_pad / 32 * nb * 1024;
  const auto ra = rsrc(act, (u32)(codes_bytes + da_bytes));
  const auto rl = rsrc(ql_plane, (u32)(n_pad * nb * 128));
  const auto rhq = rsrc(qh_plane, (u32)(n_pad * nb * 64));
  const auto rs = rsrc(sc_plane, (u32)(n_pad * nb * 16));
  const auto rd = rsrc(d_plane, (u32)(n_pad * nb * 2));

  // ---- this wave's loads. Operands of super-block s: blocks jb = 8 P wave + i (i < 8 P)
  // of the buffer; with piece 0 the activation scales of tile wave (waves 0, 1). The wave's
  // weight row: group g0 + wave / 2, row 32 (wave & 1) + li.
  const u32 g0 = (u32)(nbase >> 6);
  const u32 G = g0 + (u32)(wave >> 1), r64 = (u32)(32 * (wave & 1) + li);
  constexpr int kPieces = 8 * kP;  // 1 KB pieces per wave and super-block
  auto issue_piece = [&](int s, int i) {
    uint8_t* P = lds + (s & 1) * X::kBuf;
    const int jb = kPieces * wave + i;  // = (k * 2 + tt) * planes + p
    const int p = kI16 ? (jb & 1) : 0, kt = kI16 ? (jb >> 1) : jb;
    const int64_t T = 2 * (int64_t)tm + (kt & 1);
    const int k = kt >> 1;
    dma16(ra, P + jb * 1024, (u32)(lane * 16), (u32)((((T * nb + s) * 16 + k) * kP + p) * 1024));
    if (i == 0 && wave < 2) {
      const int64_t Tb = 2 * (int64_t)tm + wave;
      dma16(ra, P + X::kDa + wave * 1024, (u32)(lane * 16), (u32)(codes_bytes + (Tb * nb + s) * 1024));
    }
  };
  // The weight row's planes of super-block s (past the end: the last one again), one
  // register set: each chunk is reloaded with the next super-block's right after the
  // operand build that last reads it (ql chunks 0, 1 and qh chunk 0 after block 2's
  // build, the rest after block 6's); the scales and d of the next super-block go to
  // sc_n / d_n at the start of a super-block.
  struct W6 {
    v4u ql[4], qh[2], sc;
    u32 d;
  };
  auto wofs = [&](int s) -> u32 { return G * (u32)nb + (u32)(s < nb ? s : nb - 1); };
  auto ld_ql = [&](int s, int i) { return ld16(rl, ((wofs(s) * 8u + 2u * (u32)i + (u32)hh) * 64u + r64) * 16u); };
  auto ld_qh = [&](int s, int i) { return ld16(rhq, ((wofs(s) * 4u + 2u * (u32)i + (u32)hh) * 64u + r64) * 16u); };
  auto ld_sc = [&](int s) { return ld16(rs, (wofs(s) * 64u + r64) * 16u); };
  auto ld_d = [&](int s) { return ld2(rd, (wofs(s) * 64u + r64) * 2u); };
  // The A operands of block j (K-steps 2 j + h, h = 0, 1) for this lane's row and unit
  // u = 2 j + hh: w = sc (q - 32) = a_hi + a_lo with a_hi = fh (q - 32), a_lo = fl (q - 32),
  // fh = 16 (sc >> 4) in [-128, 112], fl = sc & 15, each scaled by 2^-24 and built by one
  // exact packed fma from q 2^-24 (q as raw f16 bits): fma(q 2^-24, f, -32 f 2^-24).
  struct Unit {
    h2_t fh, ch, fl, cl;
  };
  auto unit = [&](const v4u& scv, int j) -> Unit {
    const int sc = (int)(int8_t)((u32)scv[j >> 1] >> (8 * (2 * (j & 1) + hh)));
    const _Float16 fh = (_Float16)(short)(sc & -16), fl = (_Float16)(short)(sc & 15);
    constexpr _Float16 kC = (_Float16)-0x1p-19f;  // -32 * 2^-24
    Unit u;
    u.fh = h2_t{fh, fh};
    u.fl = h2_t{fl, fl};
    u.ch = u.fh * h2_t{kC, kC};
    u.cl = u.fl * h2_t{kC, kC};
    return u;
  };
  // K-step 2 j + h's operands (a_hi, a_lo)
  auto build = [&](const W6& w, const Unit& u, int j, int h, v4u& hi, v4u& lo) {
    const int n = j >> 2, qd = j & 3;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      u32 x = w.ql[2 * n + (qd & 1)][2 * h + e], yq = w.qh[n][2 * h + e];
      asm volatile("" : "+v"(x), "+v"(yq));  // keeps this operand build here
      const u32 q = ((qd < 2 ? x : x >> 4) & 0x0F0F0F0Fu) | (((yq >> (2 * qd)) & 0x03030303u) << 4);
      const h2_t q02 = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0u, q, 0x0C020C00u));  // values 4 e + 0, + 2
      const h2_t q13 = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0u, q, 0x0C030C01u));  // values 4 e + 1, + 3
      hi[2 * e] = __builtin_bit_cast(u32, __builtin_elementwise_fma(q02, u.fh, u.ch));
      hi[2 * e + 1] = __builtin_bit_cast(u32, __builtin_elementwise_fma(q13, u.fh, u.ch));
      lo[2 * e] = __builtin_bit_cast(u32, __builtin_elementwise_fma(q02, u.fl, u.cl));
      lo[2 * e + 1] = __builtin_bit_cast(u32, __builtin_elementwise_fma(q13, u.fl, u.cl));
    }
  };

  v16f_t acc[2], S[2], T[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    acc[mt] = v16f_t{};
    T[mt] = v16f_t{};
  }
  W6 w;
  v4u sc_n;
  u32 d_n;
  v4u Ah[2], Al[2], Nh[2], Nl[2];  // this block's and the next block's operands (K-steps 2 j, 2 j + 1)

  // Super-block s, per block j in two phases: tile 0's MFMA chain (both K-steps, every
  // plane, a_hi then a_lo) beside the fold of tile 1's previous block and half the next
  // block's operand build; then tile 1's chain beside the fold of tile 0's block j and the
  // other half. Each accumulator is folded while the other tile's MFMAs run, then
  // restarted from zero.
  auto run_sb = [&](int s) {
    const bool next = s + 1 < nb;
    sc_n = ld_sc(s + 1);
    d_n = ld_d(s + 1);
    const uint8_t* P = lds + __builtin_amdgcn_readfirstlane((s & 1) * X::kBuf);
    auto ld_da = [&](int tt, int j) { return as_f(lds4v(P + X::kDa + ((tt * 8 + j) * 32 + li) * 4)); };
    auto chain = [&](int tt, int j) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int p = 0; p < kP; ++p) {
          const v4u b = lds16(P + (((2 * (2 * j + h) + tt) * kP + p) * 64 + lane) * 16);
          S[tt] = mfma_h(Ah[h], b, h == 0 && p == 0 ? v16f_t{} : S[tt]);
          S[tt] = mfma_h(Al[h], b, S[tt]);
        }
      }
    };
    // per phase: the LDS reads, then each MFMA followed by a share of the VALU work
    auto interleave = [&]() {
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * kP + 1, 0);  // DS reads
#pragma unroll
      for (int i = 0; i < 4 * kP; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);           // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 28 / (4 * kP), 0);  // VALU
      }
    };
    float da1p = 0.0f;
    Unit un;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int jn = (j + 1) & 7;
      // phase 0
      const float da0 = ld_da(0, j), da1 = ld_da(1, j);
      chain(0, j);
      if (j > 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) T[1][r] = fmaf(da1p, S[1][r], T[1][r]);
        asm volatile("" : "+v"(T[1]));  // the fold happens here, not where T is next read
      }
      un = unit(j < 7 ? w.sc : sc_n, jn);
      build(w, un, jn, 0, Nh[0], Nl[0]);
      interleave();
      __builtin_amdgcn_sched_barrier(0);
      // phase 1
      chain(1, j);
#pragma unroll
      for (int r = 0; r < 16; ++r) T[0][r] = fmaf(da0, S[0][r], T[0][r]);
      asm volatile("" : "+v"(T[0]));
      build(w, un, jn, 1, Nh[1], Nl[1]);
      interleave();
      // chunks whose last read was this build: the next super-block's
      if (j == 2) {
        w.ql[0] = ld_ql(s + 1, 0);
        w.ql[1] = ld_ql(s + 1, 1);
        w.qh[0] = ld_qh(s + 1, 0);
      } else if (j == 6) {
        w.ql[2] = ld_ql(s + 1, 2);
        w.ql[3] = ld_ql(s + 1, 3);
        w.qh[1] = ld_qh(s + 1, 1);
      }
      if (next) {
        // the next super-block's pieces, one (two) per block
#pragma unroll
        for (int i = 0; i < kP; ++i) issue_piece(s + 1, kP * j + i);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        Ah[h] = Nh[h];
        Al[h] = Nl[h];
      }
      da1p = da1;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) T[1][r] = fmaf(da1p, S[1][r], T[1][r]);
    // acc += d 2^24 T: d of the lane's 16 result rows 8 (r / 4) + 4 hh + r % 4, which lanes
    // 0-31 hold (one weight row each); T = 0
    const float d24 = h2f(w.d) * 16777216.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int src = 8 * (r >> 2) + 4 * hh + (r & 3);
      const float dr = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * src, __builtin_bit_cast(int, d24)));
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        acc[tt][r] = fmaf(dr, T[tt][r], acc[tt][r]);
        T[tt][r] = 0.0f;
      }
    }
    w.sc = sc_n;
    w.d = d_n;
  };

  // prologue: the first super-block's operands and weights, block 0's A operands
#pragma unroll
  for (int i = 0; i < kPieces; ++i) issue_piece(0, i);
#pragma unroll
  for (int i = 0; i < 4; ++i) w.ql[i] = ld_ql(0, i);
#pragma unroll
  for (int i = 0; i < 2; ++i) w.qh[i] = ld_qh(0, i);
  w.sc = ld_sc(0);
  w.d = ld_d(0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  {
    const Unit u0 = unit(w.sc, 0);
#pragma unroll
    for (int h = 0; h < 2; ++h) build(w, u0, 0, h, Ah[h], Al[h]);
  }
  lds_barrier();
#pragma unroll 1
  for (int s = 0; s < nb; ++s) {
    run_sb(s);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
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
