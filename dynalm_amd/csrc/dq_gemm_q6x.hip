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
// and 256 hi, each scaled by 2^-24, two more MFMAs): every product is exact, and a
// block's sum |sum w a| <= 32 * 4096 * 127 < 2^24 (in units of 2^-24) is exact (int16:
// rounded to fp32 where the running sum passes 2^24 units of 2^-48). Then, as the per-32
// GEMM (dq_gemm_p32.hip) does,
//   per block:        T = fma(da_j, S_j, T)
//   per super-block:  acc = fma(d 2^24 (int16: d 2^48), T, acc)
// The order is not the reference's: the outputs agree within the fp32 tolerance of a
// K-term dot product, not bit for bit.
//
// Work split. A workgroup owns 32 TT activation rows (TT = 2 tiles of 32, or 1 up to 32
// rows) x 128 weight rows with 4 waves, and a range of super-blocks; wave w owns weight
// rows 32 w .. 32 w + 31 (lane l builds row l % 32's operands for lane half hh = l / 32
// from the Q6_K planes it loads itself) against the activation tiles. Where the tiles
// leave workgroup slots idle (two per CU) the super-blocks split into up to 16 ranges, one
// workgroup each, whose partial outputs a second launch adds in range order
// (deterministic). A wave overlaps its own MFMAs and VALU work: per block, tile 0's MFMA
// chain runs beside the fold of tile 1's previous block and half of the next block's
// operand build, then tile 1's chain beside the fold of tile 0's block and the other half
// (TT = 1: the tile's chain beside the fold of its previous block and the whole build). A
// super-block's activation codes (16 KB per tile) and scales (1 KB per tile) go to LDS one interval ahead by direct-to-LDS loads spread over the
// blocks, into a ring of two; each weight plane chunk is reloaded for the next
// super-block right after its last read. The per-32 codes are f16 B operands in LDS
// already (2 B per value: the kernel is bound by VALU issue, and converting narrow codes
// in registers cost 16 VALU per tile and block); the int16 codes stay 16-bit there and
// become their two f16 operands in registers (as f16 pairs they would take 4 B per value,
// twice the LDS, and leave room for one workgroup per CU).
//
// Activation layouts (written from the quantized rows by k_q6x_act / k_q6x_quant), for
// M_pad = m rounded up to the workgroup's 32 TT rows (zero rows past m), T = M_pad / 32 row
// tiles and nb super-blocks; lane l is row 32 T + l % 32, half hh = l / 32, and K-step
// k = 2 j + h of a lane half takes values 32 j + 16 hh + 8 h + {0, 2, 1, 3, 4, 6, 5, 7} of
// the super-block (the weight operand's order: packed 16-bit lanes take bytes (0, 2) and
// (1, 3) of a dword):
//   per-32 ("act8h") codes [T][nb][j (8)][h (2)][lane (64)][8 x f16]: the int8 code of
//                    value i as f16 (exact)
//   int16 ("act16b") codes [T][nb][j (8)][h (2)][lane (64)][8 x u16]: v + 32768 of value i;
//                    the B operands are lo = v & 255 as raw f16 bits (the subnormal
//                    lo 2^-24) and 256 hi 2^-24 = hi 2^-16 through 0x2400 | (hi + 128)
//                    (= 2^-6 + (hi + 128) 2^-16) minus 2^-6 + 128 2^-16; both exact
//   da               [T][nb][j (8)][32 rows] floats, after the codes
// Values 32 j + 16 hh + 8 h + t of a super-block are, in its half n = j / 4 and quarter
// qd = j % 4, ql byte n 64 + 32 (qd & 1) + 16 hh + 8 h + t (the low nibble for qd < 2,
// else the high one: ql chunk 4 n + 2 (qd & 1) + hh, dwords 2 h, 2 h + 1) with qh bits
// 2 qd, 2 qd + 1 of qh byte n 32 + 16 hh + 8 h + t (qh chunk 2 n + hh), scale sc of unit
// 2 j + hh.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dq_device.h"
#include "dq_f16mma.h"
#include "dq_internal.h"
#include "dq_mfma.h"
#include "dq_quant.h"

namespace dq {

namespace {

constexpr int kXN = 128;        // weight rows per workgroup
constexpr int kXThreads = 256;  // 4 waves, one per SIMD

// Super-block buffer of a workgroup with TT 32-row activation tiles (TT = 2, or 1 for few
// rows): activation codes [j (8)][h (int16: 2)][t (TT)][lane (64)][16 B], then the
// activation scales [t (TT)][j (8)][row (32)].
template <bool kI16, int TT>
struct XLds {
  static constexpr int kH = 2;  // 1 KB pieces per block and tile (one per K-step)
  static constexpr int kCodes = 8 * kH * TT * 1024;
  static constexpr int kDa = kCodes;
  static constexpr int kBuf = kDa + TT * 1024;
  static constexpr int kTotal = 2 * kBuf;
};
static_assert(XLds<true, 2>::kTotal <= 160 * 1024, "LDS");

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

constexpr int kPerm[8] = {0, 2, 1, 3, 4, 6, 5, 7};  // the K-step's value order

// Activation tiles per workgroup by rows: one for few rows, so no MFMA runs on padding.
int q6x_tt(int64_t m) { return m <= 32 ? 1 : 2; }
// Rows of the operand layout: whole workgroup tiles.
int64_t q6x_rows(int64_t m) {
  const int64_t am = 32 * q6x_tt(m);
  return (m + am - 1) / am * am;
}

}  // namespace

// ---------------------------------------------------------------- layout writer

// Per-32 rows (40 B per 32 values: float d, int32 code sum, int8 codes[32]) -> act8h, or
// ActBlockQ16 rows (72 B: float d, int32 sum, int16 codes[32]) -> act16b. Workgroup
// (s, T): one 32-row tile's super-block s; rows past m are zeros (codes 0 stored biased).
template <bool kI16>
__global__ __launch_bounds__(256) void k_q6x_act(const uint8_t* __restrict__ acts, int64_t arb, int64_t m, int nb,
                                                 int64_t m_pad, uint8_t* __restrict__ out) {
  constexpr int kH = 2, kBlk = kI16 ? 72 : 40;
  const int t = threadIdx.x;
  const int s = blockIdx.x;
  const int64_t T = blockIdx.y;
  const int64_t codes_bytes = m_pad * nb * 256 * kH;
#pragma unroll
  for (int e = 0; e < 2 * kH; ++e) {
    // unit u = ((j, h), lane) of the (T, s) block: 16 bytes
    const int u = t + 256 * e, l = u & 63, hh = l >> 5;
    const int j = u >> 7, h0 = (u >> 6) & 1;
    const int64_t row = 32 * T + (l & 31);
    u32 o[4];
    if (row < m) {
      const uint8_t* b = acts + row * arb + (int64_t)(8 * s + j) * kBlk + 8;
      if (kI16) {
        const int16_t* q = reinterpret_cast<const int16_t*>(b) + 16 * hh + 8 * h0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          o[i] = (u32)(uint16_t)(q[kPerm[2 * i]] + 32768) | ((u32)(uint16_t)(q[kPerm[2 * i + 1]] + 32768) << 16);
        }
      } else {
        const int8_t* q = reinterpret_cast<const int8_t*>(b) + 16 * hh + 8 * h0;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = f16_pair(q[kPerm[2 * i]], q[kPerm[2 * i + 1]]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = kI16 ? 0x80008000u : 0u;
    }
    *reinterpret_cast<v4u*>(out + ((((T * nb + s) * 8 + j) * kH + h0) * 64 + l) * 16) = v4u{o[0], o[1], o[2], o[3]};
  }
  {
    // da: thread t = 32 j + r
    const int j = t >> 5;
    const int64_t row = 32 * T + (t & 31);
    const float d = row < m ? *reinterpret_cast<const float*>(acts + row * arb + (int64_t)(8 * s + j) * kBlk) : 0.0f;
    *reinterpret_cast<float*>(out + codes_bytes + (T * nb + s) * 1024 + t * 4) = d;
  }
}

// fp32 rows -> act8h / act16b directly, with the standalone quantizers' arithmetic
// (per32_quant / q16_quant: the layout equals k_q6x_act's of the rows they write). One
// wave per (super-block, padded row); lane l = 8 j + 4 hh + 2 h + p quantizes values
// 4 l .. 4 l + 3, the half p of K-step 2 j + h's unit of lane half hh. per-32: each lane
// writes its half; int16: even lanes write the unit with lane l + 1's codes.
template <bool kI16>
__global__ __launch_bounds__(64) void k_q6x_quant(const float* __restrict__ x, int64_t x_stride, int64_t m, int64_t k,
                                                  int64_t m_pad, uint8_t* __restrict__ out) {
  constexpr int kH = 2;
  const int l = threadIdx.x;
  const int s = blockIdx.x;
  const int64_t row = blockIdx.y;
  const int nb = (int)(k / 256);
  const auto rx = rsrc(x + (row < m ? row * x_stride : 0), row < m ? (u32)(k * 4) : 0u);
  float v[4];
  load4f(rx, (u32)(((int64_t)s * 256 + 4 * l) * 4), v);
  float d;
  int sum;
  const int64_t T = row >> 5, r = row & 31;
  const int64_t codes_bytes = m_pad * nb * 256 * kH;
  const int j = l >> 3, hh = (l >> 2) & 1;
  if (kI16) {
    const v2u c = q16_quant(v, d, sum);
    const int src = 4 * ((l + 1) & 63);
    const u32 n0 = (u32)__builtin_amdgcn_ds_bpermute(src, (int)c.x), n1 = (u32)__builtin_amdgcn_ds_bpermute(src, (int)c.y);
    if ((l & 1) == 0) {
      // halves (v0, v2), (v1, v3) of this lane, (v4, v6), (v5, v7) of the next, plus 32768
      const int h = (l >> 1) & 1;
      const v4u o = {__builtin_amdgcn_perm(c.y, c.x, 0x05040100u) ^ 0x80008000u,
                     __builtin_amdgcn_perm(c.y, c.x, 0x07060302u) ^ 0x80008000u,
                     __builtin_amdgcn_perm(n1, n0, 0x05040100u) ^ 0x80008000u,
                     __builtin_amdgcn_perm(n1, n0, 0x07060302u) ^ 0x80008000u};
      *reinterpret_cast<v4u*>(out + ((((T * nb + s) * 8 + j) * 2 + h) * 64 + 32 * hh + r) * 16) = o;
    }
  } else {
    const u32 c = per32_quant(v, d, sum);
    // this lane's values 4 l .. 4 l + 3 as f16 pairs (0, 2), (1, 3): half p = l & 1 of
    // K-step h = (l >> 1) & 1's unit
    const int h = (l >> 1) & 1, p = l & 1;
    auto code = [&](int i) { return (int)(int8_t)(c >> (8 * i)); };
    *reinterpret_cast<v2u*>(out + ((((T * nb + s) * 8 + j) * 2 + h) * 64 + 32 * hh + r) * 16 + 8 * p) =
        v2u{f16_pair(code(0), code(2)), f16_pair(code(1), code(3))};
  }
  if ((l & 7) == 0) reinterpret_cast<float*>(out + codes_bytes + (T * nb + s) * 1024)[j * 32 + r] = d;
}

// ---------------------------------------------------------------- the GEMM

// One workgroup: activation rows [32 TT tm, + 32 TT) x weight rows [nbase0 + 128 tn, + 128),
// super-blocks of range sp of nsplit. Arguments as launch_gemm_q6x; part: the ranges'
// partial outputs [nsplit][m][W] (nsplit > 1), W = 128 tiles_n.
template <bool kI16, int TT>
__global__ __launch_bounds__(kXThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_q6k_x(
    const uint8_t* __restrict__ ql_plane, const uint8_t* __restrict__ qh_plane, const uint8_t* __restrict__ sc_plane,
    const uint8_t* __restrict__ d_plane, int nb, int64_t nbase0, int64_t n_pad, int64_t n0, int64_t n1,
    const uint8_t* __restrict__ act, int64_t m_pad, int64_t m, float* __restrict__ y, int64_t ys,
    const float* __restrict__ bias, int tiles_m, int tiles_n, int nsplit, float* __restrict__ part) {
  using X = XLds<kI16, TT>;
  constexpr int kH = X::kH;
  extern __shared__ __align__(16) uint8_t lds[];
  const int t = threadIdx.x, lane = t & 63;
  const int li = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int L = blockIdx.x;
  const int tiles = tiles_m * tiles_n;
  const int sp = __builtin_amdgcn_readfirstlane(L / tiles), Lt = L - sp * tiles;
  // Workgroups are dealt to the 8 XCDs round-robin: with tiles_n a multiple of 8, the
  // activation tiles of one weight tile go to one XCD, so they share its L2's copy of the
  // weight rows.
  int tn, tm;
  if (tiles_n % 8 == 0) {
    tn = 8 * (Lt / (8 * tiles_m)) + (Lt & 7);
    tm = (Lt >> 3) % tiles_m;
  } else {
    tn = Lt / tiles_m;
    tm = Lt - tn * tiles_m;
  }
  tn = __builtin_amdgcn_readfirstlane(tn);
  tm = __builtin_amdgcn_readfirstlane(tm);
  const int64_t nbase = nbase0 + (int64_t)kXN * tn;
  const int64_t mbase = (int64_t)tm * 32 * TT;
  const int sb0 = __builtin_amdgcn_readfirstlane(sp * nb / nsplit), sb1 = __builtin_amdgcn_readfirstlane((sp + 1) * nb / nsplit);

  const int64_t codes_bytes = m_pad * nb * 256 * kH, da_bytes = m_pad / 32 * nb * 1024;
  const auto ra = rsrc(act, (u32)(codes_bytes + da_bytes));
  const auto rl = rsrc(ql_plane, (u32)(n_pad * nb * 128));
  const auto rhq = rsrc(qh_plane, (u32)(n_pad * nb * 64));
  const auto rs = rsrc(sc_plane, (u32)(n_pad * nb * 16));
  const auto rd = rsrc(d_plane, (u32)(n_pad * nb * 2));

  // ---- this wave's loads. Codes of super-block s: pieces jb = 2 kH TT wave + i
  // (i < 2 kH TT) of the buffer, jb = (j kH + h) TT + tt; with piece 0 the activation scales
  // of tile wave (waves < TT). The wave's weight row: group g0 + wave / 2, row
  // 32 (wave & 1) + li.
  const u32 g0 = (u32)(nbase >> 6);
  const u32 G = g0 + (u32)(wave >> 1), r64 = (u32)(32 * (wave & 1) + li);
  constexpr int kPieces = 2 * kH * TT;  // 1 KB pieces per wave and super-block
  auto issue_piece = [&](int s, int buf, int i) {
    uint8_t* P = lds + buf * X::kBuf;
    const int jb = kPieces * wave + i;
    const int tt = jb % TT, jh = jb / TT;  // jh = j kH + h
    const int64_t T = (int64_t)TT * tm + tt;
    dma16(ra, P + jb * 1024, (u32)(lane * 16), (u32)(((T * nb + s) * 8 * kH + jh) * 1024));
    if (i == 0 && wave < TT) {
      const int64_t Tb = (int64_t)TT * tm + wave;
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
  // B operands. per-32: the layout's f16 codes as they are.
  // int16: a dword of two biased codes -> (lo_a, lo_b) 2^-24 and (hi_a, hi_b) 2^-16
  auto b16lo = [](u32 x) -> u32 { return __builtin_amdgcn_perm(0u, x, 0x0C020C00u); };
  auto b16hi = [](u32 x) -> u32 {
    constexpr _Float16 kOff = (_Float16)(0x1p-6f + 0x1p-9f);  // 2^-6 + 128 2^-16
    const h2_t v = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x24242424u, x, 0x04030401u));
    return __builtin_bit_cast(u32, v - h2_t{kOff, kOff});
  };

  // TT = 2: S[tt] is tile tt's block sum; TT = 1: S[j & 1] is block j's
  v16f_t acc[TT], S[2], T[TT];
#pragma unroll
  for (int mt = 0; mt < TT; ++mt) {
    acc[mt] = v16f_t{};
    T[mt] = v16f_t{};
  }
  W6 w;
  v4u sc_n;
  u32 d_n;
  v4u Ah[2][2], Al[2][2];  // [block parity][K-step h]: block j's operands, then block j + 1's

  // Super-block s, per block j in two phases (TT = 2), each in a fixed issue order: tile
  // tt's MFMA chain (K-steps 2 j, 2 j + 1; a_hi, a_lo) with a share of independent VALU work
  // between consecutive MFMAs (B conversions, the other tile's fold, the next block's
  // operand build), so that each MFMA's predecessor has finished when it issues and the
  // matrix core runs beside the VALU. Phase 0: tile 0 beside the fold of tile 1's previous
  // block and the next block's K-step 0 operands; phase 1: tile 1 beside the fold of tile
  // 0's block j and the next block's K-step 1 operands. TT = 1: one phase, the tile's chain
  // into S[j & 1] beside the fold of block j - 1 (S[(j + 1) & 1]) and the next block's
  // operands.
#define SB() __builtin_amdgcn_sched_barrier(0)
  auto run_sb = [&](int s) {
    const bool next = s + 1 < sb1;
    sc_n = ld_sc(s + 1);
    d_n = ld_d(s + 1);
    const uint8_t* P = lds + __builtin_amdgcn_readfirstlane((s & 1) * X::kBuf);
    auto ld_da = [&](int tt, int j) { return as_f(lds4v(P + X::kDa + ((tt * 8 + j) * 32 + li) * 4)); };
    // the codes of block j, tile tt (int16: K-step h); int16 reads both K-steps
    auto ld_x = [&](int j, int tt, int h) { return lds16(P + ((((j * kH + h) * TT) + tt) * 64 + lane) * 16); };
    auto fold = [&](int tt, float da, int r0) {
#pragma unroll
      for (int r = r0; r < r0 + 8; ++r) T[tt][r] = fmaf(da, S[tt][r], T[tt][r]);
    };
    float da1p = 0.0f;
    v4u xa = ld_x(0, 0, 0), xb = ld_x(0, 0, 1);  // this phase's codes (K-steps 0, 1)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int jn = (j + 1) & 7, c = j & 1, cn = c ^ 1;
      const Unit un = unit(j < 7 ? w.sc : sc_n, jn);
      if constexpr (TT == 1) {
        const float daj = ld_da(0, j);
        // prefetch block j + 1's codes
        v4u ya = xa, yb = xb;
        if (j < 7) {
          ya = ld_x(j + 1, 0, 0);
          yb = ld_x(j + 1, 0, 1);
        }
        const bool do_fold = j > 0;
        auto foldp = [&](int r0) {
#pragma unroll
          for (int r = r0; r < r0 + 8; ++r) T[0][r] = fmaf(da1p, S[cn][r], T[0][r]);
        };
        if (kI16) {
          v4u bl0 = {b16lo(xa[0]), b16lo(xa[1]), b16lo(xa[2]), b16lo(xa[3])};
          SB();
          S[c] = mfma_h(Ah[c][0], bl0, v16f_t{});
          SB();
          v4u bh0 = {b16hi(xa[0]), b16hi(xa[1]), b16hi(xa[2]), b16hi(xa[3])};
          SB();
          S[c] = mfma_h(Al[c][0], bl0, S[c]);
          SB();
          v4u bl1 = {b16lo(xb[0]), b16lo(xb[1]), b16lo(xb[2]), b16lo(xb[3])};
          if (do_fold) foldp(0);
          SB();
          S[c] = mfma_h(Ah[c][0], bh0, S[c]);
          SB();
          v4u bh1 = {b16hi(xb[0]), b16hi(xb[1]), b16hi(xb[2]), b16hi(xb[3])};
          SB();
          S[c] = mfma_h(Al[c][0], bh0, S[c]);
          SB();
          if (do_fold) {
            foldp(8);
            asm volatile("" : "+v"(T[0]));  // the fold happens here, not where T is next read
          }
          SB();
          S[c] = mfma_h(Ah[c][1], bl1, S[c]);
          SB();
          build(w, un, jn, 0, Ah[cn][0], Al[cn][0]);
          SB();
          S[c] = mfma_h(Al[c][1], bl1, S[c]);
          SB();
          build(w, un, jn, 1, Ah[cn][1], Al[cn][1]);
          SB();
          S[c] = mfma_h(Ah[c][1], bh1, S[c]);
          SB();
          S[c] = mfma_h(Al[c][1], bh1, S[c]);
          SB();
        } else {
          const v4u b0 = xa, b1 = xb;
          SB();
          S[c] = mfma_h(Ah[c][0], b0, v16f_t{});
          SB();
          S[c] = mfma_h(Al[c][0], b0, S[c]);
          SB();
          if (do_fold) foldp(0);
          SB();
          S[c] = mfma_h(Ah[c][1], b1, S[c]);
          SB();
          if (do_fold) {
            foldp(8);
            asm volatile("" : "+v"(T[0]));
          }
          SB();
          S[c] = mfma_h(Al[c][1], b1, S[c]);
          SB();
          build(w, un, jn, 0, Ah[cn][0], Al[cn][0]);
          build(w, un, jn, 1, Ah[cn][1], Al[cn][1]);
          SB();
        }
        xa = ya;
        xb = yb;
        // the scale of the block folded next
        da1p = daj;
      } else {
      float da[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        if (tt == 0) {
          da[0] = ld_da(0, j);
          da[1] = ld_da(1, j);
        }
        // prefetch the next phase's codes: tile 1 of block j, or tile 0 of block j + 1
        v4u ya, yb;
        if (tt == 0) {
          ya = ld_x(j, 1, 0);
          yb = ld_x(j, 1, 1);
        } else if (j < 7) {
          ya = ld_x(j + 1, 0, 0);
          yb = ld_x(j + 1, 0, 1);
        }
        const int ot = tt ^ 1;  // the tile folded in this phase
        const bool do_fold = tt == 1 || j > 0;
        const float fda = tt == 0 ? da1p : da[0];
        if (kI16) {
          // 8 MFMAs: (h, plane) = (0, lo) (0, hi) (1, lo) (1, hi), a_hi then a_lo each
          v4u bl0 = {b16lo(xa[0]), b16lo(xa[1]), b16lo(xa[2]), b16lo(xa[3])};
          SB();
          S[tt] = mfma_h(Ah[c][0], bl0, v16f_t{});
          SB();
          v4u bh0 = {b16hi(xa[0]), b16hi(xa[1]), b16hi(xa[2]), b16hi(xa[3])};
          SB();
          S[tt] = mfma_h(Al[c][0], bl0, S[tt]);
          SB();
          v4u bl1 = {b16lo(xb[0]), b16lo(xb[1]), b16lo(xb[2]), b16lo(xb[3])};
          if (do_fold) fold(ot, fda, 0);
          SB();
          S[tt] = mfma_h(Ah[c][0], bh0, S[tt]);
          SB();
          v4u bh1 = {b16hi(xb[0]), b16hi(xb[1]), b16hi(xb[2]), b16hi(xb[3])};
          SB();
          S[tt] = mfma_h(Al[c][0], bh0, S[tt]);
          SB();
          if (do_fold) {
            fold(ot, fda, 8);
            asm volatile("" : "+v"(T[ot]));  // the fold happens here, not where T is next read
          }
          SB();
          S[tt] = mfma_h(Ah[c][1], bl1, S[tt]);
          SB();
          build(w, un, jn, tt, Ah[cn][tt], Al[cn][tt]);
          SB();
          S[tt] = mfma_h(Al[c][1], bl1, S[tt]);
          SB();
          S[tt] = mfma_h(Ah[c][1], bh1, S[tt]);
          SB();
          S[tt] = mfma_h(Al[c][1], bh1, S[tt]);
          SB();
        } else {
          const v4u b0 = xa, b1 = xb;
          SB();
          S[tt] = mfma_h(Ah[c][0], b0, v16f_t{});
          SB();
          S[tt] = mfma_h(Al[c][0], b0, S[tt]);
          SB();
          if (do_fold) fold(ot, fda, 0);
          SB();
          S[tt] = mfma_h(Ah[c][1], b1, S[tt]);
          SB();
          if (do_fold) {
            fold(ot, fda, 8);
            asm volatile("" : "+v"(T[ot]));
          }
          SB();
          S[tt] = mfma_h(Al[c][1], b1, S[tt]);
          SB();
          build(w, un, jn, tt, Ah[cn][tt], Al[cn][tt]);
          SB();
        }
        if (tt == 0 || j < 7) {
          xa = ya;
          xb = yb;
        }
      }
      da1p = da[1];
      }
      // chunks whose last read was this block's build: the next super-block's
      if (j == 2) {
        w.ql[0] = ld_ql(s + 1, 0);
        w.ql[1] = ld_ql(s + 1, 1);
        w.qh[0] = ld_qh(s + 1, 0);
      } else if (j == 6) {
        w.ql[2] = ld_ql(s + 1, 2);
        w.ql[3] = ld_ql(s + 1, 3);
        w.qh[1] = ld_qh(s + 1, 1);
      }
      // the next super-block's pieces into the other buffer (past the range: this one's
      // again, unread), evenly over the blocks
      {
        constexpr int kEvery = 8 / kPieces;
        const int sn = next ? s + 1 : s;
        if (j % kEvery == 0) issue_piece(sn, (s + 1) & 1, j / kEvery);
      }
      SB();
    }
    // the last fold: tile 1's block 7 (TT = 2), block 7 (TT = 1)
#pragma unroll
    for (int r = 0; r < 16; ++r) T[TT - 1][r] = fmaf(da1p, S[1][r], T[TT - 1][r]);
    // acc += d 2^24 T (int16: d 2^48 T): d of the lane's 16 result rows 8 (r / 4) + 4 hh +
    // r % 4, which lanes 0-31 hold (one weight row each); T = 0
    const float dsc = h2f(w.d) * (kI16 ? 0x1p48f : 0x1p24f);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int src = 8 * (r >> 2) + 4 * hh + (r & 3);
      const float dr = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * src, __builtin_bit_cast(int, dsc)));
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        acc[tt][r] = fmaf(dr, T[tt][r], acc[tt][r]);
        T[tt][r] = 0.0f;
      }
    }
    w.sc = sc_n;
    w.d = d_n;
  };
#undef SB

  // prologue: the first super-block's codes and weights, block 0's A operands
#pragma unroll
  for (int i = 0; i < kPieces; ++i) issue_piece(sb0, sb0 & 1, i);
#pragma unroll
  for (int i = 0; i < 4; ++i) w.ql[i] = ld_ql(sb0, i);
#pragma unroll
  for (int i = 0; i < 2; ++i) w.qh[i] = ld_qh(sb0, i);
  w.sc = ld_sc(sb0);
  w.d = ld_d(sb0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  {
    const Unit u0 = unit(w.sc, 0);
#pragma unroll
    for (int h = 0; h < 2; ++h) build(w, u0, 0, h, Ah[0][h], Al[0][h]);
  }
  lds_barrier();
#pragma unroll 1
  for (int s = sb0; s < sb1; ++s) {
    run_sb(s);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
  }

  // ---- outputs: activation row 32 mt + li, weight rows nbase + 32 wave + 8 (r / 4) + 4 hh
  // + r % 4; with one range y (+ bias) in [n0, n1), else the range's partial tile
  const int64_t mrows = m - mbase < 32 * TT ? m - mbase : 32 * TT;
  const int64_t W = (int64_t)kXN * tiles_n;
#pragma unroll
  for (int mt = 0; mt < TT; ++mt) {
    const int row = 32 * mt + li;
    if (row >= mrows) continue;
    float* yr = y + (mbase + row) * ys;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t nq = nbase + 32 * wave + 8 * q + 4 * hh;
      if (nsplit > 1) {
        float* pr = part + ((int64_t)sp * m + mbase + row) * W + (nq - nbase0);
        *reinterpret_cast<float4*>(pr) = float4{acc[mt][4 * q], acc[mt][4 * q + 1], acc[mt][4 * q + 2], acc[mt][4 * q + 3]};
        continue;
      }
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

// y[r, n] = sum over the N ranges, in range order, of part[range][r][n - nbase0] (+ bias[n]),
// n in [n0, n1): one thread per output, rows in the grid's y dimension. N is a template
// argument so that the N loads issue together before the first add.
template <int N>
__global__ __launch_bounds__(256) void k_split_sum(const float* __restrict__ part, int64_t m, int64_t W,
                                                 int64_t nbase0, int64_t n0, int64_t n1, float* __restrict__ y,
                                                 int64_t ys, const float* __restrict__ bias) {
  const int64_t n = n0 + (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t r = blockIdx.y;
  if (n >= n1) return;
  const float* p = part + r * W + (n - nbase0);
  float v[N];
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = p[(int64_t)i * m * W];
  float acc = v[0];
#pragma unroll
  for (int i = 1; i < N; ++i) acc += v[i];
  y[r * ys + n] = bias ? acc + bias[n] : acc;
}

// ---------------------------------------------------------------- host

namespace {

struct Q6xGrid {
  int64_t nbase0, tiles_n, tiles_m;
  int nsplit;
};

Q6xGrid q6x_grid(const WeightDev& w, int64_t m, int64_t n0, int64_t n1) {
  Q6xGrid g;
  g.nbase0 = n0 / kRowGroup * kRowGroup;
  g.tiles_n = (n1 - g.nbase0 + kXN - 1) / kXN;
  g.tiles_m = (m + 32 * q6x_tt(m) - 1) / (32 * q6x_tt(m));
  // two workgroups fit a CU (4 waves, at most 68 KB of LDS): ranges for two per CU, so
  // that each SIMD holds two waves to hide the other's waits
  g.nsplit = split_ranges(g.tiles_n * g.tiles_m, 2 * (w.cus > 0 ? w.cus : 256), w.nblk);
  return g;
}

}  // namespace

int64_t q6x_act_bytes(int af, int64_t m, int64_t k) {
  (void)af;  // per-32 and int16 layouts: 2 B per value
  const int64_t mp = q6x_rows(m), nb = k / 256;
  return mp * nb * 256 * 2 + mp / 32 * nb * 1024;
}

int64_t q6x_part_bytes(const WeightDev& w, int64_t m, int64_t n0, int64_t n1) {
  const Q6xGrid g = q6x_grid(w, m, n0, n1);
  return g.nsplit > 1 ? (int64_t)g.nsplit * m * kXN * g.tiles_n * 4 : 0;
}

bool gemm_q6x_ok(const WeightDev& w, int af, int64_t m, int64_t n0, int64_t n1) {
  if (w.dtype != kQ6_K || (af != kActPer32 && af != kActQ16) || m <= 0 || n1 <= n0 || w.nblk <= 0) return false;
  // 32-bit buffer offsets: the ql plane plus one tile's rows past its end, and the layout;
  // the layout writer's grid has one row of workgroups per 32 padded rows, the sum's one
  // per row
  if ((w.n_pad + 2 * kRowGroup) * w.nblk * 128 >= (1ll << 32)) return false;
  if (q6x_act_bytes(af, m, w.k) >= (1ll << 32) || q6x_rows(m) / 32 > 65535) return false;
  const Q6xGrid g = q6x_grid(w, m, n0, n1);
  if (g.nsplit > 1 && m > 65535) return false;
  return g.tiles_m * g.tiles_n * g.nsplit < (1ll << 31);
}

hipError_t launch_q6x_act(int af, const uint8_t* acts, int64_t arb, int64_t m, int64_t k, uint8_t* out,
                          hipStream_t s) {
  const int64_t mp = q6x_rows(m);
  if (mp / 32 > 65535 || k % 256 != 0 || (af != kActPer32 && af != kActQ16)) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(k / 256), (unsigned)(mp / 32));
  if (af == kActQ16) {
    hipLaunchKernelGGL(k_q6x_act<true>, grid, dim3(256), 0, s, acts, arb, m, (int)(k / 256), mp, out);
  } else {
    hipLaunchKernelGGL(k_q6x_act<false>, grid, dim3(256), 0, s, acts, arb, m, (int)(k / 256), mp, out);
  }
  return hipGetLastError();
}

hipError_t launch_q6x_quant(int af, const float* x, int64_t x_stride, int64_t m, int64_t k, uint8_t* out,
                            hipStream_t s) {
  const int64_t mp = q6x_rows(m);
  if (mp > 65535 || k % 256 != 0 || (af != kActPer32 && af != kActQ16)) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(k / 256), (unsigned)mp);
  if (af == kActQ16) {
    hipLaunchKernelGGL(k_q6x_quant<true>, grid, dim3(64), 0, s, x, x_stride, m, k, mp, out);
  } else {
    hipLaunchKernelGGL(k_q6x_quant<false>, grid, dim3(64), 0, s, x, x_stride, m, k, mp, out);
  }
  return hipGetLastError();
}

hipError_t launch_gemm_q6x(const WeightDev& w, int af, const uint8_t* act, int64_t m, int64_t n0, int64_t n1, float* y,
                           int64_t ys, const float* bias, float* part, hipStream_t s) {
  if (!gemm_q6x_ok(w, af, m, n0, n1)) return hipErrorInvalidValue;
  const Q6xGrid g = q6x_grid(w, m, n0, n1);
  if (g.nsplit > 1 && part == nullptr) return hipErrorInvalidValue;
  const int64_t mp = q6x_rows(m);
  const dim3 grid((unsigned)(g.tiles_n * g.tiles_m * g.nsplit));
  hipError_t e = hipSuccess;
#define DQ_Q6X_LAUNCH(I16, TTV)                                                                                      \
  {                                                                                                                  \
    const int lds = XLds<I16, TTV>::kTotal;                                                                          \
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm_q6k_x<I16, TTV>),                                 \
                            hipFuncAttributeMaxDynamicSharedMemorySize, lds);                                        \
    if (e != hipSuccess) return e;                                                                                   \
    hipLaunchKernelGGL((k_gemm_q6k_x<I16, TTV>), grid, dim3(kXThreads), lds, s, w.plane[0], w.plane[1], w.plane[2], \
                       w.plane[3], (int)w.nblk, g.nbase0, w.n_pad, n0, n1, act, mp, m, y, ys, bias, (int)g.tiles_m,  \
                       (int)g.tiles_n, g.nsplit, part);                                                              \
  }
  const bool one = q6x_tt(m) == 1;
  if (af == kActQ16) {
    if (one) DQ_Q6X_LAUNCH(true, 1) else DQ_Q6X_LAUNCH(true, 2)
  } else {
    if (one) DQ_Q6X_LAUNCH(false, 1) else DQ_Q6X_LAUNCH(false, 2)
  }
#undef DQ_Q6X_LAUNCH
  if (g.nsplit > 1) {
    const hipError_t e2 = hipGetLastError();
    if (e2 != hipSuccess) return e2;
    return launch_split_sum(part, g.nsplit, m, (int64_t)kXN * g.tiles_n, g.nbase0, n0, n1, y, ys, bias, s);
  }
  return hipGetLastError();
}

namespace {

template <int N>
void split_sum_n(const float* part, int64_t m, int64_t W, int64_t nbase0, int64_t n0, int64_t n1, float* y,
                 int64_t ys, const float* bias, hipStream_t s) {
  hipLaunchKernelGGL(k_split_sum<N>, dim3((unsigned)((n1 - n0 + 255) / 256), (unsigned)m), dim3(256), 0, s, part, m,
                     W, nbase0, n0, n1, y, ys, bias);
}

using SplitSumFn = void (*)(const float*, int64_t, int64_t, int64_t, int64_t, int64_t, float*, int64_t,
                            const float*, hipStream_t);
constexpr SplitSumFn kSplitSum[17] = {
    nullptr,           &split_sum_n<1>,   &split_sum_n<2>,   &split_sum_n<3>,  &split_sum_n<4>,  &split_sum_n<5>,
    &split_sum_n<6>,   &split_sum_n<7>,   &split_sum_n<8>,   &split_sum_n<9>,  &split_sum_n<10>, &split_sum_n<11>,
    &split_sum_n<12>,  &split_sum_n<13>,  &split_sum_n<14>,  &split_sum_n<15>, &split_sum_n<16>};

}  // namespace

hipError_t launch_split_sum(const float* part, int nsplit, int64_t m, int64_t W, int64_t nbase0, int64_t n0,
                            int64_t n1, float* y, int64_t ys, const float* bias, hipStream_t s) {
  if (m <= 0 || m > 65535 || n1 <= n0 || nsplit < 1 || nsplit > 16) return hipErrorInvalidValue;
  kSplitSum[nsplit](part, m, W, nbase0, n0, n1, y, ys, bias, s);
  return hipGetLastError();
}

}  // namespace dq
