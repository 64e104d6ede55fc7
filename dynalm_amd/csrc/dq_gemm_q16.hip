// dq_gemm_q16.hip -- prefill GEMM for Q4_K weights x int16 activations (the int16
// contract: int16 codes with one scale d and one code sum per 32 values, the
// reference's ActBlockQ16, dynacore/cpu/avx2/kernels_avx2.cpp:1631-1652, and qmm's
// int16 mode) on the f16 matrix cores, and the activation layout it reads.
//
// Arithmetic. Per sub-block j (32 values) of every super-block the contract sums
//   acc += (d sc_j) da_j P_j - (dmin m_j) c_j,   P_j = sum_t q_t a_t,  c_j = da_j (code sum)
// (the int16 row kernel, kernels_avx2.cpp:1697-1729; qmm's dot_row_ref in int16 mode,
// qmm_reference.cpp:68-93). An int16 code a = 256 hi + lo splits into two integers
// that f16 holds exactly: lo (0 .. 255) and 256 hi (-32768 .. 32512). Both run on
// v_mfma_f32_32x32x16_f16 against the weight operand sc_j q as the raw 16-bit integer
// (at most 945, read as the f16 subnormal sc_j q 2^-24), two K-steps per sub-block
// and two MFMAs per K-step into one fresh accumulator: every product is exact and the
// accumulator ends at sc_j P_j 2^-24, rounded to fp32 where the running sum passes
// 2^24 (|sc_j P_j| reaches 945 * 32767 * 32 ~ 2^29.9, so a few roundings of relative
// size 2^-24). Then, as the per-32 GEMM (dq_gemm_p32.hip) does,
//   per sub-block:    T = fma(da_j, sc_j P_j 2^-24, T)
//   per super-block:  acc = fma(d 2^24, T, acc)
// and the mins term as fp32 matrix products straight into acc. The summation order
// is not the reference's: outputs agree within the fp32 tolerance of a K-term dot
// product, not bit for bit.
//
// Work split. A workgroup owns 64 activation rows x 256 weight rows with 8 waves, two
// per SIMD; wave w owns weight rows 32 w .. 32 w + 31 (the A operand, built by each
// lane from its own row's nibbles) against the two 32-row activation tiles (the B
// operands, lo and 256 hi). A super-block's operands (64 rows x 256 values x two
// planes as f16, 64 KB), activation scales and mins operands (2 + 2 KB) go to LDS
// one interval ahead by direct-to-LDS loads spread over the K-steps, into a ring of
// two (the 128-row tile of the per-32 GEMM would need twice the LDS).
//
// Activation layout ("act16i", k_act16i_from_q16 from ActBlockQ16 rows), for M_pad =
// m rounded up to the workgroup's 32 TT rows (zero rows past m), T = M_pad / 32 row
// tiles, nb super-blocks:
//   codes  [T][nb][k (16)][p (2)][lane (64)][8 halves]  p = 0: lo, p = 1: 256 hi; lane
//          l: row 32 T + l % 32, half hh = l / 32; K-step k = 2 j + h holds values
//          32 j + 16 hh + 8 h + {0, 2, 1, 3, 4, 6, 5, 7} of the super-block
//   da     [T][nb][j (8)][32 rows] floats
//   c      [T][nb][kk (4)][lane (64)] floats: c of row l % 32, sub-block 2 kk + l / 32
// The K order is the per-32 GEMM's: the order in which a lane's weight operand comes
// out of two dwords of its row's nibbles.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dq_device.h"
#include "dq_f16mma.h"
#include "dq_internal.h"
#include "dq_mfma.h"
#include "dq_quant.h"

namespace dq {

namespace {

constexpr int kQN = 256;  // weight rows per workgroup (activation rows: 32 TT)
constexpr int kQThreads = 512;      // 8 waves, two per SIMD
// Super-block buffer: operands [k (16)][t (2)][p (2)][lane (64)][16 B], then the
// activation scales [t (2)][j (8)][row (32)] and the mins operands [t (2)][kk (4)][lane (64)].
// With TT 32-row activation tiles per workgroup (TT = 2, or 1 for few rows): operands
// 32 TT KB, scales and mins operands TT KB each.
template <int TT>
struct QLds {
  static constexpr int kCodes = 32 * TT * 1024, kDa = kCodes, kC = kDa + TT * 1024;
  static constexpr int kBuf = kC + TT * 1024;
  static constexpr int kTotal = 2 * kBuf;
};
static_assert(QLds<2>::kTotal <= 160 * 1024, "LDS");

DQ_DEV v16f_t mfma_f32_k2(float a, float b, v16f_t c) { return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0); }

// Two integers (exact in f16) as the packed halves of a dword.
DQ_DEV u32 f16x2(int a, int b) {
  const _Float16 ha = (_Float16)(float)a, hb = (_Float16)(float)b;
  return (u32)__builtin_bit_cast(uint16_t, ha) | ((u32)__builtin_bit_cast(uint16_t, hb) << 16);
}

}  // namespace

// ---------------------------------------------------------------- act16i writer

// ActBlockQ16 rows (72 B per 32 values: float d, int32 code sum, int16 codes[32]) ->
// act16i. Workgroup (s, T): one 32-row tile's super-block s; rows past m are zeros.
__global__ __launch_bounds__(256) void k_act16i_from_q16(const uint8_t* __restrict__ acts, int64_t arb, int64_t m,
                                                         int nb, int64_t m_pad, uint8_t* __restrict__ out) {
  const int t = threadIdx.x;
  const int s = blockIdx.x;
  const int64_t T = blockIdx.y;
  const int64_t codes_bytes = m_pad * nb * 1024, da_bytes = m_pad / 32 * nb * 1024;
  constexpr int kPerm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    // unit u = (k, p, lane) of the (T, s) block
    const int u = t + 256 * e, k = u >> 7, p = (u >> 6) & 1, l = u & 63, hh = l >> 5;
    const int64_t row = 32 * T + (l & 31);
    v4u o = {0u, 0u, 0u, 0u};
    if (row < m) {
      const int16_t* q = reinterpret_cast<const int16_t*>(acts + row * arb + (int64_t)(8 * s + (k >> 1)) * 72 + 8) +
                         16 * hh + 8 * (k & 1);
      int v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int a = q[kPerm[i]];
        v[i] = p ? (a >> 8) * 256 : (a & 255);
      }
      o = v4u{f16x2(v[0], v[1]), f16x2(v[2], v[3]), f16x2(v[4], v[5]), f16x2(v[6], v[7])};
    }
    *reinterpret_cast<v4u*>(out + (((T * nb + s) * 16 + k) * 2 + p) * 1024 + l * 16) = o;
  }
  {
    // da: thread t = 32 j + r
    const int j = t >> 5;
    const int64_t row = 32 * T + (t & 31);
    const float d = row < m ? *reinterpret_cast<const float*>(acts + row * arb + (int64_t)(8 * s + j) * 72) : 0.0f;
    *reinterpret_cast<float*>(out + codes_bytes + (T * nb + s) * 1024 + t * 4) = d;
  }
  {
    // c = d * (code sum): thread t = 64 kk + lane, sub-block 2 kk + lane / 32
    const int l = t & 63, j = 2 * (t >> 6) + (l >> 5);
    const int64_t row = 32 * T + (l & 31);
    float c = 0.0f;
    if (row < m) {
      const uint8_t* b = acts + row * arb + (int64_t)(8 * s + j) * 72;
      c = *reinterpret_cast<const float*>(b) * (float)*reinterpret_cast<const int32_t*>(b + 4);
    }
    *reinterpret_cast<float*>(out + codes_bytes + da_bytes + (T * nb + s) * 1024 + t * 4) = c;
  }
}

// fp32 rows -> act16i directly, with the int16 quantizer's arithmetic (q16_quant, the
// same device function as the standalone quantizer: the layout equals k_act16i_from_q16's
// of the rows it writes). One wave per (super-block, padded row); lane l quantizes values
// 4 l .. 4 l + 3, and even lane e = 8 j + 4 hh + 2 h writes both planes of K-step 2 j + h
// of lane half hh with lane e + 1's codes.
__global__ __launch_bounds__(64) void k_act16i_quant(const float* __restrict__ x, int64_t x_stride, int64_t m,
                                                     int64_t k, int64_t m_pad, uint8_t* __restrict__ out) {
  const int l = threadIdx.x;
  const int s = blockIdx.x;
  const int64_t row = blockIdx.y;
  const int nb = (int)(k / 256);
  const auto rx = rsrc(x + (row < m ? row * x_stride : 0), row < m ? (u32)(k * 4) : 0u);
  float v[4];
  load4f(rx, (u32)(((int64_t)s * 256 + 4 * l) * 4), v);
  float d;
  int sum;
  const v2u c = q16_quant(v, d, sum);
  const int src = 4 * ((l + 1) & 63);
  const u32 n0 = (u32)__builtin_amdgcn_ds_bpermute(src, (int)c.x), n1 = (u32)__builtin_amdgcn_ds_bpermute(src, (int)c.y);
  const int64_t T = row >> 5, r = row & 31;
  const int64_t codes_bytes = m_pad * nb * 1024, da_bytes = m_pad / 32 * nb * 1024;
  const int j = l >> 3;
  if ((l & 1) == 0) {
    const int hh = (l >> 2) & 1, kk = 2 * j + ((l >> 1) & 1);
    // values {0, 2, 1, 3} of this lane, {4, 6, 5, 7} of the next: int16 halves of c / n
    const int a[8] = {(int16_t)(c.x & 0xFFFFu), (int16_t)(c.y & 0xFFFFu), (int16_t)(c.x >> 16), (int16_t)(c.y >> 16),
                      (int16_t)(n0 & 0xFFFFu),  (int16_t)(n1 & 0xFFFFu),  (int16_t)(n0 >> 16),  (int16_t)(n1 >> 16)};
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      int q[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = p ? (a[i] >> 8) * 256 : (a[i] & 255);
      *reinterpret_cast<v4u*>(out + (((T * nb + s) * 16 + kk) * 2 + p) * 1024 + (32 * hh + r) * 16) =
          v4u{f16x2(q[0], q[1]), f16x2(q[2], q[3]), f16x2(q[4], q[5]), f16x2(q[6], q[7])};
    }
  }
  if ((l & 7) == 0) {
    float* dab = reinterpret_cast<float*>(out + codes_bytes + (T * nb + s) * 1024);
    dab[j * 32 + r] = d;
    float* cb = reinterpret_cast<float*>(out + codes_bytes + da_bytes + (T * nb + s) * 1024);
    cb[(j >> 1) * 64 + 32 * (j & 1) + r] = d * (float)sum;
  }
}

// ---------------------------------------------------------------- the GEMM

// One workgroup: activation rows [64 tm, + 64) x weight rows [nbase0 + 256 tn, + 256),
// all super-blocks. Arguments as launch_gemm_q16.
template <int TT>
__global__ __launch_bounds__(kQThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_q4k_q16(
    const uint8_t* __restrict__ qs_plane, const uint8_t* __restrict__ hdr_plane, int nb, int64_t nbase0, int64_t n_pad,
    int64_t n0, int64_t n1, const uint8_t* __restrict__ act, int64_t m_pad, int64_t m, float* __restrict__ y,
    int64_t ys, const float* __restrict__ bias, int tiles_m, int xcd_map, int tiles_n, int nsplit,
    float* __restrict__ part) {
  using X = QLds<TT>;
  extern __shared__ __align__(16) uint8_t lds[];
  const int t = threadIdx.x, lane = t & 63;
  const int li = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);

  // Workgroups with the same weight rows on one XCD (workgroups are dealt to the 8
  // XCDs round-robin), so the activation tiles of a weight tile share its L2.
  // Range sp of nsplit: super-blocks [sb0, sb1) (partial outputs to part when split).
  const int tiles = tiles_m * tiles_n;
  const int sp = __builtin_amdgcn_readfirstlane((int)blockIdx.x / tiles);
  const int L = (int)blockIdx.x - sp * tiles;
  const int sb0 = __builtin_amdgcn_readfirstlane(sp * nb / nsplit), sb1 = __builtin_amdgcn_readfirstlane((sp + 1) * nb / nsplit);
  int tn, tm;
  if (xcd_map) {
    tn = 8 * (L / (8 * tiles_m)) + (L & 7);
    tm = (L >> 3) % tiles_m;
  } else {
    tn = L / tiles_m;
    tm = L - tn * tiles_m;
  }
  tn = __builtin_amdgcn_readfirstlane(tn);
  tm = __builtin_amdgcn_readfirstlane(tm);
  const int64_t nbase = nbase0 + (int64_t)kQN * tn;
  const int64_t mbase = (int64_t)tm * 32 * TT;

  const int64_t codes_bytes = m_pad * nb * 1024, da_bytes = m_pad / 32 * nb * 1024;
  const auto ra = rsrc(act, (u32)(codes_bytes + 2 * da_bytes));
  const auto rq = rsrc(qs_plane, (u32)(n_pad * nb * 128));
  const auto rh = rsrc(hdr_plane, (u32)(n_pad * nb * 16));

  // ---- this wave's loads. Operands of super-block s: blocks jb = 8 wave + i (i < 8) of
  // the buffer = (K-step jb / 4, tile (jb / 2) % 2, plane jb % 2); with piece 0 the
  // activation scales (waves 0, 1) or mins operands (waves 2, 3) of tile wave % 2. The
  // wave's weight row: 64-row group g0 + wave / 2, row 32 (wave & 1) + li; lane half hh
  // loads qs chunks hh, 2 + hh, 4 + hh, 6 + hh of it and its header.
  const u32 g0 = (u32)(nbase >> 6);
  const u32 G = g0 + (u32)(wave >> 1), r64 = (u32)(32 * (wave & 1) + li);
  const u32 vq = (G * (u32)nb * 8u + (u32)hh) * 1024u + r64 * 16u;  // + (s * 8 + 2 g) * 1024
  const u32 vh = (G * (u32)nb * 64u + r64) * 16u;                  // + s * 1024

  auto issue_piece = [&](int s, int i) {
    uint8_t* P = lds + (s & 1) * X::kBuf;
    const int jb = 4 * TT * wave + i;  // = (K-step TT + tile) 2 + plane
    const int kt = jb >> 1;
    const int64_t T = (int64_t)TT * tm + (kt % TT);
    dma16(ra, P + jb * 1024, (u32)(lane * 16), (u32)((((T * nb + s) * 16 + kt / TT) * 2 + (jb & 1)) * 1024));
    if (i == 0 && wave < 4) {
      const int tt = wave & 1;
      const int64_t Tb = (int64_t)TT * tm + tt;
      if (wave < TT) {
        dma16(ra, P + X::kDa + tt * 1024, (u32)(lane * 16), (u32)(codes_bytes + (Tb * nb + s) * 1024));
      } else if (wave >= 2 && wave < 2 + TT) {
        dma16(ra, P + X::kC + tt * 1024, (u32)(lane * 16), (u32)(codes_bytes + da_bytes + (Tb * nb + s) * 1024));
      }
    }
  };
  // The nibbles of the current super-block: nib[g] = qs chunk 2 g + hh, read by the
  // K-steps of sub-blocks 2 g and 2 g + 1 (K-steps 4 g .. 4 g + 3); the MFMA phase
  // reloads nib[g] with the next super-block's after its last use. Super-blocks past
  // the end reload the last one.
  v4u nib[4], hdr, hdr_n;
  auto ld_nib = [&](int s, int g) { return ld16(rq, vq + (u32)((s < nb ? s : nb - 1) * 8 + 2 * g) * 1024u); };
  auto ld_hdr = [&](int s) { return ld16(rh, vh + (u32)(s < nb ? s : nb - 1) * 1024u); };

  v16f_t acc[TT], S[TT], T[TT];
#pragma unroll
  for (int mt = 0; mt < TT; ++mt) {
    acc[mt] = v16f_t{};
    S[mt] = v16f_t{};
  }

  // Super-block s: per sub-block j its two K-steps (two tiles x two planes) and then its
  // fold into T; the next super-block's loads spread over the K-steps, and one of the
  // mins products per sub-block; at the end T into acc.
  auto run_sb = [&](int s) {
    const bool next = s + 1 < sb1;
    hdr_n = ld_hdr(s + 1);
    const uint8_t* P = lds + __builtin_amdgcn_readfirstlane((s & 1) * X::kBuf);
    // this lane's weight row (get_scale_min_k4, quant_formats.h:62-70): sc_j as (sc, sc)
    // 16-bit pairs, m_j, d and dmin
    const u32 scA = hdr.y & 0x3F3F3F3Fu;
    const u32 scB = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
    const u32 mA = hdr.z & 0x3F3F3F3Fu;
    const u32 mB = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
    const float ndm = -h2f(hdr.x >> 16);
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) T[tt] = v16f_t{};
    // mins product kk of tile tt: A = -dmin m_j of this lane's row, B = c of the lane's
    // activation row, K index hh: sub-block 2 kk + hh
    auto mins = [&](int tt, int kk) {
      const int j = 2 * kk + hh;
      const float am = ndm * (float)((j < 4 ? mA : mB) >> (8 * (j & 3)) & 0xFFu);
      const float cv = as_f(lds4v(P + X::kC + ((tt * 4 + kk) * 64 + lane) * 4));
      acc[tt] = mfma_f32_k2(am, cv, acc[tt]);
    };
    // weight operand of K-step k = 2 j + h: sc_j times 8 nibbles of two dwords, in the
    // pair order
    auto build = [&](int k) -> v4u {
      const int j = k >> 1, h = k & 1;
      u32 x0 = nib[j >> 1][2 * h], x1 = nib[j >> 1][2 * h + 1];
      asm volatile("" : "+v"(x0), "+v"(x1));  // keeps this K-step's operand build here
      const u32 sp = __builtin_amdgcn_perm(0u, j < 4 ? scA : scB, sel_u16x2(j & 3));
      if (j & 1) {
        x0 ^= 0x80808080u;  // the plane's high nibbles XOR 8, undone
        x1 ^= 0x80808080u;
        return v4u{mul_bytes((x0 >> 4) & 0x000F000Fu, sp), mul_bytes((x0 >> 12) & 0x000F000Fu, sp),
                   mul_bytes((x1 >> 4) & 0x000F000Fu, sp), mul_bytes((x1 >> 12) & 0x000F000Fu, sp)};
      }
      return v4u{mul_bytes(x0 & 0x000F000Fu, sp), mul_bytes((x0 >> 8) & 0x000F000Fu, sp),
                 mul_bytes(x1 & 0x000F000Fu, sp), mul_bytes((x1 >> 8) & 0x000F000Fu, sp)};
    };
    // da_j of this lane's activation row in tile tt
    auto ld_da = [&](int tt, int j) { return as_f(lds4v(P + X::kDa + ((tt * 8 + j) * 32 + li) * 4)); };
    float da[TT];
    v4u w = build(0);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      __builtin_amdgcn_s_setprio(2);
      if ((k & 1) == 0) {
        // the sub-block's activation scales, used after its two K-steps; the super-block's
        // 4 TT mins products q = tile 4 + pair over the even K-steps (TT = 2: one per even
        // K-step; 1: one every other)
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) da[tt] = ld_da(tt, k >> 1);
        if (TT == 2) {
          mins(k >> 3, (k >> 1) & 3);
        } else if ((k & 3) == 0) {
          mins(0, k >> 2);
        }
      }
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        const v4u alo = lds16(P + (((TT * k + tt) * 2) * 64 + lane) * 16);
        const v4u ahi = lds16(P + (((TT * k + tt) * 2 + 1) * 64 + lane) * 16);
        S[tt] = mfma_h(w, alo, (k & 1) == 0 ? v16f_t{} : S[tt]);
        S[tt] = mfma_h(w, ahi, S[tt]);
      }
      if (k < 15) w = build(k + 1);
      // the next super-block's 4 TT pieces of this wave, evenly over the K-steps
      if (k % (4 / TT) == 0 && next) issue_piece(s + 1, k / (4 / TT));
      if ((k & 3) == 3) nib[k >> 2] = ld_nib(s + 1, k >> 2);
      __builtin_amdgcn_sched_barrier(0);
      if (k & 1) {
        // sub-block j = k / 2 done: T += da_j sc_j P_j over the tiles
        __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
#pragma unroll
          for (int r = 0; r < 16; ++r) T[tt][r] = fmaf(da[tt], S[tt][r], T[tt][r]);
          asm volatile("" : "+v"(T[tt]));  // the sub-block's results exist here, not after later MFMAs
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // acc += d 2^24 T: d of the lane's 16 result rows 8 (r / 4) + 4 hh + r % 4, which lanes
    // 0-31 hold (one weight row each)
    const float d24 = h2f(hdr.x) * 16777216.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int src = 8 * (r >> 2) + 4 * hh + (r & 3);
      const float dr = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * src, __builtin_bit_cast(int, d24)));
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) acc[tt][r] = fmaf(dr, T[tt][r], acc[tt][r]);
    }
  };

  // prologue: the first super-block's operands and weights
#pragma unroll
  for (int i = 0; i < 4 * TT; ++i) issue_piece(sb0, i);
  hdr = ld_hdr(sb0);
#pragma unroll
  for (int g = 0; g < 4; ++g) nib[g] = ld_nib(sb0, g);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  lds_barrier();
#pragma unroll 1
  for (int s = sb0; s < sb1; ++s) {
    run_sb(s);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    hdr = hdr_n;
  }

  // ---- outputs (+ bias): activation row 32 mt + li, weight rows nbase + 32 wave +
  // 8 (r / 4) + 4 hh + r % 4 (four consecutive rows per r / 4)
  const int64_t mrows = m - mbase < 32 * TT ? m - mbase : 32 * TT;
#pragma unroll
  for (int mt = 0; mt < TT; ++mt) {
    const int row = 32 * mt + li;
    if (row >= mrows) continue;
    float* yr = y + (mbase + row) * ys;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t nq = nbase + 32 * wave + 8 * q + 4 * hh;
      if (nsplit > 1) {
        float* pr = part + ((int64_t)sp * m + mbase + row) * ((int64_t)kQN * tiles_n) + (nq - nbase0);
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

// ---------------------------------------------------------------- host

namespace {

// Activation tiles per workgroup by rows: one for few rows, so no MFMA runs on padding.
int q16_tt(int64_t m) { return m <= 32 ? 1 : 2; }

}  // namespace

// Rows of the act16i layout: whole workgroup tiles (32 q16_tt(m) rows).
int64_t act16i_rows(int64_t m) {
  const int64_t am = 32 * q16_tt(m);
  return (m + am - 1) / am * am;
}

int64_t act16i_bytes(int64_t m, int64_t k) {
  const int64_t mp = act16i_rows(m), nb = k / 256;
  return mp * nb * 1024 + 2 * (mp / 32) * nb * 1024;
}

bool gemm_q16_ok(const WeightDev& w, int64_t m, int64_t n0, int64_t n1) {
  if (w.dtype != kQ4_K || m <= 0 || n1 <= n0 || w.nblk <= 0) return false;
  // 32-bit buffer offsets: the qs plane plus one tile's rows past its end, and act16i;
  // the writer's grid has one row of workgroups per 32 padded rows
  if ((w.n_pad + 4 * kRowGroup) * w.nblk * 128 >= (1ll << 32)) return false;
  if (act16i_bytes(m, w.k) >= (1ll << 32) || act16i_rows(m) / 32 > 65535) return false;
  return true;
}

hipError_t launch_act16i_from_q16(const uint8_t* acts, int64_t arb, int64_t m, int64_t k, uint8_t* out,
                                  hipStream_t s) {
  const int64_t mp = act16i_rows(m);
  if (mp / 32 > 65535 || k % 256 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_act16i_from_q16, dim3((unsigned)(k / 256), (unsigned)(mp / 32)), dim3(256), 0, s, acts, arb, m,
                     (int)(k / 256), mp, out);
  return hipGetLastError();
}

int64_t q16_part_bytes(const WeightDev& w, int64_t m, int64_t n0, int64_t n1) {
  const int64_t nbase0 = n0 / kRowGroup * kRowGroup, am = 32 * q16_tt(m);
  const int64_t tiles_n = (n1 - nbase0 + kQN - 1) / kQN, tiles_m = (m + am - 1) / am;
  const int sp = split_ranges(tiles_n * tiles_m, w.cus > 0 ? w.cus : 256, w.nblk);
  return sp > 1 ? (int64_t)sp * m * kQN * tiles_n * 4 : 0;
}

hipError_t launch_act16i_quant(const float* x, int64_t x_stride, int64_t m, int64_t k, uint8_t* out,
                               hipStream_t s) {
  const int64_t mp = act16i_rows(m);
  if (mp > 65535 || k % 256 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_act16i_quant, dim3((unsigned)(k / 256), (unsigned)mp), dim3(64), 0, s, x, x_stride, m, k, mp,
                     out);
  return hipGetLastError();
}

hipError_t launch_gemm_q16(const WeightDev& w, const uint8_t* act, int64_t m, int64_t n0, int64_t n1, float* y,
                           int64_t ys, const float* bias, float* part, hipStream_t s) {
  if (!gemm_q16_ok(w, m, n0, n1)) return hipErrorInvalidValue;
  const int tt = q16_tt(m);
  const int64_t nbase0 = n0 / kRowGroup * kRowGroup;
  const int64_t tiles_n = (n1 - nbase0 + kQN - 1) / kQN;
  const int64_t tiles_m = (m + 32 * tt - 1) / (32 * tt);
  const int nsplit = split_ranges(tiles_n * tiles_m, w.cus > 0 ? w.cus : 256, w.nblk);
  if (nsplit > 1 && (part == nullptr || m > 65535)) return hipErrorInvalidValue;
  const int xcd_map = tiles_n % 8 == 0 ? 1 : 0;
  const void* fn = tt == 1 ? reinterpret_cast<const void*>(&k_gemm_q4k_q16<1>)
                           : reinterpret_cast<const void*>(&k_gemm_q4k_q16<2>);
  const int lds = tt == 1 ? QLds<1>::kTotal : QLds<2>::kTotal;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  const dim3 grid((unsigned)(tiles_n * tiles_m * nsplit));
  if (tt == 1) {
    hipLaunchKernelGGL(k_gemm_q4k_q16<1>, grid, dim3(kQThreads), lds, s, w.plane[0], w.plane[1], (int)w.nblk, nbase0,
                       w.n_pad, n0, n1, act, act16i_rows(m), m, y, ys, bias, (int)tiles_m, xcd_map, (int)tiles_n,
                       nsplit, part);
  } else {
    hipLaunchKernelGGL(k_gemm_q4k_q16<2>, grid, dim3(kQThreads), lds, s, w.plane[0], w.plane[1], (int)w.nblk, nbase0,
                       w.n_pad, n0, n1, act, act16i_rows(m), m, y, ys, bias, (int)tiles_m, xcd_map, (int)tiles_n,
                       nsplit, part);
  }
  if (nsplit > 1) {
    const hipError_t e2 = hipGetLastError();
    if (e2 != hipSuccess) return e2;
    return launch_split_sum(part, nsplit, m, kQN * tiles_n, nbase0, n0, n1, y, ys, bias, s);
  }
  return hipGetLastError();
}

}  // namespace dq
