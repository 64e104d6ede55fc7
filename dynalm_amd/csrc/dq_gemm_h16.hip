// dq_gemm_h16.hip -- prefill GEMM for Q4_K weights x Q8_K activations on the f16
// matrix cores, with operands that hold the integers exactly, and the activation
// layout it reads.
//
// Arithmetic. Per super-block b and output (m, n) the exact integers of the
// reference's super-block kernel (dynacore/cpu/avx2/kernels_avx2.cpp:976-1014),
//   S  = sum_j sc_j * P_j,   P_j = sum_t q_{j,t} a_{j,t}   (q: the nibbles, a: Q8_K codes)
//   Mn = sum_j m_j * (code sum of sub-block j)
// then the library's canonical fp32 order
//   u = d * (float)S;  u = fma(-dmin, Mn, u);  acc = fma(da, u, acc).
// S runs on v_mfma_f32_32x32x16_f16 with
//   A = the activation codes as f16 (integers of at most 127: exact), and
//   B = sc_j * q as the raw 16-bit integer (at most 63 * 15 = 945 < 1024), which the
//       matrix core reads as the f16 subnormal sc_j * q * 2^-24,
// so every product is exact in fp32 and every partial sum is a multiple of 2^-24:
// while every partial |S| stays below 2^24 the accumulator ends at exactly S * 2^-24,
// and u = (S * 2^-24) * (d * 2^24) rounds once, as d * (float)S does. Mn likewise:
// A = the 16 bsums as f16 (|bsum| <= 2048, exact), B = m_j as raw bits (m_j * 2^-24),
// and fma(-dmin * 2^24, Mn * 2^-24, u) is fma(-dmin, Mn, u). The outputs are then
// bit-identical to the GEMV kernels and the oracle. |S| can pass 2^24 only when codes
// and scales are both close to saturated over most of a super-block (its bound is
// 128 * 945 * 256 = 2^24.9); past it the matrix core rounds the running sum to fp32,
// a relative error of at most 2^-24 per K-step, which stays far inside the fp32
// tolerance (the GEMV, summing in int32, stays exact there). The B operands are built
// with integer operations only (mask, shift, one packed 16-bit multiply per two
// values), 12 per K-step; fp32 VALU work interferes with the matrix core on gfx950
// far more than integer work does.
//
// Work split. A workgroup owns 128 activation rows x 256 weight rows with 8 waves,
// two per SIMD. Wave w owns weight rows 32 w .. 32 w + 31 of the tile against all
// four 32-row activation tiles; each lane holds one weight row (its output column)
// and builds that row's B operands in registers from nibbles it loads itself, each
// B operand serving four MFMAs (four independent accumulation chains). Interval s is
// super-block s for every wave: its 64 MFMAs, between which the wave issues its
// eighth of super-block s + 1's activation operands (one 1 KB direct-to-LDS buffer
// load every other K-step: a burst of them stalls the wave's in-order issue) and
// reloads its nibbles as they free up; then the fp32 epilogue of super-block s; then
// a wait for its own loads and one workgroup barrier. The operands of a super-block
// (128 rows x 256 codes as f16, 64 KB) and its bsums and scales are loaded one
// interval ahead into a ring of two.
//
// Activation layout ("act16", written by k_act16_from_q8k from Q8_K rows or by
// k_act16_quant from fp32 rows), for M_pad = m rounded up to 128 rows (zero rows
// past m), T = M_pad / 32 row tiles and nb super-blocks per row:
//   codes  [T][nb][k (16)][lane (64)][8 halves]  lane l: row 32 T + l % 32, half
//          hh = l / 32; halves i = values v + {0, 2, 1, 3, 32, 34, 33, 35} of the
//          super-block, v = 64 (2 hh + k / 8) + 4 (k % 8)
//   bsums  [T][nb][lane (64)][8 halves]  bsum groups 8 hh .. 8 hh + 7 as f16
//   da     [nb][M_pad] floats
// so each MFMA operand block (one K-step of 32 rows) is 1 KB contiguous, in the
// lane order the matrix core reads it. The K order is the one in which a lane's
// B operand comes out of one dword of its weight row's nibbles: K-step k of lane
// half hh is qs dword 16 hh + k, whose four bytes hold values v .. v + 3 (low
// nibbles, sub-block 2 g) and v + 32 .. v + 35 (high nibbles, sub-block 2 g + 1),
// g = 2 hh + k / 8 (quant_formats.cpp:150-167; the plane stores the high nibbles
// XOR 8).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dq_device.h"
#include "dq_f16mma.h"
#include "dq_internal.h"
#include "dq_mfma.h"
#include "dq_quant.h"

namespace dq {

namespace {

constexpr int kHM = 128, kHN = 256;  // activation rows x weight rows per workgroup
constexpr int kHThreads = 512;       // 8 waves, two per SIMD
// Operand buffer of a super-block: activation operands [k (16)][t (4)][lane (64)][16 B].
constexpr int kHPos = 65536;
// Super-block buffer: bsums [t (4)][lane (64)][16 B], then 128 activation scales.
constexpr int kHBs = 0, kHDa = 4096, kHSb = 4608;
constexpr int kHSbBase = 2 * kHPos;
constexpr int kHLds = kHSbBase + 2 * kHSb;
static_assert(kHLds <= 160 * 1024, "LDS");

}  // namespace

// ---------------------------------------------------------------- act16 writers

// Q8_K rows (292 B per super-block: float d, int8 codes[256], int16 bsums[16]) ->
// act16. Workgroup (s, T): one 32-row tile's super-block s; rows past m are zeros.
__global__ __launch_bounds__(256) void k_act16_from_q8k(const uint8_t* __restrict__ acts, int64_t arb, int64_t m,
                                                        int nb, int64_t m_pad, uint8_t* __restrict__ out) {
  const int t = threadIdx.x;
  const int s = blockIdx.x;
  const int64_t T = blockIdx.y;
  const int64_t codes_bytes = m_pad * nb * 512, bs_bytes = m_pad / 32 * nb * 1024;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int u = t + 256 * e, k = u >> 6, l = u & 63, hh = l >> 5;
    const int64_t row = 32 * T + (l & 31);
    const int v = 64 * (2 * hh + (k >> 3)) + 4 * (k & 7);
    v4u o = {0u, 0u, 0u, 0u};
    if (row < m) {
      const uint8_t* q = acts + row * arb + (int64_t)s * 292 + 4;
      o = codes_f16(*reinterpret_cast<const u32*>(q + v), *reinterpret_cast<const u32*>(q + v + 32));
    }
    *reinterpret_cast<v4u*>(out + ((T * nb + s) * 16 + k) * 1024 + l * 16) = o;
  }
  if (t < 64) {
    const int l = t, hh = l >> 5;
    const int64_t row = 32 * T + (l & 31);
    v4u o = {0u, 0u, 0u, 0u};
    if (row < m) {
      const int16_t* bs = reinterpret_cast<const int16_t*>(acts + row * arb + (int64_t)s * 292 + 260) + 8 * hh;
      o = v4u{f16_pair(bs[0], bs[1]), f16_pair(bs[2], bs[3]), f16_pair(bs[4], bs[5]), f16_pair(bs[6], bs[7])};
    }
    *reinterpret_cast<v4u*>(out + codes_bytes + (T * nb + s) * 1024 + l * 16) = o;
  } else if (t < 96) {
    const int64_t row = 32 * T + (t - 64);
    const float d = row < m ? *reinterpret_cast<const float*>(acts + row * arb + (int64_t)s * 292) : 0.0f;
    *reinterpret_cast<float*>(out + codes_bytes + bs_bytes + ((int64_t)s * m_pad + row) * 4) = d;
  }
}

// fp32 rows -> act16 directly, with the Q8_K quantizer's arithmetic (q8k_quant, the
// same device function as k_quant_q8k: the codes, bsums and d are its bytes). One
// wave per (super-block, row) of the padded rows; rows past m read zeros.
__global__ __launch_bounds__(64) void k_act16_quant(const float* __restrict__ x, int64_t x_stride, int64_t m,
                                                    int64_t k, int64_t m_pad, uint8_t* __restrict__ out) {
  __shared__ int bsl[16];
  const int l = threadIdx.x;
  const int s = blockIdx.x;
  const int64_t row = blockIdx.y;
  const int nb = (int)(k / 256);
  const auto rx = rsrc(x + (row < m ? row * x_stride : 0), row < m ? (u32)(k * 4) : 0u);
  float v[4];
  load4f(rx, (u32)(((int64_t)s * 256 + 4 * l) * 4), v);
  float d;
  int bsum;
  const u32 packed = q8k_quant(v, d, bsum);
  // lane L (L % 16 < 8) writes the unit of K-step k = 8 ((L / 16) & 1) + L % 8, half
  // hh = L / 32: its own codes (values 4 L ..) and those of lane L + 8 (values 4 L + 32 ..)
  const u32 other = (u32)dpp<kRowRor8>((int)packed);
  const int64_t T = row >> 5;
  const int64_t codes_bytes = m_pad * nb * 512, bs_bytes = m_pad / 32 * nb * 1024;
  if ((l & 15) < 8) {
    const int hh = l >> 5, kk = 8 * ((l >> 4) & 1) + (l & 7);
    *reinterpret_cast<v4u*>(out + ((T * nb + s) * 16 + kk) * 1024 + (32 * hh + (row & 31)) * 16) =
        codes_f16(packed, other);
  }
  if ((l & 3) == 0) bsl[l >> 2] = bsum;
  __syncthreads();
  if (l < 2) {
    const int* b = bsl + 8 * l;
    *reinterpret_cast<v4u*>(out + codes_bytes + (T * nb + s) * 1024 + (32 * l + (row & 31)) * 16) =
        v4u{f16_pair(b[0], b[1]), f16_pair(b[2], b[3]), f16_pair(b[4], b[5]), f16_pair(b[6], b[7])};
  } else if (l == 2) {
    *reinterpret_cast<float*>(out + codes_bytes + bs_bytes + ((int64_t)s * m_pad + row) * 4) = d;
  }
}

// ---------------------------------------------------------------- the GEMM

// One workgroup: activation rows [128 tm, + 128) x weight rows [nbase0 + 256 tn, + 256),
// all super-blocks. Arguments as launch_gemm_h16.
__global__ __launch_bounds__(kHThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_q4k_h16(
    const uint8_t* __restrict__ qs_plane, const uint8_t* __restrict__ hdr_plane, int nb, int64_t nbase0, int64_t n_pad,
    int64_t n0, int64_t n1, const uint8_t* __restrict__ act16, int64_t m_pad, int64_t m, float* __restrict__ y,
    int64_t ys, const float* __restrict__ bias, int tiles_m, int xcd_map) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int t = threadIdx.x, lane = t & 63;
  const int li = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);

  // Workgroups with the same weight rows on one XCD (workgroups are dealt to the 8
  // XCDs round-robin), so the activation tiles of a weight tile share its L2.
  const int L = blockIdx.x;
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
  const int64_t nbase = nbase0 + (int64_t)kHN * tn;
  const int64_t mbase = (int64_t)tm * kHM;

  const int64_t codes_bytes = m_pad * nb * 512, bs_bytes = m_pad / 32 * nb * 1024;
  const auto ra = rsrc(act16, (u32)(codes_bytes + bs_bytes + (int64_t)nb * m_pad * 4));
  const auto rq = rsrc(qs_plane, (u32)(n_pad * nb * 128));
  const auto rh = rsrc(hdr_plane, (u32)(n_pad * nb * 16));

  // ---- this wave's loads. Activation operands of super-block s: blocks j = 8 wave + i
  // (i < 8) of the operand buffer, K-step j / 4 of tile j % 4; bsums of tile `wave`
  // (waves 0-3) or 64 activation scales (waves 4, 5). The wave's weight row: 64-row
  // group g0 + wave / 2, row 32 (wave & 1) + li; lane half hh loads qs chunks
  // 4 hh .. 4 hh + 3 of it and its header.
  const u32 g0 = (u32)(nbase >> 6);
  const u32 G = g0 + (u32)(wave >> 1), r64 = (u32)(32 * (wave & 1) + li);
  const u32 vq = (G * (u32)nb * 8u + 4u * (u32)hh) * 1024u + r64 * 16u;  // + (s * 8 + e) * 1024
  const u32 vh = (G * (u32)nb * 64u + r64) * 16u;                        // + s * 1024

  // Piece i (< 8) of super-block s's operands into buffer s & 1 (and, with piece 0,
  // its bsums or scales into super-block buffer s & 1).
  auto issue_piece = [&](int s, int i) {
    uint8_t* P = lds + (s & 1) * kHPos;
    const int j = 8 * wave + i;
    const int64_t T = 4 * (int64_t)tm + (j & 3);
    dma16(ra, P + j * 1024, (u32)(lane * 16), (u32)(((T * nb + s) * 16 + (j >> 2)) * 1024));
    if (i == 0) {
      uint8_t* B = lds + kHSbBase + (s & 1) * kHSb;
      if (wave < 4) {
        const int64_t Tb = 4 * (int64_t)tm + wave;
        dma16(ra, B + kHBs + wave * 1024, (u32)(lane * 16), (u32)(codes_bytes + (Tb * nb + s) * 1024));
      } else if (wave < 6) {
        dma4(ra, B + kHDa + (wave - 4) * 256, (u32)(lane * 4),
             (u32)(codes_bytes + bs_bytes + ((int64_t)s * m_pad + mbase + 64 * (wave - 4)) * 4));
      }
    }
  };
  // The nibbles of the current super-block (dword k = 4 e + i of nib[e] is K-step k);
  // the MFMA phase reloads nib[e] with the next super-block's once its last K-step has
  // used it. Super-blocks past the end reload the last one.
  v4u nib[4], hdr, hdr_n;
  auto ld_nib = [&](int s, int e) { return ld16(rq, vq + (u32)((s < nb ? s : nb - 1) * 8 + e) * 1024u); };
  auto ld_hdr = [&](int s) { return ld16(rh, vh + (u32)(s < nb ? s : nb - 1) * 1024u); };

  float acc[4][16];
  v16f_t S[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[mt][r] = 0.0f;
    S[mt] = v16f_t{};
  }

  // MFMAs of super-block s (header hdr, nibbles nib): four chains, one per activation
  // tile. Spread over its K-steps, the next super-block's loads: its operands into the
  // other buffer (read one interval earlier), its header and, as they free up, its
  // nibbles. Issuing the operands in one burst instead stalls the waves at the
  // interval start (in-order issue behind the queued loads).
  auto mfma_sb = [&](int s) {
    // the MFMA phase outranks the other wave's epilogue: a dense fp32 VALU stream from
    // one wave otherwise delays the other's MFMA issue (measured: 4% per launch)
    __builtin_amdgcn_s_setprio(2);
    const bool next = s + 1 < nb;
    hdr_n = ld_hdr(s + 1);
    const uint8_t* P = lds + __builtin_amdgcn_readfirstlane((s & 1) * kHPos);
    // scale pairs (sc_j, sc_j) of this lane's sub-blocks 4 hh .. 4 hh + 3
    // (get_scale_min_k4, quant_formats.h:62-70)
    const u32 scA = hdr.y & 0x3F3F3F3Fu;
    const u32 scB = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
    const u32 scx = hh ? scB : scA;
    const u32 sp0 = __builtin_amdgcn_perm(0u, scx, sel_u16x2(0)), sp1 = __builtin_amdgcn_perm(0u, scx, sel_u16x2(1));
    const u32 sp2 = __builtin_amdgcn_perm(0u, scx, sel_u16x2(2)), sp3 = __builtin_amdgcn_perm(0u, scx, sel_u16x2(3));
    // Software pipeline: K-step k issues its four MFMAs, then builds step k + 1's B
    // operand and reads step k + 1's activation operands while the matrix core works.
    auto build = [&](int k) -> v4u {
      u32 x = nib[k >> 2][k & 3];
      asm volatile("" : "+v"(x));  // keeps this K-step's operand build here
      const u32 y = x ^ 0x80808080u;  // the plane's high nibbles XOR 8, undone
      const u32 lo = k < 8 ? sp0 : sp2, hi = k < 8 ? sp1 : sp3;
      return v4u{mul_bytes(x & 0x000F000Fu, lo), mul_bytes((x >> 8) & 0x000F000Fu, lo),
                 mul_bytes((y >> 4) & 0x000F000Fu, hi), mul_bytes((y >> 12) & 0x000F000Fu, hi)};
    };
    v4u a[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) a[t] = lds16(P + (t * 64 + lane) * 16);
    v4u b = build(0);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      v4u an[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        S[t] = mfma_h(a[t], b, k == 0 ? v16f_t{} : S[t]);
        an[t] = k < 15 ? lds16(P + ((4 * (k + 1) + t) * 64 + lane) * 16) : a[t];
      }
      if (k < 15) b = build(k + 1);
#pragma unroll
      for (int t = 0; t < 4; ++t) a[t] = an[t];
      if ((k & 1) == 0 && next) issue_piece(s + 1, k >> 1);
      if ((k & 3) == 3) nib[k >> 2] = ld_nib(s + 1, k >> 2);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // The canonical epilogue of super-block s's four tiles, header he.
  auto epi_sb = [&](int s, const v4u& he) {
    __builtin_amdgcn_s_setprio(0);
    const uint8_t* SB = lds + kHSbBase + __builtin_amdgcn_readfirstlane((s & 1) * kHSb);
    const float d24 = h2f(he.x) * 16777216.0f, ndm24 = -h2f(he.x >> 16) * 16777216.0f;
    // Mn's B operand: m_j of sub-blocks 4 hh .. 4 hh + 3, each for two bsum groups, raw bits
    const u32 mA = he.z & 0x3F3F3F3Fu;
    const u32 mB = ((he.w >> 4) & 0x0F0F0F0Fu) | ((he.z >> 2) & 0x30303030u);
    u32 mx = hh ? mB : mA;
    // the epilogue's operands are made here, not hoisted into the MFMA phase before it
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" : "+v"(mx));
    const v4u bmn = {__builtin_amdgcn_perm(0u, mx, sel_u16x2(0)), __builtin_amdgcn_perm(0u, mx, sel_u16x2(1)),
                     __builtin_amdgcn_perm(0u, mx, sel_u16x2(2)), __builtin_amdgcn_perm(0u, mx, sel_u16x2(3))};
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      // the tile's loads together: bsums, then the activation scales of rows
      // 32 tt + 8 q + 4 hh .. + 3 (results r = 4 q .. 4 q + 3)
      const v4u bs = lds16v(SB + kHBs + (tt * 64 + lane) * 16);
      v4u da[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) da[q] = lds16v(SB + kHDa + (32 * tt + 8 * q + 4 * hh) * 4);
      const v16f_t Mn = mfma_h(bs, bmn, v16f_t{});
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float u = S[tt][r] * d24;
        u = fmaf(ndm24, Mn[r], u);
        acc[tt][r] = fmaf(as_f(da[r >> 2][r & 3]), u, acc[tt][r]);
      }
      // this tile's results exist before the next tile's loads
#pragma unroll
      for (int r = 0; r < 16; r += 4)
        asm volatile("" ::"v"(acc[tt][r]), "v"(acc[tt][r + 1]), "v"(acc[tt][r + 2]), "v"(acc[tt][r + 3]));
    }
  };

  // prologue: the first super-block's operands and weights
#pragma unroll
  for (int i = 0; i < 8; ++i) issue_piece(0, i);
  hdr = ld_hdr(0);
#pragma unroll
  for (int e = 0; e < 4; ++e) nib[e] = ld_nib(0, e);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  lds_barrier();
  // Interval s: the MFMAs of super-block s (and the next one's loads), then its
  // epilogue; then every load of the interval has landed and the workgroup barrier.
#pragma unroll 1
  for (int s = 0; s < nb; ++s) {
    mfma_sb(s);
    epi_sb(s, hdr);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    hdr = hdr_n;
  }

  // ---- outputs (+ bias): rows 32 mt + 8 (r / 4) + 4 hh + r % 4, weight row nbase + 32 wave + li
  const int64_t n = nbase + 32 * wave + li;
  const int64_t mrows = m - mbase < kHM ? m - mbase : kHM;
  if (n >= n0 && n < n1) {
    const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 32 * mt + 8 * (r >> 2) + 4 * hh + (r & 3);
        if (row < mrows) {
          const float v = acc[mt][r];
          y[(mbase + row) * ys + n] = bias ? v + bv : v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------- host side

int64_t act16_rows(int64_t m) { return (m + kHM - 1) / kHM * kHM; }

int64_t act16_bytes(int64_t m, int64_t k) {
  const int64_t mp = act16_rows(m), nb = k / 256;
  return mp * k * 2 + mp / 32 * nb * 1024 + nb * mp * 4;
}

bool gemm_h16_ok(const WeightDev& w, int64_t m, int64_t n0, int64_t n1) {
  if (w.dtype != kQ4_K || m <= 0 || n1 <= n0 || w.nblk <= 0) return false;
  // 32-bit buffer offsets: the qs plane plus one tile's rows past its end, and act16;
  // the act16 quantizer's grid has one row of workgroups per padded row
  if ((w.n_pad + 4 * kRowGroup) * w.nblk * 128 >= (1ll << 32)) return false;
  if (act16_bytes(m, w.k) >= (1ll << 32) || act16_rows(m) > 65535) return false;
  return true;
}

bool gemm_h16_pays(const WeightDev& w, int64_t m, int64_t n0, int64_t n1) {
  if (m <= 128 || !gemm_h16_ok(w, m, n0, n1)) return false;
  const int cus = w.cus > 0 ? w.cus : 256;
  const int64_t rows = n1 - (n0 / kRowGroup) * kRowGroup;
  const int64_t wgs = (rows + kHN - 1) / kHN * ((m + kHM - 1) / kHM);
  return wgs * 8 >= (int64_t)cus * 5;
}

hipError_t launch_act16_from_q8k(const uint8_t* acts, int64_t arb, int64_t m, int64_t k, uint8_t* out,
                                 hipStream_t s) {
  const int64_t mp = act16_rows(m);
  hipLaunchKernelGGL(k_act16_from_q8k, dim3((unsigned)(k / 256), (unsigned)(mp / 32)), dim3(256), 0, s, acts, arb, m,
                     (int)(k / 256), mp, out);
  return hipGetLastError();
}

hipError_t launch_act16_quant(const float* x, int64_t x_stride, int64_t m, int64_t k, uint8_t* out, hipStream_t s) {
  const int64_t mp = act16_rows(m);
  if (mp > 65535 || k % 256 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_act16_quant, dim3((unsigned)(k / 256), (unsigned)mp), dim3(64), 0, s, x, x_stride, m, k, mp,
                     out);
  return hipGetLastError();
}

hipError_t launch_gemm_h16(const WeightDev& w, const uint8_t* act16, int64_t m, int64_t n0, int64_t n1, float* y,
                           int64_t ys, const float* bias, hipStream_t s) {
  if (!gemm_h16_ok(w, m, n0, n1)) return hipErrorInvalidValue;
  const int64_t nbase0 = n0 / kRowGroup * kRowGroup;
  const int64_t tiles_n = (n1 - nbase0 + kHN - 1) / kHN;
  const int64_t tiles_m = (m + kHM - 1) / kHM;
  const int xcd_map = tiles_n % 8 == 0 ? 1 : 0;
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm_q4k_h16),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kHLds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_gemm_q4k_h16, dim3((unsigned)(tiles_n * tiles_m)), dim3(kHThreads), kHLds, s, w.plane[0],
                     w.plane[1], (int)w.nblk, nbase0, w.n_pad, n0, n1, act16, act16_rows(m), m, y, ys, bias,
                     (int)tiles_m, xcd_map);
  return hipGetLastError();
}

}  // namespace dq
