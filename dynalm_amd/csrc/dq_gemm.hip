// dq_gemm.hip -- prefill GEMM for Q4_K and Q6_K weights x Q8_K activations on gfx950 int8
// MFMA (v_mfma_i32_16x16x64_i8) with the mins on fp16 MFMA (v_mfma_f32_16x16x16_f16).
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
// S: the effective integer weight sc*q (0..945) does not fit int8. With
// sc = 8*sh + sl (sh, sl in 0..7), sh*q and sl*q are at most 105, so each fits a
// byte and a packed 16-bit multiply of four nibble bytes by sh (or sl) makes four
// of them at once without carries. Two int8 MFMA chains per output give
//   S = 8 * sum(sh*q*a) + sum(sl*q*a)
// exactly in int32.
// Mn: the Q8_K block carries the code sums of its 16-value groups (|bsum| <= 2048,
// exact in fp16) and m_j <= 63, so one fp16 MFMA over the 16 bsums against m_j
// sums 16 integer products of at most 2^17 each to at most 2^21: every partial sum
// is an integer below 2^24, so the fp32 result is exactly (float)Mn.
//
// Two kernel families, both with 16 x 16 output tiles per MFMA and one wave owning
// 16 MTW (64 unless stated) activation rows x 16*NT weight rows:
// - k_gemm_q4k<WM, NT, MTW> (up to 128 rows): 4 waves, one per SIMD, WM along the
//   activation rows (MTW = 1, 2 or 4 activation tiles each: shorter waves and more
//   workgroups for small launches). Per super-block a wave holds its rows' activation
//   operands (4 KB per tile) in registers and walks its
//   NT weight tiles; for each it unpacks the nibbles, scales and mins of 16 weight
//   rows itself (three stages: LDS reads of tile nt + 2, unpacking of nt + 1, MFMAs
//   of nt). Activation codes (swizzled), nibbles and headers reach LDS by
//   direct-to-LDS buffer loads into two buffers (loads of b + 1 issued when b
//   starts, one barrier per super-block).
// - k_gemm_q4k_big<WM, WN, NT> (more rows): WM x WN waves, two per SIMD. Each
//   16-row weight tile is unpacked once per workgroup into the sh*q / sl*q bytes of
//   the MFMA operand layout in LDS (phase 1), then every wave runs its MFMAs and
//   epilogues reading them (phase 2, software-pipelined: a tile's epilogue runs
//   after the next tile's MFMAs are issued).
// On gfx950 the matrix core hides about two VALU operations per MFMA and little
// more (measured with microbenchmarks on MI355X), so the kernels are arranged to
// keep the VALU work per MFMA low rather than to overlap large VALU phases.
//
// MFMA operand layout (16x16x64 i8): lane l supplies row (A) / column (B) l%16 and
// 16 K-values of lane group g = l/16; the result lane l holds column l%16, rows
// 4g .. 4g+3. The 256 values of a super-block are dealt to (K-step s, lane group
// g) so that each lane's 16 values are one half of one 16-byte nibble chunk of the
// weight row: chunk c = g + 4*(s>>1), low nibbles for even s, high for odd s. Chunk
// c holds values 64(c>>1) + 16(c&1) + i (low) and the same + 32 (high)
// (dynacore/src/quantization/quant_formats.cpp:150-167), so lane group g at step
// s covers values 16*q .. 16*q + 15 with q = 4(g>>1) + (g&1) + 8(s>>1) + 2(s&1),
// all of sub-block j = 2(g>>1) + 4(s>>1) + (s&1). The activation operand takes the
// same 16 values, so the product is the plain dot product in a permuted K order.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <array>
#include <cstdlib>

#include "dq_device.h"
#include "dq_internal.h"
#include "dq_mfma.h"

namespace dq {

namespace {

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 waves, one per SIMD

// LDS layout of one super-block's operands (bytes); two such buffers. WM waves along the
// activation rows, each owning MTW 16-row activation tiles.
template <int WM, int NT, int MTW = 4>
struct Cfg {
  static constexpr int kWN = 4 / WM;               // waves along the weight rows
  static constexpr int kBM = 16 * MTW * WM;        // activation rows per workgroup
  static constexpr int kBN = kWN * 16 * NT;        // weight rows per workgroup
  static constexpr int kWB = (kBN + 63) / 64;      // 64-row load blocks of weight rows
  static constexpr int kWRows = 64 * kWB;
  static constexpr int kA = 0;                     // [kBM][16 chunks][16 B] codes, chunk q at slot q ^ (row & 15)
  static constexpr int kW = kA + kBM * 256;        // [8 chunks][kWRows][16 B] nibbles as in the weight plane
  static constexpr int kH = kW + 8 * kWRows * 16;  // [kWRows][16 B] Q4_K headers {d, dmin, scales[12]}
  static constexpr int kBS = kH + kWRows * 16;     // [kBM][16] bsums as fp16
  static constexpr int kDA = kBS + kBM * 32;       // [kBM] activation scale d (float)
  static constexpr int kBuf = kDA + kBM * 4;
  static constexpr int kLds = 2 * kBuf;
};

DQ_DEV v4u lds_ld16(const uint8_t* lds, int off) { return *reinterpret_cast<const v4u*>(lds + off); }
DQ_DEV v2u lds_ld8(const uint8_t* lds, int off) { return *reinterpret_cast<const v2u*>(lds + off); }

DQ_DEV f4_t mfma_h(h4_t a, h4_t b, f4_t c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }

// Direct-to-LDS buffer load: lane l's `bytes` land at lds_dst + l * bytes.
DQ_DEV void ld_lds16(__amdgpu_buffer_rsrc_t r, uint8_t* lds_dst, u32 voff, u32 soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_dst, 16, voff, soff, 0, 0);
}
DQ_DEV void ld_lds4(__amdgpu_buffer_rsrc_t r, uint8_t* lds_dst, u32 voff, u32 soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_dst, 4, voff, soff, 0, 0);
}

// Eight int16 bsums -> eight fp16 (exact: |bsum| <= 2048).
DQ_DEV v4u bsums_f16(v4u v) {
  v4u o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const _Float16 lo = (_Float16)(short)(v[i] & 0xFFFFu), hi = (_Float16)(short)(v[i] >> 16);
    o[i] = (u32)__builtin_bit_cast(uint16_t, lo) | ((u32)__builtin_bit_cast(uint16_t, hi) << 16);
  }
  return o;
}

// The B side of one 16-row weight tile: raw LDS words, then the MFMA operands.
struct RawB {
  v4u hd, w0, w1;  // header; nibble chunks lg and lg + 4 of the lane's row
};
struct PrepB {
  v4u H[4], L[4];  // sh*q and sl*q bytes of the 4 K-steps
  h4_t mb;         // m_{2lg}, m_{2lg}, m_{2lg+1}, m_{2lg+1} (fp16)
  float d, dmin;
};

// m_{2lg}, m_{2lg}, m_{2lg+1}, m_{2lg+1} of a Q4_K header as fp16 ((1024 + m) - 1024,
// exact), the B operand of the mins MFMA for lane group lg (selector sel_mn).
DQ_DEV h4_t mins_f16(v4u hd, u32 sel_mn) {
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  const u32 mn_lo = hd.z & 0x3F3F3F3Fu;
  const u32 mn_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
  const u32 mm = __builtin_amdgcn_perm(0u, __builtin_amdgcn_perm(mn_hi, mn_lo, sel_mn), 0x0C010C00u) | 0x64006400u;
  const h2_t mf = __builtin_bit_cast(h2_t, mm) - h2_t{(_Float16)1024.0f, (_Float16)1024.0f};
  const u32 mfu = __builtin_bit_cast(u32, mf);
  return __builtin_bit_cast(h4_t, v2u{__builtin_amdgcn_perm(mfu, mfu, 0x01000100u),
                                      __builtin_amdgcn_perm(mfu, mfu, 0x03020302u)});
}

// Unpacks one tile's header and nibbles for this lane (lane group lg: sub-block
// scale bytes selected by sel_sc, mins by sel_mn).
DQ_DEV PrepB prep_tile(const RawB& r, u32 sel_sc, u32 sel_mn) {
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  PrepB p;
  p.d = h2f(r.hd.x);
  p.dmin = h2f(r.hd.x >> 16);
  // get_scale_min_k4 (dynacore/include/dynacore/quantization/quant_formats.h:62-70)
  // for all eight sub-blocks as bytes: sc_lo / mn_lo j = 0..3, sc_hi / mn_hi j = 4..7
  const u32 sc_lo = r.hd.y & 0x3F3F3F3Fu, mn_lo = r.hd.z & 0x3F3F3F3Fu;
  const u32 sc_hi = (r.hd.w & 0x0F0F0F0Fu) | ((r.hd.y >> 2) & 0x30303030u);
  const u32 mn_hi = ((r.hd.w >> 4) & 0x0F0F0F0Fu) | ((r.hd.z >> 2) & 0x30303030u);
  const u32 sc = __builtin_amdgcn_perm(sc_hi, sc_lo, sel_sc);  // byte s: scale of step s
  const u32 SH = (sc >> 3) & 0x07070707u, SL = sc & 0x07070707u;
  // m_{2lg}, m_{2lg+1} as fp16: (1024 + m) - 1024, exact
  const u32 mm = __builtin_amdgcn_perm(0u, __builtin_amdgcn_perm(mn_hi, mn_lo, sel_mn), 0x0C010C00u) | 0x64006400u;
  const h2_t mf = __builtin_bit_cast(h2_t, mm) - h2_t{(_Float16)1024.0f, (_Float16)1024.0f};
  const u32 mfu = __builtin_bit_cast(u32, mf);
  p.mb = __builtin_bit_cast(h4_t, v2u{__builtin_amdgcn_perm(mfu, mfu, 0x01000100u),
                                      __builtin_amdgcn_perm(mfu, mfu, 0x03020302u)});
  // the 4 steps' nibbles as bytes (high nibbles are stored XOR 8, dq_layout.h)
  v4u qb[4];
  qb[0] = r.w0 & 0x0F0F0F0Fu;
  qb[1] = ((r.w0 >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
  qb[2] = r.w1 & 0x0F0F0F0Fu;
  qb[3] = ((r.w1 >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const u32 kh = __builtin_amdgcn_perm(0u, SH, sel_u16x2(s));
    const u32 kl = __builtin_amdgcn_perm(0u, SL, sel_u16x2(s));
    p.H[s] = v4u{mul_bytes(qb[s].x, kh), mul_bytes(qb[s].y, kh), mul_bytes(qb[s].z, kh), mul_bytes(qb[s].w, kh)};
    p.L[s] = v4u{mul_bytes(qb[s].x, kl), mul_bytes(qb[s].y, kl), mul_bytes(qb[s].z, kl), mul_bytes(qb[s].w, kl)};
  }
  return p;
}

// The B operands of one Q6_K tile row for lane group lg: K-step s takes unit lg + 4s,
// the low (even s) or high (odd s) nibbles of ql chunk lg + 4(s>>1) -- values
// 128p + 16(c%4) + i (+ 64 for the high nibbles) with p = c/4
// (dynacore/src/quantization/quant_formats.cpp:192-216) -- with their top two bits
// from qh chunk 2p + c%2, bit pair (c%4)/2 (+2 for the high nibbles).
DQ_DEV PrepB prep_tile_q6(v4u scw, v4u w0, v4u w1, v4u h0, v4u h1, int lg) {
  PrepB p;
  p.d = 0.0f;
  p.dmin = 0.0f;
  const int sh = 2 * (lg >> 1);
  v4u q[4];
  q[0] = (w0 & 0x0F0F0F0Fu) | (((h0 >> sh) & 0x03030303u) << 4);
  q[1] = ((w0 >> 4) & 0x0F0F0F0Fu) | (((h0 >> (sh + 4)) & 0x03030303u) << 4);
  q[2] = (w1 & 0x0F0F0F0Fu) | (((h1 >> sh) & 0x03030303u) << 4);
  q[3] = ((w1 >> 4) & 0x0F0F0F0Fu) | (((h1 >> (sh + 4)) & 0x03030303u) << 4);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int sc = sbfe(scw[s], 8 * lg, 8);  // scale byte lg + 4s
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      u32 h, l;
      q6_split(q[s][w], sc, h, l);
      p.H[s][w] = h;
      p.L[s][w] = l;
    }
  }
  return p;
}

}  // namespace

template <int WM, int NT, int MTW>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_gemm_q4k(
    const uint8_t* __restrict__ qs_plane, const uint8_t* __restrict__ hdr_plane, int nb, int64_t n_pad, int64_t nt0,
    int64_t n0, int64_t n1, const uint8_t* __restrict__ acts, int64_t arb, int64_t m, float* __restrict__ y, int64_t ys,
    const float* __restrict__ bias, int tiles_n, int tiles_m) {
  using C = Cfg<WM, NT, MTW>;
  extern __shared__ __align__(16) uint8_t lds[];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave % WM, wn = wave / WM;
  const int wr = 16 * MTW * wm;  // the wave's first activation row in the tile
  const int li = lane & 15, lg = lane >> 4;

  // Tile order: workgroup i runs on XCD i % 8; consecutive logical tiles (the
  // activation tiles of one weight tile) go to one XCD so that its L2 serves the
  // weight tile to all of them.
  int L = blockIdx.x;
  const int per = (tiles_n * tiles_m) / 8;
  if (L < 8 * per) L = (L % 8) * per + L / 8;
  const int tn = __builtin_amdgcn_readfirstlane(L / tiles_m);
  const int tm = __builtin_amdgcn_readfirstlane(L - tn * tiles_m);
  const int64_t nbase = nt0 + (int64_t)tn * C::kBN;  // first weight row of the tile
  const int64_t mbase = (int64_t)tm * C::kBM;
  const int64_t mrows = m - mbase < C::kBM ? m - mbase : C::kBM;

  // ---- global sources (buffer resources: reads past the end return zeros)
  const auto ra = rsrc(acts + mbase * arb, (u32)(mrows * arb));
  const int64_t G0 = nbase >> 6;
  const int goff = (int)(nbase & 63);
  const int64_t gl = n_pad / kRowGroup - G0;
  const int64_t gspan = gl < C::kWB + 1 ? gl : C::kWB + 1;
  const auto rq = rsrc(qs_plane + G0 * nb * 8192, (u32)(gspan * nb * 8192));
  const auto rh = rsrc(hdr_plane + G0 * nb * 1024, (u32)(gspan * nb * 1024));

  // Per-lane source offsets (super-block 0).
  u32 woff[C::kWB], hoff[C::kWB];
#pragma unroll
  for (int k = 0; k < C::kWB; ++k) {
    const int rr = goff + 64 * k + lane;
    woff[k] = (u32)((rr >> 6) * nb * 8192 + (rr & 63) * 16);
    hoff[k] = (u32)((rr >> 6) * nb * 1024 + (rr & 63) * 16);
  }
  constexpr int kAI = C::kBM / 16;  // activation-code load instructions per wave (4 rows each)
  u32 aoff[kAI];
#pragma unroll
  for (int j = 0; j < kAI; ++j) {
    const int row = 4 * (wave * kAI + j) + (lane >> 4);
    const int q = (lane & 15) ^ (row & 15);
    aoff[j] = (u32)(row * arb + 4 + 16 * q);
  }
  const bool bs_role = t < 2 * C::kBM;
  const int bs_row = t >> 1, bs_half = t & 1;
  const u32 bs_off = (u32)(bs_row * arb + 260 + 16 * bs_half);

  auto issue = [&](int b, uint8_t* Lb) {
    // activation codes
#pragma unroll
    for (int j = 0; j < kAI; ++j) ld_lds16(ra, Lb + C::kA + 4 * (wave * kAI + j) * 256, aoff[j], (u32)(b * 292));
    // weight nibbles: wave w stages chunks 2w and 2w + 1 of every 64-row block
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      const int c = 2 * wave + cc;
#pragma unroll
      for (int k = 0; k < C::kWB; ++k) {
        if (k + 1 < C::kWB || 64 * k + lane < C::kBN) {
          ld_lds16(rq, Lb + C::kW + (c * C::kWRows + 64 * k) * 16, woff[k], (u32)(b * 8192 + c * 1024));
        }
      }
    }
    // headers
#pragma unroll
    for (int k = 0; k < C::kWB; ++k) {
      if (k % 4 == wave && (k + 1 < C::kWB || 64 * k + lane < C::kBN)) {
        ld_lds16(rh, Lb + C::kH + 64 * k * 16, hoff[k], (u32)(b * 1024));
      }
    }
    // activation scales
#pragma unroll
    for (int k = 0; k < (C::kBM + 63) / 64; ++k) {
      if (wave == 3 - k && 64 * k + lane < C::kBM) {
        ld_lds4(ra, Lb + C::kDA + 256 * k, (u32)((64 * k + lane) * arb), (u32)(b * 292));
      }
    }
  };
  auto bs_load = [&](int b) -> v4u { return bs_role ? ld16(ra, bs_off + (u32)(b * 292)) : v4u{0, 0, 0, 0}; };
  auto bs_store = [&](v4u v, uint8_t* Lb) {
    if (bs_role) *reinterpret_cast<v4u*>(Lb + C::kBS + bs_row * 32 + 16 * bs_half) = bsums_f16(v);
  };

  // ---- per-lane LDS read offsets
  const int qlg = 4 * (lg >> 1) + (lg & 1);
  const int arow = wr + li;
  int a_rd[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) a_rd[s] = C::kA + arow * 256 + 16 * ((qlg ^ li) ^ (8 * (s >> 1) + 2 * (s & 1)));
  const int bs_rd = C::kBS + arow * 32 + 8 * lg;
  const int da_rd = C::kDA + (wr + 4 * lg) * 4;
  const int wrow = 16 * NT * wn + li;
  const int w_rd = C::kW + (lg * C::kWRows + wrow) * 16;
  const int h_rd = C::kH + wrow * 16;
  // v_perm selectors: this lane's sub-block scales (j = 2h, 2h+1, 4+2h, 5+2h with
  // h = lg >> 1) and mins (j = 2lg, 2lg + 1)
  const u32 sel_sc = (lg >> 1) ? 0x07060302u : 0x05040100u;
  const u32 sel_mn = 0x0C0C0000u | ((u32)(2 * lg + 1) << 8) | (u32)(2 * lg);
  auto load_b = [&](const uint8_t* Lc, int nt) -> RawB {
    return RawB{lds_ld16(Lc, h_rd + nt * 256), lds_ld16(Lc, w_rd + nt * 256),
                lds_ld16(Lc, w_rd + nt * 256 + 4 * C::kWRows * 16)};
  };
  auto prep_b = [&](const RawB& r) -> PrepB { return prep_tile(r, sel_sc, sel_mn); };

  f4_t acc[NT][MTW];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) acc[nt][mt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // ---- prologue: super-block 0 into buffer 0
  {
    issue(0, lds);
    const v4u v = bs_load(0);
    __builtin_amdgcn_s_waitcnt(0);
    bs_store(v, lds);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

#pragma unroll 1
  for (int b = 0; b < nb; ++b) {
    const uint8_t* Lc = lds + (b & 1) * C::kBuf;
    uint8_t* Ln = lds + ((b & 1) ^ 1) * C::kBuf;
    v4u bsn = {0, 0, 0, 0};
    if (b + 1 < nb) {
      issue(b + 1, Ln);
      bsn = bs_load(b + 1);
    }

    // this super-block's activation operands
    v4u a[MTW][4];
    h4_t am[MTW];
    f4_t da[MTW];
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) {
#pragma unroll
      for (int s = 0; s < 4; ++s) a[mt][s] = lds_ld16(Lc, a_rd[s] + mt * 16 * 256);
      am[mt] = __builtin_bit_cast(h4_t, lds_ld8(Lc, bs_rd + mt * 16 * 32));
      da[mt] = __builtin_bit_cast(f4_t, lds_ld16(Lc, da_rd + mt * 16 * 4));
    }

    // Three stages over the weight tiles, one region per tile: the LDS reads of
    // tile nt + 2, the unpacking of tile nt + 1 and the MFMAs and epilogues of tile
    // nt. The scheduling barrier between regions keeps the compiler from hoisting
    // every tile's operands at once (which would exceed the register file).
    RawB raw[NT];
    PrepB pb[NT];
    raw[0] = load_b(Lc, 0);
    if (NT > 1) raw[1] = load_b(Lc, 1);
    pb[0] = prep_b(raw[0]);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (nt + 2 < NT) raw[nt + 2] = load_b(Lc, nt + 2);
      if (nt + 1 < NT) pb[nt + 1] = prep_b(raw[nt + 1]);
      v4i_t tH[MTW], tL[MTW];
      f4_t tM[MTW];
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) {
        const v4i_t z = {0, 0, 0, 0};
        tH[mt] = mfma(a[mt][0], pb[nt].H[0], z);
        tL[mt] = mfma(a[mt][0], pb[nt].L[0], z);
#pragma unroll
        for (int s = 1; s < 4; ++s) {
          tH[mt] = mfma(a[mt][s], pb[nt].H[s], tH[mt]);
          tL[mt] = mfma(a[mt][s], pb[nt].L[s], tL[mt]);
        }
        tM[mt] = mfma_h(am[mt], pb[nt].mb, f4_t{0.0f, 0.0f, 0.0f, 0.0f});
      }
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int S = tL[mt][e] + (tH[mt][e] << 3);
          float u = pb[nt].d * (float)S;
          u = fmaf(-pb[nt].dmin, tM[mt][e], u);
          acc[nt][mt][e] = fmaf(da[mt][e], u, acc[nt][mt][e]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    if (b + 1 < nb) {
      __builtin_amdgcn_s_waitcnt(0);
      bs_store(bsn, Ln);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // ---- store
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int64_t n = nbase + 16 * NT * wn + 16 * nt + li;
    if (n < n0 || n >= n1) continue;
    const float bn_ = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t mm = mbase + wr + 16 * mt + 4 * lg + e;
        if (mm < m) y[mm * ys + n] = bias ? acc[nt][mt][e] + bn_ : acc[nt][mt][e];
      }
    }
  }
}


// ---------------------------------------------------------------------------
// Large-M kernel: WM x WN waves (two per SIMD), each owning 64 activation rows x
// 16 NT weight rows. Per super-block the B operands are built once per workgroup:
// each wave unpacks 16-row weight tiles into the sh*q / sl*q bytes of the MFMA
// operand layout and stores them in LDS, so the VALU work per MFMA left in the
// compute phase is the fp32 epilogue, about two operations per MFMA.
template <int WT, int WM, int WN, int NT>
struct Big {
  static constexpr bool kQ6 = WT == kQ6_K;
  static constexpr int kWaves = WM * WN, kThreads = 64 * kWaves;
  static constexpr int kBM = 64 * WM, kBN = 16 * NT * WN;  // activation rows x weight rows
  static constexpr int kTiles = NT * WN;                    // 16-row weight tiles
  static constexpr int kPrep = kTiles / kWaves;             // tiles unpacked per wave
  static constexpr int kGroups = kBN / 64;                  // 64-row groups of the weight layout
  static constexpr int kA = 0;                        // [kBM rows][16 slots][16 B] codes, chunk q at slot q ^ (row & 15)
  static constexpr int kHL = kA + kBM * 256;          // [tiles][4 steps][H, L][64 lanes][16 B] B operands
  static constexpr int kW = kHL + kTiles * 8192;      // [8 chunks][kBN rows][16 B] nibbles (Q6_K: ql) as in the plane
  static constexpr int kH = kW + 8 * kBN * 16;        // [kBN rows][16 B] headers (Q6_K: the 16 scales)
  static constexpr int kQH = kH + kBN * 16;           // Q6_K: [4 chunks][kBN rows][16 B] qh
  static constexpr int kBS = kQH + (kQ6 ? 4 * kBN * 16 : 0);  // Q4_K: [kBM rows][16] bsums; Q6_K: [kBN] fp16 d
  static constexpr int kDA = kBS + (kQ6 ? kBN * 2 : kBM * 32);  // [2][kBM rows] activation scale d (two buffers)
  static constexpr int kLds = kDA + 2 * kBM * 4;
  static_assert(kPrep >= 1 && kTiles % kWaves == 0, "each wave unpacks whole tiles");
  static_assert(kBN % 64 == 0 && (8 * kGroups) % kWaves == 0, "staging roles");
  static_assert(kQ6 ? (4 * kGroups) % kWaves == 0 : kBM / 32 <= kWaves, "staging roles");
  static constexpr int kAJ = kBM / (4 * kWaves);  // activation-code instructions per wave (4 rows each)
  static_assert(kBM % (16 * kWaves) == 0 && kAJ <= 8, "staging roles");
  static_assert(kLds <= 160 * 1024, "LDS");
};

template <int WT, int WM, int WN, int NT>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_q4k_big(
    const uint8_t* __restrict__ qs_plane, const uint8_t* __restrict__ hdr_plane, const uint8_t* __restrict__ plane2,
    const uint8_t* __restrict__ plane3, int nb, int64_t n_pad, int64_t nt0,
    int64_t n0, int64_t n1, const uint8_t* __restrict__ acts, int64_t arb, int64_t m, float* __restrict__ y, int64_t ys,
    const float* __restrict__ bias, int tiles_n, int tiles_m) {
  using C = Big<WT, WM, WN, NT>;
  constexpr bool kQ6 = C::kQ6;
  constexpr int kBM = C::kBM, kBN = C::kBN, kA = C::kA, kHL = C::kHL, kW = C::kW, kH = C::kH, kQH = C::kQH,
                kBS = C::kBS, kDA = C::kDA;
  extern __shared__ __align__(16) uint8_t lds[];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave % WM, wn = wave / WM;  // 64 activation rows x 16 NT weight rows per wave
  const int li = lane & 15, lg = lane >> 4;

  int L = blockIdx.x;
  const int per = (tiles_n * tiles_m) / 8;
  if (L < 8 * per) L = (L % 8) * per + L / 8;
  const int tn = __builtin_amdgcn_readfirstlane(L / tiles_m);
  const int tm = __builtin_amdgcn_readfirstlane(L - tn * tiles_m);
  const int64_t nbase = nt0 + (int64_t)tn * kBN;  // multiple of 64
  const int64_t mbase = (int64_t)tm * kBM;
  const int64_t mrows = m - mbase < kBM ? m - mbase : kBM;

  const auto ra = rsrc(acts + mbase * arb, (u32)(mrows * arb));
  const int64_t G0 = nbase >> 6;
  const int64_t gl = n_pad / kRowGroup - G0;
  const int64_t gspan = gl < C::kGroups ? gl : C::kGroups;
  // Q4_K planes: qs (128 B per row and super-block), header (16 B). Q6_K: ql (128 B),
  // qh (64 B), scales (16 B), d (2 B).
  const auto rq = rsrc(qs_plane + G0 * nb * 8192, (u32)(gspan * nb * 8192));
  const uint8_t* hp = kQ6 ? plane2 : hdr_plane;
  const auto rh = rsrc(hp + G0 * nb * 1024, (u32)(gspan * nb * 1024));
  const auto rqh = rsrc((kQ6 ? hdr_plane : qs_plane) + G0 * nb * 4096, (u32)(gspan * nb * 4096));
  const auto rd6 = rsrc((kQ6 ? plane3 : qs_plane) + G0 * nb * 128, (u32)(gspan * nb * 128));

  // ---- staging roles (direct-to-LDS, per super-block)
  // activation codes: wave w, instruction j < kAJ fills rows kBM / kWaves w + 4 j .. + 3;
  // the per-lane part of the source offset repeats with period 4 in j
  constexpr int kAJ = C::kAJ, kAW = kBM / C::kWaves;
  u32 aoff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = kAW * wave + 4 * j + (lane >> 4);
    aoff[j] = (u32)(row * arb + 4 + 16 * ((lane & 15) ^ (row & 15)));
  }
  // bsums: wave w < kBM / 32 fills rows 32 w .. 32 w + 31
  const u32 bsoff = (u32)((32 * wave + (lane >> 1)) * arb + 260 + 16 * (lane & 1));
  constexpr int kWI = 8 * C::kGroups / C::kWaves;  // nibble instructions per wave
  auto issue = [&](int b) {
#pragma unroll
    for (int j = 0; j < kAJ; ++j) {
      ld_lds16(ra, lds + kA + (kAW * wave + 4 * j) * 256, aoff[j & 3], (u32)(b * 292 + (j >> 2) * 16 * arb));
    }
    // nibbles: instruction i = kWI w + j stages chunk i / kGroups of 64-row group i % kGroups
#pragma unroll
    for (int j = 0; j < kWI; ++j) {
      const int i = kWI * wave + j, c = i / C::kGroups, k = i % C::kGroups;
      ld_lds16(rq, lds + kW + (c * kBN + 64 * k) * 16, (u32)(k * nb * 8192 + lane * 16), (u32)(b * 8192 + c * 1024));
    }
    if (wave < C::kGroups) {
      ld_lds16(rh, lds + kH + 64 * wave * 16, (u32)(wave * nb * 1024 + lane * 16), (u32)(b * 1024));
    }
    if constexpr (kQ6) {
      // qh: instruction i = kHI w + j stages chunk i / kGroups of group i % kGroups
      constexpr int kHI = 4 * C::kGroups / C::kWaves;
#pragma unroll
      for (int j = 0; j < kHI; ++j) {
        const int i = kHI * wave + j, c = i / C::kGroups, k = i % C::kGroups;
        ld_lds16(rqh, lds + kQH + (c * kBN + 64 * k) * 16, (u32)(k * nb * 4096 + lane * 16), (u32)(b * 4096 + c * 1024));
      }
      // d: 64 rows x 2 B per group, one 4-byte piece per lane
      if (wave == 0 && lane < 32 * C::kGroups) {
        ld_lds4(rd6, lds + kBS, (u32)((lane >> 5) * nb * 128 + 4 * (lane & 31)), (u32)(b * 128));
      }
    } else {
      if (wave < kBM / 32) ld_lds16(ra, lds + kBS + 32 * wave * 32, bsoff, (u32)(b * 292));
    }
    constexpr int kDI = kBM / 64;  // activation-scale instructions, on the last waves
    if (wave >= C::kWaves - kDI) {
      const int k = wave - (C::kWaves - kDI);
      ld_lds4(ra, lds + kDA + (b & 1) * kBM * 4 + 256 * k, (u32)((64 * k + lane) * arb), (u32)(b * 292));
    }
  };

  // ---- per-lane LDS read offsets
  const int qlg = 4 * (lg >> 1) + (lg & 1);
  const int arow = 64 * wm + li;
  int a_rd[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    // Q4_K: chunk qlg + 8(s>>1) + 2(s&1); Q6_K: unit lg + 4s (see prep_tile_q6)
    a_rd[s] = kQ6 ? kA + arow * 256 + 16 * ((lg ^ li) ^ (4 * s))
                  : kA + arow * 256 + 16 * ((qlg ^ li) ^ (8 * (s >> 1) + 2 * (s & 1)));
  }
  const int bs_rd = kBS + arow * 32 + 8 * lg;
  const int da_rd = kDA + (64 * wm + 4 * lg) * 4;
  const u32 sel_sc = (lg >> 1) ? 0x07060302u : 0x05040100u;
  const u32 sel_mn = 0x0C0C0000u | ((u32)(2 * lg + 1) << 8) | (u32)(2 * lg);

  f4_t acc[NT][4];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[nt][mt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  issue(0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  struct Sc {
    float d, dmin;
    h4_t mb;
  };
  struct Tacc {
    v4i_t H, L;
    f4_t M;
  };

#pragma unroll 1
  for (int b = 0; b < nb; ++b) {
    // ---- phase 1: B operands of this wave's weight tiles into LDS; this wave's
    // activation operands and the scales of its NT weight tiles into registers
#pragma unroll
    for (int i = 0; i < C::kPrep; ++i) {
      const int p = C::kPrep * wave + i;
      const int row = 16 * p + li;
      PrepB q;
      if constexpr (kQ6) {
        q = prep_tile_q6(lds_ld16(lds, kH + row * 16), lds_ld16(lds, kW + (lg * kBN + row) * 16),
                         lds_ld16(lds, kW + ((lg + 4) * kBN + row) * 16),
                         lds_ld16(lds, kQH + ((lg & 1) * kBN + row) * 16),
                         lds_ld16(lds, kQH + ((2 + (lg & 1)) * kBN + row) * 16), lg);
      } else {
        const RawB r{lds_ld16(lds, kH + row * 16), lds_ld16(lds, kW + (lg * kBN + row) * 16),
                     lds_ld16(lds, kW + ((lg + 4) * kBN + row) * 16)};
        q = prep_tile(r, sel_sc, sel_mn);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        *reinterpret_cast<v4u*>(lds + kHL + ((p * 4 + s) * 2 + 0) * 1024 + lane * 16) = q.H[s];
        *reinterpret_cast<v4u*>(lds + kHL + ((p * 4 + s) * 2 + 1) * 1024 + lane * 16) = q.L[s];
      }
    }
    v4u a[4][4];
    h4_t am[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int s = 0; s < 4; ++s) a[mt][s] = lds_ld16(lds, a_rd[s] + mt * 16 * 256);
      if constexpr (!kQ6) {
        const v2u bs = lds_ld8(lds, bs_rd + mt * 16 * 32);
        const v4u bsf = bsums_f16(v4u{bs.x, bs.y, 0, 0});
        am[mt] = __builtin_bit_cast(h4_t, v2u{bsf.x, bsf.y});
      }
    }
    Sc sc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int row = 16 * NT * wn + 16 * nt + li;
      if constexpr (kQ6) {
        sc[nt] = Sc{h2f(*reinterpret_cast<const uint16_t*>(lds + kBS + 2 * row)), 0.0f, h4_t{}};
      } else {
        const v4u hd = lds_ld16(lds, kH + row * 16);
        sc[nt] = Sc{h2f(hd.x), h2f(hd.x >> 16), mins_f16(hd, sel_mn)};
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // ---- the next super-block's loads go into the buffers just read (the
    // activation scales, read in the compute phase, have two buffers)
    if (b + 1 < nb) issue(b + 1);
    const int da_buf = (b & 1) * kBM * 4;

    // ---- phase 2: MFMAs and the fp32 epilogue, software-pipelined: each 16 x 16
    // tile's epilogue runs after the next tile's MFMAs are issued (its results are
    // complete by then). Per tile the 4 H-chain MFMAs run before the 4 L-chain ones,
    // so the next weight tile's H operands load during the last tile's L chain and
    // its L operands during the first tile's H chain.
    auto load4 = [&](int tile, int hl) {
      v4u r[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) r[s] = lds_ld16(lds, kHL + ((tile * 4 + s) * 2 + hl) * 1024 + lane * 16);
      return std::array<v4u, 4>{r[0], r[1], r[2], r[3]};
    };
    auto epi = [&](const Tacc& r, const Sc& c, int nt, int mt, f4_t da) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (kQ6) {
          // S = 64 sum(wh a) + sum(wl a); u = d (float)S; acc = fma(da, u, acc)
          const int S = r.L[e] + (r.H[e] << 6);
          acc[nt][mt][e] = fmaf(da[e], c.d * (float)S, acc[nt][mt][e]);
        } else {
          const int S = r.L[e] + (r.H[e] << 3);
          float u = c.d * (float)S;
          u = fmaf(-c.dmin, r.M[e], u);
          acc[nt][mt][e] = fmaf(da[e], u, acc[nt][mt][e]);
        }
      }
    };
    // The two waves of a SIMD (w and w + 4) leave the barrier together; starting
    // the second ~128 clocks later lets one wave's MFMA burst run while the other
    // runs its epilogue (measured: -5% at M = 512 and 2048).
    if (C::kWaves == 8 && wave >= 4) __builtin_amdgcn_s_sleep(2);
    std::array<v4u, 4> Hc = load4(NT * wn, 0), Lc = load4(NT * wn, 1), Hn, Ln;
    Tacc prev;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int pn = mt ? nt : nt - 1, pm = mt ? mt - 1 : 3;
        // the activation scales of the previous tile's epilogue, read before this
        // tile's MFMAs so that they have landed when the epilogue runs
        f4_t dp = {0.0f, 0.0f, 0.0f, 0.0f};
        if (nt + mt > 0) dp = __builtin_bit_cast(f4_t, lds_ld16(lds, da_buf + da_rd + pm * 16 * 4));
        Tacc cur;
        const v4i_t z = {0, 0, 0, 0};
        // a wave issuing its MFMA burst goes first, so bursts of the two waves of a
        // SIMD do not interleave (and end together)
        __builtin_amdgcn_s_setprio(1);
        cur.H = mfma(a[mt][0], Hc[0], z);
#pragma unroll
        for (int s = 1; s < 4; ++s) cur.H = mfma(a[mt][s], Hc[s], cur.H);
        if (mt == 0 && nt > 0) Lc = Ln;
        if (mt == 3 && nt + 1 < NT) Hn = load4(NT * wn + nt + 1, 0);
        cur.L = mfma(a[mt][0], Lc[0], z);
#pragma unroll
        for (int s = 1; s < 4; ++s) cur.L = mfma(a[mt][s], Lc[s], cur.L);
        if constexpr (!kQ6) cur.M = mfma_h(am[mt], sc[nt].mb, f4_t{0.0f, 0.0f, 0.0f, 0.0f});
        __builtin_amdgcn_s_setprio(0);
        if (nt + mt > 0) epi(prev, sc[pn], pn, pm, dp);
        prev = cur;
        if (mt == 3 && nt + 1 < NT) Hc = Hn;
      }
      if (nt + 1 < NT) Ln = load4(NT * wn + nt + 1, 1);
    }
    epi(prev, sc[NT - 1], NT - 1, 3, __builtin_bit_cast(f4_t, lds_ld16(lds, da_buf + da_rd + 3 * 16 * 4)));
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // ---- store, through LDS (free after the last barrier): the wave's 64 x 16 NT
  // tile is written in MFMA order (rows padded by 4 floats, so the four lane groups
  // hit distinct banks) and read back as 16-byte row pieces, so each store
  // instruction writes 4 rows of 64 NT contiguous bytes instead of 64-byte pieces.
  {
    constexpr int kRow = 16 * NT + 4;  // floats per staged row
    static_assert(C::kWaves * 64 * kRow * 4 <= C::kLds, "staged output fits the LDS");
    float* tile = reinterpret_cast<float*>(lds) + wave * 64 * kRow;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) tile[(16 * mt + 4 * lg + e) * kRow + 16 * nt + li] = acc[nt][mt][e];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    constexpr int kLanesPerRow = 16 * NT / 4;  // 16-byte pieces per row
    constexpr int kRowsPerStep = 64 / kLanesPerRow;
    const int pr = lane / kLanesPerRow, pc = 4 * (lane % kLanesPerRow);
    const int64_t n = nbase + 16 * NT * wn + pc;  // first of this lane's 4 columns
    const bool vec = ((reinterpret_cast<uintptr_t>(y) | (uintptr_t)(ys * 4)) & 15) == 0 && n >= n0 && n + 4 <= n1;
    f4_t bv = {0.0f, 0.0f, 0.0f, 0.0f};
    if (bias) {
#pragma unroll
      for (int c = 0; c < 4; ++c) bv[c] = n + c >= n0 && n + c < n1 ? bias[n + c] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 64 / kRowsPerStep; ++i) {
      const int row = kRowsPerStep * i + pr;
      const int64_t mm = mbase + 64 * wm + row;
      if (mm >= m) continue;
      f4_t v = *reinterpret_cast<const f4_t*>(tile + row * kRow + pc);
      if (bias) v = v + bv;
      float* dst = y + mm * ys + n;
      if (vec) {
        *reinterpret_cast<f4_t*>(dst) = v;
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (n + c >= n0 && n + c < n1) dst[c] = v[c];
        }
      }
    }
  }
}

bool gemm_supported(int dtype, int af) {
  return ((dtype == kQ4_K || dtype == kQ6_K) && (af == kActQ8_K || af == kActPer32 || af == kActQ16)) ||
         gemm_b32_supported(dtype, af);
}

namespace {

template <int WM, int NT, int MTW = 4>
hipError_t launch_cfg(const WeightDev& w, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0, int64_t n1,
                      float* y, int64_t ys, const float* bias, hipStream_t s) {
  using C = Cfg<WM, NT, MTW>;
  static_assert(C::kLds <= 160 * 1024, "LDS");
  static bool attr_set[64] = {};
  const int dev = w.device < 64 ? w.device : 63;
  if (!attr_set[dev]) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm_q4k<WM, NT, MTW>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, C::kLds);
    if (e != hipSuccess) return e;
    attr_set[dev] = true;
  }
  const int64_t nt0 = (n0 / kRowGroup) * kRowGroup;
  const int64_t tiles_n = (n1 - nt0 + C::kBN - 1) / C::kBN;
  const int64_t tiles_m = (m + C::kBM - 1) / C::kBM;
  // buffer offsets are 32-bit: one tile's weight span and activation rows must fit
  if ((int64_t)(C::kWB + 1) * w.nblk * 8192 >= (1ll << 32) || (int64_t)C::kBM * arb >= (1ll << 32) ||
      tiles_n * tiles_m >= (1ll << 31)) {
    return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL((k_gemm_q4k<WM, NT, MTW>), dim3((unsigned)(tiles_n * tiles_m)), dim3(kThreads), C::kLds, s,
                     w.plane[0], w.plane[1], (int)w.nblk, w.n_pad, nt0, n0, n1, acts, arb, m, y, ys, bias,
                     (int)tiles_n, (int)tiles_m);
  return hipGetLastError();
}

template <int WT, int WM, int WN, int NT>
hipError_t launch_big(const WeightDev& w, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0, int64_t n1,
                      float* y, int64_t ys, const float* bias, hipStream_t s) {
  using C = Big<WT, WM, WN, NT>;
  static bool attr_set[64] = {};
  const int dev = w.device < 64 ? w.device : 63;
  if (!attr_set[dev]) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm_q4k_big<WT, WM, WN, NT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, C::kLds);
    if (e != hipSuccess) return e;
    attr_set[dev] = true;
  }
  const int64_t nt0 = (n0 / kRowGroup) * kRowGroup;
  const int64_t tiles_n = (n1 - nt0 + C::kBN - 1) / C::kBN;
  const int64_t tiles_m = (m + C::kBM - 1) / C::kBM;
  if ((int64_t)C::kGroups * w.nblk * 8192 >= (1ll << 32) || (int64_t)C::kBM * arb >= (1ll << 32) ||
      tiles_n * tiles_m >= (1ll << 31)) {
    return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL((k_gemm_q4k_big<WT, WM, WN, NT>), dim3((unsigned)(tiles_n * tiles_m)), dim3(C::kThreads), C::kLds,
                     s, w.plane[0], w.plane[1], w.plane[2], w.plane[3], (int)w.nblk, w.n_pad, nt0, n0, n1, acts, arb, m,
                     y, ys, bias, (int)tiles_n, (int)tiles_m);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0, int64_t n1,
                       float* y, int64_t ys, const float* bias, hipStream_t s) {
  if (gemm_b32_supported(w.dtype, af)) return launch_gemm_b32(w, af, acts, arb, m, n0, n1, y, ys, bias, s);
  if (!gemm_supported(w.dtype, af)) return hipErrorInvalidValue;
  if (m == 0 || n1 <= n0) return hipSuccess;
  const int cus = w.cus > 0 ? w.cus : 256;
  const int64_t rows = n1 - (n0 / kRowGroup) * kRowGroup;
  if (w.dtype == kQ6_K || m > 128) {
    // the 8-wave 256 x 128 tile when its grid fills the GPU (M = 512 at N = 14336:
    // 224 workgroups, one round), else the 4-wave 128 x 64 tile (two per CU); Q6_K has
    // only these kernels
    const int64_t wgs = (rows + 127) / 128 * ((m + 255) / 256);
    if (w.dtype == kQ6_K) {
      if (wgs * 8 >= (int64_t)cus * 7) return launch_big<kQ6_K, 4, 2, 4>(w, acts, arb, m, n0, n1, y, ys, bias, s);
      // 64 x 64 tiles (4 waves, each 64 activation rows x 16 weight rows) while they are one
      // per CU at most: the 128 x 64 tiles would leave half the CUs idle or more (K = 14336,
      // N = 4096: 87-92 against 113-121 us at 65..256 rows; at 384 rows, 384 of them took
      // 140 against 123 us); Q4_K below likewise
      if ((rows + 63) / 64 * ((m + 63) / 64) <= cus) {
        return launch_big<kQ6_K, 1, 4, 1>(w, acts, arb, m, n0, n1, y, ys, bias, s);
      }
      return launch_big<kQ6_K, 2, 2, 2>(w, acts, arb, m, n0, n1, y, ys, bias, s);
    }
    if (wgs * 8 >= (int64_t)cus * 7) return launch_big<kQ4_K, 4, 2, 4>(w, acts, arb, m, n0, n1, y, ys, bias, s);
    if ((rows + 63) / 64 * ((m + 63) / 64) <= cus) {
      return launch_big<kQ4_K, 1, 4, 1>(w, acts, arb, m, n0, n1, y, ys, bias, s);
    }
    return launch_big<kQ4_K, 2, 2, 2>(w, acts, arb, m, n0, n1, y, ys, bias, s);
  }
  // up to 128 rows: the 4-wave kernel in the shape (waves along the activation rows, weight
  // tiles per wave, activation tiles per wave) whose rounds of workgroups over the CUs
  // times its measured time per super-block (1 workgroup per CU; K = 4096 and 14336,
  // N = 4096 and 14336) is least: 32 x 32 tiles 0.68 us, 32 x 64 (two activation tiles
  // per wave) 0.93, 64 x 64 1.38, 128 x 64 2.53.
  struct Shape {
    int wm, nt, mtw, us100;
  };
  constexpr Shape kShapes[] = {{2, 1, 1, 68}, {1, 1, 2, 93}, {1, 1, 4, 138}, {2, 2, 4, 253}};
  const int64_t ntn = n1 - (n0 / kRowGroup) * kRowGroup;
  int best = 0;
  int64_t best_cost = -1;
  for (int i = 0; i < 4; ++i) {
    const Shape& c = kShapes[i];
    const int64_t bm = 16 * c.mtw * c.wm, bn = (4 / c.wm) * 16 * c.nt;
    const int64_t wgs = (ntn + bn - 1) / bn * ((m + bm - 1) / bm);
    const int64_t cost = (wgs + cus - 1) / cus * c.us100;
    if (best_cost < 0 || cost < best_cost) {
      best = i;
      best_cost = cost;
    }
  }
  switch (best) {
    case 0: return launch_cfg<2, 1, 1>(w, acts, arb, m, n0, n1, y, ys, bias, s);
    case 1: return launch_cfg<1, 1, 2>(w, acts, arb, m, n0, n1, y, ys, bias, s);
    case 2: return launch_cfg<1, 1, 4>(w, acts, arb, m, n0, n1, y, ys, bias, s);
    default: return launch_cfg<2, 2, 4>(w, acts, arb, m, n0, n1, y, ys, bias, s);
  }
}

}  // namespace dq
