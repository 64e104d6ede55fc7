// dq_skinny.hip -- the decode-batch GEMV for gfx950: Q4_K / Q6_K weights x Q8_K
// activations for 2..16 activation rows, on int8 MFMA (v_mfma_i32_16x16x64_i8), and
// its grouped launches (one launch for several matmuls, dq_matmul_many).
//
// Arithmetic contract per super-block b (256 values), activation row mm, weight row n:
//   Q4_K: S = sum_j sc_j P_j, Mn = sum_j m_j (code sum of sub-block j),
//         t = fma(-dmin, (float)Mn, d * (float)S)      (kernels_avx2.cpp:976-1014)
//   Q6_K: S = sum_u sc_u P_u over 16-value sub-blocks with codes q - 32,
//         t = d * (float)S                              (kernels_avx2.cpp:1016-1058)
// and y = the chain acc = fma(da_b, t_b, acc) over b in order: the library's
// canonical fp32 order, so outputs are bit-identical to the M = 1 GEMV, the GEMM
// and the CPU oracle.
//
// MFMA mapping: the 16 activation rows are the rows of the A operand (rows past m
// read zeros), 16 weight rows the columns of B. Q4_K: the effective weight sc*q
// (0..945) does not fit int8, so sc = 8 sh + sl and the B operands are sh*q and
// sl*q (bytes <= 105, one packed 16-bit multiply per 4 nibbles); a third operand
// holds m_j at every position of sub-block j, so its MFMA sum is exactly Mn.
// Q6_K: in K-step s lane group g of B holds sub-block 4s + g (one scale), so the
// effective weight w = sc_u (q - 32) splits exactly into int8 operands w = 64 wh + wl
// and two MFMA chains give S (dequantize_q6_K layout, quant_formats.cpp:192-216).
//
// Workgroup: 4 or 8 waves over 16 * CT weight rows (CT MFMA column tiles) and all
// super-blocks, wave w taking a contiguous slice of super-blocks. CT = 4 (a whole
// 64-row group) reads each activation super-block once per 64 weight rows instead
// of once per 16 (for launches with many workgroups); CT = 1 gives 4x the
// workgroups for small matmuls and prefetches the next super-block's weights while
// it computes the current one. Per super-block each wave writes its t-terms to
// LDS; after one barrier all waves share the in-order chains of the 16 x 16 CT
// outputs.
//
// kFused: the activations arrive as fp32 rows and each wave quantizes the 16 rows
// of its super-block itself (d = amax / 127, codes round half to even at 1 / d:
// dynacore/cpu/avx2/kernels_avx2.cpp:638-644), with the standalone quantizer's code
// routine (codes4_rne, dq_quant.h) and an order-independent amax, so the codes are
// the bytes k_quant_q8k writes. One launch then does what a quantize launch plus a
// GEMV launch do.
//
// Grouping: the grid is the concatenation of the jobs' workgroup ranges; each
// workgroup finds its job in a table passed by value, and Q4_K and Q6_K jobs mix
// in one launch (as dynacore's Device::matmul_many runs every job's row chunks in
// one parallel region, dynacore/cpu/cpu_device.cpp:500-692).
//
// kGated: a job carries a second weight of the same type and shape (the up
// projection) and writes act(x . Wg^T) * (x . Wu^T), the gated MLP projection of
// dynacore's Device::matmul_gated (dynacore/include/dynacore/device/device.h:188-199).
// Half the waves of a workgroup run the gate tile and half the up tile of the same
// 16 rows (each wave the single-weight pipeline over twice the super-blocks), the
// t-terms of both go to LDS, and the chains end in act(g) * u: one launch and no
// gate / up round trip through memory, as CpuDevice's decode path applies the
// activation per 16-column chunk (dynacore/cpu/cpu_device.cpp:1940-1979).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "dq_act.h"
#include "dq_device.h"
#include "dq_internal.h"
#include "dq_mfma.h"
#include "dq_quant.h"

namespace dq {

namespace {

struct SkinnyJob {
  const uint8_t* p[4];        // weight planes (dq_layout.h)
  const uint8_t* pu[4];       // kGated: the up projection's planes (same type and shape)
  int64_t n_pad, t0, n0, n1;  // rows (padded to 64), first tile, output row range
  const uint8_t* acts;        // !kFused: m rows of Q8_K, arb bytes apart
  int64_t arb;
  const float* x;  // kFused: m rows of fp32, xs floats apart
  int64_t xs;
  float* y;
  int64_t ys;
  const float* bias;
  int dtype, m;
  int act;  // kGated: the activation applied to the gate projection
  int wg0;  // first workgroup of this job in the grid
};
constexpr int kSkinnyMaxJobs = 8;
struct SkinnyGroup {
  SkinnyJob job[kSkinnyMaxJobs];
  int count;
  int nblk;  // super-blocks per row, the same for every job of a group
};

constexpr int kSkinnyWaves = 8;

// The activation operand of one super-block for MT tiles of 16 activation rows:
// lane (li, lg) holds the codes of activation row 16 mt + li at values
// 64 s + 16 lg .. + 15 (K-step s), and that row's d.
template <int MT>
struct ActSB {
  v4u a[MT][4];
  float da[MT];
};

// fp32 values of one super-block for the fused path: x[li][64 s + 16 lg + 4 c + i].
struct XSB {
  v4u v[4][4];
};

template <bool kFused>
struct ActSrc {
  __amdgpu_buffer_rsrc_t r;
  int64_t stride;  // bytes between rows
  DQ_DEV void init(const SkinnyJob& J) {
    if (kFused) {
      r = rsrc(J.x, (u32)(J.m * J.xs * 4));
      stride = J.xs * 4;
    } else {
      r = rsrc(J.acts, (u32)(J.m * J.arb));
      stride = J.arb;
    }
  }
};

DQ_DEV void load_x(const ActSrc<true>& src, int b, int li, int lg, XSB& o) {
  const u32 base = (u32)(li * src.stride + ((int64_t)b * 256 + 16 * lg) * 4);
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int c = 0; c < 4; ++c) o.v[s][c] = ld16(src.r, base + (u32)((64 * s + 4 * c) * 4));
}

// Q8_K quantization of row li's super-block from the 64 values of each of the 4
// lanes (li, 0..3): amax across them, d = amax / 127, codes RNE at 1 / d.
DQ_DEV void quant_x(const XSB& x, ActSB<1>& o) {
  float amax = 0.0f;
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(as_f(x.v[s][c].x)), fabsf(as_f(x.v[s][c].y))),
                               fmaxf(fabsf(as_f(x.v[s][c].z)), fabsf(as_f(x.v[s][c].w)))));
    }
  amax = fmaxf(amax, __shfl_xor(amax, 16));
  amax = fmaxf(amax, __shfl_xor(amax, 32));
  const float d = amax / 127.0f;
  const float id = d > 0 ? 1.0f / d : 0.0f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    u32 w[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float v[4] = {as_f(x.v[s][c].x), as_f(x.v[s][c].y), as_f(x.v[s][c].z), as_f(x.v[s][c].w)};
      int unused = 0;
      w[c] = codes4_rne(v, id, unused);
    }
    o.a[0][s] = v4u{w[0], w[1], w[2], w[3]};
  }
  o.da[0] = d;
}

template <int MT>
DQ_DEV void load_codes(const ActSrc<false>& src, int b, int li, int lg, ActSB<MT>& o) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const u32 base = (u32)((16 * mt + li) * src.stride + (int64_t)b * 292);
#pragma unroll
    for (int s = 0; s < 4; ++s) o.a[mt][s] = ld16(src.r, base + 4 + 64 * s + 16 * lg);
    o.da[mt] = as_f(ld4(src.r, base));
  }
}

// Sub-scaled activations (ActSuperQ8, 320 bytes per super-block: codes, u @256, the
// sub-block multipliers m_b as int16 @260; kernels_avx2.cpp:1077-1096): the codes as
// in ActSB, u of row 16 mt + li in da (the chain's per-super-block factor), and the
// eight m_b of each of this lane's output rows 16 mt + 4 lg + e (dword s holds
// m_{2s} | m_{2s+1} << 16).
template <int MT>
struct ActSBX {
  v4u a[MT][4];
  float da[MT];
  v4u mb[MT][4];
};

template <int MT>
DQ_DEV void load_codes_sx(const ActSrc<false>& src, int b, int li, int lg, ActSBX<MT>& o) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const u32 base = (u32)((16 * mt + li) * src.stride + (int64_t)b * 320);
#pragma unroll
    for (int s = 0; s < 4; ++s) o.a[mt][s] = ld16(src.r, base + 64 * s + 16 * lg);
    o.da[mt] = as_f(ld4(src.r, base + 256));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o.mb[mt][e] = ld16(src.r, (u32)((16 * mt + 4 * lg + e) * src.stride + (int64_t)b * 320 + 260));
    }
  }
}

// ---- weights of one super-block for CT column tiles (row r0 + 16 ct + li of row group G)
template <int WT, int CT>
struct WSB;

template <int CT>
struct WSB<kQ4_K, CT> {
  v4u hd[CT], q[CT][4];
  DQ_DEV void load(const __amdgpu_buffer_rsrc_t& rq, const __amdgpu_buffer_rsrc_t& rh, int b, int r0, int li,
                   int lg) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int r = r0 + 16 * ct + li;
      hd[ct] = ld16nt(rh, (u32)((b * 64 + r) * 16));
#pragma unroll
      for (int s = 0; s < 4; ++s) q[ct][s] = ld16nt(rq, (u32)(((b * 8 + 2 * s + (lg & 1)) * 64 + r) * 16));
    }
  }
};

template <int CT>
struct WSB<kQ6_K, CT> {
  v4u l0[CT], l1[CT], h0[CT], h1[CT], sc[CT];
  u32 dw[CT];
  DQ_DEV void load(const __amdgpu_buffer_rsrc_t* rp, int b, int r0, int li, int lg) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int r = r0 + 16 * ct + li;
      // lane (row, group g): ql chunks g and 4 + g (values of K-steps 0, 1 and 2, 3 in
      // the low and high nibbles), qh chunks g & 1 and 2 + (g & 1), the 16 scales, d
      l0[ct] = ld16nt(rp[0], (u32)(((b * 8 + lg) * 64 + r) * 16));
      l1[ct] = ld16nt(rp[0], (u32)(((b * 8 + 4 + lg) * 64 + r) * 16));
      h0[ct] = ld16nt(rp[1], (u32)(((b * 4 + (lg & 1)) * 64 + r) * 16));
      h1[ct] = ld16nt(rp[1], (u32)(((b * 4 + 2 + (lg & 1)) * 64 + r) * 16));
      sc[ct] = ld16nt(rp[2], (u32)((b * 64 + r) * 16));
      dw[ct] = ld2nt(rp[3], (u32)((b * 64 + r) * 2));
    }
  }
};

// t-terms of column tile ct for one super-block: for each activation tile mt the 4
// outputs of this lane (activation rows 16 mt + 4 lg + e, weight row 16 ct + li of
// the tile). The weight operands of a K-step are built once and multiplied with
// every activation tile.
template <int CT, int MT>
DQ_DEV void tterms(const WSB<kQ4_K, CT>& w, int ct, const ActSB<MT>& A, int lg, float t[MT][4]) {
  const int hi = lg >> 1;
  const u32 shift = 4u * (u32)hi, flip = hi ? 0x08080808u : 0u;  // high nibbles are stored XOR 8
  const v4u hd = w.hd[ct];
  // scales and mins of sub-blocks 2s + hi as bytes s (get_scale_min_k4, quant_formats.h:62-70)
  const u32 sc_lo = hd.y & 0x3F3F3F3Fu, mn_lo = hd.z & 0x3F3F3F3Fu;
  const u32 sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
  const u32 mn_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
  const u32 sc = __builtin_amdgcn_perm(sc_hi, sc_lo, sel_subblocks(hi));
  const u32 KH = (sc >> 3) & 0x07070707u, KL = sc & 0x07070707u;
  const u32 MN = __builtin_amdgcn_perm(mn_hi, mn_lo, sel_subblocks(hi));
  v4i_t acc[MT][3];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const v4u qb = ((w.q[ct][s] >> shift) & 0x0F0F0F0Fu) ^ flip;
    const u32 kh = __builtin_amdgcn_perm(0u, KH, sel_u16x2(s));
    const u32 kl = __builtin_amdgcn_perm(0u, KL, sel_u16x2(s));
    const u32 mm4 = __builtin_amdgcn_perm(0u, MN, sel_x4(s));
    const v4u H = {mul_bytes(qb.x, kh), mul_bytes(qb.y, kh), mul_bytes(qb.z, kh), mul_bytes(qb.w, kh)};
    const v4u Lo = {mul_bytes(qb.x, kl), mul_bytes(qb.y, kl), mul_bytes(qb.z, kl), mul_bytes(qb.w, kl)};
    const v4u Mp = {mm4, mm4, mm4, mm4};
    const v4i_t z = {0, 0, 0, 0};
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc[mt][0] = mfma(A.a[mt][s], H, s == 0 ? z : acc[mt][0]);
      acc[mt][1] = mfma(A.a[mt][s], Lo, s == 0 ? z : acc[mt][1]);
      acc[mt][2] = mfma(A.a[mt][s], Mp, s == 0 ? z : acc[mt][2]);
    }
  }
  const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int S = acc[mt][1][e] + (acc[mt][0][e] << 3);
      const float u = d * (float)S;
      t[mt][e] = fmaf(-dmin, (float)acc[mt][2][e], u);
    }
}

template <int CT, int MT>
DQ_DEV void tterms(const WSB<kQ6_K, CT>& w, int ct, const ActSB<MT>& A, int lg, float t[MT][4]) {
  // lane group g at K-step s holds sub-block u = 4s + g (one scale): w = sc_u (q - 32)
  // split exactly into int8 operands w = 64 wh + wl (q6_split), two MFMA chains give
  // S = 64 sum(wh a) + sum(wl a) = sum_u sc_u sum((q - 32) a), and t = d (float)S
  v4i_t H[MT], L[MT];
  const int sh = 2 * (lg >> 1);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    // codes of sub-block 4s + g: the low (even s) or high nibbles of ql chunk g + 4(s>>1)
    // with their top two bits from qh chunk 2(s>>1) + (g&1), bit pair g/2 (+2 for odd s)
    const v4u lo = (s >> 1) ? w.l1[ct] : w.l0[ct], hb = (s >> 1) ? w.h1[ct] : w.h0[ct];
    const u32 qsh = (u32)(sh + 4 * (s & 1));
    const v4u q = ((lo >> (u32)(4 * (s & 1))) & 0x0F0F0F0Fu) | (((hb >> qsh) & 0x03030303u) << 4);
    const u32 sw = s == 0 ? w.sc[ct].x : s == 1 ? w.sc[ct].y : s == 2 ? w.sc[ct].z : w.sc[ct].w;
    const int sc = sbfe(sw, 8 * lg, 8);
    v4u bh, bl;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32 h, l;
      q6_split(q[i], sc, h, l);
      bh[i] = h;
      bl[i] = l;
    }
    const v4i_t z = {0, 0, 0, 0};
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      H[mt] = mfma(A.a[mt][s], bh, s == 0 ? z : H[mt]);
      L[mt] = mfma(A.a[mt][s], bl, s == 0 ? z : L[mt]);
    }
  }
  const float d = h2f(w.dw[ct]);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int e = 0; e < 4; ++e) t[mt][e] = d * (float)((H[mt][e] << 6) + L[mt][e]);
}

// Sub-scaled activations (kernels_avx2.cpp:1117-1216): the super-block integers carry
// the activation multiplier of each 32-value sub-block b, S = sum_b m_b S_b, which
// differs per activation row, so it cannot ride in the weight operand. K-step s
// spans sub-blocks 2 s (lane groups 0, 1) and 2 s + 1 (lane groups 2, 3): each chain
// runs twice per step on the activation operand with the other half's lanes zeroed,
// and the exact products m_b S_b (below 2^31 each) are added into a 64-bit S. Then
// the canonical order of the Q8_K pair: t = d (float)S (Q4_K: t = fma(-dmin, Mn, t)
// with Mn = sum_b m_b m_j (code sum of sub-block b)), the chain multiplies by u.
DQ_DEV void halves(v4u a, int lg, v4u& a0, v4u& a1) {
  const u32 keep0 = lg < 2 ? 0xFFFFFFFFu : 0u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a0[i] = a[i] & keep0;
    a1[i] = a[i] & ~keep0;
  }
}
DQ_DEV int mb_lo(v4u mb, int s) { return (int)((s == 0 ? mb.x : s == 1 ? mb.y : s == 2 ? mb.z : mb.w) & 0xFFFFu); }
DQ_DEV int mb_hi(v4u mb, int s) { return (int)((s == 0 ? mb.x : s == 1 ? mb.y : s == 2 ? mb.z : mb.w) >> 16); }

template <int CT, int MT>
DQ_DEV void tterms(const WSB<kQ4_K, CT>& w, int ct, const ActSBX<MT>& A, int lg, float t[MT][4]) {
  const int hi = lg >> 1;
  const u32 shift = 4u * (u32)hi, flip = hi ? 0x08080808u : 0u;  // high nibbles are stored XOR 8
  const v4u hd = w.hd[ct];
  const u32 sc_lo = hd.y & 0x3F3F3F3Fu, mn_lo = hd.z & 0x3F3F3F3Fu;
  const u32 sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
  const u32 mn_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
  const u32 sc = __builtin_amdgcn_perm(sc_hi, sc_lo, sel_subblocks(hi));
  const u32 KH = (sc >> 3) & 0x07070707u, KL = sc & 0x07070707u;
  const u32 MN = __builtin_amdgcn_perm(mn_hi, mn_lo, sel_subblocks(hi));
  int64_t S[MT][4];
  int Mn[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      S[mt][e] = 0;
      Mn[mt][e] = 0;
    }
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const v4u qb = ((w.q[ct][s] >> shift) & 0x0F0F0F0Fu) ^ flip;
    const u32 kh = __builtin_amdgcn_perm(0u, KH, sel_u16x2(s));
    const u32 kl = __builtin_amdgcn_perm(0u, KL, sel_u16x2(s));
    const u32 mm4 = __builtin_amdgcn_perm(0u, MN, sel_x4(s));
    const v4u H = {mul_bytes(qb.x, kh), mul_bytes(qb.y, kh), mul_bytes(qb.z, kh), mul_bytes(qb.w, kh)};
    const v4u Lo = {mul_bytes(qb.x, kl), mul_bytes(qb.y, kl), mul_bytes(qb.z, kl), mul_bytes(qb.w, kl)};
    const v4u Mp = {mm4, mm4, mm4, mm4};
    const v4i_t z = {0, 0, 0, 0};
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      v4u a0, a1;
      halves(A.a[mt][s], lg, a0, a1);
      const v4i_t h0 = mfma(a0, H, z), l0 = mfma(a0, Lo, z), m0 = mfma(a0, Mp, z);
      const v4i_t h1 = mfma(a1, H, z), l1 = mfma(a1, Lo, z), m1 = mfma(a1, Mp, z);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int f0 = mb_lo(A.mb[mt][e], s), f1 = mb_hi(A.mb[mt][e], s);
        S[mt][e] += (int64_t)(((h0[e] << 3) + l0[e]) * f0) + (int64_t)(((h1[e] << 3) + l1[e]) * f1);
        Mn[mt][e] += m0[e] * f0 + m1[e] * f1;
      }
    }
  }
  const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float u = d * (float)S[mt][e];
      t[mt][e] = fmaf(-dmin, (float)Mn[mt][e], u);
    }
}

template <int CT, int MT>
DQ_DEV void tterms(const WSB<kQ6_K, CT>& w, int ct, const ActSBX<MT>& A, int lg, float t[MT][4]) {
  int64_t S[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int e = 0; e < 4; ++e) S[mt][e] = 0;
  const int sh = 2 * (lg >> 1);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const v4u lo = (s >> 1) ? w.l1[ct] : w.l0[ct], hb = (s >> 1) ? w.h1[ct] : w.h0[ct];
    const u32 qsh = (u32)(sh + 4 * (s & 1));
    const v4u q = ((lo >> (u32)(4 * (s & 1))) & 0x0F0F0F0Fu) | (((hb >> qsh) & 0x03030303u) << 4);
    const u32 sw = s == 0 ? w.sc[ct].x : s == 1 ? w.sc[ct].y : s == 2 ? w.sc[ct].z : w.sc[ct].w;
    const int sc = sbfe(sw, 8 * lg, 8);
    v4u bh, bl;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32 h, l;
      q6_split(q[i], sc, h, l);
      bh[i] = h;
      bl[i] = l;
    }
    const v4i_t z = {0, 0, 0, 0};
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      v4u a0, a1;
      halves(A.a[mt][s], lg, a0, a1);
      const v4i_t h0 = mfma(a0, bh, z), l0 = mfma(a0, bl, z);
      const v4i_t h1 = mfma(a1, bh, z), l1 = mfma(a1, bl, z);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // |64 H + L| <= 32 * 128 * 32 * 127 per half step, times m_b <= 128: below 2^31
        const int f0 = mb_lo(A.mb[mt][e], s), f1 = mb_hi(A.mb[mt][e], s);
        S[mt][e] += (int64_t)(((h0[e] << 6) + l0[e]) * f0) + (int64_t)(((h1[e] << 6) + l1[e]) * f1);
      }
    }
  }
  const float d = h2f(w.dw[ct]);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int e = 0; e < 4; ++e) t[mt][e] = d * (float)S[mt][e];
}

template <int WT, int CT>
struct WRes;
template <int CT>
struct WRes<kQ4_K, CT> {
  __amdgpu_buffer_rsrc_t rq, rh;
  DQ_DEV void init(const uint8_t* const* p, int64_t G, int nblk, bool ok) {
    rq = rsrc(p[0] + G * nblk * 8192, ok ? (u32)(nblk * 8192) : 0u);
    rh = rsrc(p[1] + G * nblk * 1024, ok ? (u32)(nblk * 1024) : 0u);
  }
  DQ_DEV void load(WSB<kQ4_K, CT>& w, int b, int r0, int li, int lg) const { w.load(rq, rh, b, r0, li, lg); }
};
template <int CT>
struct WRes<kQ6_K, CT> {
  __amdgpu_buffer_rsrc_t rp[4];
  DQ_DEV void init(const uint8_t* const* p, int64_t G, int nblk, bool ok) {
    rp[0] = rsrc(p[0] + G * nblk * 8192, ok ? (u32)(nblk * 8192) : 0u);
    rp[1] = rsrc(p[1] + G * nblk * 4096, ok ? (u32)(nblk * 4096) : 0u);
    rp[2] = rsrc(p[2] + G * nblk * 1024, ok ? (u32)(nblk * 1024) : 0u);
    rp[3] = rsrc(p[3] + G * nblk * 128, ok ? (u32)(nblk * 128) : 0u);
  }
  DQ_DEV void load(WSB<kQ6_K, CT>& w, int b, int r0, int li, int lg) const { w.load(rp, b, r0, li, lg); }
};

// One wave's super-blocks [b0, b1) of one weight (planes p) of a job: activations,
// weights, t-terms to LDS. CT == 1 keeps the next super-block's weight loads in
// flight during the compute (activation loads of b are issued before the weight
// loads of b + 1, so waiting for them does not wait for the prefetch: loads retire
// in order).
template <int WT, int CT, int MT, bool kFused, int D, bool kSx>
DQ_DEV void skinny_wave(const SkinnyJob& J, const uint8_t* const* p, int nblk, int64_t G, int r0, bool ok, int b0,
                        int b1, float* tt, float* dal, int li, int lg) {
  constexpr int NC = 16 * CT, NR = 16 * MT;
  static_assert(!kSx || !kFused, "sub-scaled rows arrive quantized");
  using Act = std::conditional_t<kSx, ActSBX<MT>, ActSB<MT>>;
  WRes<WT, CT> res;
  res.init(p, G, nblk, ok);
  ActSrc<kFused> src;
  src.init(J);
  auto emit = [&](const WSB<WT, CT>& w, const Act& A, int b) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      float t[MT][4];
      tterms<CT, MT>(w, ct, A, lg, t);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) tt[(b * NR + 16 * mt + 4 * lg + e) * NC + 16 * ct + li] = t[mt][e];
    }
    if (lg == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) dal[b * NR + 16 * mt + li] = A.da[mt];
    }
  };
  auto act = [&](int b, Act& A) {
    if constexpr (kSx) {
      load_codes_sx<MT>(src, b, li, lg, A);
    } else if constexpr (kFused) {
      static_assert(MT == 1, "in-kernel quantization covers one activation tile");
      XSB x;
      load_x(src, b, li, lg, x);
      quant_x(x, A);
    } else {
      load_codes<MT>(src, b, li, lg, A);
    }
  };
  if (b0 >= b1) return;
  if constexpr (CT == 1 && D > 1) {
    static_assert(D % 2 == 0, "the activation double buffer alternates with the slot index");
    // D super-blocks of weights in flight: slot i holds super-block b0 + i (mod D) and
    // is refilled with b + D after b's t-terms. Each step issues the activations of
    // b + 1 before it waits for b, and the refills come after: loads retire in order,
    // so waiting for b's activations never waits for a refill.
    WSB<WT, CT> w[D];
#pragma unroll
    for (int i = 0; i < D; ++i)
      if (b0 + i < b1) res.load(w[i], b0 + i, r0, li, lg);
    Act A[2];
    act(b0, A[0]);
#pragma unroll 1
    for (int bb = b0; bb < b1; bb += D) {
#pragma unroll
      for (int i = 0; i < D; ++i) {
        const int b = bb + i;
        if (b < b1) {
          if (b + 1 < b1) act(b + 1, A[(i + 1) & 1]);
          emit(w[i], A[i & 1], b);
          if (b + D < b1) res.load(w[i], b + D, r0, li, lg);
        }
      }
    }
  } else if constexpr (CT == 1) {
    WSB<WT, CT> cur;
    res.load(cur, b0, r0, li, lg);
    for (int b = b0; b < b1; ++b) {
      Act A;
      act(b, A);
      WSB<WT, CT> nxt;
      res.load(nxt, b + 1 < b1 ? b + 1 : b, r0, li, lg);
      emit(cur, A, b);
      cur = nxt;
    }
  } else {
    // CT == 4: the weight loads of all tiles first (the longer latency), then the
    // activations (L2-resident), which keeps the fp32 values out of the weights'
    // live range
    for (int b = b0; b < b1; ++b) {
      WSB<WT, CT> w;
      res.load(w, b, r0, li, lg);
      __builtin_amdgcn_sched_barrier(0);
      Act A;
      act(b, A);
      emit(w, A, b);
    }
  }
}

// W waves per workgroup (4 or 8; launch_group picks it from the launch's shape); D
// super-blocks of weights in flight per wave (launch_group picks 4 for one round of
// workgroups with several super-blocks per wave).
template <int CT, int MT, bool kFused, bool kGated, int W, int D = 1, bool kSx = false>
__global__ __launch_bounds__(W * 64) void k_skinny(SkinnyGroup g) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int NC = 16 * CT, NR = 16 * MT;
  const int wg = blockIdx.x;
  int j = 0;
  while (j + 1 < g.count && wg >= g.job[j + 1].wg0) ++j;
  const SkinnyJob& J = g.job[j];
  const int nblk = g.nblk;
  float* tt = reinterpret_cast<float*>(lds);        // [nblk][NR activation rows][NC weight rows]
  float* tu = tt + (kGated ? nblk * NR * NC : 0);  // kGated: the up projection's, same shape
  float* dal = tu + nblk * NR * NC;                // [nblk][NR] activation d (kGated: twice)
  const int l = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = l & 15, lg = l >> 4;
  const int64_t row0 = (J.t0 + (wg - J.wg0)) * NC;  // first weight row of the tile
  const int64_t G = row0 / kRowGroup;
  const int r0 = (int)(row0 % kRowGroup);
  const bool ok = row0 < J.n_pad;
  // kGated: waves W/2.. run the up projection over the same tile, each half with its
  // own t-term and activation-d regions (both halves write the same d values)
  constexpr int WH = kGated ? W / 2 : W;
  const int half = kGated && wave >= WH ? 1 : 0;
  const int wl = wave - half * WH;
  const int b0 = wl * nblk / WH, b1 = (wl + 1) * nblk / WH;
  const uint8_t* const* planes = half ? J.pu : J.p;
  float* tw = half ? tu : tt;
  float* dw = dal + half * nblk * NR;
  if (J.dtype == kQ6_K) {
    skinny_wave<kQ6_K, CT, MT, kFused, D, kSx>(J, planes, nblk, G, r0, ok, b0, b1, tw, dw, li, lg);
  } else {
    skinny_wave<kQ4_K, CT, MT, kFused, D, kSx>(J, planes, nblk, G, r0, ok, b0, b1, tw, dw, li, lg);
  }
  __syncthreads();
  // the in-order chains of the tile's NR x NC outputs, shared by all waves
  for (int o = threadIdx.x; o < NR * NC; o += W * 64) {
    const int mm = o / NC, c = o % NC;
    float v = 0.0f, vu = 0.0f;
#pragma unroll 8
    for (int b = 0; b < nblk; ++b) {
      const float da = dal[b * NR + mm];
      v = fmaf(da, tt[(b * NR + mm) * NC + c], v);
      if (kGated) vu = fmaf(da, tu[(b * NR + mm) * NC + c], vu);
    }
    const int64_t n = row0 + c;
    if (mm < J.m && n >= J.n0 && n < J.n1) {
      if (kGated) {
        J.y[mm * J.ys + n] = act_apply(J.act, v) * vu;
      } else {
        J.y[mm * J.ys + n] = J.bias ? v + J.bias[n] : v;
      }
    }
  }
}

// ---- long Q6_K rows on few 16-row tiles (an FFN down projection at up to 16
// activation rows: Q6_K 1536 x 8960 is 96 tiles of 35 super-blocks). k_skinny runs
// one workgroup per tile there, so 96 CUs each stream ~280 KB (weights and the
// tile's activation super-blocks), and a CU streams at most ~20 KB per microsecond
// on this GPU. k_skinny_split spreads the row over ~all CUs: a workgroup takes one
// 64-row group and a slice of kSplitWaves super-blocks, one wave per super-block with
// k_skinny's CT = 4 step (each activation super-block is read once per 64 weight
// rows, a quarter of the 16-row tiles' activation traffic), and stores the t-terms
// in T[group][b][16 activation rows][64 weight rows]. k_skinny_chain then runs the
// in-order chains acc = fma(d_b, t_b, acc) with d from the Q8_K rows. Same t-terms,
// same chains: bit-equal to k_skinny.
constexpr int kSplitWaves = 4;

template <int WT>
DQ_DEV void split_wave(const SkinnyJob& J, int nblk, int64_t G, int b, float* tb, int li, int lg) {
  WRes<WT, 4> res;
  res.init(J.p, G, nblk, true);
  WSB<WT, 4> w;
  res.load(w, b, 0, li, lg);
  __builtin_amdgcn_sched_barrier(0);  // the weight loads first (the longer latency)
  ActSrc<false> src;
  src.init(J);
  ActSB<1> A;
  load_codes<1>(src, b, li, lg, A);
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    float t[1][4];
    tterms<4, 1>(w, ct, A, lg, t);
#pragma unroll
    for (int e = 0; e < 4; ++e) tb[(4 * lg + e) * 64 + 16 * ct + li] = t[0][e];
  }
}

__global__ __launch_bounds__(kSplitWaves * 64) void k_skinny_split(SkinnyJob J, int nblk, int slices, int64_t g0,
                                                                   float* __restrict__ T) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63;
  const int64_t gi = blockIdx.x / slices;
  const int b = (int)(blockIdx.x % slices) * kSplitWaves + wave;
  if (b >= nblk) return;
  float* tb = T + (gi * nblk + b) * 16 * 64;
  if (J.dtype == kQ6_K) {
    split_wave<kQ6_K>(J, nblk, g0 + gi, b, tb, l & 15, l >> 4);
  } else {
    split_wave<kQ4_K>(J, nblk, g0 + gi, b, tb, l & 15, l >> 4);
  }
}

// The chains of k_skinny_split's t-terms: one wave per (64-row group g0 + blockIdx.x,
// activation row blockIdx.y), lane r = weight row (one-wave workgroups spread the
// t-term reads over all CUs). Every load of a chain (nblk <= NB t-terms and d values)
// is issued before its first FMA, so the chain waits on one round trip.
template <int NB>
__global__ __launch_bounds__(64) void k_skinny_chain(const float* __restrict__ T, const uint8_t* __restrict__ acts,
                                                     int64_t arb, int m, int nblk, int64_t g0, int64_t n0, int64_t n1,
                                                     float* __restrict__ y, int64_t ys, const float* __restrict__ bias) {
  const int r = threadIdx.x, mm = (int)blockIdx.y;
  const int64_t n = (g0 + blockIdx.x) * kRowGroup + r;
  const float* tp = T + ((int64_t)blockIdx.x * nblk * 16 + mm) * 64 + r;
  const uint8_t* ap = acts + mm * arb;
  float t[NB], d[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int bc = b < nblk ? b : nblk - 1;  // past the row: a repeat, not used
    t[b] = tp[bc * 16 * 64];
    d[b] = *reinterpret_cast<const float*>(ap + bc * 292);
  }
  float v = 0.0f;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b < nblk) v = fmaf(d[b], t[b], v);
  }
  if (n >= n0 && n < n1) y[mm * ys + n] = bias ? v + bias[n] : v;
}

size_t skinny_lds(int64_t nblk, int ct, int mt, bool gated = false) {
  return (size_t)nblk * (16 * mt * (16 * ct + 1)) * (gated ? 2 : 1) * sizeof(float);
}
constexpr size_t kSkinnyMaxLds = 160 * 1024;

template <int CT, int MT, bool kFused, bool kGated = false, int W = kSkinnyWaves, int D = 1, bool kSx = false>
hipError_t skinny_launch(const SkinnyGroup& g, int wgs, hipStream_t s) {
  const size_t lds = skinny_lds(g.nblk, CT, MT, kGated);
  if (lds > kSkinnyMaxLds) return hipErrorInvalidValue;
  if (lds > 64 * 1024) {
    const hipError_t e =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&k_skinny<CT, MT, kFused, kGated, W, D, kSx>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((k_skinny<CT, MT, kFused, kGated, W, D, kSx>), dim3((unsigned)wgs), dim3(W * 64), lds, s, g);
  return hipGetLastError();
}

SkinnyJob skinny_job(const WeightDev& w, int64_t m, int64_t n0, int64_t n1, float* y, int64_t ys, const float* bias) {
  SkinnyJob J{};
  for (int i = 0; i < 4; ++i) J.p[i] = w.plane[i];
  J.n_pad = w.n_pad;
  J.n0 = n0;
  J.n1 = n1;
  J.y = y;
  J.ys = ys;
  J.bias = bias;
  J.dtype = w.dtype;
  J.m = (int)m;
  return J;
}

// Tiles of 64 rows when the group has work for very many workgroups (at 16-row
// tiles at least 16 per CU, e.g. an LM head) and their LDS fits; else 16-row tiles.
// More than 16 activation rows take 4 activation tiles and 16-row weight tiles.
int skinny_ct(int64_t wgs16, int64_t nblk, int cus, int mt) {
  return mt == 1 && wgs16 >= 16 * (int64_t)cus && skinny_lds(nblk, 4, 1) <= kSkinnyMaxLds ? 4 : 1;
}

// Bytes of k_skinny_split's t-terms for rows [n0, n1) of nblk super-blocks.
int64_t split_t_bytes(int64_t n0, int64_t n1, int64_t nblk) {
  return ((n1 + kRowGroup - 1) / kRowGroup - n0 / kRowGroup) * nblk * 16 * 64 * (int64_t)sizeof(float);
}

// ws: room for the split launch's t-terms (none: launches of one long-row job on few
// tiles run k_skinny with 4 super-blocks of weights in flight per wave instead).
hipError_t launch_group(SkinnyGroup& g, const int64_t* first_row, const int64_t* last_row, bool fused, bool gated,
                        int cus, hipStream_t s, bool sx = false, const Workspace* ws = nullptr) {
  int mmax = 0;
  int64_t wgs16 = 0;
  for (int i = 0; i < g.count; ++i) {
    wgs16 += (last_row[i] + 15) / 16 - first_row[i] / 16;
    mmax = g.job[i].m > mmax ? g.job[i].m : mmax;
  }
  const int mt = mmax > 16 ? 4 : 1;
  if (mt == 4 && (fused || sx)) return hipErrorInvalidValue;
  if (sx && (fused || gated)) return hipErrorInvalidValue;
  const int ct = gated ? 1 : skinny_ct(wgs16, g.nblk, cus, mt);
  const int nc = 16 * ct;
  int64_t wgs = 0;
  for (int i = 0; i < g.count; ++i) {
    g.job[i].t0 = first_row[i] / nc;
    g.job[i].wg0 = (int)wgs;
    wgs += (last_row[i] + nc - 1) / nc - first_row[i] / nc;
  }
  if (wgs >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  // Waves per workgroup: launches of more tiles than CUs whose tiles have few
  // super-blocks (at most 12, gate and up counted), and the 64-row tiles, run 4
  // waves so that more workgroups are resident (measured at M = 16: gate 8960 x 1536
  // 7.3 -> 6.7 us, gated 13.3 -> 11.2 us, a 151936 x 1536 Q6_K LM head 80 -> 68 us).
  const bool four = ct == 4 || (!fused && mt == 1 && wgs > cus && g.nblk * (gated ? 2 : 1) <= 12);
  if (gated) {
    if (mt == 4) return skinny_launch<1, 4, false, true>(g, (int)wgs, s);
    if (fused) return skinny_launch<1, 1, true, true>(g, (int)wgs, s);
    return four ? skinny_launch<1, 1, false, true, 4>(g, (int)wgs, s) : skinny_launch<1, 1, false, true>(g, (int)wgs, s);
  }
  if (sx) {
    // sub-scaled rows (up to 16): the launch shapes of the Q8_K rows below
    if (ct == 4) return skinny_launch<4, 1, false, false, 4, 1, true>(g, (int)wgs, s);
    if (four) return skinny_launch<1, 1, false, false, 4, 1, true>(g, (int)wgs, s);
    if (wgs <= cus && g.nblk >= 3 * kSkinnyWaves) {  // 2 in flight: the m_b words take the registers of 2 more
      return skinny_launch<1, 1, false, false, kSkinnyWaves, 2, true>(g, (int)wgs, s);
    }
    return skinny_launch<1, 1, false, false, kSkinnyWaves, 1, true>(g, (int)wgs, s);
  }
  if (mt == 4) return skinny_launch<1, 4, false>(g, (int)wgs, s);
  if (ct == 4) return fused ? skinny_launch<4, 1, true, false, 4>(g, (int)wgs, s)
                            : skinny_launch<4, 1, false, false, 4>(g, (int)wgs, s);
  if (fused) return skinny_launch<1, 1, true>(g, (int)wgs, s);
  if (four) return skinny_launch<1, 1, false, false, 4>(g, (int)wgs, s);
  // One round of 8-wave workgroups with at least 3 super-blocks per wave (a long-K
  // matmul such as an FFN down projection): the waves' dependent load steps, not the
  // bytes, set the time, so 4 super-blocks of weights stay in flight per wave.
  if (wgs <= cus && g.nblk >= 3 * kSkinnyWaves) {
    if (g.count == 1 && g.job[0].dtype == kQ6_K && g.nblk >= 32 && g.nblk <= 64 && 2 * wgs <= cus && ws != nullptr &&
        ws->bytes >= (size_t)split_t_bytes(first_row[0], last_row[0], g.nblk)) {
      // one matmul: the t-terms of 64-row groups x super-block slices, then the chains
      const SkinnyJob& J = g.job[0];
      const int64_t g0 = first_row[0] / kRowGroup, g1 = (last_row[0] + kRowGroup - 1) / kRowGroup;
      const int slices = (g.nblk + kSplitWaves - 1) / kSplitWaves;
      float* T = reinterpret_cast<float*>(ws->p);
      hipLaunchKernelGGL(k_skinny_split, dim3((unsigned)((g1 - g0) * slices)), dim3(kSplitWaves * 64), 0, s, J, g.nblk,
                         slices, g0, T);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      const dim3 grid((unsigned)(g1 - g0), (unsigned)J.m);
      if (g.nblk <= 40) {
        hipLaunchKernelGGL(k_skinny_chain<40>, grid, dim3(64), 0, s, T, J.acts, J.arb, J.m, g.nblk, g0, J.n0, J.n1,
                           J.y, J.ys, J.bias);
      } else {
        hipLaunchKernelGGL(k_skinny_chain<64>, grid, dim3(64), 0, s, T, J.acts, J.arb, J.m, g.nblk, g0, J.n0, J.n1,
                           J.y, J.ys, J.bias);
      }
      return hipGetLastError();
    }
    return skinny_launch<1, 1, false, false, kSkinnyWaves, 4>(g, (int)wgs, s);
  }
  return skinny_launch<1, 1, false>(g, (int)wgs, s);
}

}  // namespace

bool gemv_mma_supported(int dtype, int af, int64_t m) {
  if (dtype != kQ4_K && dtype != kQ6_K) return false;
  if (af == kActQ8_K) return m >= 2 && m <= kSkinnyMaxRows;
  return af == kActSX && m >= 2 && m <= kSkinnySxMaxRows;
}

// Sub-scaled rows: the MFMA GEMV costs the same from 2 to 16 rows, the VALU GEMV grows
// with the rows but is cheaper for a few rows of a launch with many 16-row tiles.
// Measured (graph replay, rotated weights; skinny vs VALU GEMV at m = 2 / 4 / 8):
// Q4_K 8960 x 1536 11.8 / 11.9 / 12.3 vs 8.2 / 10.6 / 15.3 us; Q4_K 14336 x 4096
// 23.2 / 23.3 / 23.6 vs 13.2 / 17.5 / 25.0; Q6_K 151936 x 1536 (64-row tiles) 128 / 128 /
// 130 vs 71 / 100 / 156; one round of tiles (Q4_K 1536 x 1536, 4096 x 14336; Q6_K
// 1536 x 8960, 4096 x 14336) 6.5 / 20.8 / 16.1 / 24.5 vs 7.3 / 23.6 / 23.8 / 34.1 at m = 2.
bool skinny_sx_pays(const WeightDev& w, int64_t m, int64_t n0, int64_t n1) {
  const int64_t tiles = (n1 + 15) / 16 - n0 / 16;
  const int64_t cus = w.cus > 0 ? w.cus : 256;
  return m >= 8 || tiles <= cus || (w.dtype == kQ6_K && tiles < 16 * cus);
}

bool gemv_mma_lds_ok(int64_t nblk, int64_t m, bool gated) {
  return skinny_lds(nblk, 1, m > 16 ? 4 : 1, gated) <= kSkinnyMaxLds;
}

int64_t skinny_units(const GemvJob* jobs, int count) {
  if (count <= 0) return 0;
  int64_t wgs16 = 0;
  for (int i = 0; i < count; ++i) wgs16 += (jobs[i].w->n + 15) / 16;
  int64_t mmax = 0;
  for (int i = 0; i < count; ++i) mmax = jobs[i].m > mmax ? jobs[i].m : mmax;
  const int ct = jobs[0].wu != nullptr ? 1 : skinny_ct(wgs16, jobs[0].w->nblk, jobs[0].w->cus, mmax > 16 ? 4 : 1);
  int64_t wgs = 0;
  for (int i = 0; i < count; ++i) wgs += (jobs[i].w->n + 16 * ct - 1) / (16 * ct);
  return wgs * jobs[0].w->nblk;
}

// The split route pays for Q6_K rows of at least 32 super-blocks on at most half as
// many 16-row tiles as CUs. Measured (graph replay, M = 2 / 8 / 16, split vs k_skinny):
// Q6_K 1536 x 8960 9.3 / 9.4 / 9.9 vs 10.7 / 10.8 / 11.5 us; with every CU holding a
// tile it loses (Q6_K 4096 x 14336: 20.7 / 21.7 / 25.2 vs 16.0 / 16.2 / 17.7), and so it
// does for Q4_K's lighter super-blocks (1536 x 6144: 7.6 / 7.8 / 8.0 vs 6.1 / 6.2 / 6.8).
int64_t skinny_split_bytes(const WeightDev& w, int af, int64_t m, int64_t n0, int64_t n1) {
  const int64_t tiles = (n1 + 15) / 16 - n0 / 16;
  if (af != kActQ8_K || w.dtype != kQ6_K || m < 2 || m > 16 || n1 <= n0 || 2 * tiles > w.cus || w.nblk < 32 ||
      w.nblk > 64) {
    return 0;
  }
  return split_t_bytes(n0, n1, w.nblk);
}

hipError_t launch_gemv_mma(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0,
                           int64_t n1, float* y, int64_t ys, const float* bias, hipStream_t s, const Workspace* ws) {
  if (!gemv_mma_supported(w.dtype, af, m)) return hipErrorInvalidValue;
  if (n1 <= n0) return hipSuccess;
  SkinnyGroup g;
  g.job[0] = skinny_job(w, m, n0, n1, y, ys, bias);
  g.job[0].acts = acts;
  g.job[0].arb = arb;
  g.count = 1;
  g.nblk = (int)w.nblk;
  return launch_group(g, &n0, &n1, false, false, w.cus, s, af == kActSX, ws);
}

hipError_t launch_gemv_mma_many(const GemvJob* jobs, int count, hipStream_t s, const Workspace* ws) {
  for (int i0 = 0; i0 < count; i0 += kSkinnyMaxJobs) {
    SkinnyGroup g;
    g.count = count - i0 < kSkinnyMaxJobs ? count - i0 : kSkinnyMaxJobs;
    g.nblk = (int)jobs[i0].w->nblk;
    const bool fused = jobs[i0].x != nullptr, gated = jobs[i0].wu != nullptr;
    int64_t first[kSkinnyMaxJobs], last[kSkinnyMaxJobs];
    for (int i = 0; i < g.count; ++i) {
      const GemvJob& q = jobs[i0 + i];
      if (q.w->nblk != g.nblk || !gemv_mma_supported(q.w->dtype, kActQ8_K, q.m) || (q.x != nullptr) != fused ||
          (q.wu != nullptr) != gated) {
        return hipErrorInvalidValue;
      }
      if (gated && (q.wu->dtype != q.w->dtype || q.wu->n != q.w->n || q.wu->k != q.w->k || q.bias != nullptr ||
                    !act_ok(q.act))) {
        return hipErrorInvalidValue;
      }
      g.job[i] = skinny_job(*q.w, q.m, 0, q.w->n, q.y, q.ys, q.bias);
      if (gated) {
        for (int p = 0; p < 4; ++p) g.job[i].pu[p] = q.wu->plane[p];
        g.job[i].act = q.act;
      }
      g.job[i].acts = q.acts;
      g.job[i].arb = q.arb;
      g.job[i].x = q.x;
      g.job[i].xs = q.xs;
      first[i] = 0;
      last[i] = q.w->n;
    }
    const hipError_t e = launch_group(g, first, last, fused, gated, jobs[i0].w->cus, s, false, ws);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace dq
