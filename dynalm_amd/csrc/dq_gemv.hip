// dq_gemv.hip -- the decode GEMV for gfx950 (M <= 4 activation rows per pass,
// int8 dot products against the 64-row weight layout) and its host launchers.
//
// Arithmetic contracts follow the reference's integer sums and fp32 combination:
//   dynacore/cpu/generic/kernels_generic.cpp:210-310 (per-32 activations),
//   dynacore/cpu/avx2/kernels_avx2.cpp:976-1058 (one activation scale per 256 values).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "dq_act.h"
#include "dq_device.h"
#include "dq_internal.h"
#include "dq_quant.h"

namespace dq {

// ===================================================================== GEMV
// Lane r of every wave owns weight row 64*G + r of the workgroup's row group G
// (the 64-row layout of dq_layout.h), so at each step all lanes multiply their
// own weight bytes with the same activation values: those are wave-uniform and
// come through scalar loads, the weights through 1 KB-contiguous vector loads,
// and a row's sums need no cross-lane reduction. The W waves of a workgroup
// split the row's blocks into W contiguous slices (W times more bytes in flight
// per row group).
//
// fp32 order. K-quants x Q8_K: each lane computes its super-blocks' exact S, Mn
// and t = fma(-dmin, (float)Mn, d*(float)S) and writes t to LDS; after a barrier
// lane r of wave 0 runs acc = fma(da, t, acc) over all super-blocks in order --
// the canonical order of the CPU oracle, so outputs are bit-identical to it.
// Per-32 activations: each wave accumulates its slice in the reference's generic
// per-block order; the W slice sums are then added in slice order.

typedef u32 v4ua __attribute__((ext_vector_type(4), aligned(4)));

// Wave-uniform loads (scalar loads when base and offset are uniform).
DQ_DEV u32 uld(const uint8_t* __restrict__ p, u32 off) { return *reinterpret_cast<const u32*>(p + off); }
DQ_DEV v4u uld16(const uint8_t* __restrict__ p, u32 off) {
  const v4ua v = *reinterpret_cast<const v4ua*>(p + off);
  return v4u{v.x, v.y, v.z, v.w};
}
DQ_DEV int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Activation codes 16c .. 16c+15 of a 32-value per-32 / GGUF-Q8_0 block at base (uniform).
template <int AF>
DQ_DEV void act_codes32(const uint8_t* __restrict__ a, u32 base, v4u& x0, v4u& x1) {
  if (AF == kActPer32) {
    x0 = uld16(a, base + 8);
    x1 = uld16(a, base + 24);
  } else {  // GGUF Q8_0: codes at byte 2 of the 34-byte block
    const u32 off = base + 2, al = off & ~3u;
    const v4u y0 = uld16(a, al), y1 = uld16(a, al + 16);
    const u32 y2 = uld(a, al + 32);
    if ((off & 3u) == 0) {
      x0 = y0;
      x1 = y1;
    } else {
      x0 = v4u{__builtin_amdgcn_alignbyte(y0.y, y0.x, 2), __builtin_amdgcn_alignbyte(y0.z, y0.y, 2),
               __builtin_amdgcn_alignbyte(y0.w, y0.z, 2), __builtin_amdgcn_alignbyte(y1.x, y0.w, 2)};
      x1 = v4u{__builtin_amdgcn_alignbyte(y1.y, y1.x, 2), __builtin_amdgcn_alignbyte(y1.z, y1.y, 2),
               __builtin_amdgcn_alignbyte(y1.w, y1.z, 2), __builtin_amdgcn_alignbyte(y2, y1.w, 2)};
    }
  }
}

// ---- per-format weight chunks: the vector loads of U consecutive blocks of the
// lane's row (blocks past the wave's slice read as zeros and are not used).
struct Rsrcs {
  __amdgpu_buffer_rsrc_t r0, r1, r2, r3;
};

template <int WT, int U>
struct Chunk;

template <int U>
struct Chunk<kQ4_K, U> {
  v4u q[U][8], hd[U];
  DQ_DEV void load(const Rsrcs& rs, int bb, int b1, int nblk, int r) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = bb + u < b1 ? bb + u : nblk;
      // header first: the scales are needed by the first sub-block pair
      hd[u] = ld16nt(rs.r1, (u32)((b * 64 + r) * 16));
#pragma unroll
      for (int c = 0; c < 8; ++c) q[u][c] = ld16nt(rs.r0, (u32)(((b * 8 + c) * 64 + r) * 16));
    }
  }
};

template <int U>
struct Chunk<kQ6_K, U> {
  v4u L[U][8], H[U][4], SC[U];
  u32 DW[U];
  DQ_DEV void load(const Rsrcs& rs, int bb, int b1, int nblk, int r) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = bb + u < b1 ? bb + u : nblk;
#pragma unroll
      for (int c = 0; c < 8; ++c) L[u][c] = ld16nt(rs.r0, (u32)(((b * 8 + c) * 64 + r) * 16));
#pragma unroll
      for (int c = 0; c < 4; ++c) H[u][c] = ld16nt(rs.r1, (u32)(((b * 4 + c) * 64 + r) * 16));
      SC[u] = ld16nt(rs.r2, (u32)((b * 64 + r) * 16));
      DW[u] = ld2nt(rs.r3, (u32)((b * 64 + r) * 2));
    }
  }
};

template <int WT, int U>
struct Chunk32 {  // Q8_0 (2 chunks of 16 B per block) and Q4_0 (1)
  static constexpr int kC = WT == kQ8_0 ? 2 : 1;
  v4u q[U][kC];
  u32 DW[U];
  DQ_DEV void load(const Rsrcs& rs, int bb, int b1, int nblk, int r) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = bb + u < b1 ? bb + u : nblk;
#pragma unroll
      for (int c = 0; c < kC; ++c) q[u][c] = ld16nt(rs.r0, (u32)(((b * kC + c) * 64 + r) * 16));
      DW[u] = ld2nt(rs.r1, (u32)((b * 64 + r) * 2));
    }
  }
};
template <int U>
struct Chunk<kQ8_0, U> : Chunk32<kQ8_0, U> {};
template <int U>
struct Chunk<kQ4_0, U> : Chunk32<kQ4_0, U> {};

// Activations staged in LDS (both the plain and the fused path), 16-byte aligned
// so that compute reads them with broadcast ds_read_b128 at wave-uniform addresses:
//   Q8_K super-block (336 B):  d float @0, codes int8[256] @16, bsums int16[16] @272,
//       and the 32-value sub-block code sums s_j (j = 0..7) in two more forms:
//       int8 pairs s_j >> 7 @304 + j and s_j & 127 @312 + j (s_j = 128 (s_j >> 7) +
//       (s_j & 127), |s_j| <= 4064), and 128 s_j of the odd sub-blocks @320 + 4 (j / 2)
//   32-value block   (48 B):   d float @0, code sum int32 @4, codes int8[32] @16
// (per-32 ActBlockQ8 and GGUF Q8_0 activations both stage as the latter; the GGUF
// fp16 d converts exactly to float).
//   sub-scaled super-block (352 B): u float @0, codes int8[256] @16, the block
//       multipliers m_j int32[8] @272, m_j * s_j int32[8] @304 (s_j the code sum of
//       32-value block j), and 128 s_j of the odd blocks int32[4] @336
//   int16 32-value block (80 B): d float @0, code sum int32 @4, the code sums of
//       values 0..15 and 16..31 int32 @8, @12, and each code split as 256 hi + lo:
//       hi int8[32] @16, lo uint8[32] @48 (dynacore's split_act16,
//       dynacore/cpu/generic/kernels_generic.cpp:334-350)
constexpr int kStageQ8K = 336;
constexpr int kStageSX = 352;
constexpr int kStage32 = 48;
constexpr int kStage16 = 80;
constexpr int kStageF32 = 144;
// Staged bytes per 32-value block of the per-32 activation formats.
constexpr int stage_b32(int af) { return af == kActQ16 ? kStage16 : af == kActF32 ? kStageF32 : kStage32; }

// fp32 activations (the reference's kF32 contract, dynacore/cpu/generic/kernels_generic.cpp:67-150):
// a staged 32-value block is the 32 floats @0 and their sum, added in index order, @128.
// The four bytes of a dword as floats (v_cvt_f32_ubyte0..3).
DQ_DEV void ubytes_f32(u32 w, float* f) {
#pragma unroll
  for (int e = 0; e < 4; ++e) f[e] = (float)((w >> (8 * e)) & 0xFFu);
}
// dot + sum_{i < n} q[i] * x[i] in index order, x from a staged block (wave-uniform
// LDS address: broadcast reads); every product and sum rounds where written.
template <int N>
DQ_DEV float dot_f32(float dot, const float* q, const uint8_t* x) {
#pragma unroll
  for (int i = 0; i < N; i += 4) {
    const v4u xv = *reinterpret_cast<const v4u*>(x + 4 * i);
#pragma unroll
    for (int e = 0; e < 4; ++e) dot = dot + q[i + e] * as_f(xv[e]);
  }
  return dot;
}
// Staged bytes per super-block of the 256-value activation formats.
constexpr int stage_sb(int af) { return af == kActSX ? kStageSX : kStageQ8K; }

// Writes the derived forms of sub-block sum s of sub-block j of a staged Q8_K block.
DQ_DEV void stage_subsum(uint8_t* o, int j, int s) {
  o[304 + j] = (uint8_t)(s >> 7);
  o[312 + j] = (uint8_t)(s & 127);
  if (j & 1) *reinterpret_cast<int32_t*>(o + 320 + 2 * (j - 1)) = s * 128;
}

DQ_DEV v4u lds16(const uint8_t* p) { return *reinterpret_cast<const v4u*>(p); }
DQ_DEV u32 lds4(const uint8_t* p) { return *reinterpret_cast<const u32*>(p); }

// Per-lane state the compute steps write: Q8_K t-terms and da go to LDS (rec,
// dav); per-32 sums accumulate in acc.
template <int M>
struct Out {
  float* rec;
  float* dav;
  float acc[M];
  float cor[M];  // Q4_K x int16: the mins term, subtracted at the end
  int32_t* dbg;
  int64_t dbg_n, n;
  int nblk, r;
};

// Q4_K. Low nibbles (sub-block 2jp of pair jp) are unsigned bytes after one AND;
// high nibbles are stored XOR 8 (dq_layout.h), so `q & 0xF0F0F0F0` is the int8
// 16 * (q - 8) and a dot product seeded with 128 * s_j (the staged odd-sub-block
// sum) is exactly 16 * P_j.
template <int AF, int M, int U>
DQ_DEV void compute(const Chunk<kQ4_K, U>& ch, int bb, const uint8_t* st, Out<M>& o, int nv = U) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (u >= nv) break;
    const int b = bb + u;
    // the 6-bit scales sc_j (bits 0..5 of byte j&3 of sc_lo / sc_hi) and the mins m_j
    // as clean bytes (get_scale_min_k4, quant_formats.h:62-70)
    const u32 s0 = ch.hd[u].y, s1 = ch.hd[u].z, s2 = ch.hd[u].w;
    const u32 sc_lo = s0;
    const u32 sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0xF0F0F0F0u);
    const u32 mn_lo = s1 & 0x3F3F3F3Fu;
    const u32 mn_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
    const float d = h2f(ch.hd[u].x), dmin = h2f(ch.hd[u].x >> 16);
    if constexpr (AF == kActF32) {
      // vec_dot_q4_K (kernels_generic.cpp:108-130): per 64 values, dot_lo / sum_lo over
      // the low nibbles (sub-block 2jp) and dot_hi / sum_hi over the high ones (2jp + 1),
      // then sum += d*sc*dot - dmin*m*sum_x for each
#pragma unroll
      for (int jp = 0; jp < 4; ++jp) {
        float qlo[32], qhi[32];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const v4u c = ch.q[u][2 * jp + h];
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            ubytes_f32(c[w] & 0x0F0F0F0Fu, qlo + 16 * h + 4 * w);
            ubytes_f32(((c[w] >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u, qhi + 16 * h + 4 * w);
          }
        }
        const u32 scw = jp < 2 ? sc_lo : sc_hi, mnw = jp < 2 ? mn_lo : mn_hi;
        const int e = 16 * (jp & 1);
        const float sl = (float)bfe(scw, e, 6), sh = (float)bfe(scw, e + 8, 6);
        const float ml = (float)bfe(mnw, e, 8), mh = (float)bfe(mnw, e + 8, 8);
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
          const uint8_t* al = st + (mm * o.nblk * 8 + b * 8 + 2 * jp) * kStageF32;
          const uint8_t* ah = al + kStageF32;
          const float dlo = dot_f32<32>(0.0f, qlo, al), dhi = dot_f32<32>(0.0f, qhi, ah);
          o.acc[mm] = o.acc[mm] + ((d * sl) * dlo - (dmin * ml) * as_f(lds4(al + 128)));
          o.acc[mm] = o.acc[mm] + ((d * sh) * dhi - (dmin * mh) * as_f(lds4(ah + 128)));
        }
      }
      continue;
    }
#pragma unroll
    for (int mm = 0; mm < M; ++mm) {
      if (AF == kActQ8_K) {
        const uint8_t* ab = st + (mm * o.nblk + b) * kStageQ8K;
        const v4u sj = lds16(ab + 304);   // s_j >> 7 (j = 0..3, 4..7), s_j & 127 (0..3, 4..7)
        const v4u codd = lds16(ab + 320);  // 128 s_j, j = 1, 3, 5, 7
        // One row, one super-block per chunk (the decode launch): all sixteen code
        // reads are issued here, before the first wait on the weights, so a wave whose
        // weights land last computes without further LDS round trips (64 VGPRs).
        constexpr bool kAll = M == 1 && U == 1;
        v4u av[kAll ? 16 : 1];
        if constexpr (kAll) {
#pragma unroll
          for (int i = 0; i < 16; ++i) av[i] = lds16(ab + 16 + 16 * i);
          __builtin_amdgcn_sched_barrier(0);
        }
        int S = 0;
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) {
          const v4u c0 = ch.q[u][2 * jp], c1 = ch.q[u][2 * jp + 1];
          const uint8_t* cp = ab + 16 + 64 * jp;
          const v4u a0 = kAll ? av[kAll ? 4 * jp : 0] : lds16(cp), a1 = kAll ? av[kAll ? 4 * jp + 1 : 0] : lds16(cp + 16);
          const v4u a2 = kAll ? av[kAll ? 4 * jp + 2 : 0] : lds16(cp + 32);
          const v4u a3 = kAll ? av[kAll ? 4 * jp + 3 : 0] : lds16(cp + 48);
          const int pe = sdot16(c1 & 0x0F0F0F0Fu, a1, sdot16(c0 & 0x0F0F0F0Fu, a0, 0));
          const int x16 = sdot16(c1 & 0xF0F0F0F0u, a3, sdot16(c0 & 0xF0F0F0F0u, a2, (int)codd[jp]));
          const int po = x16 >> 4;
          const u32 scw = jp < 2 ? sc_lo : sc_hi;
          const int e = 16 * (jp & 1);
          S += __builtin_amdgcn_sbfe(pe, 0, 24) * (int)bfe(scw, e, 6);
          S += __builtin_amdgcn_sbfe(po, 0, 24) * (int)bfe(scw, e + 8, 6);
        }
        // Mn = sum_j m_j s_j = 128 sum_j m_j (s_j >> 7) + sum_j m_j (s_j & 127)
        const int mh = sdot4(mn_hi, sj.y, sdot4(mn_lo, sj.x, 0));
        const int ml = sdot4(mn_hi, sj.w, sdot4(mn_lo, sj.z, 0));
        const int Mn = (mh << 7) + ml;
        float t = d * (float)S;
        t = fmaf(-dmin, (float)Mn, t);
        o.rec[(mm * o.nblk + b) * 64 + o.r] = t;
        if (o.r == 0) o.dav[mm * o.nblk + b] = as_f(lds4(ab));
        if (o.dbg != nullptr && o.n < o.dbg_n) {
          int32_t* p = o.dbg + (((int64_t)mm * o.dbg_n + o.n) * o.nblk + b) * 2;
          p[0] = S;
          p[1] = Mn;
        }
      } else if (AF == kActSX) {
        // sub-scaled (kernels_avx2.cpp:1117-1163): S = sum_j sc_j m_j P_j in 64 bits,
        // Mn = sum_j mn_j (m_j s_j); the Q8_K pair's canonical order with u for da
        const uint8_t* ab = st + (mm * o.nblk + b) * kStageSX;
        const v4u codd = lds16(ab + 336);  // 128 s_j, j = 1, 3, 5, 7
        const v4i mul0 = __builtin_bit_cast(v4i, lds16(ab + 272)), mul1 = __builtin_bit_cast(v4i, lds16(ab + 288));
        const v4i ms0 = __builtin_bit_cast(v4i, lds16(ab + 304)), ms1 = __builtin_bit_cast(v4i, lds16(ab + 320));
        int64_t S = 0;
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) {
          const v4u c0 = ch.q[u][2 * jp], c1 = ch.q[u][2 * jp + 1];
          const uint8_t* cp = ab + 16 + 64 * jp;
          const int pe = sdot16(c1 & 0x0F0F0F0Fu, lds16(cp + 16), sdot16(c0 & 0x0F0F0F0Fu, lds16(cp), 0));
          const int x16 = sdot16(c1 & 0xF0F0F0F0u, lds16(cp + 48), sdot16(c0 & 0xF0F0F0F0u, lds16(cp + 32), (int)codd[jp]));
          const int po = x16 >> 4;
          const u32 scw = jp < 2 ? sc_lo : sc_hi;
          const int e = 16 * (jp & 1);
          const v4i mj = jp < 2 ? mul0 : mul1;
          S += (int64_t)pe * (int)(bfe(scw, e, 6) * (u32)mj[2 * (jp & 1)]);
          S += (int64_t)po * (int)(bfe(scw, e + 8, 6) * (u32)mj[2 * (jp & 1) + 1]);
        }
        int Mn = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          Mn += (int)bfe(mn_lo, 8 * j, 8) * ms0[j];
          Mn += (int)bfe(mn_hi, 8 * j, 8) * ms1[j];
        }
        float t = d * (float)S;
        t = fmaf(-dmin, (float)Mn, t);
        o.rec[(mm * o.nblk + b) * 64 + o.r] = t;
        if (o.r == 0) o.dav[mm * o.nblk + b] = as_f(lds4(ab));
      } else if (AF == kActQ16) {
        // int16 activations (kernels_avx2.cpp:1697-1729): P_j = sum q a over the
        // 32 values of sub-block j, exactly 256 sum(q hi) + sum(q lo) (the nibbles
        // are valid signed and unsigned bytes); acc += (float)(sc_j P_j) (d da) and
        // the mins term dmin (m_j da (float)sum) gathered apart and subtracted
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int jp = j >> 1;
          const uint8_t* ab = st + (mm * o.nblk * 8 + b * 8 + j) * kStage16;
          const v4u c0 = ch.q[u][2 * jp], c1 = ch.q[u][2 * jp + 1];
          const v4u q0 = (j & 1) ? ((c0 >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u : c0 & 0x0F0F0F0Fu;
          const v4u q1 = (j & 1) ? ((c1 >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u : c1 & 0x0F0F0F0Fu;
          const int ph = sdot16(q1, lds16(ab + 32), sdot16(q0, lds16(ab + 16), 0));
          const int pl = (int)udot16(q1, lds16(ab + 64), udot16(q0, lds16(ab + 48), 0u));
          const int P = ph * 256 + pl;
          const u32 scw = j < 4 ? sc_lo : sc_hi;
          const u32 mnw = j < 4 ? mn_lo : mn_hi;
          const int sc = (int)bfe(scw, 8 * (j & 3), 6), mn = (int)bfe(mnw, 8 * (j & 3), 8);
          const float ad = as_f(lds4(ab));
          o.acc[mm] = o.acc[mm] + (float)(sc * P) * (d * ad);
          o.cor[mm] = o.cor[mm] + dmin * (((float)mn * ad) * (float)(int)lds4(ab + 4));
        }
      } else {
        // per-32 activations, sub-block order j = 0..7 (kernels_generic.cpp:267-275)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int jp = j >> 1;
          const uint8_t* ab = st + (mm * o.nblk * 8 + b * 8 + j) * kStage32;
          const v4u c0 = ch.q[u][2 * jp], c1 = ch.q[u][2 * jp + 1];
          const int sum = (int)lds4(ab + 4);
          int P;
          if (j & 1) {
            P = sdot16(c1 & 0xF0F0F0F0u, lds16(ab + 32), sdot16(c0 & 0xF0F0F0F0u, lds16(ab + 16), sum * 128)) >> 4;
          } else {
            P = sdot16(c1 & 0x0F0F0F0Fu, lds16(ab + 32), sdot16(c0 & 0x0F0F0F0Fu, lds16(ab + 16), 0));
          }
          const u32 scw = j < 4 ? sc_lo : sc_hi;
          const u32 mnw = j < 4 ? mn_lo : mn_hi;
          const int sc = (int)bfe(scw, 8 * (j & 3), 6), mn = (int)bfe(mnw, 8 * (j & 3), 8);
          const float ad = as_f(lds4(ab));
          const float t = (d * (float)sc) * (float)P - (dmin * (float)mn) * (float)sum;
          o.acc[mm] = o.acc[mm] + ad * t;
        }
      }
    }
  }
}

template <int AF, int M, int U>
DQ_DEV void compute(const Chunk<kQ6_K, U>& ch, int bb, const uint8_t* st, Out<M>& o, int nv = U) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (u >= nv) break;
    const int b = bb + u;
    const float d = h2f(ch.DW[u]);
    if constexpr (AF == kActF32) {
      // vec_dot_q6_K (kernels_generic.cpp:132-150): per 16-value unit u (values 16u ..
      // 16u + 15) s_u = sum (q - 32) x in index order; sum += d*sc_u*s_u, units in order.
      // ql chunk c: half p = c/4, values 128p + 16(c%4) + i (low nibbles) and + 64
      // (high); top bits from qh chunk 2p + c%2, bit pairs s and s+2 (s = (c%4)/2).
#pragma unroll
      for (int uu = 0; uu < 16; ++uu) {
        const int p = uu >> 3, cc = uu & 3, c = 4 * p + cc, sh = cc >> 1;
        const v4u hb = ch.H[u][2 * p + (c & 1)];
        const v4u qv = (uu & 4) ? ((ch.L[u][c] >> 4) & 0x0F0F0F0Fu) | (((hb >> (2 * sh + 4)) & 0x03030303u) << 4)
                                : (ch.L[u][c] & 0x0F0F0F0Fu) | (((hb >> (2 * sh)) & 0x03030303u) << 4);
        float q[16];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          ubytes_f32(qv[w], q + 4 * w);
#pragma unroll
          for (int e = 0; e < 4; ++e) q[4 * w + e] = q[4 * w + e] - 32.0f;
        }
        const u32 sw = uu < 4 ? ch.SC[u].x : uu < 8 ? ch.SC[u].y : uu < 12 ? ch.SC[u].z : ch.SC[u].w;
        const float ds = d * (float)sbfe(sw, 8 * (uu & 3), 8);
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
          const uint8_t* ab = st + (mm * o.nblk * 8 + b * 8 + uu / 2) * kStageF32 + 64 * (uu & 1);
          o.acc[mm] = o.acc[mm] + ds * dot_f32<16>(0.0f, q, ab);
        }
      }
      continue;
    }
    // ql chunk c: half p = c/4, values 128p + 16(c%4) + i (low nibbles) and + 64
    // (high); their top bits are qh chunk 2p + c%2 at bit pairs s and s+2,
    // s = (c%4)/2 (quant_formats.cpp:192-216). Units u_lo = 8p + c%4, u_hi = u_lo + 4.
    v4u qlo[8], qhi[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int p = c >> 2, cc = c & 3, s = cc >> 1;
      const v4u hb = ch.H[u][2 * p + (c & 1)];
      qlo[c] = (ch.L[u][c] & 0x0F0F0F0Fu) | (((hb >> (2 * s)) & 0x03030303u) << 4);
      qhi[c] = ((ch.L[u][c] >> 4) & 0x0F0F0F0Fu) | (((hb >> (2 * s + 4)) & 0x03030303u) << 4);
    }
#pragma unroll
    for (int mm = 0; mm < M; ++mm) {
      if (AF == kActQ8_K) {
        const uint8_t* ab = st + (mm * o.nblk + b) * kStageQ8K;
        int S = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const int ulo = 8 * (c >> 2) + (c & 3), uhi = ulo + 4;
          const u32 bsl = lds4(ab + 272 + 4 * (ulo >> 1)), bsh = lds4(ab + 272 + 4 * (uhi >> 1));
          const int sl = (int)(int16_t)(bsl >> (16 * (ulo & 1))), sh = (int)(int16_t)(bsh >> (16 * (uhi & 1)));
          const int plo = sdot16(qlo[c], lds16(ab + 16 + 16 * ulo), 0) - 32 * sl;
          const int phi = sdot16(qhi[c], lds16(ab + 16 + 16 * uhi), 0) - 32 * sh;
          const u32 wl = ulo < 4 ? ch.SC[u].x : ulo < 8 ? ch.SC[u].y : ulo < 12 ? ch.SC[u].z : ch.SC[u].w;
          const u32 wh = uhi < 4 ? ch.SC[u].x : uhi < 8 ? ch.SC[u].y : uhi < 12 ? ch.SC[u].z : ch.SC[u].w;
          S += sbfe(wl, 8 * (ulo & 3), 8) * plo + sbfe(wh, 8 * (uhi & 3), 8) * phi;
        }
        o.rec[(mm * o.nblk + b) * 64 + o.r] = d * (float)S;
        if (o.r == 0) o.dav[mm * o.nblk + b] = as_f(lds4(ab));
        if (o.dbg != nullptr && o.n < o.dbg_n) {
          int32_t* p = o.dbg + (((int64_t)mm * o.dbg_n + o.n) * o.nblk + b) * 2;
          p[0] = S;
          p[1] = 0;
        }
      } else if (AF == kActSX) {
        // sub-scaled (kernels_avx2.cpp:1165-1216): S = sum_u sc_u m_(u/2) P_u in 64 bits,
        // the 16-value code sums for the -32 correction from the staged codes
        const uint8_t* ab = st + (mm * o.nblk + b) * kStageSX;
        const v4i mul0 = __builtin_bit_cast(v4i, lds16(ab + 272)), mul1 = __builtin_bit_cast(v4i, lds16(ab + 288));
        const v4u ones = {0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};
        int64_t S = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const int ulo = 8 * (c >> 2) + (c & 3), uhi = ulo + 4;
          const v4u alo = lds16(ab + 16 + 16 * ulo), ahi = lds16(ab + 16 + 16 * uhi);
          const int plo = sdot16(qlo[c], alo, 0) - 32 * sdot16(ones, alo, 0);
          const int phi = sdot16(qhi[c], ahi, 0) - 32 * sdot16(ones, ahi, 0);
          const u32 wl = ulo < 4 ? ch.SC[u].x : ulo < 8 ? ch.SC[u].y : ulo < 12 ? ch.SC[u].z : ch.SC[u].w;
          const u32 wh = uhi < 4 ? ch.SC[u].x : uhi < 8 ? ch.SC[u].y : uhi < 12 ? ch.SC[u].z : ch.SC[u].w;
          const int mlo = (ulo >> 1) < 4 ? mul0[(ulo >> 1) & 3] : mul1[(ulo >> 1) & 3];
          const int mhi = (uhi >> 1) < 4 ? mul0[(uhi >> 1) & 3] : mul1[(uhi >> 1) & 3];
          S += (int64_t)plo * (sbfe(wl, 8 * (ulo & 3), 8) * mlo) + (int64_t)phi * (sbfe(wh, 8 * (uhi & 3), 8) * mhi);
        }
        o.rec[(mm * o.nblk + b) * 64 + o.r] = d * (float)S;
        if (o.r == 0) o.dav[mm * o.nblk + b] = as_f(lds4(ab));
      } else if (AF == kActQ16) {
        // int16 activations (kernels_avx2.cpp:1732-1765): per 16-value unit the exact
        // P = sum (q - 32) a = 256 sum(q hi) + sum(q lo) - 32 sum(a); acc += (float)(sc P) (d da)
#pragma unroll
        for (int uu = 0; uu < 16; ++uu) {
          const int p = uu >> 3, cc = uu & 3, c = 4 * p + cc;  // unit uu lives in chunk c
          const v4u qv = (uu & 4) ? qhi[c] : qlo[c];
          const uint8_t* ab = st + (mm * o.nblk * 8 + b * 8 + uu / 2) * kStage16;
          const int h = uu & 1;
          const int P = sdot16(qv, lds16(ab + 16 + 16 * h), 0) * 256 + (int)udot16(qv, lds16(ab + 48 + 16 * h), 0u) -
                        32 * (int)lds4(ab + 8 + 4 * h);
          const u32 sw = uu < 4 ? ch.SC[u].x : uu < 8 ? ch.SC[u].y : uu < 12 ? ch.SC[u].z : ch.SC[u].w;
          o.acc[mm] = o.acc[mm] + (float)(sbfe(sw, 8 * (uu & 3), 8) * P) * (d * as_f(lds4(ab)));
        }
      } else {
        // per-32 activations, units of 16 in order (kernels_generic.cpp:299-306)
        const v4u ones = {0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};
#pragma unroll
        for (int uu = 0; uu < 16; ++uu) {
          const int p = uu >> 3, cc = uu & 3, c = 4 * p + cc;  // unit uu lives in chunk c
          const v4u qv = (uu & 4) ? qhi[c] : qlo[c];
          const uint8_t* ab = st + (mm * o.nblk * 8 + b * 8 + uu / 2) * kStage32;
          const v4u av = lds16(ab + 16 + 16 * (uu & 1));
          const int P = sdot16(qv, av, 0) - 32 * sdot16(ones, av, 0);
          const u32 sw = uu < 4 ? ch.SC[u].x : uu < 8 ? ch.SC[u].y : uu < 12 ? ch.SC[u].z : ch.SC[u].w;
          o.acc[mm] = o.acc[mm] + ((as_f(lds4(ab)) * d) * (float)sbfe(sw, 8 * (uu & 3), 8)) * (float)P;
        }
      }
    }
  }
}

template <int WT, int AF, int M, int U>
DQ_DEV void compute32(const Chunk32<WT, U>& ch, int bb, const uint8_t* st, Out<M>& o, int nv) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (u >= nv) break;
    const int b = bb + u;
    const float dw = h2f(ch.DW[u]);
    if constexpr (AF == kActF32) {
      float q[32];
      if (WT == kQ8_0) {
        // vec_dot_q8_0 (kernels_generic.cpp:67-76): s = sum q x in index order
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int w = 0; w < 4; ++w)
#pragma unroll
            for (int e = 0; e < 4; ++e) q[16 * c + 4 * w + e] = (float)(int)sbfe(ch.q[u][c][w], 8 * e, 8);
      } else {
        // vec_dot_q4_0 (kernels_generic.cpp:78-90): for j < 16 the low nibble of byte j
        // (value j) and then its high nibble (value j + 16) go into one sum
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          float lo[4], hi[4];
          ubytes_f32(ch.q[u][0][w] & 0x0F0F0F0Fu, lo);
          ubytes_f32((ch.q[u][0][w] >> 4) & 0x0F0F0F0Fu, hi);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            q[2 * (4 * w + e)] = lo[e] - 8.0f;
            q[2 * (4 * w + e) + 1] = hi[e] - 8.0f;
          }
        }
      }
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        const uint8_t* ab = st + (mm * o.nblk + b) * kStageF32;
        float sum = 0.0f;
        if (WT == kQ8_0) {
          sum = dot_f32<32>(0.0f, q, ab);
        } else {
#pragma unroll
          for (int j = 0; j < 16; j += 4) {
            const v4u xl = *reinterpret_cast<const v4u*>(ab + 4 * j), xh = *reinterpret_cast<const v4u*>(ab + 64 + 4 * j);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              sum = sum + q[2 * (j + e)] * as_f(xl[e]);
              sum = sum + q[2 * (j + e) + 1] * as_f(xh[e]);
            }
          }
        }
        o.acc[mm] = o.acc[mm] + dw * sum;
      }
      continue;
    }
#pragma unroll
    for (int mm = 0; mm < M; ++mm) {
      if (AF == kActQ16) {
        const uint8_t* ab = st + (mm * o.nblk + b) * kStage16;
        int P;
        if (WT == kQ8_0) {
          // int16 activations, Q8_0 (kernels_avx2.cpp:1662-1676): the exact
          // P = sum q a = 256 sum(q hi) + sum(q (lo - 128)) + 128 sum(q)
          const v4u q0 = ch.q[u][0], q1 = ch.q[u][Chunk32<WT, U>::kC - 1];
          const v4u ones = {0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};
          const v4u flip = {0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
          const int ph = sdot16(q1, lds16(ab + 32), sdot16(q0, lds16(ab + 16), 0));
          const int pl = sdot16(q1, lds16(ab + 64) ^ flip, sdot16(q0, lds16(ab + 48) ^ flip, 0));
          const int sq = sdot16(q1, ones, sdot16(q0, ones, 0));
          P = ph * 256 + pl + 128 * sq;
        } else {
          // int16 activations, Q4_0 (qmm's dot_row_ref, qmm_reference.cpp:68-93, codes
          // nibble - 8 as qmm_unpack.h:61-75 unpacks them): low nibbles are values 0..15,
          // high nibbles 16..31; the exact P = 256 sum(nib hi) + sum(nib lo) - 8 sum(a)
          // (|sum nib a| <= 15 * 32768 * 32 < 2^31)
          const v4u q0 = ch.q[u][0] & 0x0F0F0F0Fu, q1 = (ch.q[u][0] >> 4) & 0x0F0F0F0Fu;
          const int ph = sdot16(q1, lds16(ab + 32), sdot16(q0, lds16(ab + 16), 0));
          const int pl = (int)udot16(q1, lds16(ab + 64), udot16(q0, lds16(ab + 48), 0u));
          P = ph * 256 + pl - 8 * (int)lds4(ab + 4);
        }
        // acc += (float)P (dw da): the reference's (dw da) P for both formats
        o.acc[mm] = o.acc[mm] + (float)P * (dw * as_f(lds4(ab)));
        continue;
      }
      const uint8_t* ab = st + (mm * o.nblk + b) * kStage32;
      const v4u x0 = lds16(ab + 16), x1 = lds16(ab + 32);
      int P;
      if (WT == kQ8_0) {
        P = sdot16(ch.q[u][Chunk32<WT, U>::kC - 1], x1, sdot16(ch.q[u][0], x0, 0));
      } else {
        // low nibbles are values 0..15, high nibbles 16..31; code = nibble - 8
        P = sdot16((ch.q[u][0] >> 4) & 0x0F0F0F0Fu, x1, sdot16(ch.q[u][0] & 0x0F0F0F0Fu, x0, 0)) -
            8 * (int)lds4(ab + 4);
      }
      // generic order: acc += (dw * da) * (float)P (kernels_generic.cpp:220,235)
      o.acc[mm] = o.acc[mm] + (dw * as_f(lds4(ab))) * (float)P;
    }
  }
}
template <int AF, int M, int U>
DQ_DEV void compute(const Chunk<kQ8_0, U>& ch, int bb, const uint8_t* st, Out<M>& o, int nv = U) {
  compute32<kQ8_0, AF, M, U>(ch, bb, st, o, nv);
}
template <int AF, int M, int U>
DQ_DEV void compute(const Chunk<kQ4_0, U>& ch, int bb, const uint8_t* st, Out<M>& o, int nv = U) {
  compute32<kQ4_0, AF, M, U>(ch, bb, st, o, nv);
}

// ---- staging a wave's slice of activations into LDS. Loads are issued first
// (issue), the weight loads after them, then commit() waits for the activation
// loads only (vector loads complete in order) and writes the staged layout.

// Copies this wave's slice (weight blocks [b0, b1); bpu 32-value activation blocks
// per weight block for per-32 formats) of M pre-quantized rows into the staged
// LDS layout.
template <int AF, int M>
DQ_DEV void stage_acts(const uint8_t* __restrict__ acts, int64_t arb, int nblk, int b0, int b1, int bpu, int r,
                       uint8_t* st) {
  // For each block the loads of all M rows go out together, then the stores:
  // M loads in flight per round trip instead of one.
  const auto ra = rsrc(acts, (u32)(M * arb));
  if constexpr (AF == kActSX) {
    // lane r: codes dword r; lanes 0..4 also u and the m pairs. The block sums s_j
    // come from the codes (8 lanes per 32-value block), m_j from lane 1 + j / 2.
    for (int b = b0; b < b1; ++b) {
      u32 v[M][2];
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        const u32 base = (u32)(mm * arb + (int64_t)b * 320);
        v[mm][0] = ld4(ra, base + 4 * r);
        v[mm][1] = ld4(ra, base + 256 + 4 * (r < 5 ? r : 0));
      }
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        uint8_t* o = st + (mm * nblk + b) * kStageSX;
        const int j = r >> 3;
        const int sj = red8(sdot4(v[mm][0], 0x01010101u, 0));
        const u32 mw = (u32)__shfl((int)v[mm][1], 1 + (j >> 1));
        const int mj = (int)(int16_t)(mw >> (16 * (j & 1)));
        *reinterpret_cast<u32*>(o + 16 + 4 * r) = v[mm][0];
        if (r == 0) *reinterpret_cast<u32*>(o) = v[mm][1];
        if ((r & 7) == 0) {
          *reinterpret_cast<int*>(o + 272 + 4 * j) = mj;
          *reinterpret_cast<int*>(o + 304 + 4 * j) = mj * sj;
          if (j & 1) *reinterpret_cast<int*>(o + 336 + 4 * (j >> 1)) = 128 * sj;
        }
      }
    }
  } else if constexpr (AF == kActQ8_K) {
    for (int b = b0; b < b1; ++b) {
      u32 v[M][2];
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        const u32 base = (u32)(mm * arb + (int64_t)b * 292);
        v[mm][0] = ld4(ra, base + 4 * r);
        v[mm][1] = ld4(ra, r < 9 ? base + 4 * (64 + r) : (u32)(M * arb));
      }
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        uint8_t* o = st + (mm * nblk + b) * kStageQ8K;
        // dword j of the block: 0 -> d @0, 1..64 -> codes @16, 65..72 -> bsums @272
        *reinterpret_cast<u32*>(o + (r == 0 ? 0 : 16 + 4 * (r - 1))) = v[mm][0];
        if (r < 9) *reinterpret_cast<u32*>(o + (r == 0 ? 16 + 4 * 63 : 272 + 4 * (r - 1))) = v[mm][1];
        if (r >= 1 && r < 9) stage_subsum(o, r - 1, bsum_pair(v[mm][1]));
      }
    }
  } else if constexpr (AF == kActF32) {
    // lane r: one 32-value block of fp32 values per round, and their sum in index order
    for (int blk = b0 * bpu + r; blk < b1 * bpu; blk += 64) {
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        const u32 base = (u32)(mm * arb + (int64_t)blk * 128);
        v4u w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = ld16(ra, base + 16 * i);
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) sum = sum + as_f(w[i][e]);
        uint8_t* o = st + (mm * nblk * bpu + blk) * kStageF32;
#pragma unroll
        for (int i = 0; i < 8; ++i) *reinterpret_cast<v4u*>(o + 16 * i) = w[i];
        *reinterpret_cast<v4u*>(o + 128) = v4u{as_u(sum), 0u, 0u, 0u};
      }
    }
  } else if constexpr (AF == kActQ16) {
    // lane r: one 32-value block per round; the int16 codes split into bytes
    for (int blk = b0 * bpu + r; blk < b1 * bpu; blk += 64) {
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        const u32 base = (u32)(mm * arb + (int64_t)blk * 72);
        const v2u ds = ld8(ra, base);
        const v4u w0 = ld16(ra, base + 8), w1 = ld16(ra, base + 24), w2 = ld16(ra, base + 40), w3 = ld16(ra, base + 56);
        const u32 w[16] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w, w2.x, w2.y, w2.z, w2.w, w3.x, w3.y, w3.z, w3.w};
        u32 hi[8], lo[8];
        int a16[2] = {0, 0};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          lo[i] = __builtin_amdgcn_perm(w[2 * i + 1], w[2 * i], 0x06040200u);
          hi[i] = __builtin_amdgcn_perm(w[2 * i + 1], w[2 * i], 0x07050301u);
          a16[i >> 2] = sdot2w(w[2 * i + 1], sdot2w(w[2 * i], a16[i >> 2]));
        }
        uint8_t* o = st + (mm * nblk * bpu + blk) * kStage16;
        *reinterpret_cast<v4u*>(o) = v4u{ds.x, ds.y, (u32)a16[0], (u32)a16[1]};
        *reinterpret_cast<v4u*>(o + 16) = v4u{hi[0], hi[1], hi[2], hi[3]};
        *reinterpret_cast<v4u*>(o + 32) = v4u{hi[4], hi[5], hi[6], hi[7]};
        *reinterpret_cast<v4u*>(o + 48) = v4u{lo[0], lo[1], lo[2], lo[3]};
        *reinterpret_cast<v4u*>(o + 64) = v4u{lo[4], lo[5], lo[6], lo[7]};
      }
    }
  } else {
    constexpr int kG = M < 4 ? M : 4;  // rows per batch of loads
    for (int blk = b0 * bpu + r; blk < b1 * bpu; blk += 64) {
#pragma unroll
      for (int m0 = 0; m0 < M; m0 += kG) {
        u32 w[kG][10];
#pragma unroll
        for (int g = 0; g < kG; ++g) {
          const int mm = m0 + g < M ? m0 + g : M - 1;
          const u32 base = AF == kActPer32 ? (u32)(mm * arb + (int64_t)blk * 40)
                                           : ((u32)(mm * arb + (int64_t)blk * 34) & ~3u);
#pragma unroll
          for (int i = 0; i < 10; ++i) w[g][i] = ld4(ra, base + 4 * i);
        }
#pragma unroll
        for (int g = 0; g < kG; ++g) {
          const int mm = m0 + g;
          if (mm >= M) break;
          uint8_t* o = st + (mm * nblk * bpu + blk) * kStage32;
          if constexpr (AF == kActPer32) {
            *reinterpret_cast<v2u*>(o) = v2u{w[g][0], w[g][1]};
            *reinterpret_cast<v4u*>(o + 16) = v4u{w[g][2], w[g][3], w[g][4], w[g][5]};
            *reinterpret_cast<v4u*>(o + 32) = v4u{w[g][6], w[g][7], w[g][8], w[g][9]};
          } else {  // GGUF Q8_0: fp16 d at 0, codes at 2 (the block is 2-byte aligned)
            const bool sh = (((int64_t)mm * arb + (int64_t)blk * 34) & 3) != 0;
            u32 cw[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) cw[i] = sh ? w[g][i + 1] : __builtin_amdgcn_alignbyte(w[g][i + 1], w[g][i], 2);
            const float d = h2f(sh ? (w[g][0] >> 16) : w[g][0]);
            const v4u ones = {0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};
            const v4u c0 = {cw[0], cw[1], cw[2], cw[3]}, c1 = {cw[4], cw[5], cw[6], cw[7]};
            const int sum = sdot16(ones, c1, sdot16(ones, c0, 0));
            *reinterpret_cast<v2u*>(o) = v2u{as_u(d), (u32)sum};
            *reinterpret_cast<v4u*>(o + 16) = c0;
            *reinterpret_cast<v4u*>(o + 32) = c1;
          }
        }
      }
    }
  }
}

// Activation loads of a wave's slice (one activation row) held in registers
// between issue() and commit(), so they go out before the weight loads: vector
// loads retire in order, so commit() waits for these loads only. Every load is
// issued unconditionally (blocks past the slice read zeros through the buffer
// bound), so no branch separates the loads from their uses and the compiler's
// waits stay exact. Q8_K: at most E super-blocks; 32-value blocks: one per lane.
template <int AF, int E>
struct ActRegs {
  u32 v[AF == kActQ8_K ? 2 * E : 10];
  v2u pd;      // per-32: {d, sum}
  v4u pc[2];   // per-32: the 32 codes
  DQ_DEV void issue(const uint8_t* __restrict__ acts, int64_t arb, int b0, int b1, int bpu, int r) {
    const auto ra = rsrc(acts, (u32)arb);
    if constexpr (AF == kActQ8_K) {
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const bool ok = b0 + i < b1;
        const u32 base = (u32)((int64_t)(b0 + i) * 292);
        v[2 * i] = ld4(ra, ok ? base + 4 * r : (u32)arb);
        v[2 * i + 1] = ld4(ra, ok && r < 9 ? base + 4 * (64 + r) : (u32)arb);
      }
    } else {
      const int nsl = (b1 - b0) * bpu;
      const int blk = b0 * bpu + (r < nsl ? r : 0);
      if constexpr (AF == kActPer32) {
        const u32 base = (u32)((int64_t)blk * 40);
        pd = ld8(ra, base);
        pc[0] = ld16(ra, base + 8);
        pc[1] = ld16(ra, base + 24);
      } else {
        const u32 base = (u32)((int64_t)blk * 34) & ~3u;
#pragma unroll
        for (int i = 0; i < 10; ++i) v[i] = ld4(ra, base + 4 * i);
      }
    }
  }
  // The stores are unconditional: blocks outside the slice go to a per-lane dummy
  // area (kDummyBytes at `dummy`), so the loads above have no conditional use that
  // the compiler could sink them into (below the weight loads).
  DQ_DEV void commit(int64_t arb, int nblk, int b0, int b1, int bpu, int r, uint8_t* st, uint8_t* dummy) {
    if constexpr (AF == kActQ8_K) {
#pragma unroll
      for (int i = 0; i < E; ++i) {
        uint8_t* o = b0 + i < b1 ? st + (b0 + i) * kStageQ8K : dummy;
        // dword j of the block: 0 -> d @0, 1..64 -> codes @16, 65..72 -> bsums @272
        *reinterpret_cast<u32*>(o + (r == 0 ? 0 : 16 + 4 * (r - 1))) = v[2 * i];
        if (r < 9) *reinterpret_cast<u32*>(o + (r == 0 ? 16 + 4 * 63 : 272 + 4 * (r - 1))) = v[2 * i + 1];
        if (r >= 1 && r < 9) stage_subsum(o, r - 1, bsum_pair(v[2 * i + 1]));
      }
    } else {
      const int nsl = (b1 - b0) * bpu;
      const int blk = b0 * bpu + r;
      uint8_t* o = r < nsl ? st + blk * kStage32 : dummy + r * kStage32;
      if constexpr (AF == kActPer32) {
        *reinterpret_cast<v2u*>(o) = pd;
        *reinterpret_cast<v4u*>(o + 16) = pc[0];
        *reinterpret_cast<v4u*>(o + 32) = pc[1];
      } else {  // GGUF Q8_0: fp16 d at byte 0, codes at byte 2 of the 2-byte-aligned block
        const bool sh = (((int64_t)blk * 34) & 3) != 0;  // the block starts at byte 2 of v[0]
        u32 cw[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) cw[i] = sh ? v[i + 1] : __builtin_amdgcn_alignbyte(v[i + 1], v[i], 2);
        const float d = h2f(sh ? (v[0] >> 16) : v[0]);
        const v4u ones = {0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};
        const v4u c0 = {cw[0], cw[1], cw[2], cw[3]}, c1 = {cw[4], cw[5], cw[6], cw[7]};
        const int sum = sdot16(ones, c1, sdot16(ones, c0, 0));
        *reinterpret_cast<v2u*>(o) = v2u{as_u(d), (u32)sum};
        *reinterpret_cast<v4u*>(o + 16) = c0;
        *reinterpret_cast<v4u*>(o + 32) = c1;
      }
    }
  }
};

// Per-lane dummy LDS area of the early-activation path (64 lanes x one 32-value
// stage block; a Q8_K stage block fits too).
constexpr int kDummyBytes = 64 * kStage32;
static_assert(kDummyBytes >= kStageQ8K, "dummy area holds a Q8_K stage block");

// Makes this wave's LDS writes visible to its own later LDS reads (each wave
// stages and reads only its own slice, so no workgroup barrier is needed).
DQ_DEV void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Quantize this wave's blocks [b0, b1) of M fp32 rows into the staged LDS layout
// (the fused decode path), with the standalone quantizers' device functions. bpu:
// 32-value activation blocks per weight block (8 for K-quant weights with per-32
// activations, else 1).
template <int AF, int M>
DQ_DEV void quantize_slice(const float* __restrict__ x, int64_t xs, int nblk, int b0, int b1, int bpu, int r,
                           uint8_t* st) {
  // For each block the fp32 loads of all M rows go out together, then the M
  // quantizations: M loads in flight per round trip instead of one.
  constexpr bool kSb = AF == kActQ8_K;
  const int64_t kk = (int64_t)nblk * (kSb ? 256 : 32 * bpu);
  if constexpr (kSb) {
    for (int b = b0; b < b1; ++b) {
      float v[M][4];
#pragma unroll
      for (int mm = 0; mm < M; ++mm) load4f(rsrc(x + mm * xs, (u32)(kk * 4)), (u32)((b * 256 + 4 * r) * 4), v[mm]);
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        float d;
        int bsum;
        const u32 packed = q8k_quant(v[mm], d, bsum);
        const int s32 = bsum + dpp<kHalfMirror>(bsum);  // the other 4-lane group of the 32-value sub-block
        uint8_t* o = st + (mm * nblk + b) * kStageQ8K;
        *reinterpret_cast<u32*>(o + 16 + 4 * r) = packed;
        if ((r & 3) == 0) *reinterpret_cast<int16_t*>(o + 272 + 2 * (r >> 2)) = (int16_t)bsum;
        if ((r & 7) == 0) stage_subsum(o, r >> 3, s32);
        if (r == 0) *reinterpret_cast<float*>(o) = d;
      }
    }
  } else {
    const int e0 = b0 * bpu, e1 = b1 * bpu;  // this slice's 32-value blocks
    for (int bb = e0; bb < e1; bb += 8) {
      const int blk = bb + (r >> 3);
      float v[M][4];
#pragma unroll
      for (int mm = 0; mm < M; ++mm) load4f(rsrc(x + mm * xs, (u32)(kk * 4)), (u32)((blk * 32 + 4 * (r & 7)) * 4), v[mm]);
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        float d;
        int sum;
        const u32 packed = per32_quant(v[mm], d, sum);
        if (blk < e1) {
          uint8_t* o = st + (mm * nblk * bpu + blk) * kStage32;
          *reinterpret_cast<u32*>(o + 16 + 4 * (r & 7)) = packed;
          if ((r & 7) == 0) {
            *reinterpret_cast<float*>(o) = d;
            *reinterpret_cast<int32_t*>(o + 4) = sum;
          }
        }
      }
    }
  }
}

// kFuse: the activations arrive as fp32 rows (x, row stride xs floats) and each
// wave quantizes its own slice into LDS with the standalone quantizers' device
// functions (q8k_quant / per32_quant), so the codes are the same bytes.
// kEarly (one activation row only): 0 = activations staged by loops after the
// first weight loads; E > 0 = each wave holds at most E Q8_K super-blocks (or, for
// 32-value formats, at most 64 blocks) and loads them ahead of the weights.
// kGated (K-quants, one fused row): q0..q3 are a second weight of the same type and
// shape (the up projection); waves W/2.. run it over the same row group with their
// own LDS regions, and y = act(x . gate) * (x . up) (dynacore's Device::matmul_gated,
// dynacore/include/dynacore/device/device.h:188-199).
template <int WT, int AF, int M, int W, int U, bool kFuse, int kEarly, bool kGated = false, bool kSplit = false>
__global__ __launch_bounds__(W * 64) void k_gemv(const uint8_t* __restrict__ p0, const uint8_t* __restrict__ p1,
                                                 const uint8_t* __restrict__ p2, const uint8_t* __restrict__ p3,
                                                 int nblk, int64_t g0, int64_t n0, int64_t n1,
                                                 const uint8_t* __restrict__ acts, int64_t arb,
                                                 const float* __restrict__ x, int64_t xs,
                                                 float* __restrict__ y, int64_t ys, const float* __restrict__ bias,
                                                 int32_t* __restrict__ dbg, int64_t dbg_n,
                                                 const uint8_t* __restrict__ q0, const uint8_t* __restrict__ q1,
                                                 const uint8_t* __restrict__ q2, const uint8_t* __restrict__ q3,
                                                 int act, int splits, float* __restrict__ part) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr bool kSb = AF == kActQ8_K || AF == kActSX;
  static_assert(!kGated || (kSb && M == 1 && kFuse), "the gated GEMV takes one fp32 row and K-quant weights");
  static_assert((AF != kActSX && AF != kActQ16 && AF != kActF32) || (!kFuse && kEarly == 0),
                "sub-scaled, int16 and fp32 activations arrive ready and are staged by loops");
  // LDS: Q8_K t-terms [M][nblk][64] + da [M][nblk]  |  per-32 slice sums [W][M][64];
  // then the staged activation rows [M][nblk (blocks of 32 for per-32)][stage bytes].
  // kGated: one t-term region and one stage region per weight.
  constexpr int WH = kGated ? W / 2 : W;  // waves per weight
  const int r = threadIdx.x & 63, wave = wave_id();
  const int half = kGated && wave >= WH ? 1 : 0;
  const int wl = wave - half * WH;
  // split-K (splits > 1): workgroup L takes K-range L % splits of row group L / splits
  const int sk = kSplit ? (int)(blockIdx.x % (unsigned)splits) : 0;
  const int64_t G = g0 + (kSplit ? (int64_t)(blockIdx.x / (unsigned)splits) : (int64_t)blockIdx.x);
  const size_t region = kSb ? ((size_t)M * nblk * 65 * 4 + 15) / 16 * 16 : (size_t)W * M * 64 * 4;
  Out<M> o;
  o.rec = reinterpret_cast<float*>(smem + half * region);
  o.dav = o.rec + M * nblk * 64;
  o.dbg = dbg;
  o.dbg_n = dbg_n;
  o.n = G * kRowGroup + r;
  o.nblk = nblk;
  o.r = r;
#pragma unroll
  for (int mm = 0; mm < M; ++mm) o.acc[mm] = o.cor[mm] = 0.0f;
  const int kb0 = kSplit ? sk * nblk / splits : 0, kb1 = kSplit ? (sk + 1) * nblk / splits : nblk;  // this workgroup's blocks
  const int b0 = kb0 + wl * (kb1 - kb0) / WH, b1 = kb0 + (wl + 1) * (kb1 - kb0) / WH;  // this wave's
  // bytes of the staged activation rows (the dummy area of the early path follows)
  const int stage_bytes =
      kSb ? M * nblk * stage_sb(AF) : M * nblk * ((WT == kQ4_K || WT == kQ6_K) ? 8 : 1) * stage_b32(AF);
  uint8_t* st = smem + (kGated ? 2 : 1) * region + half * stage_bytes;

  // plane buffer resources of this row group (64 rows x nblk blocks)
  const int u0 = plane_unit(WT, 0), u1 = plane_unit(WT, 1);
  const uint8_t* w0 = half ? q0 : p0;
  const uint8_t* w1 = half ? q1 : p1;
  Rsrcs rs;
  rs.r0 = rsrc(w0 + G * nblk * 64 * u0, (u32)(nblk * 64 * u0));
  rs.r1 = rsrc(w1 + G * nblk * 64 * u1, (u32)(nblk * 64 * u1));
  rs.r2 = rs.r0;
  rs.r3 = rs.r0;
  if (WT == kQ6_K) {
    const uint8_t* w2 = half ? q2 : p2;
    const uint8_t* w3 = half ? q3 : p3;
    rs.r2 = rsrc(w2 + G * nblk * 64 * 16, (u32)(nblk * 64 * 16));
    rs.r3 = rsrc(w3 + G * nblk * 64 * 2, (u32)(nblk * 64 * 2));
  }

  // Activations of this slice first, so their latency hides behind the weight
  // loads issued next (each wave stages only its own slice). With kEarly the
  // activation loads and the first weight chunk are issued unconditionally, in
  // straight-line code, so the waits before their uses count exactly these loads.
  const int bpu = (WT == kQ4_K || WT == kQ6_K) && !kSb ? 8 : 1;
  constexpr int kE = kEarly > 0 ? kEarly : 1;
  float xv[kE][4];
  ActRegs<AF, kE> ar;
  if constexpr (kEarly > 0) {
    if constexpr (kFuse) {  // Q8_K, one row: the fp32 values of this wave's super-blocks
      const auto rx = rsrc(x, (u32)(nblk * 256 * 4));
#pragma unroll
      for (int i = 0; i < kE; ++i) load4f(rx, (u32)(((b0 + i) * 256 + 4 * r) * 4), xv[i]);
    } else {
      ar.issue(acts, arb, b0, b1, bpu, r);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weight loads
  Chunk<WT, U> c0;
  c0.load(rs, b0, b1, nblk, r);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (kEarly > 0) {
    if constexpr (kFuse) {
      // quantized unconditionally (so the loads above stay ahead of the weight
      // loads); only a super-block of this slice is stored
#pragma unroll
      for (int i = 0; i < kE; ++i) {
        float d;
        int bsum;
        const u32 packed = q8k_quant(xv[i], d, bsum);
        const int s32 = bsum + dpp<kHalfMirror>(bsum);  // the other 4-lane group of the sub-block
        if (b0 + i < b1) {
          uint8_t* ob = st + (b0 + i) * kStageQ8K;
          *reinterpret_cast<u32*>(ob + 16 + 4 * r) = packed;
          if ((r & 3) == 0) *reinterpret_cast<int16_t*>(ob + 272 + 2 * (r >> 2)) = (int16_t)bsum;
          if ((r & 7) == 0) stage_subsum(ob, r >> 3, s32);
          if (r == 0) *reinterpret_cast<float*>(ob) = d;
        }
      }
    } else {
      ar.commit(arb, nblk, b0, b1, bpu, r, st, st + stage_bytes);
    }
  } else if constexpr (kFuse) {
    quantize_slice<AF, M>(x, xs, nblk, b0, b1, bpu, r, st);
  } else {
    stage_acts<AF, M>(acts, arb, nblk, b0, b1, bpu, r, st);
  }
  wave_lds_sync();

  // the first chunk holds blocks [b0, b0 + U); those at or past b1 read as zeros
  const int nv0 = b1 - b0 < U ? b1 - b0 : U;
  if (nv0 > 0) compute<AF, M, U>(c0, b0, st, o, nv0);
  int bb = b0 + U;
  for (; bb + U <= b1; bb += U) {
    Chunk<WT, U> c;
    c.load(rs, bb, b1, nblk, r);
    compute<AF, M, U>(c, bb, st, o);
  }
  for (; bb < b1; ++bb) {
    Chunk<WT, 1> c;
    c.load(rs, bb, b1, nblk, r);
    compute<AF, M, 1>(c, bb, st, o);
  }

  if (!kSb) {
#pragma unroll
    for (int mm = 0; mm < M; ++mm) o.rec[(wave * M + mm) * 64 + r] = AF == kActQ16 ? o.acc[mm] - o.cor[mm] : o.acc[mm];
  }
  __syncthreads();
  if constexpr (kSplit) {
    static_assert(!kGated && !kSb, "split launches: per-32 style formats");
    // Publish this workgroup's row sums (its slices added in wave order) in
    // [G][splits][M][64]; k_split_finish adds the splits in order.
    if (wave == 0) {
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) v = v + o.rec[(w * M + mm) * 64 + r];
        part[((G * splits + sk) * M + mm) * 64 + r] = v;
      }
    }
    return;
  }
  if (wave != 0) return;
  const int64_t n = o.n;
  // the canonical chain acc = fma(da_b, t_b, acc) over a t-term region
  auto chain = [&](const float* rec, int mm) {
    const float* tp = rec + mm * nblk * 64 + r;
    const float* dp = rec + M * nblk * 64 + mm * nblk;
    float v = 0.0f;
    int b = 0;
    if (nblk <= 16) {
      // short rows (K <= 4096): every read first, then the sixteen dependent FMAs
      // (indices past the row repeat its last block and are not used)
      float t[16], dv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int bc = i < nblk ? i : nblk - 1;
        t[i] = tp[bc * 64];
        dv[i] = dp[bc];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (i < nblk) v = fmaf(dv[i], t[i], v);
      }
      return v;
    }
    for (; b + 4 <= nblk; b += 4) {
      const float t0 = tp[b * 64], t1 = tp[(b + 1) * 64], t2 = tp[(b + 2) * 64], t3 = tp[(b + 3) * 64];
      const float d0 = dp[b], d1 = dp[b + 1], d2 = dp[b + 2], d3 = dp[b + 3];
      v = fmaf(d0, t0, v);
      v = fmaf(d1, t1, v);
      v = fmaf(d2, t2, v);
      v = fmaf(d3, t3, v);
    }
    for (; b < nblk; ++b) v = fmaf(dp[b], tp[b * 64], v);
    return v;
  };
#pragma unroll
  for (int mm = 0; mm < M; ++mm) {
    float v = 0.0f;
    if (kSb) {
      v = chain(o.rec, mm);
    } else {
#pragma unroll
      for (int w = 0; w < W; ++w) v = v + o.rec[(w * M + mm) * 64 + r];
    }
    if constexpr (kGated) {
      const float vu = chain(reinterpret_cast<const float*>(smem + region), mm);
      if (n >= n0 && n < n1) y[mm * ys + n] = act_apply(act, v) * vu;
    } else {
      if (n >= n0 && n < n1) y[mm * ys + n] = bias ? v + bias[n] : v;
    }
  }
}

// ---- the one-row Q4_K x Q8_K decode on every CU. k_gemv runs one workgroup per
// 64-row group, so a weight of fewer groups than CUs (config 3: 224 groups on 256
// CUs) leaves CUs idle, and with them their share of the loads in flight.
// k_gemv_slab runs workgroups of kSlabRows = 56 rows over the whole row, one wave per
// super-block (K = 256 NB): lane l < 56 holds row 56 g + l of workgroup g, so each
// vector load of a wave is one contiguous run of 896 bytes (two runs where the rows
// cross a 64-row group); lanes 56..63 read nothing (past the buffer bound) and
// store nothing. Each wave stages only its own super-block, as k_gemv's waves do.
// The compute step is k_gemv's (the same t-term per row and super-block) and the
// chain over the super-blocks runs in the same order, so the outputs are bit-equal
// to k_gemv's.
constexpr int kSlabRows = 56;

template <int NB, int AF, bool kFuse>
__global__ __launch_bounds__(NB * 64) void k_gemv_slab(const uint8_t* __restrict__ p0, const uint8_t* __restrict__ p1,
                                                       int64_t groups, int64_t n0, int64_t n1,
                                                       const uint8_t* __restrict__ acts, const float* __restrict__ x,
                                                       float* __restrict__ y, const float* __restrict__ bias,
                                                       int32_t* __restrict__ dbg, int64_t dbg_n) {
  static_assert(AF == kActQ8_K || (AF == kActPer32 && kFuse), "Q8_K rows, or fp32 rows quantized to per-32 here");
  constexpr bool kSb = AF == kActQ8_K;
  constexpr int kStage = kSb ? NB * kStageQ8K + kDummyBytes : NB * 8 * kStage32;
  __shared__ __align__(16) uint8_t st[kStage];
  __shared__ __align__(16) float rec[NB * 64 + NB];  // t-terms (per-32: sums) [b][row], then da [b]
  const int l = threadIdx.x & 63, b = wave_id();
  const int64_t g0 = n0 / kRowGroup;
  const bool live = l < kSlabRows;
  const int64_t n = g0 * kRowGroup + (int64_t)blockIdx.x * kSlabRows + (live ? l : 0);
  const int r = (int)(n % kRowGroup);
  // the planes from row group g0 on; rows past the last group read zeros, and so do
  // lanes 56..63 (block index past the resources)
  Rsrcs rs;
  rs.r0 = rsrc(p0 + g0 * NB * 64 * 128, (u32)((groups - g0) * NB * 64 * 128));
  rs.r1 = rsrc(p1 + g0 * NB * 64 * 16, (u32)((groups - g0) * NB * 64 * 16));
  rs.r2 = rs.r0;
  rs.r3 = rs.r0;
  const int bi = live ? (int)((n / kRowGroup - g0) * NB + b) : (int)((groups - g0) * NB);

  // activation loads first, then the weight loads (k_gemv's early path)
  float xv[4];
  ActRegs<kActQ8_K, 1> ar;
  if constexpr (kFuse) {
    load4f(rsrc(x, (u32)(NB * 256 * 4)), (u32)((b * 256 + 4 * l) * 4), xv);
  } else {
    ar.issue(acts, (int64_t)NB * 292, b, b + 1, 1, l);
  }
  __builtin_amdgcn_sched_barrier(0);
  Chunk<kQ4_K, 1> c;
  c.load(rs, bi, bi + 1, bi + 1, r);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!kSb) {
    // per-32: lanes 8 j .. 8 j + 7 hold the super-block's 32-value block j (values 4 l ..)
    float d;
    int sum;
    const u32 packed = per32_quant(xv, d, sum);
    uint8_t* ob = st + (8 * b + (l >> 3)) * kStage32;
    *reinterpret_cast<u32*>(ob + 16 + 4 * (l & 7)) = packed;
    if ((l & 7) == 0) {
      *reinterpret_cast<float*>(ob) = d;
      *reinterpret_cast<int32_t*>(ob + 4) = sum;
    }
  } else if constexpr (kFuse) {
    uint8_t* ob = st + b * kStageQ8K;
    float d;
    int bsum;
    const u32 packed = q8k_quant(xv, d, bsum);
    const int s32 = bsum + dpp<kHalfMirror>(bsum);
    *reinterpret_cast<u32*>(ob + 16 + 4 * l) = packed;
    if ((l & 3) == 0) *reinterpret_cast<int16_t*>(ob + 272 + 2 * (l >> 2)) = (int16_t)bsum;
    if ((l & 7) == 0) stage_subsum(ob, l >> 3, s32);
    if (l == 0) *reinterpret_cast<float*>(ob) = d;
  } else {
    ar.commit((int64_t)NB * 292, NB, b, b + 1, 1, l, st, st + NB * kStageQ8K);
  }
  wave_lds_sync();

  Out<1> o;
  o.rec = rec;
  o.dav = rec + NB * 64;
  o.dbg = dbg;
  o.dbg_n = dbg_n;
  o.n = live ? n : dbg_n;  // lanes 56..63 write no partials
  o.nblk = NB;
  o.r = l;
  o.acc[0] = o.cor[0] = 0.0f;
  compute<AF, 1, 1>(c, b, st, o);
  if (!kSb) rec[b * 64 + l] = o.acc[0];  // the super-block's sum, in sub-block order
  __syncthreads();
  if (b != 0 || !live) return;
  float v = 0.0f;
  if constexpr (kSb) {
    // k_gemv's chain: acc = fma(da_b, t_b, acc), b in order
    float t[NB], dv[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      t[i] = rec[i * 64 + l];
      dv[i] = rec[NB * 64 + i];
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) v = fmaf(dv[i], t[i], v);
  } else {
    // k_gemv's per-32 sum over its one-super-block waves, in wave order
#pragma unroll
    for (int i = 0; i < NB; ++i) v = v + rec[i * 64 + l];
  }
  if (n >= n0 && n < n1) y[n] = bias ? v + bias[n] : v;
}

// Completes split-K rows (one 64-lane workgroup per row group, lane r = row): the
// sum of the splits' row sums in split order, plus the bias.
template <int M>
__global__ __launch_bounds__(64) void k_split_finish(const float* __restrict__ part, int splits, int64_t g0, int64_t n0,
                                                     int64_t n1, float* __restrict__ y, int64_t ys,
                                                     const float* __restrict__ bias) {
  const int r = threadIdx.x;
  const int64_t G = g0 + blockIdx.x, n = G * kRowGroup + r;
#pragma unroll
  for (int mm = 0; mm < M; ++mm) {
    float v = 0.0f;
    for (int q = 0; q < splits; ++q) v = v + part[((G * splits + q) * M + mm) * 64 + r];
    if (n >= n0 && n < n1) y[mm * ys + n] = bias ? v + bias[n] : v;
  }
}

// ================================================================ launchers

// LDS of one GEMV workgroup: Q8_K t-terms [M][nblk][64] + da [M][nblk], or the
// per-32 slice sums [W][M][64]; the staged activation rows (Q8_K super-blocks of
// kStageQ8K B, 32-value blocks of kStage32 B); the dummy area of the early path.
constexpr size_t kGemvMaxLds = 160 * 1024;
static size_t gemv_lds_bytes(int wt, int af, int m, int waves, int64_t nblk, bool early) {
  const bool sb = af == kActQ8_K || af == kActSX;
  size_t lds = sb ? ((size_t)m * nblk * 65 * sizeof(float) + 15) / 16 * 16 : (size_t)waves * m * 64 * sizeof(float);
  lds += sb ? (size_t)m * nblk * stage_sb(af)
                        : (size_t)m * nblk * (wt == kQ4_K || wt == kQ6_K ? 8 : 1) * stage_b32(af);
  if (early) lds += kDummyBytes;
  return lds;
}

// Waves per workgroup. A workgroup holds one 64-row group; its waves split the
// row's blocks. When all row groups fit on the GPU at once (one workgroup per
// CU), 16 waves give each wave less work after its data lands, which shortens
// the tail; with more row groups than CUs, 8-wave workgroups (two per CU) do
// better. 16 waves leave 128 VGPRs per lane: K-quant passes of more than one
// activation row need more and keep 8 waves.
// K-ranges per row of a GEMV launch of weight w under activation format af (1: no
// split). Fewer row groups than half the CUs (e.g. N = 4096: 64 groups): each row's
// blocks split into up to 8 K-ranges over 8-wave workgroups (at least 8 blocks per
// range), so the launch covers the CUs, and a second launch finishes the rows. Only
// the formats whose rows are sums of per-slice sums (per-32 blocks: int8, int16,
// fp32) split; the Q8_K and sub-scaled super-block formats keep their in-order chain.
// The int8 per-32 formats split only long rows (K >= 8192). Measured (dq_matmul,
// N = 4096): fp32 Q6_K K=14336 75 -> 21 us; Q8_0 K=14336 M=1 / 4 22.5 -> 15.1 /
// 30.7 -> 23.7 us; at K = 4096 the int8 formats were slower split (Q8_0 M=4 10.8 ->
// 14.3 us, Q4_0 M=1 5.6 -> 6.9 us). The count depends on the weight and the device
// only, so every row-range call of one weight partitions K alike.
int gemv_splits(const WeightDev& w, int af) {
  if (af == kActQ8_K || af == kActSX) return 1;
  const bool int8 = af == kActPer32 || af == kActQ8_0;
  const int64_t groups = w.n_pad / kRowGroup;
  const int cus = w.cus > 0 ? w.cus : 256;
  int splits = 1;
  if (groups * 2 <= cus && (!int8 || w.k >= 8192)) {
    splits = (int)(cus / groups);
    if (splits > 8) splits = 8;
    while (splits > 1 && w.nblk / splits < 8) --splits;
  }
  return splits;
}

size_t gemv_split_bytes(const WeightDev& w, int af, int64_t m_pass) {
  const int splits = gemv_splits(w, af);
  return splits > 1 ? (size_t)(w.n_pad / kRowGroup) * splits * (size_t)m_pass * 64 * 4 : 0;
}

// Split-K state of one launch: the number of K-ranges per row group and the
// per-device buffer of their row sums (splits == 1: none).
struct Split {
  int splits = 1;
  float* part = nullptr;
};

// Per-device split-K part buffers, grown on demand. Split launches that overlap on
// one device from different streams race on it, as the library's other per-device
// scratch does.
struct SplitBufs {
  float* part = nullptr;
  size_t bytes = 0;
};
static std::mutex g_split_mu;
static SplitBufs g_split[64];

static hipError_t split_bufs(int device, size_t bytes, Split& sp) {
  std::lock_guard<std::mutex> lock(g_split_mu);
  SplitBufs& b = g_split[device < 64 ? device : 63];
  if (b.bytes < bytes) {
    DeviceScope ds(device);
    if (ds.err != hipSuccess) return ds.err;
    hipError_t e = hipDeviceSynchronize();  // launches on any stream may still use the old buffer
    if (e != hipSuccess) return e;
    if (b.part != nullptr && (e = hipFree(b.part)) != hipSuccess) return e;
    b.part = nullptr;
    b.bytes = 0;
    const size_t sz = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
    if ((e = hipMalloc(reinterpret_cast<void**>(&b.part), sz)) != hipSuccess) return e;
    b.bytes = sz;
  }
  sp.part = b.part;
  return hipSuccess;
}

template <int WT, int AF, int M, bool kFuse, int W, int kEarly, bool kSplit>
static hipError_t gemv_launch(const WeightDev& w, const uint8_t* acts, int64_t arb, const float* x, int64_t xs,
                              int64_t n0, int64_t n1, float* y, int64_t ys, const float* bias, int32_t* dbg,
                              const Split& sp, hipStream_t s) {
  // blocks per chunk of vector loads: two super-blocks (or 8 32-value blocks) per
  // wave step, one (or 4) when waves hold fewer blocks
  constexpr int U = (WT == kQ8_0 || WT == kQ4_0) ? (W >= 16 ? 4 : 8) : (W >= 16 ? 1 : 2);
  const int64_t g0 = n0 / kRowGroup, g1 = (n1 + kRowGroup - 1) / kRowGroup;
  const size_t lds = gemv_lds_bytes(WT, AF, M, W, w.nblk, kEarly > 0);
  if (lds > kGemvMaxLds) return hipErrorInvalidValue;
  const void* fn = reinterpret_cast<const void*>(&k_gemv<WT, AF, M, W, U, kFuse, kEarly, false, kSplit>);
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((k_gemv<WT, AF, M, W, U, kFuse, kEarly, false, kSplit>), dim3((unsigned)((g1 - g0) * sp.splits)),
                     dim3(64 * W),
                     lds, s, w.plane[0], w.plane[1], w.plane[2], w.plane[3], (int)w.nblk, g0, n0, n1, acts, arb, x, xs,
                     y, ys, bias, dbg, w.n, nullptr, nullptr, nullptr, nullptr, 0, sp.splits, sp.part);
  if (kSplit) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_split_finish<M>), dim3((unsigned)(g1 - g0)), dim3(64), 0, s, sp.part, sp.splits, g0, n0, n1, y,
                       ys, bias);
  }
  return hipGetLastError();
}

// The early-activation variant for W waves: Q8_K rows hold at most 4 super-blocks
// per wave (fused or not); 32-value formats at most 64 blocks per wave (not fused).
template <int WT, int AF, int M, bool kFuse, int W, bool kSplit>
static hipError_t gemv_early(const WeightDev& w, const uint8_t* acts, int64_t arb, const float* x, int64_t xs,
                             int64_t n0, int64_t n1, float* y, int64_t ys, const float* bias, int32_t* dbg,
                             const Split& sp, hipStream_t s) {
  const int64_t per_split = (w.nblk + sp.splits - 1) / sp.splits;
  const int64_t per_wave = (per_split + W - 1) / W;  // blocks of the largest slice
  if constexpr (M == 1 && AF == kActQ8_K) {
    if (per_wave == 1) {
      return gemv_launch<WT, AF, M, kFuse, W, 1, kSplit>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, sp, s);
    }
    if (per_wave == 2) {
      return gemv_launch<WT, AF, M, kFuse, W, 2, kSplit>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, sp, s);
    }
    if (per_wave <= 4) {  // long rows on few row groups (an FFN down projection, K = 14336)
      return gemv_launch<WT, AF, M, kFuse, W, 4, kSplit>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, sp, s);
    }
  } else if constexpr (M == 1 && !kFuse && AF != kActSX && AF != kActQ16 && AF != kActF32) {
    const int64_t bpu = WT == kQ4_K || WT == kQ6_K ? 8 : 1;
    if (per_wave * bpu <= 64) {
      return gemv_launch<WT, AF, M, kFuse, W, 1, kSplit>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, sp, s);
    }
  }
  return gemv_launch<WT, AF, M, kFuse, W, 0, kSplit>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, sp, s);
}

template <int AF, bool kFuse>
static hipError_t gemv_slab(const WeightDev& w, const uint8_t* acts, const float* x, int64_t n0, int64_t n1, float* y,
                            const float* bias, int32_t* dbg, hipStream_t s) {
  const int64_t g0 = n0 / kRowGroup, g1 = (n1 + kRowGroup - 1) / kRowGroup;
  const unsigned grid = (unsigned)(((g1 - g0) * kRowGroup + kSlabRows - 1) / kSlabRows);
  const int64_t groups = w.n_pad / kRowGroup;
  if (w.nblk == 16) {
    hipLaunchKernelGGL((k_gemv_slab<16, AF, kFuse>), dim3(grid), dim3(16 * 64), 0, s, w.plane[0], w.plane[1], groups,
                       n0, n1, acts, x, y, bias, dbg, w.n);
  } else {
    hipLaunchKernelGGL((k_gemv_slab<8, AF, kFuse>), dim3(grid), dim3(8 * 64), 0, s, w.plane[0], w.plane[1], groups, n0,
                       n1, acts, x, y, bias, dbg, w.n);
  }
  return hipGetLastError();
}

template <int WT, int AF, int M, bool kFuse>
static hipError_t gemv_waves(const WeightDev& w, const uint8_t* acts, int64_t arb, const float* x, int64_t xs,
                             int64_t n0, int64_t n1, float* y, int64_t ys, const float* bias, int32_t* dbg,
                             const Workspace* ws, hipStream_t s) {
  constexpr bool kWide = M == 1 || WT == kQ8_0 || WT == kQ4_0;
  // The launch shape (waves per workgroup, K-ranges per row) comes from the weight's
  // row groups, not from [n0, n1): a row's slices, and so its fp32 sum order, do not
  // depend on how the caller partitions the rows (qmm.h:35-36).
  const int64_t groups = w.n_pad / kRowGroup;
  if constexpr (WT == kQ4_K && M == 1 && (AF == kActQ8_K || (AF == kActPer32 && kFuse))) {
    // fewer row groups than CUs: 56-row workgroups spread the row over more CUs
    if ((w.nblk == 8 || w.nblk == 16) && groups * kRowGroup <= (int64_t)kSlabRows * w.cus &&
        (AF == kActQ8_K || gemv_splits(w, AF) == 1)) {
      return gemv_slab<AF, kFuse>(w, acts, x, n0, n1, y, bias, dbg, s);
    }
  }
  const int splits = gemv_splits(w, AF);
  if constexpr (AF != kActQ8_K && AF != kActSX) {
    if (splits > 1) {
      const size_t part = (size_t)groups * splits * M * 64 * 4;
      Split sp;
      sp.splits = splits;
      if (ws != nullptr && ws->p != nullptr) {
        // the caller's region (no allocation on this path)
        if (ws->bytes < part) return hipErrorInvalidValue;
        sp.part = reinterpret_cast<float*>(ws->p);
      } else {
        const hipError_t e = split_bufs(w.device, part, sp);
        if (e != hipSuccess) return e;
      }
      return gemv_early<WT, AF, M, kFuse, 8, true>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, sp, s);
    }
  }
  const Split none;
  if (kWide && groups <= w.cus) {
    return gemv_early<WT, AF, M, kFuse, kWide ? 16 : 8, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, none, s);
  }
  return gemv_early<WT, AF, M, kFuse, 8, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, none, s);
}

// M rows (1..4 or 8) of one pass; x != nullptr: fused quantization of fp32 rows.
template <int M>
static hipError_t gemv_pass(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, const float* x, int64_t xs,
                            int64_t n0, int64_t n1, float* y, int64_t ys, const float* bias, int32_t* dbg,
                            const Workspace* ws, hipStream_t s) {
  if (x != nullptr) {
    switch (w.dtype) {
      case kQ4_K:
        if (af == kActPer32) return gemv_waves<kQ4_K, kActPer32, M, true>(w, nullptr, 0, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
        return gemv_waves<kQ4_K, kActQ8_K, M, true>(w, nullptr, 0, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
      case kQ6_K:
        if (af == kActPer32) return gemv_waves<kQ6_K, kActPer32, M, true>(w, nullptr, 0, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
        return gemv_waves<kQ6_K, kActQ8_K, M, true>(w, nullptr, 0, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
      case kQ8_0: return gemv_waves<kQ8_0, kActPer32, M, true>(w, nullptr, 0, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
      default: return gemv_waves<kQ4_0, kActPer32, M, true>(w, nullptr, 0, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
    }
  }
  switch (w.dtype) {
    case kQ4_K:
      if (af == kActSX) return gemv_waves<kQ4_K, kActSX, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
      if (af == kActQ16) return gemv_waves<kQ4_K, kActQ16, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
      if (af == kActF32) return gemv_waves<kQ4_K, kActF32, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
      return af == kActQ8_K ? gemv_waves<kQ4_K, kActQ8_K, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s)
                            : gemv_waves<kQ4_K, kActPer32, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
    case kQ6_K:
      if (af == kActSX) return gemv_waves<kQ6_K, kActSX, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
      if (af == kActQ16) return gemv_waves<kQ6_K, kActQ16, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
      if (af == kActF32) return gemv_waves<kQ6_K, kActF32, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
      return af == kActQ8_K ? gemv_waves<kQ6_K, kActQ8_K, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s)
                            : gemv_waves<kQ6_K, kActPer32, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
    case kQ8_0:
      if (af == kActQ16) return gemv_waves<kQ8_0, kActQ16, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
      if (af == kActF32) return gemv_waves<kQ8_0, kActF32, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
      return af == kActPer32 ? gemv_waves<kQ8_0, kActPer32, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s)
                             : gemv_waves<kQ8_0, kActQ8_0, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
    default:
      if (af == kActQ16) return gemv_waves<kQ4_0, kActQ16, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
      if (af == kActF32) return gemv_waves<kQ4_0, kActF32, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
      return af == kActPer32 ? gemv_waves<kQ4_0, kActPer32, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s)
                             : gemv_waves<kQ4_0, kActQ8_0, M, false>(w, acts, arb, x, xs, n0, n1, y, ys, bias, dbg, ws, s);
  }
}

// Passes of up to 8 activation rows (each pass streams the weights once); 8-row
// passes when their LDS fits, else 4.
static hipError_t gemv_rows(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, const float* x, int64_t xs,
                            int64_t m, int64_t n0, int64_t n1, float* y, int64_t ys, const float* bias, int32_t* dbg,
                            const Workspace* ws, hipStream_t s) {
  const int paf = x != nullptr && af < 0 ? (w.dtype == kQ4_K || w.dtype == kQ6_K ? kActQ8_K : kActPer32) : af;
  // rows per pass: 8, 4, 2 or 1, the most whose staged activations fit the LDS
  int pmax = 8;
  while (pmax > 1 && gemv_lds_bytes(w.dtype, paf, pmax, 16, w.nblk, false) > kGemvMaxLds) pmax /= 2;
  for (int64_t r0 = 0; r0 < m;) {
    const int64_t left = m - r0;
    const int cap = pmax < 4 ? pmax : 4;
    const int rows = left >= 8 && pmax >= 8 ? 8 : (int)(left < cap ? left : cap);
    const uint8_t* a = acts ? acts + r0 * arb : nullptr;
    const float* xx = x ? x + r0 * xs : nullptr;
    float* yy = y + r0 * ys;
    int32_t* dd = dbg ? dbg + r0 * w.n * w.nblk * 2 : nullptr;
    hipError_t e;
    switch (rows) {
      case 1: e = gemv_pass<1>(w, af, a, arb, xx, xs, n0, n1, yy, ys, bias, dd, ws, s); break;
      case 2: e = gemv_pass<2>(w, af, a, arb, xx, xs, n0, n1, yy, ys, bias, dd, ws, s); break;
      case 3: e = gemv_pass<3>(w, af, a, arb, xx, xs, n0, n1, yy, ys, bias, dd, ws, s); break;
      case 4: e = gemv_pass<4>(w, af, a, arb, xx, xs, n0, n1, yy, ys, bias, dd, ws, s); break;
      default: e = gemv_pass<8>(w, af, a, arb, xx, xs, n0, n1, yy, ys, bias, dd, ws, s); break;
    }
    if (e != hipSuccess) return e;
    r0 += rows;
  }
  return hipSuccess;
}

// The gated M = 1 GEMV: one workgroup per 64-row group holds both weights' rows,
// W / 2 waves each, so the launch streams gate and up together and writes only
// act(g) * u. 16-wave workgroups while the row groups fit on the CUs at once.
template <int WT, int W, int kEarly>
static hipError_t gated_launch(const WeightDev& wg, const WeightDev& wu, int act, const float* x, float* y,
                               hipStream_t s) {
  constexpr int U = W >= 16 ? 1 : 2;
  const int64_t groups = (wg.n + kRowGroup - 1) / kRowGroup;
  const size_t lds = 2 * gemv_lds_bytes(WT, kActQ8_K, 1, W, wg.nblk, false) + (kEarly > 0 ? kDummyBytes : 0);
  if (lds > kGemvMaxLds) return hipErrorInvalidValue;
  const void* fn = reinterpret_cast<const void*>(&k_gemv<WT, kActQ8_K, 1, W, U, true, kEarly, true>);
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((k_gemv<WT, kActQ8_K, 1, W, U, true, kEarly, true>), dim3((unsigned)groups), dim3(64 * W), lds, s,
                     wg.plane[0], wg.plane[1], wg.plane[2], wg.plane[3], (int)wg.nblk, (int64_t)0, (int64_t)0, wg.n,
                     nullptr, (int64_t)0, x, wg.k, y, wg.n, nullptr, nullptr, wg.n, wu.plane[0], wu.plane[1],
                     wu.plane[2], wu.plane[3], act, 1, nullptr);
  return hipGetLastError();
}

template <int WT, int W>
static hipError_t gated_waves(const WeightDev& wg, const WeightDev& wu, int act, const float* x, float* y,
                              hipStream_t s) {
  const int64_t per_wave = (wg.nblk + W / 2 - 1) / (W / 2);
  if (per_wave == 1) return gated_launch<WT, W, 1>(wg, wu, act, x, y, s);
  if (per_wave == 2) return gated_launch<WT, W, 2>(wg, wu, act, x, y, s);
  return gated_launch<WT, W, 0>(wg, wu, act, x, y, s);
}

bool gemv_gated_supported(const WeightDev& wg, const WeightDev& wu) {
  if ((wg.dtype != kQ4_K && wg.dtype != kQ6_K) || wu.dtype != wg.dtype || wu.n != wg.n || wu.k != wg.k) return false;
  return 2 * gemv_lds_bytes(wg.dtype, kActQ8_K, 1, 16, wg.nblk, false) + kDummyBytes <= kGemvMaxLds &&
         wg.k * 4 < ((int64_t)1 << 32);
}

hipError_t launch_gemv_gated(const WeightDev& wg, const WeightDev& wu, int act, const float* x, float* y,
                             hipStream_t s) {
  if (!gemv_gated_supported(wg, wu) || !act_ok(act)) return hipErrorInvalidValue;
  const bool wide = (wg.n + kRowGroup - 1) / kRowGroup <= wg.cus;
  if (wg.dtype == kQ4_K) return wide ? gated_waves<kQ4_K, 16>(wg, wu, act, x, y, s) : gated_waves<kQ4_K, 8>(wg, wu, act, x, y, s);
  return wide ? gated_waves<kQ6_K, 16>(wg, wu, act, x, y, s) : gated_waves<kQ6_K, 8>(wg, wu, act, x, y, s);
}

hipError_t launch_gemv(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0, int64_t n1,
                       float* y, int64_t ys, const float* bias, int32_t* dbg, hipStream_t s, const Workspace* ws) {
  return gemv_rows(w, af, acts, arb, nullptr, 0, m, n0, n1, y, ys, bias, dbg, ws, s);
}

hipError_t launch_gemv_fused(const WeightDev& w, const float* x, int64_t xs, int64_t m, float* y, int64_t ys,
                             const float* bias, hipStream_t s, const Workspace* ws, int af) {
  if (af >= 0 && !(af == kActPer32 && (w.dtype == kQ4_K || w.dtype == kQ6_K))) return hipErrorInvalidValue;
  return gemv_rows(w, af, nullptr, 0, x, xs, m, 0, w.n, y, ys, bias, nullptr, ws, s);
}

}  // namespace dq
