// dq_gemm_p32.hip -- prefill GEMM for Q4_K weights x per-32 activations (qmm's int8
// contract: one scale d and one code sum per 32 values) on the f16 matrix cores, and
// the activation layout it reads.
//
// Arithmetic. qmm's reference for Q4_K (dot_row_ref, qmm_reference.cpp:68-93, with
// Fmt<kQ4_K>'s s32 = d sc_j and mn = dmin m_j, qmm_unpack.h) sums per sub-block j
// (32 values) of every super-block
//   acc += (d sc_j) da_j P_j - (dmin m_j) c_j,   P_j = sum_t q_t a_t,  c_j = da_j (code sum).
// sc_j P_j, an integer below 2^24 in magnitude (63 * 15 * 128 * 32), runs on
// v_mfma_f32_32x32x16_f16 with the weight operand sc_j q as the raw 16-bit integer
// (at most 945, read by the matrix core as the f16 subnormal sc_j q 2^-24) and the
// activation operand the int8 codes as f16: two K-steps per sub-block into a fresh
// accumulator, which ends at exactly sc_j P_j 2^-24. Then
//   per sub-block:    T = fma(da_j, sc_j P_j 2^-24, T)      (one VALU operation per output)
//   per super-block:  acc = fma(d 2^24, T, acc)             (one per output), T = 0
// and the mins term as fp32 matrix products on v_mfma_f32_32x32x2_f32, two
// sub-blocks per instruction straight into the output accumulator:
//   acc = acc + sum_j (-dmin m_j) c_j.
// Every product is exact or rounded once, but d multiplies the super-block's sum
// rather than each term, and the summation order is not qmm's (nor the per-32
// GEMV's, kernels_generic.cpp:261-279): the outputs agree within the fp32 tolerance of
// a K-term dot product, not bit for bit.
//
// Work split. A workgroup owns 128 activation rows x 256 weight rows with 8 waves, two
// per SIMD; wave w owns weight rows 32 w .. 32 w + 31 against the four 32-row
// activation tiles. The weight rows are the MFMA's A operand (lane l builds row l % 32's
// operand from nibbles it loads itself, each serving four MFMAs), the activation rows
// its B operand, so a lane's 16 results share one activation row and the
// per-sub-block activation scale da_j is one register per tile, read ahead of the
// sub-block. K-steps 2 j and 2 j + 1 belong to sub-block j alone; after them the wave
// folds the sub-block into T (VALU) while the SIMD's other wave runs MFMAs. A
// super-block's operands (128 rows x 256 codes as f16, 64 KB), activation scales and
// mins operands (4 + 4 KB) go to LDS one interval ahead by direct-to-LDS loads spread
// over the K-steps, into a ring of two; one barrier per super-block.
//
// Activation layout ("act32", k_act32_from_p32 from per-32 rows), for M_pad = m
// rounded up to the workgroup's 32 TT rows (zero rows past m), T = M_pad / 32 row
// tiles, nb super-blocks:
//   codes  [T][nb][k (16)][lane (64)][8 halves]  lane l: row 32 T + l % 32, half
//          hh = l / 32; K-step k = 2 j + h holds values 32 j + 16 hh + 8 h + {0, 2, 1,
//          3, 4, 6, 5, 7} of the super-block (sub-block j only)
//   da     [T][nb][j (8)][32 rows] floats
//   c      [T][nb][kk (4)][lane (64)] floats: c of row l % 32, sub-block 2 kk + l / 32
// The K order is the one in which a lane's B operand comes out of two dwords of its
// weight row's nibbles: values 32 j + t of sub-block j are the low (j even) or high
// (j odd) nibbles of qs bytes 32 (j / 2) + t (quant_formats.cpp:150-167), so K-step
// (j, h) of lane half hh reads bytes 8 h .. 8 h + 7 of qs chunk 2 (j / 2) + hh (16-byte
// chunks; the plane stores the high nibbles XOR 8).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dq_device.h"
#include "dq_f16mma.h"
#include "dq_internal.h"
#include "dq_mfma.h"
#include "dq_quant.h"

namespace dq {

namespace {

constexpr int kPN = 256;  // weight rows per workgroup (activation rows: 32 TT)
constexpr int kPThreads = 512;       // 8 waves, two per SIMD
// Super-block buffer: operands [k (16)][t (4)][lane (64)][16 B], then the activation
// scales [t (4)][j (8)][row (32)] and the mins operands [t (4)][kk (4)][lane (64)].
// With TT 32-row activation tiles per workgroup (TT = 4, or 2 / 1 for few rows): codes
// 16 TT KB, scales and mins operands TT KB each.
template <int TT>
struct PLds {
  static constexpr int kCodes = 16 * TT * 1024, kDa = kCodes, kC = kDa + TT * 1024;
  static constexpr int kBuf = kC + TT * 1024;
  static constexpr int kTotal = 2 * kBuf;
};
static_assert(PLds<4>::kTotal <= 160 * 1024, "LDS");

DQ_DEV v16f_t mfma_f32_k2(float a, float b, v16f_t c) { return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0); }

}  // namespace

// ---------------------------------------------------------------- act32 writer

// Per-32 rows (40 B per 32 values: float d, int32 code sum, int8 codes[32]) -> act32.
// Workgroup (s, T): one 32-row tile's super-block s; rows past m are zeros.
__global__ __launch_bounds__(256) void k_act32_from_p32(const uint8_t* __restrict__ acts, int64_t arb, int64_t m,
                                                        int nb, int64_t m_pad, uint8_t* __restrict__ out) {
  const int t = threadIdx.x;
  const int s = blockIdx.x;
  const int64_t T = blockIdx.y;
  const int64_t codes_bytes = m_pad * nb * 512, da_bytes = m_pad / 32 * nb * 1024;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int u = t + 256 * e, k = u >> 6, l = u & 63, hh = l >> 5;
    const int64_t row = 32 * T + (l & 31);
    v4u o = {0u, 0u, 0u, 0u};
    if (row < m) {
      const uint8_t* q = acts + row * arb + (int64_t)(8 * s + (k >> 1)) * 40 + 8 + 16 * hh + 8 * (k & 1);
      o = codes_f16(*reinterpret_cast<const u32*>(q), *reinterpret_cast<const u32*>(q + 4));
    }
    *reinterpret_cast<v4u*>(out + ((T * nb + s) * 16 + k) * 1024 + l * 16) = o;
  }
  {
    // da: thread t = 32 j + r
    const int j = t >> 5;
    const int64_t row = 32 * T + (t & 31);
    const float d = row < m ? *reinterpret_cast<const float*>(acts + row * arb + (int64_t)(8 * s + j) * 40) : 0.0f;
    *reinterpret_cast<float*>(out + codes_bytes + (T * nb + s) * 1024 + t * 4) = d;
  }
  {
    // c = d * (code sum): thread t = 64 kk + lane, sub-block 2 kk + lane / 32
    const int l = t & 63, j = 2 * (t >> 6) + (l >> 5);
    const int64_t row = 32 * T + (l & 31);
    float c = 0.0f;
    if (row < m) {
      const uint8_t* b = acts + row * arb + (int64_t)(8 * s + j) * 40;
      c = *reinterpret_cast<const float*>(b) * (float)*reinterpret_cast<const int32_t*>(b + 4);
    }
    *reinterpret_cast<float*>(out + codes_bytes + da_bytes + (T * nb + s) * 1024 + t * 4) = c;
  }
}

// fp32 rows -> act32 directly, with the per-32 quantizer's arithmetic (per32_quant, the
// same device function as the standalone quantizer: the codes, d and code sums are its
// bytes, so the layout equals k_act32_from_p32's of those rows). One wave per (super-
// block, padded row); lane l quantizes values 4 l .. 4 l + 3 (block l / 8), and even lane
// e = 8 j + 4 hh + 2 h writes K-step 2 j + h of lane half hh with lane e + 1's codes.
__global__ __launch_bounds__(64) void k_act32_quant(const float* __restrict__ x, int64_t x_stride, int64_t m,
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
  const u32 packed = per32_quant(v, d, sum);
  const u32 next = (u32)__builtin_amdgcn_ds_bpermute(4 * ((l + 1) & 63), (int)packed);
  const int64_t T = row >> 5, r = row & 31;
  const int64_t codes_bytes = m_pad * nb * 512, da_bytes = m_pad / 32 * nb * 1024;
  const int j = l >> 3;
  if ((l & 1) == 0) {
    const int hh = (l >> 2) & 1, kk = 2 * j + ((l >> 1) & 1);
    *reinterpret_cast<v4u*>(out + ((T * nb + s) * 16 + kk) * 1024 + (32 * hh + r) * 16) = codes_f16(packed, next);
  }
  if ((l & 7) == 0) {
    float* dab = reinterpret_cast<float*>(out + codes_bytes + (T * nb + s) * 1024);
    dab[j * 32 + r] = d;
    float* cb = reinterpret_cast<float*>(out + codes_bytes + da_bytes + (T * nb + s) * 1024);
    cb[(j >> 1) * 64 + 32 * (j & 1) + r] = d * (float)sum;
  }
}

// ---------------------------------------------------------------- the GEMM

// One workgroup: activation rows [128 tm, + 128) x weight rows [nbase0 + 256 tn, + 256),
// all super-blocks. Arguments as launch_gemm_p32.
template <int TT>
__global__ __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_q4k_p32(
    const uint8_t* __restrict__ qs_plane, const uint8_t* __restrict__ hdr_plane, int nb, int64_t nbase0, int64_t n_pad,
    int64_t n0, int64_t n1, const uint8_t* __restrict__ act32, int64_t m_pad, int64_t m, float* __restrict__ y,
    int64_t ys, const float* __restrict__ bias, int tiles_m, int xcd_map, int tiles_n, int nsplit,
    float* __restrict__ part) {
  using X = PLds<TT>;
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
  const int64_t nbase = nbase0 + (int64_t)kPN * tn;
  const int64_t mbase = (int64_t)tm * 32 * TT;

  const int64_t codes_bytes = m_pad * nb * 512, da_bytes = m_pad / 32 * nb * 1024;
  const auto ra = rsrc(act32, (u32)(codes_bytes + 2 * da_bytes));
  const auto rq = rsrc(qs_plane, (u32)(n_pad * nb * 128));
  const auto rh = rsrc(hdr_plane, (u32)(n_pad * nb * 16));

  // ---- this wave's loads. Operands of super-block s: blocks jb = 2 TT wave + i (i < 2 TT)
  // of the buffer, K-step jb / TT of tile jb % TT; with piece 0 the activation scales
  // (waves 0 .. TT - 1) or mins operands (waves 4 .. 3 + TT) of tile wave % 4. The wave's weight row:
  // 64-row group g0 + wave / 2, row 32 (wave & 1) + li; lane half hh loads qs chunks
  // hh, 2 + hh, 4 + hh, 6 + hh of it and its header.
  const u32 g0 = (u32)(nbase >> 6);
  const u32 G = g0 + (u32)(wave >> 1), r64 = (u32)(32 * (wave & 1) + li);
  const u32 vq = (G * (u32)nb * 8u + (u32)hh) * 1024u + r64 * 16u;  // + (s * 8 + 2 g) * 1024
  const u32 vh = (G * (u32)nb * 64u + r64) * 16u;                  // + s * 1024

  auto issue_piece = [&](int s, int i) {
    uint8_t* P = lds + (s & 1) * X::kBuf;
    const int jb = 2 * TT * wave + i;
    const int64_t T = (int64_t)TT * tm + (jb % TT);
    dma16(ra, P + jb * 1024, (u32)(lane * 16), (u32)(((T * nb + s) * 16 + (jb / TT)) * 1024));
    if (i == 0) {
      const int tt = wave & 3;
      const int64_t Tb = (int64_t)TT * tm + tt;
      if (wave < TT) {
        dma16(ra, P + X::kDa + tt * 1024, (u32)(lane * 16), (u32)(codes_bytes + (Tb * nb + s) * 1024));
      } else if (wave >= 4 && wave < 4 + TT) {
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

  // Super-block s: per sub-block j its two K-steps (TT MFMA chains, one per activation
  // tile) and then its fold into T; the next super-block's loads spread over the K-steps,
  // and the 4 TT mins products over the even K-steps; at the end T into acc.
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
        // mins products q = tile 4 + pair, 4 TT of them over the 8 even K-steps (TT = 4:
        // two per even K-step; 2: one; 1: one every other)
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) da[tt] = ld_da(tt, k >> 1);
        if (TT == 4) {
          mins(k >> 2, 2 * ((k >> 1) & 1));
          mins(k >> 2, 2 * ((k >> 1) & 1) + 1);
        } else if (TT == 2) {
          mins((k >> 1) >> 2, (k >> 1) & 3);
        } else if ((k & 3) == 0) {
          mins(0, k >> 2);
        }
      }
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        const v4u a = lds16(P + ((TT * k + tt) * 64 + lane) * 16);
        S[tt] = mfma_h(w, a, (k & 1) == 0 ? v16f_t{} : S[tt]);
      }
      if (k < 15) w = build(k + 1);
      // the next super-block's 2 TT pieces of this wave, evenly over the K-steps
      if (k % (8 / TT) == 0 && next) issue_piece(s + 1, k / (8 / TT));
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
  for (int i = 0; i < 2 * TT; ++i) issue_piece(sb0, i);
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
        float* pr = part + ((int64_t)sp * m + mbase + row) * ((int64_t)kPN * tiles_n) + (nq - nbase0);
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

// Activation tiles per workgroup by rows: fewer for few rows, so no MFMA runs on padding.
int p32_tt(int64_t m) { return m <= 32 ? 1 : m <= 64 ? 2 : 4; }

}  // namespace

// Rows of the act32 layout: whole workgroup tiles (32 p32_tt(m) rows).
int64_t act32_rows(int64_t m) {
  const int64_t am = 32 * p32_tt(m);
  return (m + am - 1) / am * am;
}

int64_t act32_bytes(int64_t m, int64_t k) {
  const int64_t mp = act32_rows(m), nb = k / 256;
  return mp * nb * 512 + 2 * (mp / 32) * nb * 1024;
}

bool gemm_p32_ok(const WeightDev& w, int64_t m, int64_t n0, int64_t n1) {
  if (w.dtype != kQ4_K || m <= 0 || n1 <= n0 || w.nblk <= 0) return false;
  // 32-bit buffer offsets: the qs plane plus one tile's rows past its end, and act32;
  // the writer's grid has one row of workgroups per 32 padded rows
  if ((w.n_pad + 4 * kRowGroup) * w.nblk * 128 >= (1ll << 32)) return false;
  if (act32_bytes(m, w.k) >= (1ll << 32) || act32_rows(m) / 32 > 65535) return false;
  return true;
}

hipError_t launch_act32_from_p32(const uint8_t* acts, int64_t arb, int64_t m, int64_t k, uint8_t* out,
                                 hipStream_t s) {
  const int64_t mp = act32_rows(m);
  if (mp / 32 > 65535 || k % 256 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_act32_from_p32, dim3((unsigned)(k / 256), (unsigned)(mp / 32)), dim3(256), 0, s, acts, arb, m,
                     (int)(k / 256), mp, out);
  return hipGetLastError();
}

hipError_t launch_act32_quant(const float* x, int64_t x_stride, int64_t m, int64_t k, uint8_t* out, hipStream_t s) {
  const int64_t mp = act32_rows(m);
  if (mp > 65535 || k % 256 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_act32_quant, dim3((unsigned)(k / 256), (unsigned)mp), dim3(64), 0, s, x, x_stride, m, k, mp, out);
  return hipGetLastError();
}

int64_t p32_part_bytes(const WeightDev& w, int64_t m, int64_t n0, int64_t n1) {
  const int64_t nbase0 = n0 / kRowGroup * kRowGroup, am = 32 * p32_tt(m);
  const int64_t tiles_n = (n1 - nbase0 + kPN - 1) / kPN, tiles_m = (m + am - 1) / am;
  const int sp = split_ranges(tiles_n * tiles_m, w.cus > 0 ? w.cus : 256, w.nblk);
  return sp > 1 ? (int64_t)sp * m * kPN * tiles_n * 4 : 0;
}

hipError_t launch_gemm_p32(const WeightDev& w, const uint8_t* act32, int64_t m, int64_t n0, int64_t n1, float* y,
                           int64_t ys, const float* bias, float* part, hipStream_t s) {
  if (!gemm_p32_ok(w, m, n0, n1)) return hipErrorInvalidValue;
  const int tt = p32_tt(m);
  const int64_t nbase0 = n0 / kRowGroup * kRowGroup;
  const int64_t tiles_n = (n1 - nbase0 + kPN - 1) / kPN;
  const int64_t tiles_m = (m + 32 * tt - 1) / (32 * tt);
  const int nsplit = split_ranges(tiles_n * tiles_m, w.cus > 0 ? w.cus : 256, w.nblk);
  if (nsplit > 1 && (part == nullptr || m > 65535)) return hipErrorInvalidValue;
  const int xcd_map = tiles_n % 8 == 0 ? 1 : 0;
  const void* fn = tt == 1   ? reinterpret_cast<const void*>(&k_gemm_q4k_p32<1>)
                   : tt == 2 ? reinterpret_cast<const void*>(&k_gemm_q4k_p32<2>)
                             : reinterpret_cast<const void*>(&k_gemm_q4k_p32<4>);
  const int lds = tt == 1 ? PLds<1>::kTotal : tt == 2 ? PLds<2>::kTotal : PLds<4>::kTotal;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  const dim3 grid((unsigned)(tiles_n * tiles_m * nsplit));
#define DQ_P32_LAUNCH(TTV)                                                                                            \
  hipLaunchKernelGGL(k_gemm_q4k_p32<TTV>, grid, dim3(kPThreads), lds, s, w.plane[0], w.plane[1], (int)w.nblk, nbase0, \
                     w.n_pad, n0, n1, act32, act32_rows(m), m, y, ys, bias, (int)tiles_m, xcd_map, (int)tiles_n,       \
                     nsplit, part)
  if (tt == 1) {
    DQ_P32_LAUNCH(1);
  } else if (tt == 2) {
    DQ_P32_LAUNCH(2);
  } else {
    DQ_P32_LAUNCH(4);
  }
#undef DQ_P32_LAUNCH
  if (nsplit > 1) {
    const hipError_t e2 = hipGetLastError();
    if (e2 != hipSuccess) return e2;
    return launch_split_sum(part, nsplit, m, kPN * tiles_n, nbase0, n0, n1, y, ys, bias, s);
  }
  return hipGetLastError();
}

}  // namespace dq
