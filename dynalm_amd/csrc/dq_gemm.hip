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

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

DQ_DEV v4i_t mfma(v4u a, v4u b, v4i_t c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i_t, a), __builtin_bit_cast(v4i_t, b), c, 0, 0,
                                               0);
}

// Four bytes (each <= 15) times k (<= 7) in two packed 16-bit lanes: bytes stay
// bytes (k * q <= 105), one v_pk_mul_lo_u16.
DQ_DEV u32 mul_bytes(u32 q, u32 kk) {
  return __builtin_bit_cast(u32, __builtin_bit_cast(u16x2, q) * __builtin_bit_cast(u16x2, kk));
}

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

// v_perm_b32 selectors: bytes (j & 3) of the lane's sub-blocks j = hi, 2 + hi,
// 4 + hi, 6 + hi out of {sc_hi, sc_lo}; and byte s of a word into both 16-bit
// lanes (0x0C selects zero) or into all four bytes.
DQ_DEV u32 sel_subblocks(int hi) { return hi ? 0x07050301u : 0x06040200u; }
DQ_DEV u32 sel_u16x2(int s) { return 0x0C000C00u | ((u32)s << 16) | (u32)s; }
DQ_DEV u32 sel_x4(int s) { return (u32)s * 0x01010101u; }

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

// ====================================================== skinny MFMA GEMV
// Q4_K / Q6_K x Q8_K for 2..16 activation rows (decode batches): one workgroup per
// 16 weight rows, its W waves splitting the super-blocks. The activation rows are
// the 16 rows of the MFMA A operand (rows past m read zeros), the 16 weight rows
// its B columns. Per super-block each wave turns its exact integer sums into
// t = fma(-dmin, Mn, d*S) (Q6_K: d*S) in LDS; after a barrier each lane chains
// acc = fma(da, t, acc) over the super-blocks in order for its 4 outputs: the
// canonical order, so outputs are bit-identical to the GEMV, the GEMM and the CPU
// oracle. 16 rows per workgroup give N/16 workgroups, enough to fill the GPU for
// N down to ~1.5K rows at 8 waves.
//
// One kernel serves a group of matmuls (dq_matmul_many: projections sharing one
// input, as dynacore's Device::matmul_many groups them,
// dynacore/include/dynacore/device/device.h:165-171): the grid is the
// concatenation of the jobs' workgroup ranges, each workgroup finds its job in a
// table passed by value, and Q4_K and Q6_K jobs mix in one launch. dq_gemv is a
// group of one.
struct SkinnyJob {
  const uint8_t* p0;  // weight planes (dq_layout.h)
  const uint8_t* p1;
  const uint8_t* p2;
  const uint8_t* p3;
  int64_t n_pad, f0, n0, n1;  // rows (padded), first 16-row tile, output row range
  const uint8_t* acts;        // m rows of Q8_K, arb bytes apart
  int64_t arb;
  float* y;
  int64_t ys;
  const float* bias;
  int dtype, m;
  int wg0;  // first workgroup of this job in the grid
};
constexpr int kSkinnyMaxJobs = 8;
struct SkinnyGroup {
  SkinnyJob job[kSkinnyMaxJobs];
  int count;
  int nblk;  // super-blocks per row, the same for every job of a group
};

// The per-lane chain of the 16 x 16 t-terms of every super-block (LDS tt, da) and
// the stores of this lane's 4 outputs.
DQ_DEV void skinny_chain(const SkinnyJob& J, int nblk, int64_t n, const float* tt, const float* dal, int li, int lg) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int mm = 4 * lg + e;
    float v = 0.0f;
    for (int b = 0; b < nblk; ++b) v = fmaf(dal[b * 16 + mm], tt[(b * 16 + mm) * 16 + li], v);
    if (mm < J.m && n >= J.n0 && n < J.n1) J.y[mm * J.ys + n] = J.bias ? v + J.bias[n] : v;
  }
}

// Q4_K: the same sh / sl / m operand planes as the GEMM.
template <int W>
DQ_DEV void skinny_q4k(const SkinnyJob& J, int nblk, int64_t tile, uint8_t* lds) {
  float* tt = reinterpret_cast<float*>(lds);  // [nblk][16 activation rows][16 weight rows]
  float* dal = tt + nblk * 256;               // [nblk][16] activation d
  const int l = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = l & 15, lg = l >> 4, hi = lg >> 1;
  const int64_t n = tile * 16 + li;  // this lane's weight row (B column)
  const int64_t G = n / kRowGroup, r = n % kRowGroup;
  const bool nok = n < J.n_pad;
  const auto rq = rsrc(J.p0 + G * nblk * 8192, nok ? (u32)(nblk * 8192) : 0u);
  const auto rh = rsrc(J.p1 + G * nblk * 1024, nok ? (u32)(nblk * 1024) : 0u);
  const auto ra = rsrc(J.acts, (u32)(J.m * J.arb));  // activation rows past m read zeros
  const int b0 = wave * nblk / W, b1 = (wave + 1) * nblk / W;
  const u32 shift = 4u * (u32)hi, flip = hi ? 0x08080808u : 0u;  // high nibbles are stored XOR 8

  for (int b = b0; b < b1; ++b) {
    // loads: header, the lane's 16 nibble bytes of each K-step, the activation codes
    const v4u hd = ld16nt(rh, (u32)((b * 64 + r) * 16));
    v4u q[4], a[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) q[s] = ld16nt(rq, (u32)(((b * 8 + 2 * s + (lg & 1)) * 64 + r) * 16));
#pragma unroll
    for (int s = 0; s < 4; ++s) a[s] = ld16(ra, (u32)(li * J.arb + (int64_t)b * 292 + 4 + 64 * s + 16 * lg));
    const u32 dau = ld4(ra, (u32)(li * J.arb + (int64_t)b * 292));

    // scales and mins of sub-blocks 2s + hi as bytes s (get_scale_min_k4, quant_formats.h:62-70)
    const u32 sc_lo = hd.y & 0x3F3F3F3Fu, mn_lo = hd.z & 0x3F3F3F3Fu;
    const u32 sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
    const u32 mn_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
    const u32 sc = __builtin_amdgcn_perm(sc_hi, sc_lo, sel_subblocks(hi));
    const u32 KH = (sc >> 3) & 0x07070707u, KL = sc & 0x07070707u;
    const u32 MN = __builtin_amdgcn_perm(mn_hi, mn_lo, sel_subblocks(hi));

    v4i_t acc[3];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const v4u qb = ((q[s] >> shift) & 0x0F0F0F0Fu) ^ flip;
      const u32 kh = __builtin_amdgcn_perm(0u, KH, sel_u16x2(s));
      const u32 kl = __builtin_amdgcn_perm(0u, KL, sel_u16x2(s));
      const u32 mm4 = __builtin_amdgcn_perm(0u, MN, sel_x4(s));
      const v4u H = {mul_bytes(qb.x, kh), mul_bytes(qb.y, kh), mul_bytes(qb.z, kh), mul_bytes(qb.w, kh)};
      const v4u Lo = {mul_bytes(qb.x, kl), mul_bytes(qb.y, kl), mul_bytes(qb.z, kl), mul_bytes(qb.w, kl)};
      const v4u Mp = {mm4, mm4, mm4, mm4};
      const v4i_t z = {0, 0, 0, 0};
      acc[0] = mfma(a[s], H, s == 0 ? z : acc[0]);
      acc[1] = mfma(a[s], Lo, s == 0 ? z : acc[1]);
      acc[2] = mfma(a[s], Mp, s == 0 ? z : acc[2]);
    }
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int S = acc[1][e] + (acc[0][e] << 3);
      float t = d * (float)S;
      t = fmaf(-dmin, (float)acc[2][e], t);
      tt[(b * 16 + 4 * lg + e) * 16 + li] = t;
    }
    if (lg == 0) dal[b * 16 + li] = as_f(dau);
  }
  __syncthreads();
  if (wave != 0) return;
  skinny_chain(J, nblk, n, tt, dal, li, lg);
}

// Q6_K. A Q6_K sub-block is 16 values with its own signed 8-bit scale; in K-step s
// (64 values) lane group g of the B operand holds exactly sub-block u = 4s + g.
// With the unsigned 6-bit codes q (the -32 offset moved into a correction term),
//   S = sum_u sc_u * P_u - 32 * sum_u sc_u * bsum_u,   P_u = sum over sub-block u of q * a,
// P_u comes from one MFMA per sub-block whose A operand keeps only lane group u,
// and sum_u sc_u * bsum_u from one MFMA whose B operand holds sc_u at every position
// of sub-block u. Q6_K layout: dequantize_q6_K, quant_formats.cpp:192-216.
template <int W>
DQ_DEV void skinny_q6k(const SkinnyJob& J, int nblk, int64_t tile, uint8_t* lds) {
  float* tt = reinterpret_cast<float*>(lds);  // [nblk][16 activation rows][16 weight rows]
  float* dal = tt + nblk * 256;               // [nblk][16] activation d
  const int l = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = l & 15, lg = l >> 4;
  const int64_t n = tile * 16 + li;
  const int64_t G = n / kRowGroup, r = n % kRowGroup;
  const bool nok = n < J.n_pad;
  const auto rl = rsrc(J.p0 + G * nblk * 8192, nok ? (u32)(nblk * 8192) : 0u);
  const auto rh = rsrc(J.p1 + G * nblk * 4096, nok ? (u32)(nblk * 4096) : 0u);
  const auto rs = rsrc(J.p2 + G * nblk * 1024, nok ? (u32)(nblk * 1024) : 0u);
  const auto rd = rsrc(J.p3 + G * nblk * 128, nok ? (u32)(nblk * 128) : 0u);
  const auto ra = rsrc(J.acts, (u32)(J.m * J.arb));
  const int b0 = wave * nblk / W, b1 = (wave + 1) * nblk / W;
  const v4u zero = {0u, 0u, 0u, 0u};

  for (int b = b0; b < b1; ++b) {
    // lane (row li, group g): ql chunks g and 4 + g (values of K-steps 0, 1 and 2, 3 in
    // the low and high nibbles), qh chunks g & 1 and 2 + (g & 1), the 16 scales, d
    const v4u l0 = ld16nt(rl, (u32)(((b * 8 + lg) * 64 + r) * 16));
    const v4u l1 = ld16nt(rl, (u32)(((b * 8 + 4 + lg) * 64 + r) * 16));
    const v4u h0 = ld16nt(rh, (u32)(((b * 4 + (lg & 1)) * 64 + r) * 16));
    const v4u h1 = ld16nt(rh, (u32)(((b * 4 + 2 + (lg & 1)) * 64 + r) * 16));
    const v4u scw = ld16nt(rs, (u32)((b * 64 + r) * 16));
    const u32 dw = ld2nt(rd, (u32)((b * 64 + r) * 2));
    v4u a[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) a[s] = ld16(ra, (u32)(li * J.arb + (int64_t)b * 292 + 4 + 64 * s + 16 * lg));
    const u32 dau = ld4(ra, (u32)(li * J.arb + (int64_t)b * 292));

    v4i_t S = {0, 0, 0, 0}, C = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      // codes of sub-block 4s + g: quarter 2(s&1) + g/2 of half s/2
      const v4u lo = (s >> 1) ? l1 : l0, hb = (s >> 1) ? h1 : h0;
      const u32 qsh = 2u * (u32)(2 * (s & 1) + (lg >> 1));
      const v4u q = ((lo >> (u32)(4 * (s & 1))) & 0x0F0F0F0Fu) | (((hb >> qsh) & 0x03030303u) << 4);
      // scales of sub-blocks 4s .. 4s + 3 (signed bytes of scale dword s)
      const u32 sw = s == 0 ? scw.x : s == 1 ? scw.y : s == 2 ? scw.z : scw.w;
      const u32 mine = (u32)sbfe(sw, 8 * lg, 8) & 0xFFu;  // this lane group's scale
      const u32 sc4 = mine * 0x01010101u;
      const v4i_t z = {0, 0, 0, 0};
      C = mfma(a[s], v4u{sc4, sc4, sc4, sc4}, C);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const v4u au = lg == u ? a[s] : zero;
        const v4i_t P = mfma(au, q, z);
        const int scu = sbfe(sw, 8 * u, 8);
#pragma unroll
        for (int e = 0; e < 4; ++e) S[e] += scu * __builtin_amdgcn_sbfe(P[e], 0, 24);
      }
    }
    const float d = h2f(dw);
#pragma unroll
    for (int e = 0; e < 4; ++e) tt[(b * 16 + 4 * lg + e) * 16 + li] = d * (float)(S[e] - 32 * C[e]);
    if (lg == 0) dal[b * 16 + li] = as_f(dau);
  }
  __syncthreads();
  if (wave != 0) return;
  skinny_chain(J, nblk, n, tt, dal, li, lg);
}

template <int W>
__global__ __launch_bounds__(W * 64) void k_gemv_mma(SkinnyGroup g) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int wg = blockIdx.x;
  int j = 0;
  while (j + 1 < g.count && wg >= g.job[j + 1].wg0) ++j;
  const SkinnyJob& J = g.job[j];
  const int64_t tile = J.f0 + (wg - J.wg0);
  if (J.dtype == kQ6_K) {
    skinny_q6k<W>(J, g.nblk, tile, lds);
  } else {
    skinny_q4k<W>(J, g.nblk, tile, lds);
  }
}

static size_t skinny_lds(int64_t nblk) { return (size_t)nblk * (256 + 16) * sizeof(float); }

// One launch over the jobs of g (count <= kSkinnyMaxJobs, wg0 set).
static hipError_t launch_skinny(SkinnyGroup& g, int wgs, hipStream_t s) {
  const size_t lds = skinny_lds(g.nblk);
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  const bool wide = g.nblk >= 8;
  const void* fn = wide ? reinterpret_cast<const void*>(&k_gemv_mma<8>) : reinterpret_cast<const void*>(&k_gemv_mma<4>);
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  if (wide) {
    hipLaunchKernelGGL(k_gemv_mma<8>, dim3((unsigned)wgs), dim3(512), lds, s, g);
  } else {
    hipLaunchKernelGGL(k_gemv_mma<4>, dim3((unsigned)wgs), dim3(256), lds, s, g);
  }
  return hipGetLastError();
}

static SkinnyJob skinny_job(const WeightDev& w, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0, int64_t n1,
                            float* y, int64_t ys, const float* bias) {
  SkinnyJob J;
  J.p0 = w.plane[0];
  J.p1 = w.plane[1];
  J.p2 = w.plane[2];
  J.p3 = w.plane[3];
  J.n_pad = w.n_pad;
  J.f0 = n0 / 16;
  J.n0 = n0;
  J.n1 = n1;
  J.acts = acts;
  J.arb = arb;
  J.y = y;
  J.ys = ys;
  J.bias = bias;
  J.dtype = w.dtype;
  J.m = (int)m;
  J.wg0 = 0;
  return J;
}

hipError_t launch_gemv_mma(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0,
                           int64_t n1, float* y, int64_t ys, const float* bias, hipStream_t s) {
  if (!gemv_mma_supported(w.dtype, af, m)) return hipErrorInvalidValue;
  if (n1 <= n0) return hipSuccess;
  SkinnyGroup g;
  g.job[0] = skinny_job(w, acts, arb, m, n0, n1, y, ys, bias);
  g.count = 1;
  g.nblk = (int)w.nblk;
  return launch_skinny(g, (int)((n1 + 15) / 16 - n0 / 16), s);
}

hipError_t launch_gemv_mma_many(const GemvJob* jobs, int count, hipStream_t s) {
  for (int i0 = 0; i0 < count; i0 += kSkinnyMaxJobs) {
    SkinnyGroup g;
    g.count = count - i0 < kSkinnyMaxJobs ? count - i0 : kSkinnyMaxJobs;
    g.nblk = (int)jobs[i0].w->nblk;
    int wgs = 0;
    for (int i = 0; i < g.count; ++i) {
      const GemvJob& q = jobs[i0 + i];
      if (q.w->nblk != g.nblk || !gemv_mma_supported(q.w->dtype, kActQ8_K, q.m)) return hipErrorInvalidValue;
      g.job[i] = skinny_job(*q.w, q.acts, q.arb, q.m, 0, q.w->n, q.y, q.ys, q.bias);
      g.job[i].wg0 = wgs;
      wgs += (int)((q.w->n + 15) / 16);
    }
    const hipError_t e = launch_skinny(g, wgs, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

bool gemv_mma_supported(int dtype, int af, int64_t m) {
  return (dtype == kQ4_K || dtype == kQ6_K) && af == kActQ8_K && m >= 2 && m <= 16;
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
