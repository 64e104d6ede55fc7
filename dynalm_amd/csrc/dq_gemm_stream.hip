// dq_gemm_stream.hip -- prefill GEMM for Q4_K weights x Q8_K activations, laid out so
// that the matrix cores, the VALU and LDS are each below their own limit at once.
//
// Arithmetic (bit-identical to the GEMV kernels, the other GEMMs and the oracle): per
// super-block b and output (m, n) the exact integer pair of the reference's super-block
// kernel (dynacore/cpu/avx2/kernels_avx2.cpp:976-1014),
//   S  = sum_j sc_j * P_j = 8 H + L,  H = sum(sh_j q a), L = sum(sl_j q a)  (sc_j = 8 sh_j + sl_j)
//   Mn = sum_j m_j * (code sum of sub-block j)
// then the library's canonical fp32 order
//   u = d * (float)S;  u = fma(-dmin, Mn, u);  acc = fma(da, u, acc).
// H and L run on v_mfma_i32_32x32x32_i8 (one sub-block per K-step; sh q and sl q are at
// most 105, so one packed 16-bit multiply turns four nibble bytes into four operand
// bytes), Mn on v_mfma_f32_32x32x16_f16 over the 16 bsums (integers below 2^24: exact).
//
// Work split. A workgroup owns 128 activation rows x 256 weight rows and 8 waves, two
// per SIMD. Wave w owns weight tile w (32 rows) against all four 32-row activation
// tiles, so each B operand it builds serves four MFMAs and no B operand goes through
// LDS: the wave unpacks its own nibbles (staged in LDS by DMA) into sh q / sl q bytes
// in registers. Only the activation codes are shared through LDS.
//
// Pipelining. The K loop runs in half super-blocks (4 sub-blocks, "positions"
// p = 2 b + h). Waves 0-3 process position t in interval t, waves 4-7 position t - 1,
// so the two waves of a SIMD are half a super-block apart: each one's fp32 epilogue
// (after its super-block's last MFMA; its H, L accumulators are reused by the next
// super-block) runs while the other wave issues MFMAs. One barrier per interval.
// Loads for position t + 2 are issued at the start of interval t as direct-to-LDS
// buffer loads into a ring of four position buffers (and a ring of three per-
// super-block buffers: headers, bsums, activation scales), and waited for at the end
// of interval t + 1.
//
// MFMA lane layout (gfx950): A lane l holds row l % 32 and K bytes 16 (l / 32) ..;
// B lane l holds column l % 32 likewise; result register r of lane l is row
// 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32 (f16 32x32x16: 8 halves of K
// 8 (l / 32) .. per lane, same result layout). Sub-block j's lane group hh takes values
// 32 j + 16 hh + i: for weights the low (j even) or high (j odd) nibbles of qs chunk
// 2 (j / 2) + hh (quant_formats.cpp:150-167; the plane stores high nibbles XOR 8), for
// activations codes 32 j + 16 hh .. of the Q8_K block. The mins MFMA's K is the 16 bsum
// groups: lane group hh takes groups 8 hh .. 8 hh + 7, i.e. m_j of sub-blocks
// 4 hh .. 4 hh + 3, each for two groups.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dq_device.h"
#include "dq_internal.h"
#include "dq_mfma.h"

namespace dq {

namespace {

typedef int v16i_t __attribute__((ext_vector_type(16)));
typedef float v16f_t __attribute__((ext_vector_type(16)));
typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

constexpr int kSM = 128, kSN = 256;  // activation rows x weight rows per workgroup
constexpr int kSThreads = 512;       // 8 waves, two per SIMD
// Position buffer (one half super-block): activation codes [4 jj][2 hh][128 rows][16 B],
// then nibbles [4 row groups][4 chunks][64 rows][16 B] (chunk c' = qs chunk 4 h + c').
constexpr int kPA = 0, kPN = 16384, kPos = 32768;
// Super-block buffer: headers [4 row groups][64 rows][16 B], bsums [128 rows][32 B],
// activation scales [128] float.
constexpr int kBH = 0, kBBs = 4096, kBDa = 8192, kBsb = 8704;
constexpr int kSbBase = 4 * kPos;
constexpr int kSLds = kSbBase + 3 * kBsb;
static_assert(kSLds <= 160 * 1024, "LDS");

DQ_DEV v16i_t mfma_i8(v4u a, v4u b, v16i_t c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i_t, a), __builtin_bit_cast(v4i_t, b), c, 0, 0, 0);
}
DQ_DEV v16f_t mfma_h(v4u a, v4u b) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h_t, a), __builtin_bit_cast(v8h_t, b), v16f_t{},
                                                0, 0, 0);
}
DQ_DEV v4u lds16(const uint8_t* p) { return *reinterpret_cast<const v4u*>(p); }

// Direct-to-LDS buffer loads: lane l's 16 (4) bytes land at dst + 16 l (4 l). The
// range check covers the vector offset only, so everything that can fall past the end
// of the buffer goes there; soff carries in-bounds offsets. (No instruction offset:
// the hardware adds it to the LDS address as well.)
DQ_DEV void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* dst, u32 voff, u32 soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, soff, 0, 0);
}
DQ_DEV void dma4(__amdgpu_buffer_rsrc_t r, uint8_t* dst, u32 voff, u32 soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 4, voff, soff, 0, 0);
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

// Interval end: this wave's loads older than its newest N are complete and its LDS
// operations are done; then the workgroup barrier. Later loads stay in flight.
template <int N>
DQ_DEV void wait_vm() {
  if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  if constexpr (N == 5) asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
  if constexpr (N == 6) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
}
DQ_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int H>
struct Half {
  static constexpr int h = H;
};

}  // namespace

// One workgroup: activation rows [128 tm, + 128) x weight rows [nbase0 + 256 tn, + 256),
// all super-blocks. Arguments as launch_gemm_stream.
__global__ __launch_bounds__(kSThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_q4k_stream(
    const uint8_t* __restrict__ qs_plane, const uint8_t* __restrict__ hdr_plane, int nb, int64_t nbase0, int64_t n_pad,
    int64_t n0, int64_t n1, const uint8_t* __restrict__ acts, int64_t arb, int64_t m, float* __restrict__ y, int64_t ys,
    const float* __restrict__ bias, int tiles_m, int xcd_map) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int t = threadIdx.x, lane = t & 63;
  const int li = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lag = wave >> 2;  // waves 4-7 run one interval behind

  // Workgroups with the same weight rows on one XCD (blocks are dealt to the 8 XCDs
  // round-robin), so the activation tiles of a weight tile share an L2.
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
  const int64_t nbase = nbase0 + (int64_t)kSN * tn;
  const int64_t mbase = (int64_t)tm * kSM;
  const int64_t mrows = m - mbase < kSM ? m - mbase : kSM;

  // Buffer resources: reads past the end return zeros (rows past m, weight rows past
  // the padded plane).
  const auto ra = rsrc(acts + mbase * arb, (u32)(mrows * arb));
  const auto rq = rsrc(qs_plane, (u32)(n_pad * nb * 128));
  const auto rh = rsrc(hdr_plane, (u32)(n_pad * nb * 16));
  const u32 g0 = (u32)(nbase >> 6);  // first 64-row group of the plane

  // ---- this wave's share of the loads: per position 2 activation + 2 nibble
  // instructions of 1 KB; with the first half of a super-block one header (waves 0-3)
  // or bsums (waves 4-7) instruction, and the activation scales on waves 0 and 4.
  // Activation instruction e of wave w: sub-block jj = w / 2, lane half ah = w % 2,
  // rows 64 e ..; nibble instruction e: row group w / 2, chunk 2 (w % 2) + e.
  const int wj = wave >> 1, wh = wave & 1;
  const u32 va0 = (u32)(lane * arb), va1 = (u32)((64 + lane) * arb);
  const u32 sa = 4 + 32 * wj + 16 * wh;
  const int adst = kPA + ((wj * 2 + wh) * 128) * 16;  // + 64 e * 16
  const u32 vn = (g0 + wj) * (u32)nb * 8192u + (u32)(2 * wh) * 1024 + lane * 16;  // + e * 1024
  const int ndst = kPN + (wj * 4 + 2 * wh) * 1024;                                 // + e * 1024
  const bool da_wave = (wave & 3) == 0;
  const u32 vx = lag ? (u32)((32 * (wave - 4) + (lane >> 1)) * arb) + 16 * (lane & 1)
                     : (g0 + wave) * (u32)nb * 1024u + lane * 16;
  const int xdst = lag ? kBBs + (wave - 4) * 1024 : kBH + wave * 1024;

  auto issue = [&](int p) {
    const int b = p >> 1, h = p & 1;
    uint8_t* P = lds + (p & 3) * kPos;
    const u32 soa = (u32)(b * 292 + 128 * h) + sa;
    dma16(ra, P + adst, va0, soa);
    dma16(ra, P + adst + 1024, va1, soa);
    const u32 son = (u32)(b * 8192 + h * 4096);
    dma16(rq, P + ndst, vn, son);
    dma16(rq, P + ndst + 1024, vn, son + 1024);
    if (h == 0) {
      uint8_t* B = lds + kSbBase + (b % 3) * kBsb;
      if (lag) {
        dma16(ra, B + xdst, vx, (u32)(b * 292 + 260));
      } else {
        dma16(rh, B + xdst, vx, (u32)(b * 1024));
      }
      if (da_wave) dma4(ra, B + kBDa + 256 * lag, lag ? va1 : va0, (u32)(b * 292));
    }
  };
  // Interval iv ends: wait for position iv + 1 (the loads issued before the newest
  // count(iv + 2), which were issued when interval iv began), barrier; then the loads
  // of position iv + 3 are issued as interval iv + 1 begins (their buffer held
  // position iv - 1, which the lagging waves read in interval iv).
  const int np = 2 * nb;
  auto interval_end = [&](int iv) {
    if (iv + 2 < np) {
      if (iv & 1) {
        wait_vm<4>();
      } else if (da_wave) {
        wait_vm<6>();
      } else {
        wait_vm<5>();
      }
    } else {
      wait_vm<0>();
    }
    lds_barrier();
    if (iv + 3 < np) issue(iv + 3);
  };

  // ---- LDS read offsets: the wave's weight rows are row group wave / 2, rows
  // 32 (wave & 1) + li; its activation operands rows 32 mt + li, lane half hh
  const int wrow = 32 * wh + li;
  const int hrd = kBH + wj * 1024 + wrow * 16;
  const int nrd = kPN + wj * 4 * 1024 + hh * 1024 + wrow * 16;  // + 2 g * 1024
  const int ard = kPA + hh * 128 * 16 + li * 16;                // + jj * 4096 + 32 mt * 16

  float acc[4][16];  // plain floats: only VALU touches them
  v16i_t sH[4], sL[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[mt][r] = 0.0f;
    sH[mt] = v16i_t{};
    sL[mt] = v16i_t{};
  }

  // MFMAs of half H of super-block b (position buffer (2 b + H) % 4; the base is a
  // run-time scalar, so that each read is one vector address plus an immediate)
  auto half = [&](int b, auto st) {
    constexpr int H = decltype(st)::h;
    const uint8_t* P = lds + __builtin_amdgcn_readfirstlane(((2 * b + H) & 3) * kPos);
    // the MFMA stream goes first when both waves of a SIMD have work ready, the other
    // wave's VALU fills the matrix core's shadow
    __builtin_amdgcn_s_setprio(1);
    const v4u hd = lds16(lds + kSbBase + (b % 3) * kBsb + hrd);
    // sc_j of sub-blocks 4 H .. 4 H + 3 as bytes (get_scale_min_k4, quant_formats.h:62-70)
    const u32 sc = H ? ((hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u)) : (hd.y & 0x3F3F3F3Fu);
    const u32 SH = (sc >> 3) & 0x07070707u, SL = sc & 0x07070707u;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const v4u w = lds16(P + nrd + 2 * g * 1024);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int jj = 2 * g + s;
        const v4u q = s ? (((w >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u) : (w & 0x0F0F0F0Fu);
        const u32 kh = __builtin_amdgcn_perm(0u, SH, sel_u16x2(jj)), kl = __builtin_amdgcn_perm(0u, SL, sel_u16x2(jj));
        const v4u bH = {mul_bytes(q.x, kh), mul_bytes(q.y, kh), mul_bytes(q.z, kh), mul_bytes(q.w, kh)};
        const v4u bL = {mul_bytes(q.x, kl), mul_bytes(q.y, kl), mul_bytes(q.z, kl), mul_bytes(q.w, kl)};
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          const v4u a = lds16(P + ard + jj * 4096 + 32 * mt * 16);
          const bool first = H == 0 && jj == 0;
          sH[mt] = mfma_i8(a, bH, first ? v16i_t{} : sH[mt]);
          sL[mt] = mfma_i8(a, bL, first ? v16i_t{} : sL[mt]);
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };
  // after super-block b's last MFMA: mins MFMAs and the canonical epilogue
  auto epilogue = [&](int b) {
    const uint8_t* B = lds + kSbBase + (b % 3) * kBsb;
    const v4u hd = lds16(B + hrd);
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    // m_{4hh} .. m_{4hh + 3}, each for two bsum groups, as fp16 ((1024 + m) - 1024, exact)
    const u32 mn = hh ? (((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u)) : (hd.z & 0x3F3F3F3Fu);
    const h2_t k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    const u32 f01 = __builtin_bit_cast(
        u32, __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0u, mn, 0x0C010C00u) | 0x64006400u) - k1024);
    const u32 f23 = __builtin_bit_cast(
        u32, __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0u, mn, 0x0C030C02u) | 0x64006400u) - k1024);
    const v4u mb = {__builtin_amdgcn_perm(f01, f01, 0x01000100u), __builtin_amdgcn_perm(f01, f01, 0x03020302u),
                    __builtin_amdgcn_perm(f23, f23, 0x01000100u), __builtin_amdgcn_perm(f23, f23, 0x03020302u)};
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const v4u bs = lds16(B + kBBs + (32 * mt + li) * 32 + 16 * hh);  // fp16 (converted in place)
      const v16f_t M = mfma_h(bs, mb);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // activation scales of rows 32 mt + 8 q + 4 hh .. + 3 (results r = 4 q .. 4 q + 3)
        const v4u da = lds16(B + kBDa + (32 * mt + 8 * q + 4 * hh) * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * q + e;
          const int S = (sH[mt][r] << 3) + sL[mt][r];
          float u = d * (float)S;
          u = fmaf(-dmin, M[r], u);
          acc[mt][r] = fmaf(as_f(da[e]), u, acc[mt][r]);
        }
      }
    }
  };

  // super-block b's bsums, int16 as loaded, to fp16 in place (exact: |bsum| <= 2048):
  // two words per thread, in the interval where both roles issue MFMAs only (the
  // leading waves' second half, the lagging waves' first), a barrier before the first
  // epilogue that reads them
  auto convert_bsums = [&](int b) {
    u32* w = reinterpret_cast<u32*>(lds + kSbBase + (b % 3) * kBsb + kBBs) + 2 * t;
    const v4u v = {w[0], w[1], 0u, 0u};
    const v4u f = bsums_f16(v);
    w[0] = f.x;
    w[1] = f.y;
  };

  // Interval iv: waves 0-3 process position iv, waves 4-7 position iv - 1. Written per
  // wave as the same loop over its own positions, the lagging waves starting with one
  // idle interval. A super-block's epilogue runs right before the first MFMA of the
  // next super-block on the leading waves, and right after the super-block's last MFMA
  // on the lagging ones: both land in the even intervals, each beside the other role's
  // MFMAs, and the odd intervals are MFMAs only. Every wave passes 2 nb + 1 barriers
  // after the first.
  issue(0);
  issue(1);
  wait_vm<4>();
  lds_barrier();
  if (np > 2) issue(2);
  if (lag) interval_end(0);
#pragma unroll 1
  for (int b = 0; b < nb; ++b) {
    if (!lag && b > 0) epilogue(b - 1);
    if (lag) convert_bsums(b);
    half(b, Half<0>{});
    interval_end(2 * b + lag);
    if (!lag) convert_bsums(b);
    half(b, Half<1>{});
    if (lag) epilogue(b);
    interval_end(2 * b + 1 + lag);
  }
  if (!lag) {
    epilogue(nb - 1);
    interval_end(np + 1);
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- outputs (+ bias): rows 32 mt + 8 (r / 4) + 4 hh + r % 4, weight row nbase + 32 wave + li
  const int64_t n = nbase + 32 * wave + li;
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

bool gemm_stream_ok(const WeightDev& w, int64_t m, int64_t n0, int64_t n1, int64_t arb) {
  if (w.dtype != kQ4_K || m <= 0 || n1 <= n0 || w.nblk <= 0) return false;
  // 32-bit buffer offsets: the qs plane plus the loads of four row groups past its end,
  // and one tile's activation rows
  if ((w.n_pad + 4 * kRowGroup) * w.nblk * 128 >= (1ll << 32) || (int64_t)kSM * arb >= (1ll << 32)) return false;
  return true;
}

hipError_t launch_gemm_stream(const WeightDev& w, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0, int64_t n1,
                              float* y, int64_t ys, const float* bias, hipStream_t s) {
  if (!gemm_stream_ok(w, m, n0, n1, arb)) return hipErrorInvalidValue;
  const int64_t nbase0 = n0 / kRowGroup * kRowGroup;
  const int64_t tiles_n = (n1 - nbase0 + kSN - 1) / kSN;
  const int64_t tiles_m = (m + kSM - 1) / kSM;
  const int xcd_map = tiles_n % 8 == 0 ? 1 : 0;
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm_q4k_stream),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kSLds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_gemm_q4k_stream, dim3((unsigned)(tiles_n * tiles_m)), dim3(kSThreads), kSLds, s, w.plane[0],
                     w.plane[1], (int)w.nblk, nbase0, w.n_pad, n0, n1, acts, arb, m, y, ys, bias, (int)tiles_m,
                     xcd_map);
  return hipGetLastError();
}

}  // namespace dq
