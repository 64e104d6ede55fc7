// dq_gemm_b32.hip -- prefill GEMM for the 32-value block types (Q8_0, Q4_0) x per-32
// activations (ActBlockQ8) on gfx950 int8 MFMA (v_mfma_i32_16x16x32_i8).
//
// Arithmetic: the reference's generic per-32 dot (dynacore/cpu/generic/kernels_generic.cpp:216-239):
// per block b the exact integer P_b = sum_{i<32} w_i a_i, then acc = acc + (dw*da)*(float)P_b
// over the blocks in order. One MFMA with K = 32 forms P_b of a 16 x 16 tile, so every
// output runs exactly that sequence and the result is bit-identical to the CPU oracle
// (and to the GEMV only up to its slice-sum order). Q4_0 codes are the nibbles minus 8:
// the MFMA takes the raw nibbles (valid int8) and P_b = P_raw - 8 * sum(a_i), with the
// code sum of the activation block.
//
// Workgroup: 4 waves (2 x 2) over a tile of activation rows x weight rows: 64 x 64 (one
// 64-row weight group; each wave 32 x 32, 2 x 2 MFMA tiles) where those tiles are enough
// to fill the CUs, else 32 x 32 (each wave one 16 x 16 MFMA tile: twice the workgroups
// per weight group, and no padded rows for m <= 32).
//
// Two LDS stages of 4 blocks (44 KB at 64 x 64: three workgroups per CU; 21.5 KB at
// 32 x 32): the direct-to-LDS loads of the next stage are in flight while one is
// computed, across an LDS-only barrier (a full __syncthreads would wait for them; a third
// stage, two workgroups per CU, measured slower). Per stage the weight codes (the plane
// layout: per block and 16-byte chunk 64 rows x 16 B, 1 KB contiguous), their fp16 scales
// and the 160 activation bytes of each row reach LDS by direct-to-LDS buffer loads (rows
// and blocks past the ends read as zeros); the activation scales, the Q4_0 offsets
// -8 sum(a_i) and the weight scales as floats are then gathered into [block][row] arrays
// (a lane reads the offsets of its four result rows with one 16-byte read, and one scale
// of each kind for the outer products below).
//
// The MFMAs write VGPRs (a budget of at most 256 registers, at least two waves per SIMD,
// selects that form: no accumulation registers to read back), the Q4_0 offset is the
// MFMA's initial accumulator, the scale products dw * da of a block come from one fp32
// MFMA of four K = 1 outer products (each a single rounded product, as the VALU's;
// subnormal products included), and the products of the next block are in flight during
// each block's epilogue (3 VALU per output and block: cvt, multiply, add).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dq_device.h"
#include "dq_internal.h"
#include "dq_mfma.h"

namespace dq {

namespace {

typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int kKB = 4;           // blocks per stage
constexpr int kARow = kKB * 40;  // staged activation bytes per row

// LDS of one stage for a tile of TM activation rows x TN weight rows (32 or 64 each)
template <int TM, int TN>
struct Tile {
  static constexpr int kA = 0;                       // [TM rows][kKB * 40 B] activation blocks as stored
  static constexpr int kB = kA + TM * kARow;         // [kKB * chunks][TN rows][16 B] weight codes
  static constexpr int kD = kB + kKB * 2 * TN * 16;  // [kKB][TN rows] fp16 weight scales
  static constexpr int kDA = kD + kKB * TN * 2;      // [kKB][TM rows] activation scales (float)
  static constexpr int kSA = kDA + kKB * TM * 4;     // [kKB][TM rows] Q4_0: -8 x activation code sums (int)
  static constexpr int kDW = kSA + kKB * TM * 4;     // [kKB][TN rows] weight scales as float
  static constexpr int kStage = kDW + kKB * TN * 4;
  static constexpr int kLds = 2 * kStage;  // two stages: 44 KB at 64 x 64 (three workgroups per CU)
  static constexpr int RT = TM / 32, CT = TN / 32;  // 16 x 16 MFMA tiles per wave (2 x 2 waves)
};

DQ_DEV void ld_lds16(__amdgpu_buffer_rsrc_t r, uint8_t* lds_dst, u32 voff, u32 soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_dst, 16, voff, soff, 0, 0);
}

// a workgroup barrier after this wave's LDS reads and writes: later direct-to-LDS loads stay
// in flight across it (__syncthreads would wait for them)
DQ_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

DQ_DEV v4i_t mfma32(v2u a, v2u b, v4i_t c) {
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, a), __builtin_bit_cast(long, b), c, 0, 0, 0);
}

typedef float f16v_t __attribute__((ext_vector_type(16)));

// Four 16 x 16 outer products in one instruction (K = 1, four blocks): lane group g
// gives column vector a (its 16 lanes' values) and row vector b of block g; registers
// 4 g' .. 4 g' + 3 of every lane hold block g' at rows 4 lg + e, column li, the layout
// of the 16 x 16 integer products. Each output is one product a_i b_j rounded once.
DQ_DEV f16v_t outer4(float a, float b) {
  return __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, f16v_t{}, 0, 0, 0);
}

template <int WT, int TM, int TN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm_b32(
    const uint8_t* __restrict__ qs_plane, const uint8_t* __restrict__ d_plane, int nblk, int64_t g0, int64_t n0,
    int64_t n1, const uint8_t* __restrict__ acts, int64_t arb, int64_t m, float* __restrict__ y, int64_t ys,
    const float* __restrict__ bias, int tiles_n, int tiles_m) {
  using C = Tile<TM, TN>;
  constexpr int RT = C::RT, CT = C::CT, kA = C::kA, kB = C::kB, kD = C::kD, kDA = C::kDA, kSA = C::kSA, kDW = C::kDW;
  constexpr int kStage = C::kStage;
  constexpr int kC = WT == kQ8_0 ? 2 : 1;  // 16-byte code chunks per block and row
  extern __shared__ __align__(16) uint8_t lds[];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave & 1, wn = wave >> 1;  // rows (TM / 2) wm, columns (TN / 2) wn of the tile
  const int li = lane & 15, lg = lane >> 4;

  // XCD-aware order: the activation tiles of one weight tile run on one XCD
  int L = blockIdx.x;
  const int per = (tiles_n * tiles_m) / 8;
  if (L < 8 * per) L = (L % 8) * per + L / 8;
  const int tn = __builtin_amdgcn_readfirstlane(L / tiles_m);
  const int tm = __builtin_amdgcn_readfirstlane(L - tn * tiles_m);
  const int64_t G = g0 + tn / (64 / TN);  // 64-row group of the plane, rows r0 .. r0 + TN - 1 of it
  const int r0 = (tn % (64 / TN)) * TN;
  const int64_t mbase = (int64_t)tm * TM;
  const int64_t mrows = m - mbase < TM ? m - mbase : TM;

  const auto ra = rsrc(acts + mbase * arb, (u32)(mrows * arb));
  const auto rq = rsrc(qs_plane + G * nblk * 64 * 16 * kC, (u32)(nblk * 64 * 16 * kC));
  const auto rd = rsrc(d_plane + G * nblk * 64 * 2, (u32)(nblk * 64 * 2));

  f4_t acc[RT][CT];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < CT; ++j) acc[i][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // staging of blocks [b, b + kKB) into buffer buf: direct-to-LDS loads only, 1 KB
  // instruction i of each kind going to wave i % 4. Every offset is in the vector offset,
  // which the buffer's range check covers (the scalar offset is not checked): blocks past
  // the row's end read as zeros instead of the bytes after the plane or the rows.
  auto issue = [&](int b, int buf) {
    uint8_t* base = lds + buf * kStage;
    // activations: piece p (16 B) of the TM x kARow region is row p / kAP, byte 16 (p % kAP)
    constexpr int kAP = kARow / 16, kAI = TM * kAP / 64;
#pragma unroll
    for (int ii = 0; ii < (kAI + 3) / 4; ++ii) {
      const int i = wave + 4 * ii;
      if (i < kAI) {
        const int p = i * 64 + lane, row = p / kAP;
        ld_lds16(ra, base + kA + i * 1024, (u32)(row * arb + 16 * (p % kAP) + b * 40), 0u);
      }
    }
    // weight codes: piece q = (block q / kC, chunk q % kC) is TN rows x 16 B of the plane's
    // 1 KB (block, chunk) record; instruction i takes 64 / TN pieces
    constexpr int kPer = 64 / TN, kWI = kKB * kC / kPer;
#pragma unroll
    for (int ii = 0; ii < (kWI + 3) / 4; ++ii) {
      const int i = wave + 4 * ii;
      if (i < kWI) {
        ld_lds16(rq, base + kB + i * 1024, (u32)((b * kC + i * kPer + lane / TN) * 1024 + (r0 + lane % TN) * 16), 0u);
      }
    }
    // fp16 weight scales: kKB x TN x 2 B, TN / 8 lanes per block (wave 3: it issues the
    // fewest activation loads)
    constexpr int kDL = TN / 8;
    if (wave == 3 && lane < kKB * kDL) {
      ld_lds16(rd, base + kD, (u32)((b + lane / kDL) * 128 + r0 * 2 + (lane % kDL) * 16), 0u);
    }
  };
  // the activation scales, code sums and weight scales of a landed stage as [block][row]
  auto gather = [&](int buf) {
    uint8_t* base = lds + buf * kStage;
    if (t < kKB * TM) {
      const int j = t / TM, row = t % TM;
      const v2u ds = *reinterpret_cast<const v2u*>(base + kA + row * kARow + j * 40);
      *reinterpret_cast<u32*>(base + kDA + t * 4) = ds.x;
      if (WT == kQ4_0) *reinterpret_cast<int*>(base + kSA + t * 4) = -8 * (int)ds.y;
    }
    if (t < kKB * TN) {
      *reinterpret_cast<float*>(base + kDW + t * 4) = h2f(*reinterpret_cast<const uint16_t*>(base + kD + t * 2));
    }
  };
  // For block j of the landed stage and this wave's RT x CT MFMA tiles: P_b (Q4_0 starts
  // the integer accumulator at -8 x the activation code sum of the row), and the scale
  // products dw * da as four outer products, tile (rt, ct) = (g >> 1, g & 1) from lane
  // group g (groups of tiles a smaller wave tile lacks compute unused products).
  const int wr = (TM / 2) * wm, wc = (TN / 2) * wn;  // the wave's first row and column in the tile
  struct Prod {
    v4i_t p[RT][CT];
    f16v_t s;
  };
  auto products = [&](const uint8_t* base, int j, Prod& pr) {
    const int grt = (lg >> 1) & (RT - 1), gct = lg & 1 & (CT - 1);
    const float sa = *reinterpret_cast<const float*>(base + kDA + (j * TM + wr + 16 * grt + li) * 4);
    const float sw = *reinterpret_cast<const float*>(base + kDW + (j * TN + wc + 16 * gct + li) * 4);
    v2u af[RT], bf[CT];
    v4i_t c[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int row = wr + 16 * rt + li;
      af[rt] = *reinterpret_cast<const v2u*>(base + kA + row * kARow + j * 40 + 8 + 8 * lg);
      c[rt] = WT == kQ4_0 ? *reinterpret_cast<const v4i_t*>(base + kSA + (j * TM + wr + 16 * rt + 4 * lg) * 4)
                          : v4i_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int col = wc + 16 * ct + li;
      if (WT == kQ8_0) {
        bf[ct] = *reinterpret_cast<const v2u*>(base + kB + ((j * 2 + (lg >> 1)) * TN + col) * 16 + 8 * (lg & 1));
      } else {
        // values 0..15 are the low nibbles of bytes 0..15, 16..31 the high ones
        const v2u raw = *reinterpret_cast<const v2u*>(base + kB + (j * TN + col) * 16 + 8 * (lg & 1));
        const u32 sh = (lg >> 1) * 4;
        bf[ct] = v2u{(raw.x >> sh) & 0x0F0F0F0Fu, (raw.y >> sh) & 0x0F0F0F0Fu};
      }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) pr.p[rt][ct] = mfma32(af[rt], bf[ct], c[rt]);
    pr.s = outer4(sa, sw);
  };
  // acc = acc + (dw * da) * (float)P_b, in block order
  auto epilogue = [&](const Prod& pr) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float t1 = pr.s[4 * (2 * rt + ct) + e];
          const float t2 = t1 * (float)pr.p[rt][ct][e];
          acc[rt][ct][e] = acc[rt][ct][e] + t2;
        }
  };

  // two stages: the loads of the next stage are in flight while this one is computed
  issue(0, 0);
  for (int b = 0, buf = 0; b < nblk; b += kKB, buf ^= 1) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of the stage have landed
    lds_barrier();                  // everyone's have, and the other stage's compute is done
    if (b + kKB < nblk) issue(b + kKB, buf ^ 1);
    gather(buf);
    lds_barrier();
    const uint8_t* base = lds + buf * kStage;
    if (nblk - b >= kKB) {
      // a full stage: the products of the next block are in flight during each epilogue
      Prod p, q;
      products(base, 0, p);
#pragma unroll
      for (int j = 0; j < kKB; j += 2) {
        products(base, j + 1, q);
        epilogue(p);
        if (j + 2 < kKB) products(base, j + 2, p);
        epilogue(q);
      }
    } else {
      for (int j = 0; j < nblk - b; ++j) {
        Prod p;
        products(base, j, p);
        epilogue(p);
      }
    }
  }

  // ---- store
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int64_t n = G * kRowGroup + r0 + wc + 16 * ct + li;
    if (n < n0 || n >= n1) continue;
    const float bn = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t mm = mbase + wr + 16 * rt + 4 * lg + e;
        if (mm < m) y[mm * ys + n] = bias ? acc[rt][ct][e] + bn : acc[rt][ct][e];
      }
    }
  }
}

template <int WT, int TM, int TN>
hipError_t launch_tile(const WeightDev& w, const uint8_t* acts, int64_t arb, int64_t m, int64_t g0, int64_t g1,
                       int64_t n0, int64_t n1, float* y, int64_t ys, const float* bias, hipStream_t s) {
  const int64_t tiles_n = (g1 - g0) * (64 / TN), tiles_m = (m + TM - 1) / TM;
  if (tiles_n * tiles_m >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  constexpr int kLds = Tile<TM, TN>::kLds;
  hipLaunchKernelGGL((k_gemm_b32<WT, TM, TN>), dim3((unsigned)(tiles_n * tiles_m)), dim3(256), kLds, s,
                     w.plane[0], w.plane[1], (int)w.nblk, g0, n0, n1, acts, arb, m, y, ys, bias, (int)tiles_n,
                     (int)tiles_m);
  return hipGetLastError();
}

template <int WT>
hipError_t launch_type(const WeightDev& w, const uint8_t* acts, int64_t arb, int64_t m, int64_t g0, int64_t g1,
                       int64_t n0, int64_t n1, float* y, int64_t ys, const float* bias, hipStream_t s, int tile) {
  if (tile == 64) return launch_tile<WT, 64, 64>(w, acts, arb, m, g0, g1, n0, n1, y, ys, bias, s);
  return launch_tile<WT, 32, 32>(w, acts, arb, m, g0, g1, n0, n1, y, ys, bias, s);
}

}  // namespace

// The tile: 64 x 64 from 33 rows where those tiles are at least 7/4 of the CUs, else
// 32 x 32. Measured at K = 4096 (graph replay; Q8_0 N = 4096 / Q4_0 N = 14336; 64 x 64
// against 32 x 32): 39.5 / 46.4 -> 25.0 / 30.6 us at 20 rows, 39.5 / 45.4 -> 24.9 /
// 42.7 at 64, 41.5 -> 28.7 at 128 (Q8_0; Q4_0 57.3 vs 68.0 keeps 64 x 64), 51.7 / 165.5
// vs 67.0 / 223.9 at 512. The mixed tiles (64 x 32, 32 x 64) were within 6% of the better
// of the two everywhere but at 256 rows of Q4_0 (98.1 vs 104.3 us).
static int b32_tile(int64_t m, int64_t groups, int cus) {
  const int64_t wgs64 = groups * ((m + 63) / 64);
  return m > 32 && 4 * wgs64 >= 7 * (int64_t)cus ? 64 : 32;
}

bool gemm_b32_supported(int dtype, int af) { return (dtype == kQ8_0 || dtype == kQ4_0) && af == kActPer32; }

hipError_t launch_gemm_b32(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0,
                           int64_t n1, float* y, int64_t ys, const float* bias, hipStream_t s) {
  if (!gemm_b32_supported(w.dtype, af)) return hipErrorInvalidValue;
  if (m == 0 || n1 <= n0) return hipSuccess;
  const int64_t g0 = n0 / kRowGroup, g1 = (n1 + kRowGroup - 1) / kRowGroup;
  // 32-bit buffer offsets: one row group's codes and 64 activation rows
  if (w.nblk * 64 * 32 >= ((int64_t)1 << 31) || 64 * arb >= ((int64_t)1 << 32)) return hipErrorInvalidValue;
  const int tile = b32_tile(m, g1 - g0, w.cus > 0 ? w.cus : 256);
  return w.dtype == kQ8_0 ? launch_type<kQ8_0>(w, acts, arb, m, g0, g1, n0, n1, y, ys, bias, s, tile)
                          : launch_type<kQ4_0>(w, acts, arb, m, g0, g1, n0, n1, y, ys, bias, s, tile);
}

}  // namespace dq
