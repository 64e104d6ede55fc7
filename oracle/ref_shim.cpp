// ref_shim.cpp -- C entry points onto the reference's own CPU kernels.
//
// TEST INFRASTRUCTURE ONLY. Compiled (by oracle/Makefile, target `ref`) together
// with the reference's sources where they lie under /root/reference into
// oracle/_ref/libdynacore_ref.so. Nothing of the reference is copied: this file
// only includes its headers at build time and forwards to its functions:
//   dynacore/include/dynacore/tensor/fp16.h:18-62          fp16 conversion
//   dynacore/src/quantization/quant_formats.cpp:12-222      dequantize_*, quantize_q8_0
//   dynacore/cpu/generic/kernels_generic.cpp:187-310        quantize_act, dot_rows_* (generic)
//   dynacore/cpu/avx2/kernels_avx2.cpp:610-1440             AVX2 quantizers and dots
//   dynacore/cpu/avx2/kernels_avx2.cpp:1631-1765            quantize_act16, dot_rows16_*
//   dynacore/cpu/generic/kernels_generic.cpp:334-346        split_act16
//   dynacore/cpu/generic/kernels_generic.cpp:67-150         vec_dot_* (fp32 activations)
//   dynacore/include/dynacore/base/fast_exp.h:16-35         exp_nonpos (SiLU)
//   dynacore/src/kernel/matmul_registry.cpp:287-429         select_matmul (kernel choice)
//   dynacore/cpu/avx2/kernels_avx2.cpp:146-230,370-466      gemm_panel, dequant_* (fp32 expand + GEMM)
//   dynacore/src/execution/thread_pool.cpp                  ThreadPool (the timed decode call)
// Used to pin the C oracle (tests) and, on the GPU box, as the timed CPU
// baseline ("reference" kind) of bench.py.

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "dynacore/base/fast_exp.h"
#include "dynacore/cpu/cpu_kernels.h"
#include "dynacore/cpu/qmm.h"
#include "dynacore/execution/thread_pool.h"
#include "dynacore/hardware/cpu_info.h"
#include "dynacore/kernel/kernel_plan.h"
#include "dynacore/kernel/matmul_registry.h"
#include "dynacore/quantization/quant_formats.h"
#include "dynacore/tensor/dtype.h"
#include "dynacore/tensor/fp16.h"

using namespace dynacore;

namespace {

const CpuKernels& generic_table() {
  static const CpuKernels k = [] {
    CpuKernels t;
    register_generic_kernels(t);
    return t;
  }();
  return k;
}

const CpuKernels& avx2_table() {
  static const CpuKernels k = [] {
    CpuKernels t;
    register_generic_kernels(t);
    register_avx2_kernels(t);
    return t;
  }();
  return k;
}

bool valid_type(int t) { return t == 6 || t == 10 || t == 14 || t == 16 || t == 17; }

std::vector<const ActBlockQ8*> row_ptrs(const void* acts, int64_t row_bytes, int m) {
  std::vector<const ActBlockQ8*> p(static_cast<size_t>(m));
  for (int r = 0; r < m; ++r) p[static_cast<size_t>(r)] = reinterpret_cast<const ActBlockQ8*>(static_cast<const uint8_t*>(acts) + r * row_bytes);
  return p;
}

}  // namespace

extern "C" {

int ref_has_avx2(void) { return cpu_info().features.avx2 ? 1 : 0; }

// select_matmul under a KernelPlan whose matmul knobs are given (the rest at the
// struct's defaults, no environment) and the MatmulCaps of the GPU library's
// backend: int8-accelerated, without interleaved copies, SME or external kernels;
// kernel table: quantize_act / _sb / _sx / 16; per-32 row dots for Q4_0, Q8_0, Q4_K,
// Q6_K; super-block and sub-scaled dots for Q4_K, Q6_K; int16 dots for all four;
// qmm int8 and int16 for all four (k % 32 == 0), each with a gemm.
// Returns the MatmulKernelId and writes the MatmulActFormat to *act.
int ref_select_matmul(int64_t m, int64_t n, int64_t k, int dtype, int x_dense, int expand_min_rows,
                      int int8_decode_max_rows, int int16_decode_max_rows, int int8_superblock_min_rows,
                      int int8_superblock_max_rows, int int8_subscale_min_rows, uint32_t disabled, int qmm,
                      int qmm_gemm_min_rows, int* act) {
  if (!valid_type(dtype) || dtype == 17) return -1;
  const DType wt = static_cast<DType>(dtype);
  MatmulShape s;
  s.m = m;
  s.n = n;
  s.k = k;
  s.weight = wt;
  s.x_dense = x_dense != 0;
  KernelPlan p;
  p.expand_min_rows = expand_min_rows;
  p.int8_decode_max_rows = int8_decode_max_rows;
  p.int16_decode_max_rows = int16_decode_max_rows;
  p.int8_superblock_min_rows = int8_superblock_min_rows;
  p.int8_superblock_max_rows = int8_superblock_max_rows;
  p.int8_subscale_min_rows = int8_subscale_min_rows;
  p.matmul_disabled = disabled;
  p.qmm = qmm != 0;
  p.qmm_gemm_min_rows = qmm_gemm_min_rows;
  const bool kq = wt == DType::kQ4_K || wt == DType::kQ6_K;
  MatmulCaps c;
  c.int8_accelerated = true;
  c.quantize_act = c.quantize_act_sb = c.quantize_act_sx = c.quantize_act16 = true;
  c.dot_q8_rows = true;
  c.dot_q8_sb_rows = kq;
  c.dot_q8_sx_rows = kq;
  c.dot_q16_rows = true;
  c.qmm_int8 = c.qmm_int16 = k % 32 == 0;
  c.qmm_gemm = wt == DType::kQ8_0 || wt == DType::kQ4_0 || wt == DType::kQ4_K || wt == DType::kQ6_K;
  const MatmulSelection sel = select_matmul(s, p, c);
  if (act != nullptr) *act = static_cast<int>(sel.act);
  return static_cast<int>(sel.id);
}
int ref_physical_cores(void) { return static_cast<int>(cpu_info().physical_cores); }
int ref_logical_cores(void) { return static_cast<int>(cpu_info().logical_cores); }

float ref_fp16_to_fp32(uint16_t h) { return fp16_to_fp32(h); }
uint16_t ref_fp32_to_fp16(float f) { return fp32_to_fp16(f); }

int ref_dequantize(int dtype, const void* blocks, float* y, int64_t n) {
  if (!valid_type(dtype)) return -1;
  const auto t = static_cast<DType>(dtype);
  const int64_t be = dtype_block_elems(t);
  if (n % be != 0) return -1;
  const int64_t nb = n / be;
  switch (t) {
    case DType::kQ4_0: quant::dequantize_q4_0(static_cast<const quant::BlockQ4_0*>(blocks), y, nb); break;
    case DType::kQ8_0: quant::dequantize_q8_0(static_cast<const quant::BlockQ8_0*>(blocks), y, nb); break;
    case DType::kQ4_K: quant::dequantize_q4_K(static_cast<const quant::BlockQ4_K*>(blocks), y, nb); break;
    case DType::kQ6_K: quant::dequantize_q6_K(static_cast<const quant::BlockQ6_K*>(blocks), y, nb); break;
    case DType::kQ8_K: quant::dequantize_q8_K(static_cast<const quant::BlockQ8_K*>(blocks), y, nb); break;
    default: return -1;
  }
  return 0;
}

int ref_quantize_q8_0(const float* x, void* out, int64_t n) {
  if (n % 32 != 0) return -1;
  quant::quantize_q8_0(x, static_cast<quant::BlockQ8_0*>(out), n / 32);
  return 0;
}

// tier: 0 = generic, 1 = AVX2.
int ref_quantize_act(int tier, const float* x, void* out, int64_t n) {
  if (n % 32 != 0) return -1;
  const CpuKernels& k = tier ? avx2_table() : generic_table();
  k.quantize_act(x, static_cast<ActBlockQ8*>(out), n);
  return 0;
}

// Super-block (one scale per 256, ActBlockQ8 layout) and sub-scaled (ActSuperQ8): AVX2 only.
int ref_quantize_act_sb(const float* x, void* out, int64_t n) {
  const CpuKernels& k = avx2_table();
  if (n % 256 != 0 || !k.quantize_act_sb) return -1;
  k.quantize_act_sb(x, static_cast<ActBlockQ8*>(out), n);
  return 0;
}

int ref_quantize_act_sx(const float* x, void* out, int64_t n) {
  const CpuKernels& k = avx2_table();
  if (n % 256 != 0 || !k.quantize_act_sx) return -1;
  k.quantize_act_sx(x, static_cast<ActBlockQ8*>(out), n);
  return 0;
}

// int16 activations (ActBlockQ16, AVX2 quantize_act16) and their split-byte form
// (ActBlockQ16S, generic split_act16).
int ref_quantize_act16(const float* x, void* out, int64_t n) {
  const CpuKernels& k = avx2_table();
  if (n % 32 != 0 || !k.quantize_act16) return -1;
  k.quantize_act16(x, static_cast<ActBlockQ16*>(out), n);
  return 0;
}

int ref_split_act16(const void* in, void* out, int64_t nblocks) {
  const CpuKernels& k = generic_table();
  if (!k.split_act16) return -1;
  k.split_act16(static_cast<const ActBlockQ16*>(in), static_cast<ActBlockQ16S*>(out), nblocks);
  return 0;
}

// fp32 activations: vec_dot of one weight row and one fp32 row (tier 0 generic,
// 1 AVX2; kernels_generic.cpp:67-150, kernels_avx2.cpp:240-364).
int ref_vec_dot(int tier, int dtype, const void* w, const float* x, int64_t k, float* out) {
  if (!valid_type(dtype) || dtype == 17) return -1;
  const CpuKernels& t = tier ? avx2_table() : generic_table();
  VecDotFn fn = t.vec_dot_for(static_cast<DType>(dtype));
  if (!fn) return -2;
  *out = fn(w, x, k);
  return 0;
}

// out[r] = dot(w row, int16 act row r), r < m <= 4 (AVX2 DotQ16RowsFn).
int ref_dot_rows16(int dtype, const void* w, const void* acts, int64_t act_row_bytes, int m, int64_t k, float* out) {
  if (!valid_type(dtype) || m < 1 || m > kDotRowsMax) return -1;
  DotQ16RowsFn fn = avx2_table().dot_q16_rows_for(static_cast<DType>(dtype));
  if (!fn) return -2;
  std::vector<const ActBlockQ16*> p(static_cast<size_t>(m));
  for (int r = 0; r < m; ++r) {
    p[static_cast<size_t>(r)] = reinterpret_cast<const ActBlockQ16*>(static_cast<const uint8_t*>(acts) + r * act_row_bytes);
  }
  fn(w, p.data(), m, k, out);
  return 0;
}

// out[r] = dot(w row, act row r), r < m <= 4 (DotQ8RowsFn). kind: 0 = generic
// per-32, 1 = AVX2 per-32, 2 = AVX2 super-block (acts from ref_quantize_act_sb),
// 3 = AVX2 sub-scaled (acts from ref_quantize_act_sx).
int ref_dot_rows(int kind, int dtype, const void* w, const void* acts, int64_t act_row_bytes, int m, int64_t k,
                 float* out) {
  if (!valid_type(dtype) || m < 1 || m > kDotRowsMax) return -1;
  const CpuKernels& t = kind == 0 ? generic_table() : avx2_table();
  const size_t i = static_cast<size_t>(dtype);
  DotQ8RowsFn fn = kind <= 1 ? t.dot_q8_rows[i] : kind == 2 ? t.dot_q8_sb_rows[i] : t.dot_q8_sx_rows[i];
  if (!fn) return -2;
  const auto p = row_ptrs(acts, act_row_bytes, m);
  fn(w, p.data(), m, k, out);
  return 0;
}

// Multi-row AVX2 kernels over weight rows [n0, n1) (DotQ8RowsNFn):
// kind 1 = per-32 (dot_q8_rows_n), 3 = sub-scaled (dot_q8_sx_rows_n).
int ref_dot_rows_n(int kind, int dtype, const void* w, int64_t w_row_bytes, int64_t n0, int64_t n1, const void* acts,
                   int64_t act_row_bytes, int m, int64_t k, float* y, int64_t y_stride, const float* bias) {
  if (!valid_type(dtype) || m < 1 || m > kDotRowsNMax) return -1;
  const CpuKernels& t = avx2_table();
  const size_t i = static_cast<size_t>(dtype);
  DotQ8RowsNFn fn = kind == 1 ? t.dot_q8_rows_n[i] : kind == 3 ? t.dot_q8_sx_rows_n[i] : nullptr;
  if (!fn) return -2;
  const auto p = row_ptrs(acts, act_row_bytes, m);
  std::vector<float*> yp(static_cast<size_t>(m));
  for (int r = 0; r < m; ++r) yp[static_cast<size_t>(r)] = y + r * y_stride;
  fn(w, w_row_bytes, n0, n1, p.data(), m, k, yp.data(), bias);
  return 0;
}

// CpuDevice::matmul's decode call for the sub-scaled int8 class (kInt8Subscaled,
// dynacore/cpu/cpu_device.cpp:941-960) timed as the reference runs it: one
// ThreadPool of `threads` (the calling thread included) created before the timed
// calls and reused by all of them (src/execution/thread_pool.cpp:31-45); each call
// quantizes the m fp32 rows with quantize_act_sx, then parallel_for over the n weight
// rows with grain_for(n, threads, 4, chunks_per_thread) (cpu_device.cpp:101-103),
// each chunk one dot_q8_sx_rows_n call (int8_rows' dot_n branch, :410-420). The
// weight copies in `w_copies` are visited in rotation. Runs `iters` calls after one
// warm-up call and returns the nanoseconds of the timed calls.
int64_t ref_bench_decode_sx(int dtype, const void* const* w_copies, int ncopies, int64_t w_row_bytes, int64_t n,
                            const float* x, int m, int64_t k, float* y, int threads, int chunks_per_thread, int iters) {
  if ((dtype != 14 && dtype != 16) || m < 1 || m > kDotRowsNMax || ncopies < 1 || threads < 1 || iters < 1 ||
      k % 256 != 0 || chunks_per_thread < 1) {
    return -1;
  }
  const CpuKernels& t = avx2_table();
  DotQ8RowsNFn fn = t.dot_q8_sx_rows_n[static_cast<size_t>(dtype)];
  if (!fn || !t.quantize_act_sx) return -2;
  const int64_t nb = k / kActQ8Block;
  std::vector<ActBlockQ8> act(static_cast<size_t>(m * nb));
  ThreadPool pool(threads);
  const size_t grain = std::max<size_t>(4, static_cast<size_t>(n) / (static_cast<size_t>(pool.size()) *
                                                                     static_cast<size_t>(chunks_per_thread)));
  auto call = [&](const void* w) {
    for (int r = 0; r < m; ++r) t.quantize_act_sx(x + r * k, act.data() + r * nb, k);
    pool.parallel_for(static_cast<size_t>(n), grain, [&](size_t begin, size_t end) {
      const ActBlockQ8* xn[kDotRowsNMax];
      float* yr[kDotRowsNMax];
      for (int r = 0; r < m; ++r) {
        xn[r] = act.data() + r * nb;
        yr[r] = y + r * n + static_cast<int64_t>(begin);
      }
      fn(w, w_row_bytes, static_cast<int64_t>(begin), static_cast<int64_t>(end), xn, m, k, yr, nullptr);
    });
  };
  call(w_copies[0]);
  const auto t0 = std::chrono::steady_clock::now();
  for (int it = 0; it < iters; ++it) call(w_copies[(it + 1) % ncopies]);
  const auto t1 = std::chrono::steady_clock::now();
  return std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count();
}

// The host's last-level cache in bytes (sysfs, the largest unified or data cache of
// cpu0), or 0 when sysfs does not say.
int64_t ref_llc_bytes(void) {
  int64_t best = 0;
  for (int i = 0; i < 16; ++i) {
    const std::string dir = "/sys/devices/system/cpu/cpu0/cache/index" + std::to_string(i) + "/";
    FILE* ft = std::fopen((dir + "type").c_str(), "r");
    if (ft == nullptr) break;
    char type[32] = {0};
    const int got = std::fscanf(ft, "%31s", type);
    std::fclose(ft);
    if (got != 1 || std::string(type) == "Instruction") continue;
    FILE* fs = std::fopen((dir + "size").c_str(), "r");
    if (fs == nullptr) continue;
    long long v = 0;
    char unit = 0;
    const int gs = std::fscanf(fs, "%lld%c", &v, &unit);
    std::fclose(fs);
    if (gs < 1) continue;
    const int64_t bytes = unit == 'K' ? v << 10 : unit == 'M' ? v << 20 : unit == 'G' ? v << 30 : v;
    best = std::max(best, bytes);
  }
  return best;
}

// e^x for x <= 0 (dynacore/include/dynacore/base/fast_exp.h:16-35), the exp of the
// reference's SiLU (dynacore/cpu/cpu_device.cpp:117-123).
float ref_exp_nonpos(float x) { return dynacore::exp_nonpos(x); }

// The x86 expansion of kF32ExpandGemm: the AVX2 table's dequant for the type
// (kernels_avx2.cpp:370-466, installed at :1925-1933). Returns -1 without AVX2.
int ref_expand_x86(int dtype, const void* blocks, float* y, int64_t n) {
  if (!valid_type(dtype) || !cpu_info().features.avx2) return -1;
  const DequantFn f = avx2_table().dequant_for(static_cast<DType>(dtype));
  if (f == nullptr || n % dtype_block_elems(static_cast<DType>(dtype)) != 0) return -1;
  f(blocks, y, n);
  return 0;
}

// kF32ExpandGemm on one thread (cpu_device.cpp:1114-1152 with gemm_k_block = 0):
// panels of 4 weight rows expanded by the AVX2 dequant, then the AVX2 gemm_panel
// against all m activation rows (x: m rows of stride k). y: m x n, stride n.
int ref_expand_gemm(int dtype, const void* w, int64_t w_row_bytes, int64_t n, const float* x, int64_t m, int64_t k,
                    float* y) {
  if (!valid_type(dtype) || !cpu_info().features.avx2) return -1;
  const CpuKernels& kt = avx2_table();
  const DequantFn f = kt.dequant_for(static_cast<DType>(dtype));
  if (f == nullptr || kt.gemm_panel == nullptr) return -1;
  std::vector<float> panel(static_cast<size_t>(4 * k));
  for (int64_t j0 = 0; j0 < n; j0 += 4) {
    const int nr = static_cast<int>(std::min<int64_t>(4, n - j0));
    for (int r = 0; r < nr; ++r) f(static_cast<const uint8_t*>(w) + (j0 + r) * w_row_bytes, panel.data() + r * k, k);
    kt.gemm_panel(panel.data(), nr, x, k, m, k, y + j0, n, false);
  }
  return 0;
}

// qmm's ActBuffer as the reference lays it out and fills it with its reference tier
// (dynacore/cpu/qmm/qmm_reference.cpp:25-51,440-488), copied out: hi / lo m_pad * k bytes,
// d / c m_pad * k / 32 floats (m_pad = m rounded up to even for the pair layout).
int ref_qmm_quantize(const float* x, int64_t x_stride, int64_t m, int64_t k, int mode, int paired, int8_t* hi,
                     uint8_t* lo, float* d, float* c) {
  if ((mode != 0 && mode != 1) || m < 0 || k <= 0 || k % 32 != 0) return -1;
  const auto am = mode == 0 ? dynacore::qmm::ActMode::kInt8 : dynacore::qmm::ActMode::kInt16;
  dynacore::qmm::ActBuffer buf;
  buf.prepare(am, m, k, paired != 0);
  buf.quantize_rows(x, x_stride, 0, m, dynacore::qmm::reference_kernels());
  const dynacore::qmm::Acts& a = buf.acts();
  const int64_t m_pad = paired ? (m + 1) / 2 * 2 : m;
  std::memcpy(hi, a.hi, static_cast<size_t>(m_pad * k));
  if (mode == 1) std::memcpy(lo, a.lo, static_cast<size_t>(m_pad * k));
  std::memcpy(d, a.d, static_cast<size_t>(m_pad * (k / 32)) * sizeof(float));
  std::memcpy(c, a.c, static_cast<size_t>(m_pad * (k / 32)) * sizeof(float));
  return 0;
}

// qmm's reference-tier gemv (dynacore/cpu/qmm/qmm_reference.cpp:68-114) over all m rows of x,
// quantized into an ActBuffer of the given mode and layout; calls of at most kGemvMaxRows rows
// (qmm.h:125-126). w: n GGUF rows of w_row_bytes; y: m x n, stride n.
int ref_qmm_gemv(int dtype, const void* w, int64_t w_row_bytes, int64_t n, const float* x, int64_t m, int64_t k, int mode,
                 int paired, float* y) {
  if (!valid_type(dtype) || (mode != 0 && mode != 1) || m <= 0 || k <= 0 || k % 32 != 0) return -1;
  if (!dynacore::qmm::supports(static_cast<DType>(dtype))) return -1;
  dynacore::qmm::ActBuffer buf;
  buf.prepare(mode == 0 ? dynacore::qmm::ActMode::kInt8 : dynacore::qmm::ActMode::kInt16, m, k, paired != 0);
  const dynacore::qmm::Kernels& kern = dynacore::qmm::reference_kernels();
  buf.quantize_rows(x, k, 0, m, kern);
  for (int64_t r0 = 0; r0 < m; r0 += dynacore::qmm::kGemvMaxRows) {
    const int rows = static_cast<int>(std::min<int64_t>(dynacore::qmm::kGemvMaxRows, m - r0));
    kern.gemv(static_cast<DType>(dtype), w, w_row_bytes, 0, n, buf.acts(), r0, rows, y, n, nullptr);
  }
  return 0;
}

}  // extern "C"
