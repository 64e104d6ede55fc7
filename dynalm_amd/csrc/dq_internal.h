// dq_internal.h -- host-side declarations shared by the C-ABI layer and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dynaq.h"
#include "dq_layout.h"

namespace dq {

// A weight on the device in the x8 layout of dq_layout.h.
struct WeightDev {
  int dtype = 0;
  int device = 0;
  int cus = 256;           // compute units of the device (launch shapes)
  int64_t n = 0, k = 0;    // logical rows and values per row
  int64_t n_pad = 0;       // rows rounded up to a multiple of kRowGroup
  int64_t nblk = 0;        // blocks (super-blocks for K-quants) per row
  uint8_t* plane[kMaxPlanes] = {nullptr, nullptr, nullptr, nullptr};
  int64_t plane_bytes[kMaxPlanes] = {0, 0, 0, 0};
};

// Records the calling thread's error message (dq_last_error) and returns code.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Makes `device` current for the scope and restores the previous device after.
struct DeviceScope {
  int prev = -1;
  hipError_t err = hipSuccess;
  explicit DeviceScope(int device) {
    err = hipGetDevice(&prev);
    if (err == hipSuccess && prev != device) err = hipSetDevice(device);
  }
  ~DeviceScope() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
  DeviceScope(const DeviceScope&) = delete;
  DeviceScope& operator=(const DeviceScope&) = delete;
};

// A device region for a launch's temporaries (split-K row sums). p == nullptr: the
// library's per-device buffer, grown with hipMalloc on demand; otherwise the
// caller's region of `bytes` bytes (a launch that needs more fails with
// hipErrorInvalidValue and allocates nothing).
struct Workspace {
  uint8_t* p = nullptr;
  size_t bytes = 0;
};

hipError_t launch_quantize(int af, const float* x, int64_t m, int64_t k, int64_t x_stride, uint8_t* out, int64_t orb,
                           hipStream_t s);
// qmm's activation buffer (dynacore/include/dynacore/cpu/qmm.h:57-86): rows [r0, r1) of x
// into the row or pair layout, int8 or int16 codes; and the zero pad row of a paired
// buffer of odd m.
hipError_t launch_qmm_quantize(const float* x, int64_t x_stride, int64_t r0, int64_t r1, int64_t k, bool i16,
                               bool paired, int8_t* hi, uint8_t* lo, float* d, float* c, hipStream_t s);
hipError_t launch_qmm_pad(int64_t m, int64_t k, int8_t* hi, uint8_t* lo, float* d, float* c, hipStream_t s);
// Rows [r0, r0 + rows) of a qmm activation buffer as per-32 ActBlockQ8 (int8) or
// ActBlockQ16 (int16) rows of orb bytes.
hipError_t launch_qmm_to_blocks(const int8_t* hi, const uint8_t* lo, const float* d, int64_t k, bool i16, bool paired,
                                int64_t r0, int64_t rows, uint8_t* out, int64_t orb, hipStream_t s);
hipError_t launch_repack(int t, const uint8_t* src, int64_t row_stride, int64_t n, int64_t nblk, uint8_t* const* planes,
                         hipStream_t s);
hipError_t launch_unpack(int t, uint8_t* dst, int64_t row_stride, int64_t n, int64_t nblk, uint8_t* const* planes,
                         hipStream_t s);
// dbg (nullable): per (row, weight row, super-block) the exact S and Mn of the
// K-quant x Q8_K kernels.
hipError_t launch_gemv(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0, int64_t n1,
                       float* y, int64_t ys, const float* bias, int32_t* dbg, hipStream_t s,
                       const Workspace* ws = nullptr);
// Decode matmul with the activation quantization fused into the GEMV (fp32 rows x,
// row stride xs floats): af < 0, the weight's activation format (dq_act_format_for);
// af = kActPer32 for Q4_K / Q6_K, per-32 rows (qmm's int8 contract), each wave
// quantizing its slice with the standalone per-32 quantizer's device function.
hipError_t launch_gemv_fused(const WeightDev& w, const float* x, int64_t xs, int64_t m, float* y, int64_t ys,
                             const float* bias, hipStream_t s, const Workspace* ws = nullptr, int af = -1);
// K-ranges per row of the GEMV on this weight under activation format af (1: no
// split-K), and the bytes of row sums a pass of up to m_pass rows then needs (0 when
// it does not split). Both depend on the weight and the device only.
int gemv_splits(const WeightDev& w, int af);
size_t gemv_split_bytes(const WeightDev& w, int af, int64_t m_pass);
hipError_t launch_units(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int32_t* units,
                        int64_t nu, hipStream_t s);
// int8 MFMA GEMM (Q4_K x Q8_K). Returns hipErrorInvalidValue for an
// unsupported pair.
hipError_t launch_gemm(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0, int64_t n1,
                       float* y, int64_t ys, const float* bias, hipStream_t s);
bool gemm_supported(int dtype, int af);
// The Q4_K x Q8_K GEMM on the f16 matrix cores (dq_gemm_h16.hip): 128 x 256 tiles,
// activation codes as f16 in the "act16" layout of act16_bytes(m, k) bytes, written
// from Q8_K rows (launch_act16_from_q8k) or from fp32 rows with the Q8_K quantizer's
// arithmetic (launch_act16_quant). gemm_h16_pays: the shapes it is used for (its grid
// fills at least 5/8 of the CUs, and the offsets fit 32 bits).
int64_t act16_bytes(int64_t m, int64_t k);
bool gemm_h16_pays(const WeightDev& w, int64_t m, int64_t n0, int64_t n1);
hipError_t launch_act16_from_q8k(const uint8_t* acts, int64_t arb, int64_t m, int64_t k, uint8_t* out, hipStream_t s);
hipError_t launch_act16_quant(const float* x, int64_t x_stride, int64_t m, int64_t k, uint8_t* out, hipStream_t s);
hipError_t launch_gemm_h16(const WeightDev& w, const uint8_t* act16, int64_t m, int64_t n0, int64_t n1, float* y,
                           int64_t ys, const float* bias, hipStream_t s);

// Split K for the tolerance-parity GEMMs (per-32 and int16 rows, dq_gemm_p32.hip,
// dq_gemm_q16.hip, dq_gemm_q6x.hip): where a launch's tiles leave workgroup slots idle,
// each tile's super-blocks split into ranges (split_ranges: as many as fit one round of the
// slots -- one workgroup per CU, two for the 4-wave Q6_K GEMM -- at least 2 super-blocks
// each, at most 16); every range writes its partial tile to
// part[range][m][W] and launch_split_sum adds the ranges in order (+ bias) into y's
// [n0, n1), so the bits do not depend on timing.
inline int split_ranges(int64_t tiles, int slots, int64_t nblk) {
  if (tiles <= 0 || tiles >= slots) return 1;
  int64_t sp = slots / tiles;
  sp = sp < nblk / 2 ? sp : nblk / 2;
  sp = sp < 16 ? sp : 16;
  return sp > 1 ? (int)sp : 1;
}
hipError_t launch_split_sum(const float* part, int nsplit, int64_t m, int64_t W, int64_t nbase0, int64_t n0,
                            int64_t n1, float* y, int64_t ys, const float* bias, hipStream_t s);
// The Q4_K x per-32 GEMM on the f16 matrix cores (dq_gemm_p32.hip), qmm's int8 gemm
// contract: 128 x 256 tiles, codes as f16 in the "act32" layout of act32_bytes(m, k)
// bytes written from per-32 rows (launch_act32_from_p32). gemm_p32_ok: Q4_K and the
// offsets fit 32 bits.
int64_t act32_bytes(int64_t m, int64_t k);
bool gemm_p32_ok(const WeightDev& w, int64_t m, int64_t n0, int64_t n1);
hipError_t launch_act32_from_p32(const uint8_t* acts, int64_t arb, int64_t m, int64_t k, uint8_t* out, hipStream_t s);
int64_t p32_part_bytes(const WeightDev& w, int64_t m, int64_t n0, int64_t n1);
// fp32 rows -> act32 with the per-32 quantizer's arithmetic (the layout of
// launch_act32_from_p32 on the rows dq_act_quantize writes), in one launch
hipError_t launch_act32_quant(const float* x, int64_t x_stride, int64_t m, int64_t k, uint8_t* out, hipStream_t s);
hipError_t launch_gemm_p32(const WeightDev& w, const uint8_t* act32, int64_t m, int64_t n0, int64_t n1, float* y,
                           int64_t ys, const float* bias, float* part, hipStream_t s);
// The Q4_K x int16 GEMM on the f16 matrix cores (dq_gemm_q16.hip), the int16 contract
// (ActBlockQ16 rows, qmm's int16 mode): 64 x 256 tiles, codes split into lo and 256 hi
// as f16 in the "act16i" layout of act16i_bytes(m, k) bytes written from ActBlockQ16
// rows (launch_act16i_from_q16). gemm_q16_ok: Q4_K and the 32-bit offset limits.
int64_t act16i_bytes(int64_t m, int64_t k);
bool gemm_q16_ok(const WeightDev& w, int64_t m, int64_t n0, int64_t n1);
hipError_t launch_act16i_from_q16(const uint8_t* acts, int64_t arb, int64_t m, int64_t k, uint8_t* out,
                                  hipStream_t s);
int64_t q16_part_bytes(const WeightDev& w, int64_t m, int64_t n0, int64_t n1);
// fp32 rows -> act16i with the int16 quantizer's arithmetic, in one launch
hipError_t launch_act16i_quant(const float* x, int64_t x_stride, int64_t m, int64_t k, uint8_t* out,
                               hipStream_t s);
hipError_t launch_gemm_q16(const WeightDev& w, const uint8_t* act, int64_t m, int64_t n0, int64_t n1, float* y,
                           int64_t ys, const float* bias, float* part, hipStream_t s);
// The Q6_K GEMM on the f16 matrix cores (dq_gemm_q6x.hip) for per-32 rows (af =
// kActPer32) and int16 rows (kActQ16): launch_q6x_act writes the rows' operand layout
// (q6x_act_bytes: per-32 codes as f16, int16 codes biased to u16), launch_gemm_q6x runs
// 32- or 64-row x 128-row tiles over it. Where the tiles
// leave CUs idle, each tile's super-blocks split into ranges whose partial outputs go to
// part (q6x_part_bytes; 0: no split, part may be null) and a second launch adds them in
// range order. gemm_q6x_ok: Q6_K, one of those formats, 32-bit offsets.
int64_t q6x_act_bytes(int af, int64_t m, int64_t k);
int64_t q6x_part_bytes(const WeightDev& w, int64_t m, int64_t n0, int64_t n1);
bool gemm_q6x_ok(const WeightDev& w, int af, int64_t m, int64_t n0, int64_t n1);
hipError_t launch_q6x_act(int af, const uint8_t* acts, int64_t arb, int64_t m, int64_t k, uint8_t* out,
                          hipStream_t s);
// fp32 rows -> the same layout with the per-32 / int16 quantizer's arithmetic, in one launch
hipError_t launch_q6x_quant(int af, const float* x, int64_t x_stride, int64_t m, int64_t k, uint8_t* out,
                            hipStream_t s);
hipError_t launch_gemm_q6x(const WeightDev& w, int af, const uint8_t* act, int64_t m, int64_t n0, int64_t n1, float* y,
                           int64_t ys, const float* bias, float* part, hipStream_t s);
// The expand-class fp32 GEMM (dq_gemm_f32.hip): weight tiles expanded to fp32 in LDS
// and contracted with the fp32 rows x (stride xs floats) on the matrix cores; any of
// the four weight types. Below kF32GemmMinRows rows the fp32 GEMV passes are faster.
hipError_t launch_gemm_f32(const WeightDev& w, const float* x, int64_t xs, int64_t m, int64_t n0, int64_t n1, float* y,
                           int64_t ys, const float* bias, hipStream_t s);
constexpr int64_t kF32GemmMinRows = DQ_F32_GEMM_MIN_ROWS;
// The 32-value block GEMM (Q8_0 / Q4_0 x per-32 ActBlockQ8) that launch_gemm dispatches to.
hipError_t launch_gemm_b32(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0,
                           int64_t n1, float* y, int64_t ys, const float* bias, hipStream_t s);
bool gemm_b32_supported(int dtype, int af);
// Skinny MFMA GEMV on pre-quantized rows: Q4_K / Q6_K x Q8_K for 2 <= m <=
// kSkinnyMaxRows, and x sub-scaled (DQ_ACT_SX) for 2 <= m <= kSkinnySxMaxRows;
// hipErrorInvalidValue otherwise. ws (may be null): room for the t-terms of the split
// launch that long Q6_K rows on few 16-row tiles take at m <= 16 (skinny_split_bytes;
// without it they run unsplit, same results).
hipError_t launch_gemv_mma(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0,
                           int64_t n1, float* y, int64_t ys, const float* bias, hipStream_t s,
                           const Workspace* ws = nullptr);
// Bytes of that split launch's t-terms for these rows (0: the launch is not split).
int64_t skinny_split_bytes(const WeightDev& w, int af, int64_t m, int64_t n0, int64_t n1);
constexpr int64_t kSkinnyMaxRows = 64;
constexpr int64_t kSkinnySxMaxRows = 16;
// Whether m sub-scaled rows over rows [n0, n1) of w run faster on the skinny MFMA GEMV
// than on the VALU GEMV (the launch shapes where it was measured faster).
bool skinny_sx_pays(const WeightDev& w, int64_t m, int64_t n0, int64_t n1);
bool gemv_mma_supported(int dtype, int af, int64_t m);
// Whether the skinny kernel's LDS holds the t-terms of nblk super-blocks for m rows
// (gated: of two weights).
bool gemv_mma_lds_ok(int64_t nblk, int64_t m, bool gated = false);
// One matmul of a grouped skinny launch: y[r, i] (+ bias) for r < m, i < w->n, from
// either pre-quantized Q8_K rows (acts, arb bytes apart) or fp32 rows that the
// kernel quantizes (x != nullptr, xs floats apart). wu != nullptr: a gated job,
// y[r, i] = act(x . w^T) * (x . wu^T) with wu of w's type and shape and no bias.
struct GemvJob {
  const WeightDev* w;
  const uint8_t* acts;
  int64_t arb;
  const float* x;
  int64_t xs;
  int64_t m;
  float* y;
  int64_t ys;
  const float* bias;
  const WeightDev* wu = nullptr;
  int act = 0;
};
// Grouped skinny MFMA GEMV: jobs of one K (same nblk) and one input kind (all
// fused or none), Q4_K / Q6_K, 2 <= m <= 64 (fused: m <= 16), in launches of up to
// 8 jobs; hipErrorInvalidValue for any other job.
hipError_t launch_gemv_mma_many(const GemvJob* jobs, int count, hipStream_t s, const Workspace* ws = nullptr);
// Work of one grouped launch of these jobs (<= 8, one nblk) in wave-sized units
// (workgroups x super-blocks): each unit of a launch on fp32 rows quantizes 16
// activation rows of one super-block again, so the caller quantizes once instead
// when this is large. The in-kernel quantization lengthens every wave's critical
// path: at M = 16 a 1536 x 1536 Q4_K matmul (576 units) ran 7.8 us fused and
// 1.8 + 3.8 us as a quantize launch plus the GEMV, so only small launches fuse.
int64_t skinny_units(const GemvJob* jobs, int count);
constexpr int64_t kSkinnyFuseMaxUnits = 128;
// The gated M = 1 decode GEMV: y[i] = act(x . wg_i) * (x . wu_i) for one fp32 row x,
// K-quant weights of one type and shape, activations quantized in the kernel.
// hipErrorInvalidValue when the pair or its LDS is not supported.
bool gemv_gated_supported(const WeightDev& wg, const WeightDev& wu);
hipError_t launch_gemv_gated(const WeightDev& wg, const WeightDev& wu, int act, const float* x, float* y,
                             hipStream_t s);
// out[r, c] = act(g[r, c]) * u[r, c] for r < m, c < n (strides in floats).
hipError_t launch_act_mul(int act, const float* g, int64_t gs, const float* u, int64_t us, int64_t m, int64_t n,
                          float* out, int64_t os, hipStream_t s);

// Where one matmul keeps its temporaries (quantized activations at the start,
// split-K row sums after them): base == nullptr selects the library's per-device
// buffers (grown with hipMalloc, shared by the device's streams); otherwise the
// caller's device region of `bytes` bytes, and nothing is allocated.
struct Region {
  uint8_t* base = nullptr;
  size_t bytes = 0;
};

// The activations of the gated projection (dynacore Activation, device/ops.h:14);
// their device code is in dq_act.h.
enum { kActSilu = 0, kActGelu = 1, kActGeluTanh = 2 };
inline bool act_ok(int act) { return act == kActSilu || act == kActGelu || act == kActGeluTanh; }

}  // namespace dq

// The library's weight handle (include/dynaq.h).
struct dq_weight {
  dq::WeightDev dev;
};

namespace dq {
// Bytes of temporaries dq_matmul (fmt < 0) or dq_matmul_act (format fmt) needs for
// m rows of w in a fixed region: an upper bound over the routes either may take.
size_t matmul_scratch_bytes(const dq_weight* w, int fmt, int64_t m);
// dq_matmul / dq_matmul_act with their temporaries in r (arguments validated).
int matmul_impl(const dq_weight* w, const float* x, int64_t m, int64_t x_stride, float* y, int64_t y_stride,
                const float* bias, hipStream_t s, const Region& r);
int matmul_act_impl(const dq_weight* w, int fmt, const float* x, int64_t m, int64_t x_stride, float* y,
                    int64_t y_stride, const float* bias, hipStream_t s, const Region& r);
// KernelPlan::defaults() (without environment overrides) and select_matmul over this
// library's kernels (dq_plan.cpp).
dq_plan default_plan();
dq_selection select(const dq_matmul_shape& s, const dq_plan& p);
// Runs selection sel for m rows of w (arguments validated), temporaries in r.
int matmul_sel_impl(const dq_weight* w, const dq_selection& sel, const float* x, int64_t m, int64_t x_stride,
                    float* y, int64_t y_stride, const float* bias, hipStream_t s, const Region& r);
// Bytes of temporaries matmul_sel_impl needs for this selection in a fixed region.
size_t sel_scratch_bytes(const dq_weight* w, const dq_selection& sel, int64_t m);
}  // namespace dq
