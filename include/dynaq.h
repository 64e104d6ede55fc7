/*
 * dynaq.h -- C ABI of the MI355X block-quantized matmul library (libdynaq.so).
 *
 * y[m, n] = sum_k x[m, k] * w[n, k] (+ bias[n]) with w stored as GGUF blocks
 * (Q8_0, Q4_0, Q4_K, Q6_K) and x quantized to int8 blocks on the GPU, behind
 * the entry points dynacore's quantized matmul exposes:
 *   dynacore/include/dynacore/device/device.h:89,103-106,161   Device::upload,
 *       prepack_weight, matmul
 *   dynacore/include/dynacore/cpu/qmm.h:116-137                qmm::Kernels
 *       {quantize_row, gemv, gemm}
 *   dynacore/include/dynacore/cpu/cpu_kernels.h:39,53-54       QuantizeActFn,
 *       DotQ8RowsNFn
 *
 * Conventions (as the reference's, dynacore/include/dynacore/device/device.h:11-13
 * and qmm.h:35-36):
 *   - every pointer argument except host_rows of dq_weight_upload and
 *     dq_weight_download is device memory owned by the caller;
 *   - `stream` is a hipStream_t (NULL = the default stream); every call only
 *     enqueues work on it, except upload/download/free, which synchronize it;
 *   - calls return a dq_status (the values of dynacore's StatusCode,
 *     dynacore/include/dynacore/base/status.h:19-32); no exception crosses the
 *     ABI; dq_last_error() describes the last failure on the calling thread;
 *   - weight handles are library-owned; calls on one stream are ordered, and
 *     dq_matmul's activation scratch is per device (concurrent dq_matmul calls
 *     on one device from different streams race, like CpuDevice's scratch,
 *     dynacore/include/dynacore/cpu/cpu_device.h:106-118).
 */
#ifndef DYNAQ_H_
#define DYNAQ_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DQ_API __attribute__((visibility("default")))

/* dynacore::StatusCode (dynacore/include/dynacore/base/status.h:19-32). */
typedef enum dq_status {
  DQ_OK = 0,
  DQ_INVALID_ARGUMENT = 1,
  DQ_NOT_FOUND = 2,
  DQ_ALREADY_EXISTS = 3,
  DQ_OUT_OF_MEMORY = 4,
  DQ_RESOURCE_EXHAUSTED = 5,
  DQ_UNSUPPORTED = 6,
  DQ_IO_ERROR = 7,
  DQ_CORRUPT = 8,
  DQ_CANCELLED = 9,
  DQ_DEADLINE_EXCEEDED = 10,
  DQ_INTERNAL = 11,
} dq_status;

/* Weight block types: dynacore::DType values (dynacore/include/dynacore/tensor/dtype.h:19-44),
 * which are also GGUF's ggml_type ids' positions in dynacore's type table
 * (dynalm/src/loader/gguf/gguf.cpp:38-48 maps GGUF ids 2/8/12/14 onto them). */
typedef enum dq_dtype {
  DQ_Q4_0 = 6,
  DQ_Q8_0 = 10,
  DQ_Q4_K = 14,
  DQ_Q6_K = 16,
} dq_dtype;

/* Quantized activation formats (m rows of dq_act_row_bytes(fmt, k) bytes each):
 *   DQ_ACT_PER32  dynacore ActBlockQ8 {float d; int32 sum; int8 q[32]}, 40 B per 32 values,
 *                 d = amax/127, codes round half to even
 *                 (dynacore/include/dynacore/cpu/cpu_kernels.h:31-37,
 *                  dynacore/cpu/generic/kernels_generic.cpp:187-207);
 *   DQ_ACT_Q8_0   GGUF block_q8_0 {fp16 d; int8 q[32]}, 34 B per 32 values, codes
 *                 round half away from zero at the fp32 d
 *                 (dynacore/src/quantization/quant_formats.cpp:60-74);
 *   DQ_ACT_Q8_K   GGUF block_q8_K {float d; int8 q[256]; int16 bsums[16]}, 292 B per 256,
 *                 d = amax256/127, codes round half to even
 *                 (dynacore/include/dynacore/quantization/quant_formats.h:30,
 *                  dynacore/cpu/avx2/kernels_avx2.cpp:638-644);
 *   DQ_ACT_SX     dynacore ActSuperQ8 {int8 q[256]; float u; int16 m[8]; float ms[8];
 *                 int32 pad[3]}, 320 B per 256: sub-scaled activations (DD-077), dynacore's
 *                 validated default for K-quant decode rows on x86. u = amax256/(127*128),
 *                 per 32 values the smallest m in 1..128 with amax32 <= 127*u*m, codes round
 *                 half to even at u*m, ms = (u*m)*sum
 *                 (dynacore/include/dynacore/cpu/cpu_kernels.h:56-70,
 *                  dynacore/cpu/avx2/kernels_avx2.cpp:1077-1096). With Q4_K / Q6_K only; the
 *                 kernels form S = sum sc_j*m_j*P_j exactly (64 bits) and the mins term from
 *                 the integer m_j*sum_j;
 *   DQ_ACT_Q16    dynacore ActBlockQ16 {float d; int32 sum; int16 q[32]}, 72 B per 32 values:
 *                 int16 activations (DD-076), dynacore's contract for inputs with outlier
 *                 channels (the FFN down projection). d = amax32/32767, codes round half to
 *                 even (saturated to int16), sum = the sum of the codes
 *                 (dynacore/include/dynacore/cpu/cpu_kernels.h:72-82,
 *                  dynacore/cpu/avx2/kernels_avx2.cpp:1631-1652). With every weight type
 *                 (Q4_0 as qmm's int16 mode runs it, qmm_reference.cpp:68-93; the reference's
 *                 AVX2 int16 kernels cover Q8_0, Q4_K and Q6_K); the GEMV forms each
 *                 32-value (Q6_K: 16-value) integer dot exactly; Q4_K's GEMM (from 6
 *                 rows) and Q6_K's (from 5) split each code into lo and 256 hi on the
 *                 f16 matrix cores;
 *   DQ_ACT_F32    no quantization: fp32 rows of k floats (4k bytes), dynacore's kF32
 *                 contract (f32_row_dot, the reference-accuracy fallback and x86 prefill
 *                 default, dynacore/src/kernel/matmul_registry.cpp:51-54) with the arithmetic
 *                 of vec_dot_* (dynacore/cpu/generic/kernels_generic.cpp:67-150): each
 *                 block's fp32 dot in index order, scaled and added block by block. With
 *                 every weight type; dq_act_quantize copies the rows, there are no integer
 *                 partials. */
typedef enum dq_act_format {
  DQ_ACT_PER32 = 0,
  DQ_ACT_Q8_0 = 1,
  DQ_ACT_Q8_K = 2,
  DQ_ACT_SX = 3,
  DQ_ACT_Q16 = 4,
  DQ_ACT_F32 = 5,
} dq_act_format;

/* Activation rows at or below which dq_matmul runs the GEMV kernels. */
#define DQ_GEMV_MAX_ROWS 16

typedef struct dq_weight dq_weight;

DQ_API const char* dq_version(void);
/* Message of the last failing call on this thread ("" if none). */
DQ_API const char* dq_last_error(void);

/* Bytes of one GGUF row of k values of dtype (-1 if k is not a whole number of
 * blocks); dynacore dtype_row_bytes (dynacore/src/tensor/dtype.cpp:50-54). */
DQ_API int64_t dq_row_bytes(int dtype, int64_t k);
/* Bytes of one quantized activation row (-1 if unsupported or misaligned). */
DQ_API int64_t dq_act_row_bytes(int fmt, int64_t k);
/* The activation format dq_matmul uses for weights of dtype: DQ_ACT_PER32 for
 * Q8_0 / Q4_0, DQ_ACT_Q8_K for Q4_K / Q6_K. */
DQ_API int dq_act_format_for(int dtype);

/* Upload n GGUF rows of k values (row stride row_bytes >= dq_row_bytes(dtype, k))
 * from host memory and repack them into the GPU layout of the current device.
 * Replaces Device::upload + Device::prepack_weight
 * (dynacore/include/dynacore/device/device.h:89,103-106) and qmm::pack_groups
 * (dynacore/include/dynacore/cpu/qmm.h:109-114). Synchronizes `stream`. */
DQ_API int dq_weight_upload(int dtype, const void* host_rows, int64_t n, int64_t k, int64_t row_bytes, void* stream,
                            dq_weight** out);
/* The same from rows already in device memory (not modified, not retained). */
DQ_API int dq_weight_upload_device(int dtype, const void* dev_rows, int64_t n, int64_t k, int64_t row_bytes,
                                   void* stream, dq_weight** out);
/* Unpack the device copy back into GGUF rows in host memory (round-trip check). */
DQ_API int dq_weight_download(const dq_weight* w, void* host_rows, int64_t row_bytes, void* stream);
DQ_API int dq_weight_free(dq_weight* w);
DQ_API int dq_weight_info(const dq_weight* w, int* dtype, int64_t* n, int64_t* k, int64_t* device_bytes);

/* Quantize m rows of k fp32 values (row stride x_stride floats) into `out`
 * (m rows of dq_act_row_bytes(fmt, k) bytes). Replaces QuantizeActFn
 * (dynacore/include/dynacore/cpu/cpu_kernels.h:39) / qmm quantize_row
 * (dynacore/include/dynacore/cpu/qmm.h:122-123); bit-identical results. */
DQ_API int dq_act_quantize(int fmt, const float* x, int64_t m, int64_t k, int64_t x_stride, void* out, void* stream);

/* qmm's activation buffer: m rows of k values (k % 32 == 0) quantized per 32-value
 * block to int8 or int16 codes with d = amax / qmax and c = d * (code sum), in the row
 * layout (gemv) or the pair-interleaved layout (gemm; rows 2p and 2p + 1 in 8-byte
 * chunks, scales interleaved). Replaces qmm::ActBuffer (dynacore/include/dynacore/cpu/
 * qmm.h:57-93) and its tier's quantize_row (qmm.h:122-123; the reference tier,
 * dynacore/cpu/qmm/qmm_reference.cpp:25-51); bit-identical bytes. */
typedef enum dq_qmm_mode { /* qmm::ActMode (qmm.h:46) */
  DQ_QMM_INT8 = 0,
  DQ_QMM_INT16 = 1 /* q = 256 * hi + lo */
} dq_qmm_mode;
/* qmm::Acts (qmm.h:71-79); the pointers are device memory inside one buffer. */
typedef struct dq_qmm_acts {
  int32_t mode;
  int32_t paired;
  int64_t m, k;
  int8_t* hi;
  uint8_t* lo; /* DQ_QMM_INT16 only, else NULL */
  float* d;
  float* c;
  uint8_t* blocks; /* the m rows as DQ_ACT_PER32 (int8) / DQ_ACT_Q16 (int16) blocks, row layout */
} dq_qmm_acts;
/* Bytes ActBuffer::prepare lays out for the shape (qmm_reference.cpp:440-454): codes,
 * low bytes (int16), d and c, each region rounded up to 64 bytes, then (past the
 * reference's regions) the rows in the block format gemv / gemm read; -1 if invalid. */
DQ_API int64_t dq_qmm_act_bytes(int mode, int64_t m, int64_t k, int paired);
/* ActBuffer::prepare on a caller's device buffer (64-byte aligned, at least
 * dq_qmm_act_bytes): fills *out and, for a paired buffer of odd m, zeroes the pad
 * row's codes and scales on `stream` (qmm_reference.cpp:455-469). */
DQ_API int dq_qmm_act_prepare(void* base, int64_t bytes, int mode, int64_t m, int64_t k, int paired,
                              dq_qmm_acts* out, void* stream);
/* ActBuffer::quantize_rows (qmm_reference.cpp:472-488): rows [r0, r1) of x (row r at
 * x + r * x_stride floats, device memory) into a prepared buffer: the codes, d and c,
 * and the same rows in the blocks region. Disjoint row ranges may be quantized by
 * separate calls. */
DQ_API int dq_qmm_quantize_rows(const float* x, int64_t x_stride, int64_t r0, int64_t r1, const dq_qmm_acts* a,
                                void* stream);
/* qmm::Kernels::gemv (dynacore/include/dynacore/cpu/qmm.h:125-126): y[(r0 + r) * y_stride + n]
 * for r < rows and n in [n0, n1), from rows [r0, r0 + rows) of a qmm buffer in either
 * layout, + bias. The codes and d equal the per-32 (int8) / int16 block formats' (same
 * quantizer arithmetic), so this is dq_gemv on DQ_ACT_PER32 / DQ_ACT_Q16 rows: bit-identical
 * to it, within the fp32 tolerance of qmm's own order (qmm_reference.cpp:68-114). No
 * kGemvMaxRows limit. Reads the buffer's blocks region only (no library state, as the
 * reference's pure functions): calls on disjoint [n0, n1) ranges may run concurrently. */
DQ_API int dq_qmm_gemv(const dq_weight* w, int64_t n0, int64_t n1, const dq_qmm_acts* a, int64_t r0, int rows,
                       float* y, int64_t y_stride, const float* bias, void* stream);
/* qmm::Kernels::gemm (qmm.h:128-129): every row of the buffer (the reference expects the
 * pair layout; both are accepted), on the MFMA GEMM where the format has one (Q8_0 / Q4_0
 * per-32), else the GEMV passes. Reads the blocks region, as dq_qmm_gemv. */
DQ_API int dq_qmm_gemm(const dq_weight* w, int64_t n0, int64_t n1, const dq_qmm_acts* a, float* y, int64_t y_stride,
                       const float* bias, void* stream);

/* y[r * y_stride + i] = dot(weight row i, activation row r) + (bias ? bias[i] : 0)
 * for r < m and i in [n0, n1). `acts`: m rows in format fmt, as dq_act_quantize
 * writes them. Replaces qmm::Kernels::gemv (dynacore/include/dynacore/cpu/qmm.h:125-126)
 * and DotQ8RowsNFn (dynacore/include/dynacore/cpu/cpu_kernels.h:53-54).
 * Any m: the weights are streamed once per pass of up to 4 activation rows. */
DQ_API int dq_gemv(const dq_weight* w, int fmt, const void* acts, int64_t m, int64_t n0, int64_t n1, float* y,
                   int64_t y_stride, const float* bias, void* stream);
/* dq_gemm runs the prefill GEMMs on the matrix cores: Q4_K and Q6_K weights with
 * DQ_ACT_Q8_K activations (the super-block pair's canonical fp32 order, bit-identical to
 * dq_gemv), Q8_0 / Q4_0 weights with DQ_ACT_PER32 (each output in the reference's
 * generic per-32 block order, kernels_generic.cpp:216-239), and Q4_K and Q6_K weights
 * with DQ_ACT_PER32 or DQ_ACT_Q16 (f16 matrix-core GEMMs that sum in an order of their
 * own: within the fp32 tolerance of a K-term dot product of the reference's); other pairs
 * return DQ_UNSUPPORTED; any m.
 * Replaces qmm::Kernels::gemm (dynacore/include/dynacore/cpu/qmm.h:128-129). */
DQ_API int dq_gemm(const dq_weight* w, int fmt, const void* acts, int64_t m, int64_t n0, int64_t n1, float* y,
                   int64_t y_stride, const float* bias, void* stream);

/* y = x . w^T (+ bias): quantize x with dq_act_format_for(w), then GEMV or GEMM by
 * m (Q4_K: GEMM above DQ_GEMV_MAX_ROWS, or above 48 rows for weights of <= 4096 rows;
 * Q8_0 / Q4_0: GEMM from 13 rows; Q6_K: GEMM
 * above 64 rows, or above 16 for weights of >= 4096 rows or long K, except long rows on
 * weights of few rows, which run the 16-row skinny GEMV per 16 rows). Every route gives
 * the same bits. Replaces Device::matmul
 * (dynacore/include/dynacore/device/device.h:161; CpuDevice::matmul,
 * dynacore/cpu/cpu_device.cpp:869-1177). Uses a per-device scratch buffer. */
DQ_API int dq_matmul(const dq_weight* w, const float* x, int64_t m, int64_t x_stride, float* y, int64_t y_stride,
                     const float* bias, void* stream);

/* Bytes of the static device array dq_matmul_noalloc keeps its temporaries in (one per GPU). */
#define DQ_NOALLOC_SCRATCH_BYTES (16u << 20)

/* dq_matmul without any device allocation: the same kernels and bits as dq_matmul,
 * with the quantized activations and split-K row sums in a static device array of
 * DQ_NOALLOC_SCRATCH_BYTES per GPU instead of buffers grown with hipMalloc. No
 * counterpart in the reference; it is for callers that cannot allocate (code under
 * HIP graph capture, serving loops that forbid hipMalloc). Calls needing more
 * scratch than the array holds (Q4_K with K = 4096: more than 3,591 rows) return
 * DQ_RESOURCE_EXHAUSTED before launching anything. Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (unordered streams or threads) race. */
DQ_API int dq_matmul_noalloc(const dq_weight* w, const float* x, int64_t m, int64_t x_stride, float* y,
                             int64_t y_stride, const float* bias, void* stream);

/* y = x . w^T (+ bias) with the activations quantized to format fmt (the caller's
 * choice of dynacore's activation contract, which KernelPlan makes per matmul:
 * dynacore/include/dynacore/kernel/kernel_plan.h:50-92). One quantize launch into
 * the per-device scratch, then dq_gemv, or dq_gemm's kernel where it supports the pair
 * and is faster at this m: for DQ_ACT_PER32 / DQ_ACT_Q16 the f16 GEMMs take Q4_K from 5
 * rows and Q6_K from 3, their quantization writing the GEMM's operand layout directly;
 * below that, DQ_ACT_PER32 on Q4_K / Q6_K quantizes inside the GEMV launch (the same
 * bits as dq_act_quantize + dq_gemv). Replaces Device::matmul under a chosen contract. */
DQ_API int dq_matmul_act(const dq_weight* w, int fmt, const float* x, int64_t m, int64_t x_stride, float* y,
                         int64_t y_stride, const float* bias, void* stream);

/* One matmul of dq_matmul_many: y = x . w^T (+ bias) for m rows of x (x_stride
 * floats apart, w's k values each) into y (y_stride floats apart). The fields are
 * those of dynacore's Device::MatmulJob {x, w, y, bias}
 * (dynacore/include/dynacore/device/device.h:165-168), with the shapes spelled out. */
typedef struct dq_matmul_job {
  const dq_weight* w;
  const float* x;
  int64_t m;
  int64_t x_stride;
  float* y;
  int64_t y_stride;
  const float* bias; /* NULL or w's n floats */
} dq_matmul_job;

/* Several independent matmuls on one stream, e.g. the projections that share one
 * input (Q/K/V, gate/up) or the experts of an MoE layer. The decode-sized K-quant
 * jobs (Q4_K: 2 <= m <= 16; Q6_K: 2 <= m <= 64) of one k run together in grouped
 * skinny-GEMV launches (up to
 * 8 jobs each, Q4_K and Q6_K mixed) that quantize each job's fp32 rows in the
 * kernel; every other job runs as dq_matmul runs it. Each job's y is
 * bit-identical to dq_matmul on that job. Replaces Device::matmul_many
 * (dynacore/include/dynacore/device/device.h:169-171; CpuDevice::matmul_many,
 * dynacore/cpu/cpu_device.cpp:500-692, which quantizes a shared input once and
 * runs all jobs' row chunks in one parallel region). */
DQ_API int dq_matmul_many(const dq_matmul_job* jobs, int64_t n_jobs, void* stream);

/* Activations of the gated MLP projection: dynacore::Activation
 * (dynacore/include/dynacore/device/ops.h:14), with the reference's fp32 formulas
 * (dynacore/cpu/cpu_device.cpp:117-134): SiLU x / (1 + e^-x) through exp_nonpos
 * (dynacore/include/dynacore/base/fast_exp.h:16-35), bit-identical to the
 * reference; GELU 0.5 x (1 + erf(x / sqrt 2)) and its tanh form, within a few ulp
 * of the reference (device erff / tanhf). */
typedef enum dq_activation {
  DQ_SILU = 0,
  DQ_GELU = 1,
  DQ_GELU_TANH = 2,
} dq_activation;

/* out[r * out_stride + c] = act(gate[r * gate_stride + c]) * up[r * up_stride + c]
 * for r < m, c < n (fp32). Replaces Device::act_mul
 * (dynacore/include/dynacore/device/device.h:186-187; CpuDevice::act_mul,
 * dynacore/cpu/cpu_device.cpp:1912-1930). out may alias gate or up. */
DQ_API int dq_act_mul(int act, const float* gate, int64_t gate_stride, const float* up, int64_t up_stride, int64_t m,
                      int64_t n, float* out, int64_t out_stride, void* stream);

/* out = act(x . w_gate^T) * (x . w_up^T): the gated MLP projection (SwiGLU /
 * GeGLU) of m rows of x (x_stride floats apart, k values each); w_gate and w_up
 * have the same n and k; out has out_stride floats per row; no bias. Replaces
 * Device::matmul_gated (dynacore/include/dynacore/device/device.h:188-199;
 * CpuDevice::matmul_gated, dynacore/cpu/cpu_device.cpp:1931-2072).
 *   - Q4_K weights with m <= 16, or Q6_K weights with m <= 64 (of one type): one
 *     fused launch that streams both
 *     weights and writes only act(g) * u (no gate / up round trip);
 *   - otherwise both projections as dq_matmul computes them, into gate_scratch and
 *     up_scratch (m rows of scratch_stride floats each, clobbered), then dq_act_mul.
 *     NULL scratch pointers (both) select a per-device library buffer.
 * Every path gives the bits of act(dq_matmul(x, w_gate)) * dq_matmul(x, w_up). */
DQ_API int dq_matmul_gated(int act, const float* x, int64_t m, int64_t x_stride, const dq_weight* w_gate,
                           const dq_weight* w_up, float* out, int64_t out_stride, float* gate_scratch,
                           float* up_scratch, int64_t scratch_stride, void* stream);

/* ---- accuracy classes: dynacore's KernelPlan and select_matmul -----------
 * Which activation contract a matmul runs under is dynacore's per-call kernel
 * selection (select_matmul, dynacore/src/kernel/matmul_registry.cpp:94-191,287-429)
 * from the step's KernelPlan (dynacore/include/dynacore/kernel/kernel_plan.h:29-192).
 * dq_select restates it for this library's kernels and dq_matmul_plan runs the
 * result; under the default plan a Q4_K / Q6_K decode row is sub-scaled int8
 * (validated), Q8_0 / Q4_0 up to 4 rows per-32 int8, larger batches fp32, and the
 * super-block (Q8_K) class that dq_matmul runs is opt-in, as in the reference. */

/* MatmulShape (dynacore/include/dynacore/kernel/matmul_registry.h:87-91). */
typedef struct dq_matmul_shape {
  int64_t m, n, k;
  int32_t dtype;
  int32_t x_dense; /* x rows are contiguous (row stride == k floats) */
} dq_matmul_shape;

/* The kernels: dynacore::MatmulKernelId values (dynacore/include/dynacore/kernel/
 * matmul_registry.h:33-51) of the ones this library implements on the GPU; the
 * others (interleaved-copy, SME, external) do not exist here. */
typedef enum dq_kernel {
  DQ_KERNEL_QMM_GEMM = 1,         /* kQmmGemm: qmm's gemm, DQ_ACT_PER32 / DQ_ACT_Q16 (validated classes) */
  DQ_KERNEL_QMM_GEMV = 2,         /* kQmmGemv: qmm's gemv, DQ_ACT_PER32 / DQ_ACT_Q16 */
  DQ_KERNEL_INT8_SUBSCALED = 7,   /* kInt8Subscaled: DQ_ACT_SX, K-quants (validated, DD-077) */
  DQ_KERNEL_INT8_SUPERBLOCK = 8,  /* kInt8Superblock: DQ_ACT_Q8_K, K-quants (fails DD-053: opt-in) */
  DQ_KERNEL_INT8_PER32 = 9,       /* kInt8Per32: DQ_ACT_PER32 (validated, DD-053) */
  DQ_KERNEL_INT16_ROWS = 13,      /* kInt16Rows: DQ_ACT_Q16, every weight type (validated, DD-076) */
  DQ_KERNEL_F32_EXPAND_GEMM = 14, /* kF32ExpandGemm: fp32 activations, dense x (reference class) */
  DQ_KERNEL_F32_ROW_DOT = 15,     /* kF32RowDot: fp32 activations (reference class) */
} dq_kernel;

/* DQ_KERNEL_F32_EXPAND_GEMM runs on the matrix cores from this many rows on: weight
 * tiles expanded to fp32 as the reference's x86 expansion does (one fma per value),
 * contracted with the fp32 rows on v_mfma_f32 (sums in the matrix cores' order, within
 * 1e-5 of sum |x_k w_k|; a row's outputs do not depend on the other rows). Fewer rows
 * run the fp32 row-dot GEMV, the same class in vec_dot order. */
#define DQ_F32_GEMM_MIN_ROWS 16

/* The matmul knobs of KernelPlan that choose among these kernels, with the
 * reference's meaning and names (kernel_plan.h:34-92,156-160); matmul_disabled is a
 * mask of (1u << dq_kernel), as KernelPlan::matmul_disabled (kernel_plan.h:144-148);
 * qmm != 0 lets the native qmm kernels take every matmul whose op allows int8 (int16)
 * activations, qmm_gemm_min_rows the rows from which qmm's gemm replaces its gemv. A
 * plan with qmm 0 selects as on a backend without qmm (the reference's x86 tiers). */
typedef struct dq_plan {
  int32_t expand_min_rows;
  int32_t int8_decode_max_rows;
  int32_t int16_decode_max_rows;
  int32_t int8_superblock_min_rows;
  int32_t int8_superblock_max_rows;
  int32_t int8_subscale_min_rows;
  uint32_t matmul_disabled;
  int32_t qmm;
  int32_t qmm_gemm_min_rows;
} dq_plan;

/* A selection: the kernel and the activation format it quantizes x to (DQ_ACT_F32
 * for the fp32 kernels), as MatmulSelection {id, act} (matmul_registry.h:143-151). */
typedef struct dq_selection {
  int32_t kernel;
  int32_t act;
} dq_selection;

/* KernelPlan::defaults() without its environment overrides (kernel_plan.cpp:22-90):
 * expand 2, int8 decode 4 rows, int16 0, super-block off (min 0, max 8), sub-scaled
 * from 1 row, nothing disabled, qmm on with its gemm from 9 rows. (The engine raises
 * int8_decode_max_rows to 2^30 on a backend whose qmm kernels are accelerated,
 * dynalm/src/runtime/engine.cpp:365-375, as this one is.) */
DQ_API int dq_plan_defaults(dq_plan* out);
/* The plan the model uses for the FFN down projection (dynalm/src/model/
 * transformer.cpp:541-550, with int8_ffn_down off and int16_ffn_down on): no int8
 * activations; int16 for up to max(int8_decode_max_rows, int8_superblock_max_rows)
 * rows while int8 decode is on. */
DQ_API int dq_plan_ffn_down(const dq_plan* base, dq_plan* out);
/* select_matmul (dynacore/src/kernel/matmul_registry.cpp:287-429) over this
 * library's kernels, with the MatmulCaps of this GPU: qmm int8 and int16 activations
 * for every weight type and a qmm gemm for Q8_0, Q4_0 and Q4_K; the int8 per-32,
 * super-block and sub-scaled row dots; int16 row dots for every weight type; no
 * interleaved copies, SME or external kernels. plan NULL: the defaults. A pure
 * function; needs no GPU. DQ_INVALID_ARGUMENT for shapes validate_matmul_shape
 * rejects. */
DQ_API int dq_select(const dq_matmul_shape* s, const dq_plan* plan, dq_selection* out);
/* y = x . w^T (+ bias) under the kernel dq_select picks for this call (plan NULL:
 * the defaults): Device::matmul with the step's KernelPlan (device.h:95,161).
 * dq_matmul is this call under the all-integer plan {int8_decode_max_rows and
 * int8_superblock_max_rows unbounded, int8_superblock_min_rows 1,
 * int8_subscale_min_rows 0, qmm 0}. */
DQ_API int dq_matmul_plan(const dq_weight* w, const dq_plan* plan, const float* x, int64_t m, int64_t x_stride,
                          float* y, int64_t y_stride, const float* bias, void* stream);

/* ---- GGUF files ----------------------------------------------------------
 * A GGUF v2 / v3 model mapped read-only (mmap): header, metadata and tensor
 * directory parsed with every length and offset checked against the file
 * (dynalm/src/loader/gguf/gguf.h:65-125, gguf.cpp:248-343). Opening the first part
 * of a split model (NAME-00001-of-0000N.gguf) opens all its parts
 * (dynalm/src/loader/gguf/gguf_model.cpp:291-331); metadata is the first part's.
 * Status codes: DQ_NOT_FOUND / DQ_IO_ERROR for files that cannot be opened,
 * DQ_CORRUPT for malformed contents, DQ_UNSUPPORTED for other versions and
 * unknown tensor types. */
typedef struct dq_gguf dq_gguf;

/* One tensor of the directory (TensorInfo, gguf.h:65-72). dims are in engine order,
 * outermost first (a weight of n rows of k values: dims {n, k}); dtype is the
 * dq_dtype of the four weight types, else -1; data points into the mapping and
 * stays valid until dq_gguf_close. */
typedef struct dq_gguf_tensor {
  const char* name;
  uint32_t ggml_type;
  int32_t dtype;
  int32_t n_dims;
  int64_t dims[4];
  uint64_t offset; /* absolute, in its part */
  uint64_t nbytes;
  int32_t part;
  const void* data;
} dq_gguf_tensor;

DQ_API int dq_gguf_open(const char* path, dq_gguf** out);
DQ_API int dq_gguf_close(dq_gguf* g);
DQ_API int dq_gguf_info(const dq_gguf* g, uint32_t* version, uint64_t* alignment, int64_t* n_tensors,
                        int64_t* n_parts);
/* Index of the tensor called name, or -1 (GgufFile::find_tensor). */
DQ_API int64_t dq_gguf_find_tensor(const dq_gguf* g, const char* name);
DQ_API int dq_gguf_tensor_info(const dq_gguf* g, int64_t i, dq_gguf_tensor* out);
/* Metadata getters (GgufFile::get_uint / get_string, gguf.h:93,97): integers of any
 * width that are >= 0; strings as (pointer into the mapping, length). */
DQ_API int dq_gguf_get_uint(const dq_gguf* g, const char* key, uint64_t* out);
DQ_API int dq_gguf_get_string(const dq_gguf* g, const char* key, const char** str, int64_t* len);
/* Upload tensor i (Q4_0 / Q8_0 / Q4_K / Q6_K, two or more dims; the outer dims are
 * its rows) from the mapping into a device weight, as dq_weight_upload does
 * (Device::upload of GgufFile::load_tensor's view, gguf.cpp:457-466). */
DQ_API int dq_gguf_upload_weight(const dq_gguf* g, int64_t i, void* stream, dq_weight** out);

/* ---- host-memory adapter ------------------------------------------------
 * The shape of dynacore's run-time extension point ExternalMatmulKernel
 * {name, eligible(const MatmulShape&, const void* weight), run(x, w, bias*, y)}
 * (dynacore/include/dynacore/cpu/cpu_device.h:22-30), which CpuDevice consults
 * before its built-in kernels (dynacore/cpu/cpu_device.cpp:810-826,909-911), for
 * an engine whose tensors live in host memory. A dq_external keeps one device copy
 * per weight it is given, keyed by the weight's host address, type, shape and row
 * stride (as CpuDevice keys its packed copies by data pointer and (n, k),
 * dynacore/include/dynacore/cpu/cpu_device.h:135-143), dropping the least recently
 * used copies beyond max_resident_bytes (0: no limit). A weight's host rows must
 * not change while a copy of them is kept (dq_external_forget drops it). Calls on
 * one dq_external are serialized. run() selects its kernel as dq_matmul_plan does,
 * under the adapter's plan (dq_external_set_plan; dynacore's defaults at creation,
 * so the accuracy class is the reference's), and its results are dq_matmul_plan's
 * on the same rows. Each adapter keeps its own device scratch: adapters on one GPU
 * do not share temporaries. */
typedef struct dq_external dq_external;

typedef struct dq_external_stats {
  int64_t runs;             /* completed dq_external_run calls */
  int64_t uploads;          /* weights copied to the device */
  int64_t hits;             /* runs that found their weight's copy */
  int64_t evictions;        /* copies dropped for the byte limit */
  int64_t resident_bytes;   /* device bytes of the copies kept now */
  int64_t resident_weights; /* copies kept now */
} dq_external_stats;

/* An adapter on GPU `device` whose eligible() accepts m >= min_rows (>= 1). */
DQ_API int dq_external_create(int device, int64_t min_rows, int64_t max_resident_bytes, dq_external** out);
DQ_API int dq_external_free(dq_external* e);
/* 1 if run() takes this shape, else 0; reads no tensor data and needs no GPU
 * (e may be NULL: min_rows 1). The rules are dq_matmul's (validate_matmul_shape,
 * dynacore/src/kernel/matmul_registry.cpp:264-278) for the four weight types. */
DQ_API int dq_external_eligible(const dq_external* e, const dq_matmul_shape* s, const void* weight);
/* y[r, i] = x[r, :] . w[i, :] (+ bias[i]) for host x (m rows, x_stride floats apart),
 * host GGUF weight rows w (n rows of k values, w_row_bytes apart), host bias (n
 * floats or NULL) and host y (m rows, y_stride floats apart). Returns when y is
 * written. */
DQ_API int dq_external_run(dq_external* e, const float* x, int64_t m, int64_t x_stride, const void* w, int dtype,
                           int64_t n, int64_t k, int64_t w_row_bytes, const float* bias, float* y, int64_t y_stride);
/* Drops the device copies of host weight rows `weight` (DQ_NOT_FOUND if none). */
DQ_API int dq_external_forget(dq_external* e, const void* weight);
DQ_API int dq_external_get_stats(dq_external* e, dq_external_stats* out);
/* The plan run() selects kernels with, as Device::set_kernel_plan (dynacore/include/
 * dynacore/device/device.h:95): an engine calls it where it sets the device's plan
 * (per step, and around the FFN down projection, transformer.cpp:538-550). A new
 * adapter starts with dq_plan_defaults. NULL: the defaults. */
DQ_API int dq_external_set_plan(dq_external* e, const dq_plan* plan);

/* Exact integer partials of every (activation row r < m, weight row i < n):
 * units[(r * n + i) * U + u] and sb[(r * n + i) * S + s], with U and S from
 * dq_partials_count; the meaning of each is that of the CPU reference's integer
 * sums (dynacore/cpu/generic/kernels_generic.cpp:210-310,
 * dynacore/cpu/avx2/kernels_avx2.cpp:976-1058). The super-block terms come from
 * the GEMV kernel's own exact reductions. sb may be NULL when S == 0. */
DQ_API int dq_partials_count(int dtype, int fmt, int64_t k, int64_t* units, int64_t* sb_terms);
DQ_API int dq_debug_partials(const dq_weight* w, int fmt, const void* acts, int64_t m, int32_t* units, int32_t* sb,
                             void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DYNAQ_H_ */
