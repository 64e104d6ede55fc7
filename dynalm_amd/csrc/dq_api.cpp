// dq_api.cpp -- the C ABI of libdynaq.so (declared in include/dynaq.h).
//
// Host-side C++: argument validation with dynacore's status codes
// (dynacore/include/dynacore/base/status.h:19-32; shape rules of
// validate_matmul_shape, dynacore/src/kernel/matmul_registry.cpp:264-278),
// weight handles, the per-device activation scratch of dq_matmul, and dispatch
// by M (GEMV up to DQ_GEMV_MAX_ROWS rows, as KernelPlan's decode row limit
// selects the decode kernels, dynacore/src/kernel/matmul_registry.cpp:287-429).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/dynaq.h"
#include "dq_internal.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

}  // namespace

int dq::set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

namespace {

int hip_fail(hipError_t e, const char* what) {
  const int code = e == hipErrorOutOfMemory ? DQ_OUT_OF_MEMORY : DQ_INTERNAL;
  return fail(code, "%s: %s", what, hipGetErrorString(e));
}

#define DQ_HIP(call, what)                        \
  do {                                            \
    const hipError_t e_ = (call);                 \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

bool weight_type_ok(int t) { return t == DQ_Q4_0 || t == DQ_Q8_0 || t == DQ_Q4_K || t == DQ_Q6_K; }
bool act_fmt_ok(int f) {
  return f == DQ_ACT_PER32 || f == DQ_ACT_Q8_0 || f == DQ_ACT_Q8_K || f == DQ_ACT_SX || f == DQ_ACT_Q16 ||
         f == DQ_ACT_F32;
}

// The (weight, activation) pairs with kernels: the per-32 formats with Q8_0 / Q4_0
// (dynacore's kInt8Per32 contract); Q8_K, sub-scaled and per-32 with the K-quants;
// int16 with Q8_0, Q4_K and Q6_K (the types dynacore has int16 kernels for,
// dynacore/cpu/avx2/kernels_avx2.cpp:1957-1960).
bool pair_ok(int t, int f) {
  if (f == DQ_ACT_F32) return true;  // every weight type has an fp32 row kernel (vec_dot_*)
  if (f == DQ_ACT_Q16) return true;  // the int16 GEMV takes every weight type
  if (t == DQ_Q8_0 || t == DQ_Q4_0) return f == DQ_ACT_PER32 || f == DQ_ACT_Q8_0;
  return f == DQ_ACT_Q8_K || f == DQ_ACT_SX || f == DQ_ACT_PER32;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// Per-device scratch buffers (grow, never shrink): g_scratch holds dq_matmul's
// quantized activations (and split-K row sums after them when a region is carved
// from it), g_fscratch the fp32 gate / up projections of dq_matmul_gated's unfused
// path (which runs dq_matmul, so the two must differ). A pool is shared by every
// stream of its device: growing it waits for the whole device before the old buffer
// is freed, since a launch on another stream may still read it.
struct Scratch {
  std::mutex mu;
  std::vector<void*> ptr;
  std::vector<size_t> bytes;
};
Scratch g_scratch;
Scratch g_fscratch;

int scratch_get(Scratch& pool, int device, size_t need, void** out) {
  std::lock_guard<std::mutex> lock(pool.mu);
  if ((int)pool.ptr.size() <= device) {
    pool.ptr.resize(device + 1, nullptr);
    pool.bytes.resize(device + 1, 0);
  }
  if (pool.bytes[device] < need) {
    dq::DeviceScope ds(device);
    DQ_HIP(ds.err, "hipSetDevice");
    if (pool.ptr[device] != nullptr) {
      DQ_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
      DQ_HIP(hipFree(pool.ptr[device]), "hipFree");
      pool.ptr[device] = nullptr;
      pool.bytes[device] = 0;
    }
    size_t sz = need < (1u << 20) ? (1u << 20) : need;
    DQ_HIP(hipMalloc(&pool.ptr[device], sz), "hipMalloc(scratch)");
    pool.bytes[device] = sz;
  }
  *out = pool.ptr[device];
  return DQ_OK;
}
int scratch_get(int device, size_t need, void** out) { return scratch_get(g_scratch, device, need, out); }

constexpr size_t round256(size_t b) { return (b + 255) / 256 * 256; }

// Rows from which dq_matmul_act runs the f16 GEMMs (split K where their tiles leave CUs
// idle; one 32-row activation tile per workgroup up to 32 rows) instead of the GEMV
// passes, which read the weight once per pass of up to 4 rows. Measured per call, fp32
// rows in (graph replay; GEMV route / GEMM route, the latter's quantization fused into
// the operand layout):
//  - Q4_K x int16 (dq_gemm_q16.hip): 5 rows 27.8 / 24.3 us at K = 4096, N = 14336,
//    25.1 / 16.3 at N = 4096, 36.8 / 26.3 at K = 14336, N = 4096; at 4 rows mixed
//    (20.6 / 24.5, 17.6 / 15.7, 26.0 / 24.9);
//  - Q4_K x per-32 (dq_gemm_p32.hip): 5 rows 22.5 / 21.2, 18.5 / 13.2, 32.6 / 21.5;
//    4 rows 15.8 / 21.0, 13.4 / 14.5, 21.2 / 21.7; 10 rows 50.5 / 21.5 at K = 14336;
//  - Q6_K x per-32 / int16 (dq_gemm_q6x.hip): 3 rows per-32 24.6 / 23.8 at K = 14336,
//    N = 4096, 16.2 / 12.6 at K = 4096, N = 4096, 15.5 / 11.7 at N = 1024; int16 26.2 /
//    26.7, 17.2 / 13.9, 16.3 / 12.8; 2 rows 20.9 / 23.8 at K = 14336.
constexpr int64_t kQ16GemmMinRows = 5;
constexpr int64_t kP32GemmMinRows = 5;
constexpr int64_t kQ6xGemmMinRows = 3;

// Per-(device, stream) workspaces of the public entry points whose kernels need device
// memory beyond their arguments (dq_gemm's f16 activation operands). Each stream has
// its own buffer, so calls on different streams do not share one; the pool lock is
// held until the caller has enqueued the launches that use the buffer, so a call on
// the same stream from another thread cannot grow (free) it before they are queued,
// and launches on one stream run in order. Growing synchronizes that stream first.
struct StreamWs {
  int device;
  void* stream;
  void* p;
  size_t bytes;
};
std::mutex g_sws_mu;
std::vector<StreamWs> g_sws;

template <class F>
int with_stream_ws(int device, void* stream, size_t need, F&& fn) {
  std::lock_guard<std::mutex> lock(g_sws_mu);
  StreamWs* e = nullptr;
  for (StreamWs& x : g_sws)
    if (x.device == device && x.stream == stream) e = &x;
  if (e == nullptr) {
    g_sws.push_back(StreamWs{device, stream, nullptr, 0});
    e = &g_sws.back();
  }
  if (e->bytes < need) {
    dq::DeviceScope ds(device);
    DQ_HIP(ds.err, "hipSetDevice");
    if (e->p != nullptr) {
      DQ_HIP(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
      DQ_HIP(hipFree(e->p), "hipFree");
      e->p = nullptr;
      e->bytes = 0;
    }
    const size_t sz = need < (1u << 20) ? (1u << 20) : need;
    DQ_HIP(hipMalloc(&e->p, sz), "hipMalloc(stream workspace)");
    e->bytes = sz;
  }
  return fn(static_cast<uint8_t*>(e->p));
}

// The quantized-activation buffer of one matmul: the start of the caller's region,
// or the per-device pool.
int acts_buffer(int device, size_t need, const dq::Region& r, void** out) {
  if (r.base == nullptr) return scratch_get(device, need, out);
  if (need > r.bytes) {
    return fail(DQ_RESOURCE_EXHAUSTED, "activations need %zu bytes of scratch, the region holds %zu", need, r.bytes);
  }
  *out = r.base;
  return DQ_OK;
}

// The split-K workspace after `used` bytes of the caller's region (none: the GEMV's
// own per-device buffer).
dq::Workspace split_ws(const dq::Region& r, size_t used) {
  dq::Workspace ws;
  if (r.base != nullptr) {
    const size_t off = round256(used);
    ws.p = r.base + (off < r.bytes ? off : r.bytes);
    ws.bytes = off < r.bytes ? r.bytes - off : 0;
  }
  return ws;
}

int validate_shape(int dtype, int64_t n, int64_t k) {
  if (!weight_type_ok(dtype)) return fail(DQ_UNSUPPORTED, "weight type %d is not supported", dtype);
  if (n <= 0 || k <= 0) return fail(DQ_INVALID_ARGUMENT, "weight dims must be positive (n %lld, k %lld)", (long long)n, (long long)k);
  const int be = dq::block_elems(dtype);
  if (k % be != 0) {
    return fail(DQ_INVALID_ARGUMENT, "k %lld is not a multiple of the block (%d)", (long long)k, be);
  }
  // Buffer resources address a plane of one 64-row group with 32-bit offsets.
  if ((k / be) * dq::kRowGroup * 128 >= (int64_t)1 << 31) return fail(DQ_UNSUPPORTED, "k %lld is too large", (long long)k);
  return DQ_OK;
}

int upload_impl(int dtype, const void* rows, bool host, int64_t n, int64_t k, int64_t row_bytes, void* stream,
                dq_weight** out) {
  if (out == nullptr || rows == nullptr) return fail(DQ_INVALID_ARGUMENT, "null argument");
  *out = nullptr;
  if (int rc = validate_shape(dtype, n, k); rc != DQ_OK) return rc;
  const int64_t rb = dq_row_bytes(dtype, k);
  if (row_bytes < rb) return fail(DQ_INVALID_ARGUMENT, "row_bytes %lld < %lld", (long long)row_bytes, (long long)rb);
  hipStream_t s = as_stream(stream);
  auto* w = new (std::nothrow) dq_weight();
  if (w == nullptr) return fail(DQ_OUT_OF_MEMORY, "host allocation failed");
  dq::WeightDev& d = w->dev;
  d.dtype = dtype;
  d.n = n;
  d.k = k;
  d.n_pad = (n + dq::kRowGroup - 1) / dq::kRowGroup * dq::kRowGroup;
  d.nblk = k / dq::block_elems(dtype);
  hipError_t e = hipGetDevice(&d.device);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, d.device);
  int rc = DQ_OK;
  const uint8_t* src = static_cast<const uint8_t*>(rows);
  void* staging = nullptr;
  for (int p = 0; p < dq::num_planes(dtype) && e == hipSuccess; ++p) {
    d.plane_bytes[p] = d.n_pad * d.nblk * dq::plane_unit(dtype, p);
    e = hipMalloc(reinterpret_cast<void**>(&d.plane[p]), (size_t)d.plane_bytes[p]);
    if (e == hipSuccess) e = hipMemsetAsync(d.plane[p], 0, (size_t)d.plane_bytes[p], s);
  }
  if (e == hipSuccess && host) {
    e = hipMalloc(&staging, (size_t)(n * row_bytes));
    if (e == hipSuccess) e = hipMemcpyAsync(staging, rows, (size_t)(n * row_bytes), hipMemcpyHostToDevice, s);
    src = static_cast<const uint8_t*>(staging);
  }
  if (e == hipSuccess) e = dq::launch_repack(dtype, src, row_bytes, n, d.nblk, d.plane, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (staging != nullptr) {
    const hipError_t ef = hipFree(staging);
    if (e == hipSuccess) e = ef;
  }
  if (e != hipSuccess) {
    rc = hip_fail(e, "weight upload");
    for (int p = 0; p < dq::kMaxPlanes; ++p)
      if (d.plane[p]) (void)hipFree(d.plane[p]);  // already failing: the first error is reported
    delete w;
    return rc;
  }
  *out = w;
  return DQ_OK;
}

int check_acts(const dq_weight* w, int fmt, const void* acts, int64_t m) {
  if (w == nullptr || acts == nullptr) return fail(DQ_INVALID_ARGUMENT, "null argument");
  if (!act_fmt_ok(fmt)) return fail(DQ_UNSUPPORTED, "activation format %d is not supported", fmt);
  if (!pair_ok(w->dev.dtype, fmt)) {
    return fail(DQ_UNSUPPORTED, "activation format %d is not supported with weight type %d", fmt, w->dev.dtype);
  }
  if (m < 0) return fail(DQ_INVALID_ARGUMENT, "m must be >= 0");
  if (dq_act_row_bytes(fmt, w->dev.k) < 0) {
    return fail(DQ_INVALID_ARGUMENT, "k %lld is not a multiple of the activation block", (long long)w->dev.k);
  }
  if (m * dq_act_row_bytes(fmt, w->dev.k) >= ((int64_t)1 << 32)) return fail(DQ_UNSUPPORTED, "activations exceed 4 GiB");
  return DQ_OK;
}

int check_out(const dq_weight* w, int64_t m, int64_t n0, int64_t n1, float* y, int64_t y_stride) {
  if (y == nullptr && m > 0) return fail(DQ_INVALID_ARGUMENT, "null output");
  if (n0 < 0 || n1 > w->dev.n || n0 > n1) {
    return fail(DQ_INVALID_ARGUMENT, "row range [%lld, %lld) outside [0, %lld)", (long long)n0, (long long)n1,
                (long long)w->dev.n);
  }
  if (m > 1 && y_stride < n1) return fail(DQ_INVALID_ARGUMENT, "y_stride %lld < n1 %lld", (long long)y_stride, (long long)n1);
  return DQ_OK;
}

// The skinny path from fp32 rows: K-quant weights, 2 <= m <= 64 (m <= DQ_GEMV_MAX_ROWS
// where the pair has a GEMM, which is faster above that: 21-23 us against 31-43 us
// for 24..64 rows at K=4096, N=14336), LDS for the weight's super-blocks, and fp32
// rows addressable with 32-bit offsets.
// Whether dq_matmul / dq_matmul_act run m rows of this pair on a GEMM: above
// DQ_GEMV_MAX_ROWS for Q4_K x Q8_K, except up to 48 rows of weights with at most 4096
// rows where the skinny GEMV's LDS holds the row (its 64-row tiles beat the GEMM's few
// workgroups there: 9.4-11.1 vs 11.8-12.2 us at K = N = 4096, 19.0-20.3 vs 22.7-23.1 at
// K = 8960, N = 1536; at N = 14336 the GEMM wins, 16.1 vs 25.2 us at 17 rows); from 13 rows for the 32-value block GEMM (Q8_0 /
// Q4_0 x per-32; dq_matmul measured at K = 4096, N = 4096 / 14336, quantization
// included: GEMV passes 27.9 / 30.9 us at 12 rows, 35.7 / 36.6 at 13, 41.5 / 43.8 at
// 18; quantize + GEMM 26.9 / 32.7 at 13, 27.0 / 32.4 at 18; at K = 14336 the two are
// equal at 13 rows, 81.7 vs 82.8 us); Q6_K x Q8_K above 64 rows, and above
// 16 where the skinny GEMV's LDS does not hold the row's super-blocks (K = 14336:
// 110 us against 171-611 us for the VALU GEMV's passes at 17..64 rows; but see
// skinny_passes16) or the weight has 4096 rows or more (the
// GEMM's grid fills the CUs: 35 vs 45 us at K = 4096, N = 14336; with N = 1536 it
// loses, 70 vs 23 us).
// K-quant x Q8_K rows too long for the 64-row skinny tiles' LDS: the 16-row skinny launch
// per 16 rows (one read of the weight each) instead of the GEMM where that is faster.
// Graph replay, quantization included, K = 14336:
//  - Q6_K, while the passes read the weight fewer than ~4 times over 4096 rows: N = 4096 at
//    24 / 48 / 64 rows 38.8 / 59.2 / 78.9 us against 86-88 for quantize + the int8 GEMM
//    (64 x 64 tiles, whose few workgroups leave most CUs idle); N = 8192 at 32 rows 74.2
//    against 86.8, at 48 110.4 against 86.9; N = 14336 at 24 rows 118.1 against 120.7
//    (128 x 64 tiles);
//  - Q4_K, two passes on weights of at most 4096 rows: N = 4096 at 24 rows 30.8 against
//    40.3 us (K = 11008: 26.5 against 31.9), at 48 48.3 against 42.0; N = 8192 at 24 rows
//    53.9 against 41.7.
bool skinny_passes16(const dq::WeightDev& w, int fmt, int64_t m) {
  if (fmt != DQ_ACT_Q8_K || m <= DQ_GEMV_MAX_ROWS || m > dq::kSkinnyMaxRows) return false;
  if (dq::gemv_mma_lds_ok(w.nblk, m) || !dq::gemv_mma_lds_ok(w.nblk, DQ_GEMV_MAX_ROWS)) return false;
  const int64_t passes = (m + DQ_GEMV_MAX_ROWS - 1) / DQ_GEMV_MAX_ROWS;
  if (w.dtype == DQ_Q6_K) return passes * w.n <= 16384;
  return w.dtype == DQ_Q4_K && passes <= 2 && w.n <= 4096;
}

bool use_gemm(const dq::WeightDev& w, int fmt, int64_t m) {
  if (!dq::gemm_supported(w.dtype, fmt)) return false;
  if (w.dtype == DQ_Q8_0 || w.dtype == DQ_Q4_0) return m >= 13;
  // K-quants x per-32 / int16: the f16 GEMMs against GEMV passes of up to 4 rows
  if (w.dtype == DQ_Q6_K && (fmt == DQ_ACT_PER32 || fmt == DQ_ACT_Q16)) {
    return m >= kQ6xGemmMinRows && dq::gemm_q6x_ok(w, fmt, m, 0, w.n);
  }
  if (fmt == DQ_ACT_PER32) return m >= kP32GemmMinRows && dq::gemm_p32_ok(w, m, 0, w.n);
  if (fmt == DQ_ACT_Q16) return m >= kQ16GemmMinRows && dq::gemm_q16_ok(w, m, 0, w.n);
  if (w.dtype == DQ_Q6_K) {
    if (skinny_passes16(w, fmt, m)) return false;
    return m > dq::kSkinnyMaxRows ||
           (m > DQ_GEMV_MAX_ROWS && (!dq::gemv_mma_lds_ok(w.nblk, m) || w.n >= 4096));
  }
  if (m > DQ_GEMV_MAX_ROWS && m <= 48 && w.n <= 4096 && dq::gemv_mma_lds_ok(w.nblk, m)) return false;
  if (skinny_passes16(w, fmt, m)) return false;
  return m > DQ_GEMV_MAX_ROWS;
}

bool skinny_ok(const dq_weight* w, const float* x, int64_t m, int64_t x_stride) {
  const int fmt = dq_act_format_for(w->dev.dtype);
  if (x == nullptr || !dq::gemv_mma_supported(w->dev.dtype, fmt, m)) return false;
  if (use_gemm(w->dev, fmt, m)) return false;
  if (!dq::gemv_mma_lds_ok(w->dev.nblk, m)) return false;
  const int64_t xs = m > 1 ? x_stride : w->dev.k;
  return m * xs * 4 < ((int64_t)1 << 32);
}

// Runs grouped skinny launches over jobs (K-quant matmuls of 2..64 rows, fp32
// inputs in GemvJob::x): batches of up to 8 jobs of one k; a batch of at most 16
// rows whose re-quantization work is small quantizes in the kernel, else each
// distinct input of the batch is quantized once into the per-device scratch first.
int run_skinny(std::vector<dq::GemvJob>& jobs, int device, hipStream_t s, const dq::Region& r) {
  std::vector<bool> done(jobs.size(), false);
  std::vector<dq::GemvJob> batch;
  for (size_t g = 0; g < jobs.size(); ++g) {
    if (done[g]) continue;
    batch.clear();
    for (size_t h = g; h < jobs.size() && batch.size() < 8; ++h) {
      if (!done[h] && jobs[h].w->nblk == jobs[g].w->nblk && (jobs[h].wu != nullptr) == (jobs[g].wu != nullptr)) {
        batch.push_back(jobs[h]);
        done[h] = true;
      }
    }
    int64_t mmax = 0;
    for (const dq::GemvJob& j : batch) mmax = j.m > mmax ? j.m : mmax;
    size_t used = 0;  // bytes of the caller's region holding quantized rows
    if (mmax > 16 || dq::skinny_units(batch.data(), (int)batch.size()) > dq::kSkinnyFuseMaxUnits) {
      // one Q8_K copy per distinct input (x, m, k, stride), as CpuDevice shares one
      // buffer between jobs that read the same activations (cpu_device.cpp:561-599)
      const int64_t arb = dq_act_row_bytes(DQ_ACT_Q8_K, batch[0].w->k);
      std::vector<size_t> off(batch.size());
      std::vector<int64_t> src(batch.size());
      size_t bytes = 0;
      for (size_t i = 0; i < batch.size(); ++i) {
        src[i] = (int64_t)i;
        for (size_t h = 0; h < i; ++h) {
          if (src[h] == (int64_t)h && batch[h].x == batch[i].x && batch[h].m == batch[i].m &&
              batch[h].xs == batch[i].xs) {
            src[i] = (int64_t)h;
            break;
          }
        }
        if (src[i] == (int64_t)i) {
          off[i] = bytes;
          bytes += (size_t)(batch[i].m * arb + 255) / 256 * 256;
        } else {
          off[i] = off[src[i]];
        }
      }
      void* scratch = nullptr;
      if (int rc = acts_buffer(device, bytes, r, &scratch); rc != DQ_OK) return rc;
      used = bytes;
      uint8_t* base = static_cast<uint8_t*>(scratch);
      for (size_t i = 0; i < batch.size(); ++i) {
        dq::GemvJob& j = batch[i];
        if (src[i] == (int64_t)i) {
          DQ_HIP(dq::launch_quantize(DQ_ACT_Q8_K, j.x, j.m, j.w->k, j.xs, base + off[i], arb, s), "quantize launch");
        }
        j.acts = base + off[i];
        j.arb = arb;
        j.x = nullptr;
        j.xs = 0;
      }
    }
    const int64_t tb = batch.size() == 1 && batch[0].x == nullptr && batch[0].wu == nullptr
                           ? dq::skinny_split_bytes(*batch[0].w, DQ_ACT_Q8_K, batch[0].m, 0, batch[0].w->n)
                           : 0;
    if (tb > 0 && r.base == nullptr) {
      // one long-row matmul on few tiles: the split launch's t-terms in this stream's workspace
      const int rc = with_stream_ws(device, static_cast<void*>(s), (size_t)tb, [&](uint8_t* p) -> int {
        const dq::Workspace ws{p, (size_t)tb};
        DQ_HIP(dq::launch_gemv_mma_many(batch.data(), 1, s, &ws), "grouped gemv launch");
        return DQ_OK;
      });
      if (rc != DQ_OK) return rc;
    } else if (tb > 0) {
      // the caller's region after the quantized rows (too small: the unsplit launch)
      const dq::Workspace ws = split_ws(r, used);
      DQ_HIP(dq::launch_gemv_mma_many(batch.data(), 1, s, &ws), "grouped gemv launch");
    } else {
      DQ_HIP(dq::launch_gemv_mma_many(batch.data(), (int)batch.size(), s), "grouped gemv launch");
    }
  }
  return DQ_OK;
}

}  // namespace

namespace dq {

size_t matmul_scratch_bytes(const dq_weight* w, int fmt, int64_t m) {
  const int f = fmt < 0 ? dq_act_format_for(w->dev.dtype) : fmt;
  if (f == DQ_ACT_F32) return gemv_split_bytes(w->dev, f, m < 8 ? m : 8);  // the rows are read in place
  size_t acts = round256((size_t)(m * dq_act_row_bytes(f, w->dev.k)));
  if (f == DQ_ACT_Q8_K && gemm_h16_pays(w->dev, m, 0, w->dev.n)) acts = round256((size_t)act16_bytes(m, w->dev.k));
  // the f16 GEMMs of the per-32 and int16 contracts: their operand layout (quantized
  // straight from the fp32 rows) and the range partials
  if (f == DQ_ACT_PER32 && w->dev.dtype == DQ_Q4_K && use_gemm(w->dev, f, m)) {
    acts = round256((size_t)act32_bytes(m, w->dev.k)) + (size_t)p32_part_bytes(w->dev, m, 0, w->dev.n);
  }
  if (f == DQ_ACT_Q16 && w->dev.dtype == DQ_Q4_K && use_gemm(w->dev, f, m)) {
    acts = round256((size_t)act16i_bytes(m, w->dev.k)) + (size_t)q16_part_bytes(w->dev, m, 0, w->dev.n);
  }
  if (w->dev.dtype == DQ_Q6_K && (f == DQ_ACT_PER32 || f == DQ_ACT_Q16) && use_gemm(w->dev, f, m)) {
    acts = round256((size_t)q6x_act_bytes(f, m, w->dev.k)) + (size_t)q6x_part_bytes(w->dev, m, 0, w->dev.n);
  }
  return acts + gemv_split_bytes(w->dev, f, m < 8 ? m : 8);
}

// Q4_K prefill on the f16 GEMM: quantize straight into its operand layout (in the
// region when one is given), then the GEMM.
static int gemm_h16_from_x(const dq_weight* w, const float* x, int64_t m, int64_t x_stride, float* y,
                           int64_t y_stride, const float* bias, hipStream_t s, const Region& r) {
  void* a16 = nullptr;
  if (int rc = acts_buffer(w->dev.device, (size_t)act16_bytes(m, w->dev.k), r, &a16); rc != DQ_OK) return rc;
  DQ_HIP(launch_act16_quant(x, m > 1 ? x_stride : w->dev.k, m, w->dev.k, static_cast<uint8_t*>(a16), s),
         "act16 quantize launch");
  DQ_HIP(launch_gemm_h16(w->dev, static_cast<const uint8_t*>(a16), m, 0, w->dev.n, y, y_stride, bias, s),
         "gemm launch");
  return DQ_OK;
}

int matmul_impl(const dq_weight* w, const float* x, int64_t m, int64_t x_stride, float* y, int64_t y_stride,
                const float* bias, hipStream_t s, const Region& r) {
  const int fmt = dq_act_format_for(w->dev.dtype);
  const int64_t arb = dq_act_row_bytes(fmt, w->dev.k);
  if (skinny_ok(w, x, m, x_stride)) {
    // decode batches of 2..64 rows: the skinny MFMA GEMV (quantizing the fp32 rows in
    // the kernel when that is cheap, else after one quantize launch)
    std::vector<GemvJob> j{GemvJob{&w->dev, nullptr, 0, x, m > 1 ? x_stride : w->dev.k, m, y, y_stride, bias}};
    return run_skinny(j, w->dev.device, s, r);
  }
  if (skinny_passes16(w->dev, fmt, m)) {
    // long K-quant rows at 17..64 rows: the skinny route per 16 rows of x (its quantized rows
    // and split t-terms in the region when one is given; a last single row on the M = 1
    // route). Every route gives the same bits.
    for (int64_t r0 = 0; r0 < m; r0 += DQ_GEMV_MAX_ROWS) {
      const int64_t rows = m - r0 < DQ_GEMV_MAX_ROWS ? m - r0 : DQ_GEMV_MAX_ROWS;
      const float* xr = x + r0 * x_stride;
      float* yr = y + r0 * y_stride;
      if (rows == 1 || !skinny_ok(w, xr, rows, x_stride)) {
        if (int rc = matmul_impl(w, xr, rows, x_stride, yr, y_stride, bias, s, r); rc != DQ_OK) return rc;
        continue;
      }
      std::vector<GemvJob> j{GemvJob{&w->dev, nullptr, 0, xr, x_stride, rows, yr, y_stride, bias}};
      if (int rc = run_skinny(j, w->dev.device, s, r); rc != DQ_OK) return rc;
    }
    return DQ_OK;
  }
  void* stream = static_cast<void*>(s);
  if (m > 1 && gemv_mma_supported(w->dev.dtype, fmt, 2) && !use_gemm(w->dev, fmt, m)) {
    // K-quants without a GEMM for this size (Q6_K), or inputs whose offsets exceed
    // 32 bits: quantize once, then skinny passes of up to 64 rows
    void* acts = nullptr;
    if (int rc = acts_buffer(w->dev.device, (size_t)(m * arb), r, &acts); rc != DQ_OK) return rc;
    if (int rc = dq_act_quantize(fmt, x, m, w->dev.k, x_stride, acts, stream); rc != DQ_OK) return rc;
    return dq_gemv(w, fmt, acts, m, 0, w->dev.n, y, y_stride, bias, stream);
  }
  if (!use_gemm(w->dev, fmt, m)) {
    // decode: quantization fused into the GEMV (one launch per pass of up to 8 rows);
    // split-K row sums in the region when one is given
    const Workspace ws = split_ws(r, 0);
    DQ_HIP(launch_gemv_fused(w->dev, x, x_stride, m, y, y_stride, bias, s, r.base ? &ws : nullptr), "gemv launch");
    return DQ_OK;
  }
  if (fmt == DQ_ACT_Q8_K && gemm_h16_pays(w->dev, m, 0, w->dev.n)) {
    return gemm_h16_from_x(w, x, m, x_stride, y, y_stride, bias, s, r);
  }
  void* acts = nullptr;
  if (int rc = acts_buffer(w->dev.device, (size_t)(m * arb), r, &acts); rc != DQ_OK) return rc;
  if (int rc = dq_act_quantize(fmt, x, m, w->dev.k, x_stride, acts, stream); rc != DQ_OK) return rc;
  return dq_gemm(w, fmt, acts, m, 0, w->dev.n, y, y_stride, bias, stream);
}

int matmul_act_impl(const dq_weight* w, int fmt, const float* x, int64_t m, int64_t x_stride, float* y,
                    int64_t y_stride, const float* bias, hipStream_t s, const Region& r) {
  const int64_t arb = dq_act_row_bytes(fmt, w->dev.k);
  void* stream = static_cast<void*>(s);
  if (fmt == DQ_ACT_F32) {
    // fp32 activations: the GEMV reads the caller's rows in place
    const int64_t xrb = (m > 1 ? x_stride : w->dev.k) * 4;
    if (m * xrb >= ((int64_t)1 << 32)) return fail(DQ_UNSUPPORTED, "activations exceed 4 GiB");
    const Workspace ws = split_ws(r, 0);
    DQ_HIP(launch_gemv(w->dev, fmt, reinterpret_cast<const uint8_t*>(x), xrb, m, 0, w->dev.n, y, y_stride, bias,
                       nullptr, s, r.base ? &ws : nullptr),
           "gemv launch");
    return DQ_OK;
  }
  if (fmt == DQ_ACT_Q8_K && use_gemm(w->dev, fmt, m) && gemm_h16_pays(w->dev, m, 0, w->dev.n)) {
    return gemm_h16_from_x(w, x, m, x_stride, y, y_stride, bias, s, r);
  }
  if (fmt == DQ_ACT_PER32 && w->dev.dtype == DQ_Q4_K && use_gemm(w->dev, fmt, m)) {
    // Q4_K x per-32 prefill: the fp32 rows quantized straight into the f16 operand layout
    // (the per-32 quantizer's codes), the f16 GEMM (all in the region when one is given)
    const size_t lay = round256((size_t)act32_bytes(m, w->dev.k)), pb = (size_t)p32_part_bytes(w->dev, m, 0, w->dev.n);
    void* buf = nullptr;
    if (int rc = acts_buffer(w->dev.device, lay + pb, r, &buf); rc != DQ_OK) return rc;
    uint8_t* a32 = static_cast<uint8_t*>(buf);
    DQ_HIP(launch_act32_quant(x, m > 1 ? x_stride : w->dev.k, m, w->dev.k, a32, s), "act32 quantize launch");
    DQ_HIP(launch_gemm_p32(w->dev, a32, m, 0, w->dev.n, y, y_stride, bias,
                           pb > 0 ? reinterpret_cast<float*>(a32 + lay) : nullptr, s),
           "gemm launch");
    return DQ_OK;
  }
  if (fmt == DQ_ACT_PER32 && (w->dev.dtype == DQ_Q4_K || w->dev.dtype == DQ_Q6_K) && m <= 8 &&
      !use_gemm(w->dev, fmt, m)) {
    // K-quants x per-32 decode (qmm's int8 gemv): one pass, each wave quantizing its
    // slice with the standalone quantizer's arithmetic (the codes dq_act_quantize writes)
    const Workspace ws = split_ws(r, 0);
    DQ_HIP(launch_gemv_fused(w->dev, x, m > 1 ? x_stride : w->dev.k, m, y, y_stride, bias, s, r.base ? &ws : nullptr,
                             kActPer32),
           "gemv launch");
    return DQ_OK;
  }
  if (w->dev.dtype == DQ_Q6_K && (fmt == DQ_ACT_PER32 || fmt == DQ_ACT_Q16) && use_gemm(w->dev, fmt, m)) {
    // Q6_K x per-32 / int16 prefill: the fp32 rows quantized straight into the narrow
    // operand layout, the f16 GEMM (and its range partials)
    const size_t lay = round256((size_t)q6x_act_bytes(fmt, m, w->dev.k));
    const size_t pb = (size_t)q6x_part_bytes(w->dev, m, 0, w->dev.n);
    void* buf = nullptr;
    if (int rc = acts_buffer(w->dev.device, lay + pb, r, &buf); rc != DQ_OK) return rc;
    uint8_t* a2 = static_cast<uint8_t*>(buf);
    DQ_HIP(launch_q6x_quant(fmt, x, m > 1 ? x_stride : w->dev.k, m, w->dev.k, a2, s), "operand layout quantize launch");
    DQ_HIP(launch_gemm_q6x(w->dev, fmt, a2, m, 0, w->dev.n, y, y_stride, bias,
                           pb > 0 ? reinterpret_cast<float*>(a2 + lay) : nullptr, s),
           "gemm launch");
    return DQ_OK;
  }
  if (fmt == DQ_ACT_Q16 && w->dev.dtype == DQ_Q4_K && use_gemm(w->dev, fmt, m)) {
    // Q4_K x int16 prefill: the fp32 rows quantized straight into the lo / 256 hi f16
    // layout (the int16 quantizer's codes), the f16 GEMM
    const size_t lay = round256((size_t)act16i_bytes(m, w->dev.k)), pb = (size_t)q16_part_bytes(w->dev, m, 0, w->dev.n);
    void* buf = nullptr;
    if (int rc = acts_buffer(w->dev.device, lay + pb, r, &buf); rc != DQ_OK) return rc;
    uint8_t* a16 = static_cast<uint8_t*>(buf);
    DQ_HIP(launch_act16i_quant(x, m > 1 ? x_stride : w->dev.k, m, w->dev.k, a16, s), "act16i quantize launch");
    DQ_HIP(launch_gemm_q16(w->dev, a16, m, 0, w->dev.n, y, y_stride, bias,
                           pb > 0 ? reinterpret_cast<float*>(a16 + lay) : nullptr, s),
           "gemm launch");
    return DQ_OK;
  }
  void* acts = nullptr;
  if (int rc = acts_buffer(w->dev.device, (size_t)(m * arb), r, &acts); rc != DQ_OK) return rc;
  if (int rc = dq_act_quantize(fmt, x, m, w->dev.k, m > 1 ? x_stride : w->dev.k, acts, stream); rc != DQ_OK) return rc;
  if (use_gemm(w->dev, fmt, m)) {
    return dq_gemm(w, fmt, acts, m, 0, w->dev.n, y, y_stride, bias, stream);
  }
  // only a GEMV that splits K needs more than the activations
  if (r.base == nullptr || gemv_splits(w->dev, fmt) == 1) {
    return dq_gemv(w, fmt, acts, m, 0, w->dev.n, y, y_stride, bias, stream);
  }
  const Workspace ws = split_ws(r, (size_t)(m * arb));
  DQ_HIP(launch_gemv(w->dev, fmt, static_cast<const uint8_t*>(acts), arb, m, 0, w->dev.n, y, y_stride, bias, nullptr,
                     s, &ws),
         "gemv launch");
  return DQ_OK;
}

int matmul_sel_impl(const dq_weight* w, const dq_selection& sel, const float* x, int64_t m, int64_t x_stride,
                    float* y, int64_t y_stride, const float* bias, hipStream_t s, const Region& r) {
  const int t = w->dev.dtype;
  switch (sel.kernel) {
    case DQ_KERNEL_INT8_SUPERBLOCK:  // Q8_K, the K-quants' dq_matmul routes
      if (t == DQ_Q4_K || t == DQ_Q6_K) return matmul_impl(w, x, m, x_stride, y, y_stride, bias, s, r);
      break;
    case DQ_KERNEL_INT8_PER32:  // per-32: dq_matmul's routes for Q8_0 / Q4_0
      if (t == DQ_Q8_0 || t == DQ_Q4_0) return matmul_impl(w, x, m, x_stride, y, y_stride, bias, s, r);
      break;
    case DQ_KERNEL_F32_EXPAND_GEMM:  // expand + GEMM on the matrix cores (cpu_device.cpp:1114-1152)
      if (m >= kF32GemmMinRows) {
        const int64_t xs = m > 1 ? x_stride : w->dev.k;
        if ((127 * xs + w->dev.k) * 4 >= ((int64_t)1 << 32)) {  // one tile's 128 rows, 32-bit offsets
          return fail(DQ_UNSUPPORTED, "128 activation rows of stride %lld exceed 4 GiB", (long long)xs);
        }
        DQ_HIP(launch_gemm_f32(w->dev, x, xs, m, 0, w->dev.n, y, y_stride, bias, s), "fp32 gemm launch");
        return DQ_OK;
      }
      break;
    default:
      break;
  }
  if (!pair_ok(t, sel.act)) {
    return fail(DQ_UNSUPPORTED, "kernel %d (activation format %d) does not take weight type %d", sel.kernel, sel.act, t);
  }
  return matmul_act_impl(w, sel.act, x, m, x_stride, y, y_stride, bias, s, r);
}

size_t sel_scratch_bytes(const dq_weight* w, const dq_selection& sel, int64_t m) {
  const size_t a = matmul_scratch_bytes(w, -1, m), b = matmul_scratch_bytes(w, sel.act, m);
  return a > b ? a : b;
}

}  // namespace dq

extern "C" {

const char* dq_version(void) { return "dynaq 0.1.0 (gfx950)"; }
const char* dq_last_error(void) { return g_err.c_str(); }

int64_t dq_row_bytes(int dtype, int64_t k) {
  if (!weight_type_ok(dtype) || k < 0) return -1;
  const int be = dq::block_elems(dtype);
  if (k % be != 0) return -1;
  return k / be * dq::block_bytes(dtype);
}

int64_t dq_act_row_bytes(int fmt, int64_t k) {
  if (!act_fmt_ok(fmt) || k < 0) return -1;
  const int be = dq::act_block_elems(fmt);
  if (k % be != 0) return -1;
  return k / be * dq::act_block_bytes(fmt);
}

int dq_act_format_for(int dtype) {
  if (dtype == DQ_Q8_0 || dtype == DQ_Q4_0) return DQ_ACT_PER32;
  if (dtype == DQ_Q4_K || dtype == DQ_Q6_K) return DQ_ACT_Q8_K;
  return -1;
}

int dq_weight_upload(int dtype, const void* host_rows, int64_t n, int64_t k, int64_t row_bytes, void* stream,
                     dq_weight** out) {
  return upload_impl(dtype, host_rows, true, n, k, row_bytes, stream, out);
}

int dq_weight_upload_device(int dtype, const void* dev_rows, int64_t n, int64_t k, int64_t row_bytes, void* stream,
                            dq_weight** out) {
  return upload_impl(dtype, dev_rows, false, n, k, row_bytes, stream, out);
}

int dq_weight_download(const dq_weight* w, void* host_rows, int64_t row_bytes, void* stream) {
  if (w == nullptr || host_rows == nullptr) return fail(DQ_INVALID_ARGUMENT, "null argument");
  const dq::WeightDev& d = w->dev;
  const int64_t rb = dq_row_bytes(d.dtype, d.k);
  if (row_bytes < rb) return fail(DQ_INVALID_ARGUMENT, "row_bytes %lld < %lld", (long long)row_bytes, (long long)rb);
  hipStream_t s = as_stream(stream);
  void* staging = nullptr;
  DQ_HIP(hipMalloc(&staging, (size_t)(d.n * row_bytes)), "hipMalloc(staging)");
  hipError_t e = hipMemsetAsync(staging, 0, (size_t)(d.n * row_bytes), s);
  if (e == hipSuccess) {
    uint8_t* planes[dq::kMaxPlanes];
    for (int p = 0; p < dq::kMaxPlanes; ++p) planes[p] = d.plane[p];
    e = dq::launch_unpack(d.dtype, static_cast<uint8_t*>(staging), row_bytes, d.n, d.nblk, planes, s);
  }
  if (e == hipSuccess) e = hipMemcpyAsync(host_rows, staging, (size_t)(d.n * row_bytes), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  const hipError_t ef = hipFree(staging);
  if (e == hipSuccess) e = ef;
  if (e != hipSuccess) return hip_fail(e, "weight download");
  return DQ_OK;
}

int dq_weight_free(dq_weight* w) {
  if (w == nullptr) return DQ_OK;
  hipError_t e = hipSuccess;  // every plane is released; the first failure is reported
  for (int p = 0; p < dq::kMaxPlanes; ++p) {
    if (w->dev.plane[p] != nullptr) {
      const hipError_t ef = hipFree(w->dev.plane[p]);
      if (e == hipSuccess) e = ef;
    }
  }
  delete w;
  if (e != hipSuccess) return hip_fail(e, "weight free");
  return DQ_OK;
}

int dq_weight_info(const dq_weight* w, int* dtype, int64_t* n, int64_t* k, int64_t* device_bytes) {
  if (w == nullptr) return fail(DQ_INVALID_ARGUMENT, "null weight");
  if (dtype) *dtype = w->dev.dtype;
  if (n) *n = w->dev.n;
  if (k) *k = w->dev.k;
  if (device_bytes) {
    int64_t total = 0;
    for (int p = 0; p < dq::kMaxPlanes; ++p) total += w->dev.plane_bytes[p];
    *device_bytes = total;
  }
  return DQ_OK;
}

int dq_act_quantize(int fmt, const float* x, int64_t m, int64_t k, int64_t x_stride, void* out, void* stream) {
  if (!act_fmt_ok(fmt)) return fail(DQ_UNSUPPORTED, "activation format %d is not supported", fmt);
  const int64_t orb = dq_act_row_bytes(fmt, k);
  if (orb < 0 || k <= 0) return fail(DQ_INVALID_ARGUMENT, "k %lld is not a multiple of the activation block", (long long)k);
  if (m < 0) return fail(DQ_INVALID_ARGUMENT, "m must be >= 0");
  if (m == 0) return DQ_OK;
  if (x == nullptr || out == nullptr) return fail(DQ_INVALID_ARGUMENT, "null argument");
  if (m > 1 && x_stride < k) return fail(DQ_INVALID_ARGUMENT, "x_stride %lld < k %lld", (long long)x_stride, (long long)k);
  if (k * 4 >= ((int64_t)1 << 32) || m > 65535) return fail(DQ_UNSUPPORTED, "activation shape too large");
  if (reinterpret_cast<uintptr_t>(out) % 4 != 0) return fail(DQ_INVALID_ARGUMENT, "out must be 4-byte aligned");
  if (fmt == DQ_ACT_F32) {  // no quantization: the rows, densely
    DQ_HIP(hipMemcpy2DAsync(out, (size_t)orb, x, (size_t)(m > 1 ? x_stride : k) * 4, (size_t)orb, (size_t)m,
                            hipMemcpyDeviceToDevice, as_stream(stream)),
           "row copy");
    return DQ_OK;
  }
  DQ_HIP(dq::launch_quantize(fmt, x, m, k, x_stride, static_cast<uint8_t*>(out), orb, as_stream(stream)),
         "quantize launch");
  return DQ_OK;
}

static int qmm_acts_ok(const dq_qmm_acts* a) {
  if (a == nullptr) return fail(DQ_INVALID_ARGUMENT, "null argument");
  if (dq_qmm_act_bytes(a->mode, a->m, a->k, a->paired) < 0 || a->hi == nullptr || a->d == nullptr || a->c == nullptr ||
      a->blocks == nullptr || (a->mode == DQ_QMM_INT16) != (a->lo != nullptr)) {
    return fail(DQ_INVALID_ARGUMENT, "qmm acts not prepared");
  }
  if (reinterpret_cast<uintptr_t>(a->hi) % 4 != 0 || (a->lo && reinterpret_cast<uintptr_t>(a->lo) % 4 != 0) ||
      reinterpret_cast<uintptr_t>(a->blocks) % 16 != 0) {
    return fail(DQ_INVALID_ARGUMENT, "qmm acts codes must be 4-byte aligned (blocks 16-byte)");
  }
  return DQ_OK;
}

static int64_t qmm_align64(int64_t v) { return (v + 63) / 64 * 64; }
// The block format a qmm mode's rows convert to: per-32 (int8) or int16.
static int qmm_fmt(int mode) { return mode == DQ_QMM_INT16 ? DQ_ACT_Q16 : DQ_ACT_PER32; }

int64_t dq_qmm_act_bytes(int mode, int64_t m, int64_t k, int paired) {
  if ((mode != DQ_QMM_INT8 && mode != DQ_QMM_INT16) || m < 0 || k <= 0 || k % 32 != 0) return -1;
  if (m > ((int64_t)1 << 24) || k > ((int64_t)1 << 30)) return -1;
  const int64_t m_pad = paired ? (m + 1) / 2 * 2 : m;
  const int64_t code = qmm_align64(m_pad * k), scale = qmm_align64(m_pad * (k / 32) * 4);
  const int64_t blocks = qmm_align64(m * dq_act_row_bytes(qmm_fmt(mode), k));
  return code * (mode == DQ_QMM_INT16 ? 2 : 1) + 2 * scale + blocks;
}

int dq_qmm_act_prepare(void* base, int64_t bytes, int mode, int64_t m, int64_t k, int paired, dq_qmm_acts* out,
                       void* stream) {
  const int64_t need = dq_qmm_act_bytes(mode, m, k, paired);
  if (need < 0) return fail(DQ_INVALID_ARGUMENT, "qmm acts: mode %d, m %lld, k %lld (k must be a positive multiple of 32)",
                            mode, (long long)m, (long long)k);
  if (base == nullptr || out == nullptr) return fail(DQ_INVALID_ARGUMENT, "null argument");
  if (reinterpret_cast<uintptr_t>(base) % 64 != 0) return fail(DQ_INVALID_ARGUMENT, "qmm acts buffer must be 64-byte aligned");
  if (bytes < need) return fail(DQ_INVALID_ARGUMENT, "qmm acts buffer of %lld bytes < %lld", (long long)bytes, (long long)need);
  const int64_t m_pad = paired ? (m + 1) / 2 * 2 : m;
  const int64_t code = qmm_align64(m_pad * k), lo_bytes = mode == DQ_QMM_INT16 ? code : 0;
  const int64_t scale = qmm_align64(m_pad * (k / 32) * 4);
  uint8_t* p = static_cast<uint8_t*>(base);
  out->mode = mode;
  out->paired = paired ? 1 : 0;
  out->m = m;
  out->k = k;
  out->hi = reinterpret_cast<int8_t*>(p);
  out->lo = mode == DQ_QMM_INT16 ? p + code : nullptr;
  out->d = reinterpret_cast<float*>(p + code + lo_bytes);
  out->c = reinterpret_cast<float*>(p + code + lo_bytes + scale);
  out->blocks = p + code + lo_bytes + 2 * scale;
  if (paired && (m & 1)) {
    DQ_HIP(dq::launch_qmm_pad(m, k, out->hi, out->lo, out->d, out->c, as_stream(stream)), "qmm pad launch");
  }
  return DQ_OK;
}

int dq_qmm_quantize_rows(const float* x, int64_t x_stride, int64_t r0, int64_t r1, const dq_qmm_acts* a, void* stream) {
  if (int rc = qmm_acts_ok(a); rc != DQ_OK) return rc;
  if (r0 < 0 || r1 < r0 || r1 > a->m) {
    return fail(DQ_INVALID_ARGUMENT, "rows [%lld, %lld) outside [0, %lld)", (long long)r0, (long long)r1, (long long)a->m);
  }
  if (r0 == r1) return DQ_OK;
  if (x == nullptr) return fail(DQ_INVALID_ARGUMENT, "null argument");
  if (r1 > 1 && x_stride < a->k) {
    return fail(DQ_INVALID_ARGUMENT, "x_stride %lld < k %lld", (long long)x_stride, (long long)a->k);
  }
  DQ_HIP(dq::launch_qmm_quantize(x, x_stride, r0, r1, a->k, a->mode == DQ_QMM_INT16, a->paired != 0, a->hi, a->lo, a->d,
                                 a->c, as_stream(stream)),
         "qmm quantize launch");
  // the same rows in the block format gemv / gemm read, from the codes just written
  const int64_t orb = dq_act_row_bytes(qmm_fmt(a->mode), a->k);
  DQ_HIP(dq::launch_qmm_to_blocks(a->hi, a->lo, a->d, a->k, a->mode == DQ_QMM_INT16, a->paired != 0, r0, r1 - r0,
                                  a->blocks + r0 * orb, orb, as_stream(stream)),
         "qmm conversion launch");
  return DQ_OK;
}

// qmm's gemv / gemm on a qmm activation buffer: the library's GEMV passes or GEMM on
// the buffer's rows in the per-32 (int8) or int16 block format, which
// dq_qmm_quantize_rows wrote beside the codes. Reads only the caller's buffer (no
// library state), so calls on disjoint [n0, n1) or row ranges may run concurrently.
// y row r0 + r for buffer row r0 + r.
static int qmm_matmul(const dq_weight* w, const dq_qmm_acts* a, int64_t r0, int64_t rows, int64_t n0, int64_t n1,
                      float* y, int64_t y_stride, const float* bias, void* stream, bool gemm) {
  if (int rc = qmm_acts_ok(a); rc != DQ_OK) return rc;
  if (w == nullptr) return fail(DQ_INVALID_ARGUMENT, "null weight");
  if (a->k != w->dev.k) return fail(DQ_INVALID_ARGUMENT, "acts k %lld != weight k %lld", (long long)a->k, (long long)w->dev.k);
  if (r0 < 0 || rows < 0 || r0 + rows > a->m) {
    return fail(DQ_INVALID_ARGUMENT, "rows [%lld, %lld) outside [0, %lld)", (long long)r0, (long long)(r0 + rows),
                (long long)a->m);
  }
  const int fmt = qmm_fmt(a->mode);
  const int64_t orb = dq_act_row_bytes(fmt, a->k);
  const uint8_t* buf = a->blocks + r0 * orb;
  if (int rc = check_acts(w, fmt, buf, rows); rc != DQ_OK) return rc;
  if (y == nullptr && rows > 0) return fail(DQ_INVALID_ARGUMENT, "null output");
  if (int rc = check_out(w, rows, n0, n1, rows > 0 ? y + r0 * y_stride : y, y_stride); rc != DQ_OK) return rc;
  if (rows == 0 || n0 == n1) return DQ_OK;
  if (gemm && use_gemm(w->dev, fmt, rows)) {
    return dq_gemm(w, fmt, buf, rows, n0, n1, y + r0 * y_stride, y_stride, bias, stream);
  }
  return dq_gemv(w, fmt, buf, rows, n0, n1, y + r0 * y_stride, y_stride, bias, stream);
}

int dq_qmm_gemv(const dq_weight* w, int64_t n0, int64_t n1, const dq_qmm_acts* a, int64_t r0, int rows, float* y,
                int64_t y_stride, const float* bias, void* stream) {
  return qmm_matmul(w, a, r0, rows, n0, n1, y, y_stride, bias, stream, false);
}

int dq_qmm_gemm(const dq_weight* w, int64_t n0, int64_t n1, const dq_qmm_acts* a, float* y, int64_t y_stride,
                const float* bias, void* stream) {
  if (int rc = qmm_acts_ok(a); rc != DQ_OK) return rc;
  return qmm_matmul(w, a, 0, a->m, n0, n1, y, y_stride, bias, stream, true);
}

int dq_gemv(const dq_weight* w, int fmt, const void* acts, int64_t m, int64_t n0, int64_t n1, float* y,
            int64_t y_stride, const float* bias, void* stream) {
  if (int rc = check_acts(w, fmt, acts, m); rc != DQ_OK) return rc;
  if (int rc = check_out(w, m, n0, n1, y, y_stride); rc != DQ_OK) return rc;
  if (m == 0 || n0 == n1) return DQ_OK;
  // passes of up to 64 rows (sub-scaled: 16); 16 where the 64-row tiles' LDS does not hold
  // the row's super-blocks
  int64_t pass = fmt == DQ_ACT_SX ? dq::kSkinnySxMaxRows : dq::kSkinnyMaxRows;
  if (m > DQ_GEMV_MAX_ROWS && !dq::gemv_mma_lds_ok(w->dev.nblk, m < pass ? m : pass)) pass = DQ_GEMV_MAX_ROWS;
  if (m >= 2 && dq::gemv_mma_supported(w->dev.dtype, fmt, 2) && dq::gemv_mma_lds_ok(w->dev.nblk, m < pass ? m : pass) &&
      (fmt != DQ_ACT_SX || dq::skinny_sx_pays(w->dev, m < pass ? m : pass, n0, n1))) {
    // K-quants x Q8_K / sub-scaled: the skinny MFMA GEMV in passes of `pass` rows (a last
    // single row goes to the M = 1 GEMV)
    const int64_t arb = dq_act_row_bytes(fmt, w->dev.k);
    const uint8_t* a = static_cast<const uint8_t*>(acts);
    for (int64_t r0 = 0; r0 < m; r0 += pass) {
      const int64_t rows = m - r0 < pass ? m - r0 : pass;
      if (rows == 1) {
        DQ_HIP(dq::launch_gemv(w->dev, fmt, a + r0 * arb, arb, 1, n0, n1, y + r0 * y_stride, y_stride, bias, nullptr,
                               as_stream(stream)),
               "gemv launch");
      } else if (const int64_t tb = dq::skinny_split_bytes(w->dev, fmt, rows, n0, n1); tb > 0) {
        // long rows on few tiles: the split launch's t-terms in this stream's workspace
        const int rc = with_stream_ws(w->dev.device, stream, (size_t)tb, [&](uint8_t* p) -> int {
          const dq::Workspace ws{p, (size_t)tb};
          DQ_HIP(dq::launch_gemv_mma(w->dev, fmt, a + r0 * arb, arb, rows, n0, n1, y + r0 * y_stride, y_stride, bias,
                                     as_stream(stream), &ws),
                 "gemv launch");
          return DQ_OK;
        });
        if (rc != DQ_OK) return rc;
      } else {
        DQ_HIP(dq::launch_gemv_mma(w->dev, fmt, a + r0 * arb, arb, rows, n0, n1, y + r0 * y_stride, y_stride, bias,
                                   as_stream(stream)),
               "gemv launch");
      }
    }
    return DQ_OK;
  }
  DQ_HIP(dq::launch_gemv(w->dev, fmt, static_cast<const uint8_t*>(acts), dq_act_row_bytes(fmt, w->dev.k), m, n0, n1, y,
                         y_stride, bias, nullptr, as_stream(stream)),
         "gemv launch");
  return DQ_OK;
}

int dq_gemm(const dq_weight* w, int fmt, const void* acts, int64_t m, int64_t n0, int64_t n1, float* y,
            int64_t y_stride, const float* bias, void* stream) {
  if (int rc = check_acts(w, fmt, acts, m); rc != DQ_OK) return rc;
  if (int rc = check_out(w, m, n0, n1, y, y_stride); rc != DQ_OK) return rc;
  if (!dq::gemm_supported(w->dev.dtype, fmt)) {
    return fail(DQ_UNSUPPORTED, "no GEMM kernel for weight type %d with activation format %d", w->dev.dtype, fmt);
  }
  if (m == 0 || n0 == n1) return DQ_OK;
  if (fmt == DQ_ACT_Q8_K && dq::gemm_h16_pays(w->dev, m, n0, n1)) {
    // Q4_K: the codes as f16 operands (one conversion launch), then the f16 GEMM
    const int64_t arb = dq_act_row_bytes(fmt, w->dev.k);
    return with_stream_ws(w->dev.device, stream, (size_t)dq::act16_bytes(m, w->dev.k), [&](uint8_t* ws) -> int {
      DQ_HIP(dq::launch_act16_from_q8k(static_cast<const uint8_t*>(acts), arb, m, w->dev.k, ws, as_stream(stream)),
             "act16 conversion launch");
      DQ_HIP(dq::launch_gemm_h16(w->dev, ws, m, n0, n1, y, y_stride, bias, as_stream(stream)), "gemm launch");
      return DQ_OK;
    });
  }
  if (fmt == DQ_ACT_PER32 && w->dev.dtype == DQ_Q4_K) {
    // Q4_K x per-32: the codes as f16 operands (one conversion launch), then the f16 GEMM
    if (!dq::gemm_p32_ok(w->dev, m, n0, n1)) return fail(DQ_UNSUPPORTED, "m too large");
    const int64_t arb = dq_act_row_bytes(fmt, w->dev.k);
    const size_t lay = round256((size_t)dq::act32_bytes(m, w->dev.k)), pb = (size_t)dq::p32_part_bytes(w->dev, m, n0, n1);
    return with_stream_ws(w->dev.device, stream, lay + pb, [&](uint8_t* ws) -> int {
      DQ_HIP(dq::launch_act32_from_p32(static_cast<const uint8_t*>(acts), arb, m, w->dev.k, ws, as_stream(stream)),
             "act32 conversion launch");
      DQ_HIP(dq::launch_gemm_p32(w->dev, ws, m, n0, n1, y, y_stride, bias,
                                 pb > 0 ? reinterpret_cast<float*>(ws + lay) : nullptr, as_stream(stream)),
             "gemm launch");
      return DQ_OK;
    });
  }
  if (w->dev.dtype == DQ_Q6_K && (fmt == DQ_ACT_PER32 || fmt == DQ_ACT_Q16)) {
    // Q6_K x per-32 / int16: the operand layout (one launch), then the f16 GEMM (and the sum
    // of its range partials)
    if (!dq::gemm_q6x_ok(w->dev, fmt, m, n0, n1)) return fail(DQ_UNSUPPORTED, "m too large");
    const int64_t arb = dq_act_row_bytes(fmt, w->dev.k);
    const size_t lay = round256((size_t)dq::q6x_act_bytes(fmt, m, w->dev.k));
    const size_t pb = (size_t)dq::q6x_part_bytes(w->dev, m, n0, n1);
    return with_stream_ws(w->dev.device, stream, lay + pb, [&](uint8_t* ws) -> int {
      DQ_HIP(dq::launch_q6x_act(fmt, static_cast<const uint8_t*>(acts), arb, m, w->dev.k, ws, as_stream(stream)),
             "operand layout launch");
      DQ_HIP(dq::launch_gemm_q6x(w->dev, fmt, ws, m, n0, n1, y, y_stride, bias,
                                 pb > 0 ? reinterpret_cast<float*>(ws + lay) : nullptr, as_stream(stream)),
             "gemm launch");
      return DQ_OK;
    });
  }
  if (fmt == DQ_ACT_Q16) {
    // Q4_K x int16: lo / 256 hi as f16 operands (one conversion launch), then the f16 GEMM
    if (!dq::gemm_q16_ok(w->dev, m, n0, n1)) return fail(DQ_UNSUPPORTED, "m too large");
    const int64_t arb = dq_act_row_bytes(fmt, w->dev.k);
    const size_t lay = round256((size_t)dq::act16i_bytes(m, w->dev.k)), pb = (size_t)dq::q16_part_bytes(w->dev, m, n0, n1);
    return with_stream_ws(w->dev.device, stream, lay + pb, [&](uint8_t* ws) -> int {
      DQ_HIP(dq::launch_act16i_from_q16(static_cast<const uint8_t*>(acts), arb, m, w->dev.k, ws, as_stream(stream)),
             "act16i conversion launch");
      DQ_HIP(dq::launch_gemm_q16(w->dev, ws, m, n0, n1, y, y_stride, bias,
                                 pb > 0 ? reinterpret_cast<float*>(ws + lay) : nullptr, as_stream(stream)),
             "gemm launch");
      return DQ_OK;
    });
  }
  if ((m + 127) / 128 > 65535) return fail(DQ_UNSUPPORTED, "m too large");
  DQ_HIP(dq::launch_gemm(w->dev, fmt, static_cast<const uint8_t*>(acts), dq_act_row_bytes(fmt, w->dev.k), m, n0, n1, y,
                         y_stride, bias, as_stream(stream)),
         "gemm launch");
  return DQ_OK;
}

int dq_matmul(const dq_weight* w, const float* x, int64_t m, int64_t x_stride, float* y, int64_t y_stride,
              const float* bias, void* stream) {
  if (w == nullptr) return fail(DQ_INVALID_ARGUMENT, "null weight");
  if (m < 0) return fail(DQ_INVALID_ARGUMENT, "m must be >= 0");
  if (m == 0) return DQ_OK;
  if (int rc = check_out(w, m, 0, w->dev.n, y, y_stride); rc != DQ_OK) return rc;
  if (x == nullptr) return fail(DQ_INVALID_ARGUMENT, "null argument");
  if (m > 1 && x_stride < w->dev.k) {
    return fail(DQ_INVALID_ARGUMENT, "x_stride %lld < k %lld", (long long)x_stride, (long long)w->dev.k);
  }
  return dq::matmul_impl(w, x, m, x_stride, y, y_stride, bias, as_stream(stream), dq::Region{});
}

int dq_matmul_plan(const dq_weight* w, const dq_plan* plan, const float* x, int64_t m, int64_t x_stride, float* y,
                   int64_t y_stride, const float* bias, void* stream) {
  if (w == nullptr) return fail(DQ_INVALID_ARGUMENT, "null weight");
  if (m < 0) return fail(DQ_INVALID_ARGUMENT, "m must be >= 0");
  if (m == 0) return DQ_OK;
  if (int rc = check_out(w, m, 0, w->dev.n, y, y_stride); rc != DQ_OK) return rc;
  if (x == nullptr) return fail(DQ_INVALID_ARGUMENT, "null argument");
  if (m > 1 && x_stride < w->dev.k) {
    return fail(DQ_INVALID_ARGUMENT, "x_stride %lld < k %lld", (long long)x_stride, (long long)w->dev.k);
  }
  const dq_matmul_shape shape{m, w->dev.n, w->dev.k, w->dev.dtype, (int32_t)(m == 1 || x_stride == w->dev.k)};
  const dq_selection sel = dq::select(shape, plan != nullptr ? *plan : dq::default_plan());
  return dq::matmul_sel_impl(w, sel, x, m, x_stride, y, y_stride, bias, as_stream(stream), dq::Region{});
}

int dq_matmul_many(const dq_matmul_job* jobs, int64_t n_jobs, void* stream) {
  if (n_jobs < 0) return fail(DQ_INVALID_ARGUMENT, "n_jobs must be >= 0");
  if (n_jobs == 0) return DQ_OK;
  if (jobs == nullptr) return fail(DQ_INVALID_ARGUMENT, "null jobs");
  // validation of every job first: nothing is launched for a call that fails
  for (int64_t i = 0; i < n_jobs; ++i) {
    const dq_matmul_job& j = jobs[i];
    if (j.w == nullptr) return fail(DQ_INVALID_ARGUMENT, "job %lld: null weight", (long long)i);
    if (j.m < 0) return fail(DQ_INVALID_ARGUMENT, "job %lld: m must be >= 0", (long long)i);
    if (j.w->dev.device != jobs[0].w->dev.device) {
      return fail(DQ_INVALID_ARGUMENT, "job %lld: weights of one call must be on one device", (long long)i);
    }
    if (j.m == 0) continue;
    if (int rc = check_out(j.w, j.m, 0, j.w->dev.n, j.y, j.y_stride); rc != DQ_OK) return rc;
    if (j.x == nullptr) return fail(DQ_INVALID_ARGUMENT, "job %lld: null x", (long long)i);
    if (j.m > 1 && j.x_stride < j.w->dev.k) {
      return fail(DQ_INVALID_ARGUMENT, "job %lld: x_stride %lld < k %lld", (long long)i, (long long)j.x_stride,
                  (long long)j.w->dev.k);
    }
  }
  hipStream_t s = as_stream(stream);
  // the grouped jobs: decode-sized K-quant matmuls (the skinny MFMA GEMV, which
  // quantizes each job's fp32 rows itself); one launch per k for up to 8 jobs
  std::vector<dq::GemvJob> grouped;
  std::vector<int64_t> others;
  for (int64_t i = 0; i < n_jobs; ++i) {
    const dq_matmul_job& j = jobs[i];
    if (j.m == 0) continue;
    if (skinny_ok(j.w, j.x, j.m, j.x_stride)) {
      grouped.push_back(dq::GemvJob{&j.w->dev, nullptr, 0, j.x, j.m > 1 ? j.x_stride : j.w->dev.k, j.m, j.y,
                                    j.y_stride, j.bias});
    } else {
      others.push_back(i);
    }
  }
  if (int rc = run_skinny(grouped, jobs[0].w->dev.device, s, dq::Region{}); rc != DQ_OK) return rc;
  for (int64_t i : others) {
    const dq_matmul_job& j = jobs[i];
    if (int rc = dq_matmul(j.w, j.x, j.m, j.x_stride, j.y, j.y_stride, j.bias, stream); rc != DQ_OK) return rc;
  }
  return DQ_OK;
}

int dq_act_mul(int act, const float* gate, int64_t gate_stride, const float* up, int64_t up_stride, int64_t m,
               int64_t n, float* out, int64_t out_stride, void* stream) {
  if (!dq::act_ok(act)) return fail(DQ_INVALID_ARGUMENT, "unknown activation %d", act);
  if (m < 0 || n < 0) return fail(DQ_INVALID_ARGUMENT, "m and n must be >= 0");
  if (m == 0 || n == 0) return DQ_OK;
  if (gate == nullptr || up == nullptr || out == nullptr) return fail(DQ_INVALID_ARGUMENT, "null argument");
  if (m > 1 && (gate_stride < n || up_stride < n || out_stride < n)) {
    return fail(DQ_INVALID_ARGUMENT, "row strides (%lld, %lld, %lld) must be >= n %lld", (long long)gate_stride,
                (long long)up_stride, (long long)out_stride, (long long)n);
  }
  const int64_t gs = m > 1 ? gate_stride : n, us = m > 1 ? up_stride : n, os = m > 1 ? out_stride : n;
  DQ_HIP(dq::launch_act_mul(act, gate, gs, up, us, m, n, out, os, as_stream(stream)), "act_mul launch");
  return DQ_OK;
}

int dq_matmul_gated(int act, const float* x, int64_t m, int64_t x_stride, const dq_weight* w_gate,
                    const dq_weight* w_up, float* out, int64_t out_stride, float* gate_scratch, float* up_scratch,
                    int64_t scratch_stride, void* stream) {
  if (!dq::act_ok(act)) return fail(DQ_INVALID_ARGUMENT, "unknown activation %d", act);
  if (w_gate == nullptr || w_up == nullptr) return fail(DQ_INVALID_ARGUMENT, "null weight");
  if (m < 0) return fail(DQ_INVALID_ARGUMENT, "m must be >= 0");
  const dq::WeightDev &g = w_gate->dev, &u = w_up->dev;
  if (g.n != u.n || g.k != u.k) {
    return fail(DQ_INVALID_ARGUMENT, "gate [%lld, %lld] and up [%lld, %lld] differ in shape", (long long)g.n,
                (long long)g.k, (long long)u.n, (long long)u.k);
  }
  if (g.device != u.device) return fail(DQ_INVALID_ARGUMENT, "gate and up weights are on different devices");
  if ((gate_scratch == nullptr) != (up_scratch == nullptr)) {
    return fail(DQ_INVALID_ARGUMENT, "gate_scratch and up_scratch are both given or both NULL");
  }
  if (m == 0) return DQ_OK;
  if (x == nullptr) return fail(DQ_INVALID_ARGUMENT, "null x");
  if (m > 1 && x_stride < g.k) return fail(DQ_INVALID_ARGUMENT, "x_stride %lld < k %lld", (long long)x_stride, (long long)g.k);
  if (int rc = check_out(w_gate, m, 0, g.n, out, out_stride); rc != DQ_OK) return rc;
  if (gate_scratch != nullptr && m > 1 && scratch_stride < g.n) {
    return fail(DQ_INVALID_ARGUMENT, "scratch_stride %lld < n %lld", (long long)scratch_stride, (long long)g.n);
  }
  hipStream_t s = as_stream(stream);
  const bool same = g.dtype == u.dtype;
  if (same && m == 1 && dq::gemv_gated_supported(g, u)) {
    // decode, one row: both weights' row groups in one GEMV launch
    DQ_HIP(dq::launch_gemv_gated(g, u, act, x, out, s), "gated gemv launch");
    return DQ_OK;
  }
  if (same && skinny_ok(w_gate, x, m, x_stride) && dq::gemv_mma_lds_ok(g.nblk, m, true)) {
    // decode batches: the skinny MFMA GEMV over both weights, act(g) * u in its chains
    std::vector<dq::GemvJob> j{
        dq::GemvJob{&g, nullptr, 0, x, m > 1 ? x_stride : g.k, m, out, m > 1 ? out_stride : g.n, nullptr, &u, act}};
    return run_skinny(j, g.device, s, dq::Region{});
  }
  // the unfused sequence of Device::matmul_gated (device.h:194-199)
  float* gp = gate_scratch;
  float* up = up_scratch;
  int64_t ss = m > 1 ? scratch_stride : g.n;
  if (gp == nullptr) {
    const int64_t plane = (m * g.n + 63) / 64 * 64;
    void* p = nullptr;
    if (int rc = scratch_get(g_fscratch, g.device, (size_t)(2 * plane) * sizeof(float), &p); rc != DQ_OK) return rc;
    gp = static_cast<float*>(p);
    up = gp + plane;
    ss = g.n;
  }
  const dq_matmul_job jobs[2] = {{w_gate, x, m, x_stride, gp, ss, nullptr}, {w_up, x, m, x_stride, up, ss, nullptr}};
  if (int rc = dq_matmul_many(jobs, 2, stream); rc != DQ_OK) return rc;
  return dq_act_mul(act, gp, ss, up, ss, m, g.n, out, out_stride, stream);
}

int dq_matmul_act(const dq_weight* w, int fmt, const float* x, int64_t m, int64_t x_stride, float* y, int64_t y_stride,
                  const float* bias, void* stream) {
  if (w == nullptr) return fail(DQ_INVALID_ARGUMENT, "null weight");
  if (!act_fmt_ok(fmt)) return fail(DQ_UNSUPPORTED, "activation format %d is not supported", fmt);
  if (!pair_ok(w->dev.dtype, fmt)) {
    return fail(DQ_UNSUPPORTED, "activation format %d is not supported with weight type %d", fmt, w->dev.dtype);
  }
  if (m < 0) return fail(DQ_INVALID_ARGUMENT, "m must be >= 0");
  if (m == 0) return DQ_OK;
  if (int rc = check_out(w, m, 0, w->dev.n, y, y_stride); rc != DQ_OK) return rc;
  if (x == nullptr) return fail(DQ_INVALID_ARGUMENT, "null argument");
  if (m > 1 && x_stride < w->dev.k) {
    return fail(DQ_INVALID_ARGUMENT, "x_stride %lld < k %lld", (long long)x_stride, (long long)w->dev.k);
  }
  if (dq_act_row_bytes(fmt, w->dev.k) < 0) {
    return fail(DQ_INVALID_ARGUMENT, "k %lld is not a multiple of the activation block", (long long)w->dev.k);
  }
  return dq::matmul_act_impl(w, fmt, x, m, x_stride, y, y_stride, bias, as_stream(stream), dq::Region{});
}

int dq_partials_count(int dtype, int fmt, int64_t k, int64_t* units, int64_t* sb_terms) {
  if (!weight_type_ok(dtype) || !act_fmt_ok(fmt) || !pair_ok(dtype, fmt) || fmt == DQ_ACT_F32) {
    return fail(DQ_UNSUPPORTED, "unsupported pair (%d, %d)", dtype, fmt);
  }
  if (dq_row_bytes(dtype, k) < 0 || dq_act_row_bytes(fmt, k) < 0) return fail(DQ_INVALID_ARGUMENT, "bad k");
  if (units) *units = dtype == DQ_Q6_K ? k / 16 : k / 32;
  if (sb_terms) *sb_terms = (dtype == DQ_Q4_K || dtype == DQ_Q6_K) && fmt == DQ_ACT_Q8_K ? 2 * (k / 256) : 0;
  return DQ_OK;
}

int dq_debug_partials(const dq_weight* w, int fmt, const void* acts, int64_t m, int32_t* units, int32_t* sb,
                      void* stream) {
  if (int rc = check_acts(w, fmt, acts, m); rc != DQ_OK) return rc;
  int64_t nu = 0, ns = 0;
  if (int rc = dq_partials_count(w->dev.dtype, fmt, w->dev.k, &nu, &ns); rc != DQ_OK) return rc;
  if (units == nullptr || (ns > 0 && sb == nullptr)) return fail(DQ_INVALID_ARGUMENT, "null output");
  if (m == 0) return DQ_OK;
  const int64_t arb = dq_act_row_bytes(fmt, w->dev.k);
  hipStream_t s = as_stream(stream);
  DQ_HIP(dq::launch_units(w->dev, fmt, static_cast<const uint8_t*>(acts), arb, m, units, nu, s), "units launch");
  if (ns > 0) {
    // The GEMV kernel writes its exact super-block reductions; y goes to scratch.
    void* yscratch = nullptr;
    if (int rc = scratch_get(w->dev.device, (size_t)(m * w->dev.n * 4), &yscratch); rc != DQ_OK) return rc;
    DQ_HIP(dq::launch_gemv(w->dev, fmt, static_cast<const uint8_t*>(acts), arb, m, 0, w->dev.n,
                           static_cast<float*>(yscratch), w->dev.n, nullptr, sb, s),
           "gemv launch");
  }
  return DQ_OK;
}

}  // extern "C"
