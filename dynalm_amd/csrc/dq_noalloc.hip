// dq_noalloc.hip -- dq_matmul_noalloc: dq_matmul with every temporary in a static
// device array, for callers that cannot allocate device memory (code under HIP
// graph capture, serving loops that forbid hipMalloc).
//
// dq_matmul keeps its temporaries -- the quantized activations of the GEMM and
// skinny routes, the split-K row sums of the decode GEMV -- in per-device buffers
// that grow with hipMalloc on first use. This entry point takes them from
// `scratch` instead: a file-scope device array of DQ_NOALLOC_SCRATCH_BYTES, which
// every GPU the library runs on holds until the process ends. Its device address
// is looked up once per device (hipGetSymbolAddress, with that device current) and
// only that address is handed to kernels: the array's name is a host-side stand-in
// in host code, not a device pointer.
//
// All calls on one GPU share that GPU's array and it keeps the last call's
// contents. Nothing in it has to start at zero: each launch writes the quantized
// rows or row sums it later reads. Calls that overlap on one GPU (from different
// streams or threads without ordering) race on the array.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/dynaq.h"
#include "dq_internal.h"

static __device__ __align__(256) uint8_t scratch[DQ_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch_ptr[kMaxDevices] = {};  // per device: the device address of scratch

// The device address of `scratch` on `device`, looked up on the first call there.
int scratch_ptr(int device, void** out) {
  if (device < 0 || device >= kMaxDevices) {
    return dq::set_error(DQ_UNSUPPORTED, "dq_matmul_noalloc: device %d is beyond the %d it tracks", device,
                         kMaxDevices);
  }
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch_ptr[device] == nullptr) {
    dq::DeviceScope ds(device);
    if (ds.err != hipSuccess) return dq::set_error(DQ_INTERNAL, "hipSetDevice: %s", hipGetErrorString(ds.err));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      return dq::set_error(DQ_INTERNAL, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    }
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return DQ_OK;
}

}  // namespace

extern "C" int dq_matmul_noalloc(const dq_weight* w, const float* x, int64_t m, int64_t x_stride, float* y,
                                 int64_t y_stride, const float* bias, void* stream) {
  if (w == nullptr) return dq::set_error(DQ_INVALID_ARGUMENT, "null weight");
  if (m < 0) return dq::set_error(DQ_INVALID_ARGUMENT, "m must be >= 0");
  if (m == 0) return DQ_OK;
  if (x == nullptr || y == nullptr) return dq::set_error(DQ_INVALID_ARGUMENT, "null argument");
  if (m > 1 && x_stride < w->dev.k) {
    return dq::set_error(DQ_INVALID_ARGUMENT, "x_stride %lld < k %lld", (long long)x_stride, (long long)w->dev.k);
  }
  if (m > 1 && y_stride < w->dev.n) {
    return dq::set_error(DQ_INVALID_ARGUMENT, "y_stride %lld < n %lld", (long long)y_stride, (long long)w->dev.n);
  }
  const size_t need = dq::matmul_scratch_bytes(w, -1, m);
  if (need > (size_t)DQ_NOALLOC_SCRATCH_BYTES) {
    return dq::set_error(DQ_RESOURCE_EXHAUSTED,
                         "dq_matmul_noalloc: %lld rows of this %lld x %lld weight need %zu bytes of scratch, more than "
                         "the %zu of DQ_NOALLOC_SCRATCH_BYTES (use dq_matmul, or fewer rows per call)",
                         (long long)m, (long long)w->dev.n, (long long)w->dev.k, need,
                         (size_t)DQ_NOALLOC_SCRATCH_BYTES);
  }
  void* p = nullptr;
  if (int rc = scratch_ptr(w->dev.device, &p); rc != DQ_OK) return rc;
  const dq::Region r{static_cast<uint8_t*>(p), (size_t)DQ_NOALLOC_SCRATCH_BYTES};
  return dq::matmul_impl(w, x, m, x_stride, y, y_stride, bias, static_cast<hipStream_t>(stream), r);
}
