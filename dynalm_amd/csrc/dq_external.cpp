// dq_external.cpp -- host-memory matmul adapter: the shape of dynacore's run-time
// extension point ExternalMatmulKernel {name, eligible(shape, weight), run(x, w,
// bias, y)} (dynacore/include/dynacore/cpu/cpu_device.h:22-30), consulted by
// CpuDevice before its built-in kernels (dynacore/cpu/cpu_device.cpp:810-826,909-911).
//
// A CPU-resident engine hands over host tensors: fp32 x rows, GGUF weight rows as
// mapped from the file, an optional fp32 bias and fp32 y rows. This adapter keeps
// one device copy per weight it has been given, keyed by the weight's host address,
// type, shape and row stride, as CpuDevice keys its prepacked copies by data pointer
// and (n, k) (dynacore/include/dynacore/cpu/cpu_device.h:135-143,188-206); copies
// of the least recently used weights are dropped when a byte limit is set. x goes
// in and y comes back through pinned staging buffers on the adapter's own stream.
// In between, the kernel dynacore would select under the adapter's KernelPlan runs
// (dq_select; the defaults until dq_external_set_plan, Device::set_kernel_plan), so
// the accuracy class is the reference's, and results are dq_matmul_plan's on the
// same rows. The adapter's temporaries live in its own device buffer, so adapters
// on one GPU never share them. A call returns when y is written.
#include <hip/hip_runtime.h>

#include <cstring>
#include <list>
#include <mutex>
#include <new>

#include "../../include/dynaq.h"
#include "dq_internal.h"
#include "dq_layout.h"

namespace {

struct Key {
  const void* w;
  int dtype;
  int64_t n, k, row_bytes;
  bool operator==(const Key& o) const {
    return w == o.w && dtype == o.dtype && n == o.n && k == o.k && row_bytes == o.row_bytes;
  }
};

struct Entry {
  Key key;
  dq_weight* h;
  int64_t bytes;
};

bool type_ok(int t) { return t == DQ_Q4_0 || t == DQ_Q8_0 || t == DQ_Q4_K || t == DQ_Q6_K; }

// Device bytes of a weight's copy: its rows padded to the 64-row group.
int64_t copy_bytes(int dtype, int64_t n, int64_t k) {
  return (n + dq::kRowGroup - 1) / dq::kRowGroup * dq::kRowGroup * dq_row_bytes(dtype, k);
}

// The shape rules of dq_weight_upload and dq_matmul (validate_matmul_shape,
// dynacore/src/kernel/matmul_registry.cpp:264-278), answered without a GPU.
bool shape_ok(int64_t m, int64_t n, int64_t k, int dtype) {
  if (!type_ok(dtype) || m <= 0 || n <= 0 || k <= 0) return false;
  const int be = dq::block_elems(dtype);
  if (k % be != 0) return false;
  return (k / be) * dq::kRowGroup * 128 < ((int64_t)1 << 31);
}

}  // namespace

struct dq_external {
  int device = 0;
  int64_t min_rows = 1;
  int64_t max_bytes = 0;  // 0: no limit
  hipStream_t stream = nullptr;
  std::mutex mu;
  std::list<Entry> lru;  // most recently used first
  int64_t resident = 0;
  dq_external_stats stats{};
  // staging: pinned host and device buffers, grown on demand
  void* h_stage = nullptr;
  size_t h_bytes = 0;
  void* d_stage = nullptr;  // x, y, bias, then this adapter's matmul temporaries
  size_t d_bytes = 0;
  dq_plan plan = dq::default_plan();  // Device::set_kernel_plan
};

namespace {

int hip_status(hipError_t e, const char* what) {
  return dq::set_error(e == hipErrorOutOfMemory ? DQ_OUT_OF_MEMORY : DQ_INTERNAL, "%s: %s", what,
                       hipGetErrorString(e));
}

using dq::DeviceScope;

int grow(dq_external* e, size_t host, size_t dev) {
  if (e->h_bytes < host) {
    if (e->h_stage != nullptr) {
      if (hipError_t r = hipHostFree(e->h_stage); r != hipSuccess) return hip_status(r, "hipHostFree");
      e->h_stage = nullptr;
      e->h_bytes = 0;
    }
    const size_t sz = host < ((size_t)1 << 20) ? ((size_t)1 << 20) : host;
    if (hipError_t r = hipHostMalloc(&e->h_stage, sz, hipHostMallocDefault); r != hipSuccess) {
      e->h_stage = nullptr;
      return hip_status(r, "hipHostMalloc(staging)");
    }
    e->h_bytes = sz;
  }
  if (e->d_bytes < dev) {
    if (e->d_stage != nullptr) {
      if (hipError_t r = hipFree(e->d_stage); r != hipSuccess) return hip_status(r, "hipFree");
      e->d_stage = nullptr;
      e->d_bytes = 0;
    }
    const size_t sz = dev < ((size_t)1 << 20) ? ((size_t)1 << 20) : dev;
    if (hipError_t r = hipMalloc(&e->d_stage, sz); r != hipSuccess) {
      e->d_stage = nullptr;
      return hip_status(r, "hipMalloc(staging)");
    }
    e->d_bytes = sz;
  }
  return DQ_OK;
}

void drop(dq_external* e, std::list<Entry>::iterator it) {
  dq_weight_free(it->h);
  e->resident -= it->bytes;
  e->lru.erase(it);
}

// The device copy of weight `key`: found (moved to the front) or uploaded (after
// dropping least recently used copies to stay within the byte limit). *transient
// is set when the weight alone exceeds the limit: the caller frees it after use.
int weight_for(dq_external* e, const Key& key, dq_weight** out, bool* transient) {
  *transient = false;
  for (auto it = e->lru.begin(); it != e->lru.end(); ++it) {
    if (it->key == key) {
      e->lru.splice(e->lru.begin(), e->lru, it);
      ++e->stats.hits;
      *out = it->h;
      return DQ_OK;
    }
  }
  const int64_t bytes = copy_bytes(key.dtype, key.n, key.k);
  if (e->max_bytes > 0) {
    while (!e->lru.empty() && e->resident + bytes > e->max_bytes) {
      drop(e, std::prev(e->lru.end()));
      ++e->stats.evictions;
    }
  }
  dq_weight* h = nullptr;
  if (int rc = dq_weight_upload(key.dtype, key.w, key.n, key.k, key.row_bytes, e->stream, &h); rc != DQ_OK) return rc;
  ++e->stats.uploads;
  if (e->max_bytes > 0 && bytes > e->max_bytes) {
    *transient = true;
  } else {
    e->lru.push_front(Entry{key, h, bytes});
    e->resident += bytes;
  }
  *out = h;
  return DQ_OK;
}

}  // namespace

extern "C" {

int dq_external_create(int device, int64_t min_rows, int64_t max_resident_bytes, dq_external** out) {
  if (out == nullptr) return dq::set_error(DQ_INVALID_ARGUMENT, "null argument");
  *out = nullptr;
  if (device < 0 || min_rows < 1 || max_resident_bytes < 0) {
    return dq::set_error(DQ_INVALID_ARGUMENT, "bad adapter settings (device %d, min_rows %lld, limit %lld)", device,
                         (long long)min_rows, (long long)max_resident_bytes);
  }
  int count = 0;
  if (hipError_t r = hipGetDeviceCount(&count); r != hipSuccess) return hip_status(r, "hipGetDeviceCount");
  if (device >= count) return dq::set_error(DQ_INVALID_ARGUMENT, "device %d of %d", device, count);
  auto* e = new (std::nothrow) dq_external();
  if (e == nullptr) return dq::set_error(DQ_OUT_OF_MEMORY, "host allocation failed");
  e->device = device;
  e->min_rows = min_rows;
  e->max_bytes = max_resident_bytes;
  DeviceScope ds(device);
  hipError_t r = ds.err;
  if (r == hipSuccess) r = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking);
  if (r != hipSuccess) {
    delete e;
    return hip_status(r, "adapter stream");
  }
  *out = e;
  return DQ_OK;
}

int dq_external_free(dq_external* e) {
  if (e == nullptr) return DQ_OK;
  DeviceScope ds(e->device);
  int rc = DQ_OK;
  if (e->stream != nullptr) {
    if (hipError_t r = hipStreamSynchronize(e->stream); r != hipSuccess) rc = hip_status(r, "hipStreamSynchronize");
  }
  while (!e->lru.empty()) drop(e, e->lru.begin());
  if (e->h_stage != nullptr) (void)hipHostFree(e->h_stage);
  if (e->d_stage != nullptr) (void)hipFree(e->d_stage);
  if (e->stream != nullptr) (void)hipStreamDestroy(e->stream);
  delete e;
  return rc;
}

int dq_external_eligible(const dq_external* e, const dq_matmul_shape* s, const void* weight) {
  if (s == nullptr || weight == nullptr) return 0;
  const int64_t min_rows = e != nullptr ? e->min_rows : 1;
  return shape_ok(s->m, s->n, s->k, s->dtype) && s->m >= min_rows ? 1 : 0;
}

int dq_external_run(dq_external* e, const float* x, int64_t m, int64_t x_stride, const void* w, int dtype, int64_t n,
                    int64_t k, int64_t w_row_bytes, const float* bias, float* y, int64_t y_stride) {
  if (e == nullptr || x == nullptr || w == nullptr || y == nullptr) {
    return dq::set_error(DQ_INVALID_ARGUMENT, "null argument");
  }
  if (!type_ok(dtype)) return dq::set_error(DQ_UNSUPPORTED, "weight type %d is not supported", dtype);
  if (!shape_ok(m, n, k, dtype)) {
    return dq::set_error(DQ_INVALID_ARGUMENT, "bad shape (m %lld, n %lld, k %lld)", (long long)m, (long long)n,
                         (long long)k);
  }
  if ((m > 1 && x_stride < k) || (m > 1 && y_stride < n)) {
    return dq::set_error(DQ_INVALID_ARGUMENT, "row strides (x %lld, y %lld) below the row lengths", (long long)x_stride,
                         (long long)y_stride);
  }
  if (w_row_bytes < dq_row_bytes(dtype, k)) {
    return dq::set_error(DQ_INVALID_ARGUMENT, "w_row_bytes %lld < %lld", (long long)w_row_bytes,
                         (long long)dq_row_bytes(dtype, k));
  }
  std::lock_guard<std::mutex> lock(e->mu);
  DeviceScope ds(e->device);
  if (ds.err != hipSuccess) return hip_status(ds.err, "hipSetDevice");
  dq_weight* h = nullptr;
  bool transient = false;
  if (int rc = weight_for(e, Key{w, dtype, n, k, w_row_bytes}, &h, &transient); rc != DQ_OK) return rc;
  // The kernel under the adapter's plan, chosen from the caller's layout of x (as
  // CpuDevice::matmul chooses, cpu_device.cpp:869-897).
  const dq_matmul_shape shape{m, n, k, dtype, (int32_t)(m == 1 || x_stride == k)};
  const dq_selection sel = dq::select(shape, e->plan);
  // dense device rows: x [m][k], y [m][n], bias [n], then the matmul's temporaries
  // (this adapter's own: adapters never share scratch); one pinned buffer for x and y
  const size_t xb = (size_t)(m * k) * 4, yb = (size_t)(m * n) * 4, bb = bias ? (size_t)n * 4 : 0;
  const size_t xo = 0, yo = (xb + 255) / 256 * 256, bo = yo + (yb + 255) / 256 * 256;
  const size_t so = bo + (bb + 255) / 256 * 256, sb = dq::sel_scratch_bytes(h, sel, m);
  int rc = grow(e, xb > yb ? xb : yb, so + sb);
  if (rc != DQ_OK) {
    if (transient) dq_weight_free(h);
    return rc;
  }
  auto* hs = static_cast<float*>(e->h_stage);
  auto* dbase = static_cast<uint8_t*>(e->d_stage);
  float* dx = reinterpret_cast<float*>(dbase + xo);
  float* dy = reinterpret_cast<float*>(dbase + yo);
  float* dbias = bias ? reinterpret_cast<float*>(dbase + bo) : nullptr;
  const dq::Region region{dbase + so, sb};
  hipError_t r = hipSuccess;
  if (bias != nullptr) r = hipMemcpyAsync(dbias, bias, bb, hipMemcpyHostToDevice, e->stream);
  for (int64_t i = 0; i < m; ++i) std::memcpy(hs + i * k, x + i * (m > 1 ? x_stride : k), (size_t)k * 4);
  if (r == hipSuccess) r = hipMemcpyAsync(dx, hs, xb, hipMemcpyHostToDevice, e->stream);
  // the pinned buffer is reused for y: x must have left it first
  if (r == hipSuccess) r = hipStreamSynchronize(e->stream);
  if (r != hipSuccess) {
    rc = hip_status(r, "adapter input copy");
  } else {
    rc = dq::matmul_sel_impl(h, sel, dx, m, k, dy, n, dbias, e->stream, region);
  }
  if (rc == DQ_OK) {
    r = hipMemcpyAsync(hs, dy, yb, hipMemcpyDeviceToHost, e->stream);
    if (r == hipSuccess) r = hipStreamSynchronize(e->stream);
    if (r != hipSuccess) {
      rc = hip_status(r, "adapter output copy");
    } else {
      for (int64_t i = 0; i < m; ++i) std::memcpy(y + i * (m > 1 ? y_stride : n), hs + i * n, (size_t)n * 4);
      ++e->stats.runs;
    }
  }
  if (transient) {
    (void)hipStreamSynchronize(e->stream);
    dq_weight_free(h);
  }
  return rc;
}

int dq_external_forget(dq_external* e, const void* weight) {
  if (e == nullptr || weight == nullptr) return dq::set_error(DQ_INVALID_ARGUMENT, "null argument");
  std::lock_guard<std::mutex> lock(e->mu);
  DeviceScope ds(e->device);
  if (hipError_t r = hipStreamSynchronize(e->stream); r != hipSuccess) return hip_status(r, "hipStreamSynchronize");
  bool found = false;
  for (auto it = e->lru.begin(); it != e->lru.end();) {
    auto next = std::next(it);
    if (it->key.w == weight) {
      drop(e, it);
      found = true;
    }
    it = next;
  }
  return found ? DQ_OK : dq::set_error(DQ_NOT_FOUND, "no device copy of that weight");
}

int dq_external_set_plan(dq_external* e, const dq_plan* plan) {
  if (e == nullptr) return dq::set_error(DQ_INVALID_ARGUMENT, "null adapter");
  std::lock_guard<std::mutex> lock(e->mu);
  e->plan = plan != nullptr ? *plan : dq::default_plan();
  return DQ_OK;
}

int dq_external_get_stats(dq_external* e, dq_external_stats* out) {
  if (e == nullptr || out == nullptr) return dq::set_error(DQ_INVALID_ARGUMENT, "null argument");
  std::lock_guard<std::mutex> lock(e->mu);
  *out = e->stats;
  out->resident_bytes = e->resident;
  out->resident_weights = (int64_t)e->lru.size();
  return DQ_OK;
}

}  // extern "C"
