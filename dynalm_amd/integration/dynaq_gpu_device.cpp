// dynaq_gpu_device.cpp -- the Device of dynaq_gpu_device.h: tensors in HIP device
// memory, quantized matmuls on libdynaq under the step's KernelPlan.
#include "dynaq_gpu_device.h"

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstring>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace dynaq_shim {

// Uploaded weights: each library handle is also its tensor's data token.
struct WeightRegistry {
  std::mutex mu;
  std::unordered_map<const void*, dq_weight*> handles;
  std::atomic<int64_t> buffer_bytes{0};  // allocate()d bytes still held
};

namespace {

using dynacore::Status;
using dynacore::StatusCode;
using dynacore::TensorView;

Status from_dq(int rc, const char* what) {
  return Status(static_cast<StatusCode>(rc), std::string(what) + ": " + dq_last_error());
}
Status from_hip(hipError_t e, const char* what) {
  return dynacore::Internal(std::string(what) + ": " + hipGetErrorString(e));
}

// Makes `device` current for the scope (the library's calls use the current device
// for launches; its own entry points switch to a weight's device as needed).
struct DeviceScope {
  int prev = -1;
  explicit DeviceScope(int device) {
    if (hipGetDevice(&prev) == hipSuccess && prev != device) (void)hipSetDevice(device);
  }
  ~DeviceScope() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

// fp32 matrices [rows, cols] (a vector is one row); row strides in floats
int64_t rows_of(const TensorView& t) { return t.rank() > 1 ? t.dim(0) : 1; }
int64_t cols_of(const TensorView& t) { return t.dim(t.rank() - 1); }
int64_t row_floats(const TensorView& t) { return t.rank() > 1 ? t.stride(0) / 4 : cols_of(t); }
bool fp32_matrix(const TensorView& t) {
  return t.dtype() == dynacore::DType::kF32 && t.rank() >= 1 && t.rank() <= 2 &&
         (t.rank() == 1 || (t.stride(1) == 4 && t.stride(0) % 4 == 0));
}

}  // namespace

dynacore::Result<std::unique_ptr<DynaqGpuDevice>> DynaqGpuDevice::create(int gpu, void* stream) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || gpu < 0 || gpu >= count) {
    return dynacore::InvalidArgument("no HIP device " + std::to_string(gpu));
  }
  return std::unique_ptr<DynaqGpuDevice>(new DynaqGpuDevice(gpu, stream));
}

DynaqGpuDevice::DynaqGpuDevice(int gpu, void* stream)
    : gpu_(gpu), stream_(stream), weights_(std::make_shared<WeightRegistry>()) {
  (void)dq_plan_defaults(&plan_);  // KernelPlan::defaults() until the engine sets a plan
}

DynaqGpuDevice::~DynaqGpuDevice() {
  DeviceScope ds(gpu_);
  (void)hipStreamSynchronize(static_cast<hipStream_t>(stream_));
}

void DynaqGpuDevice::fail(Status st) {
  std::lock_guard<std::mutex> lock(mu_);
  if (first_error_.ok()) first_error_ = std::move(st);
}
void DynaqGpuDevice::fail_dq(int rc, const char* what) { fail(from_dq(rc, what)); }
void DynaqGpuDevice::unsupported(const char* op) {
  fail(dynacore::Unsupported(std::string(op) + " is outside the quantized-matmul path of the dynaq device"));
}

dynacore::Status DynaqGpuDevice::take_error() {
  std::lock_guard<std::mutex> lock(mu_);
  Status st = std::move(first_error_);
  first_error_ = Status::Ok();
  return st;
}

// ---- memory ----------------------------------------------------------------

dynacore::Result<std::shared_ptr<dynacore::Storage>> DynaqGpuDevice::allocate(size_t bytes) {
  DeviceScope ds(gpu_);
  void* p = nullptr;
  if (hipError_t e = hipMalloc(&p, bytes > 0 ? bytes : 1); e != hipSuccess) {
    return dynacore::OutOfMemory("hipMalloc of " + std::to_string(bytes) + " bytes: " + hipGetErrorString(e));
  }
  std::shared_ptr<WeightRegistry> reg = weights_;
  reg->buffer_bytes += (int64_t)bytes;
  const int gpu = gpu_;
  std::shared_ptr<const void> keep(p, [reg, gpu, bytes](const void* q) {
    DeviceScope s(gpu);
    (void)hipFree(const_cast<void*>(q));
    reg->buffer_bytes -= (int64_t)bytes;
  });
  return dynacore::Storage::borrow(p, bytes, device(), std::move(keep));
}

void DynaqGpuDevice::copy(void* dst, const void* src, size_t bytes) {
  DeviceScope ds(gpu_);
  if (hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream_));
      e != hipSuccess) {
    fail(from_hip(e, "copy"));
  }
}

void DynaqGpuDevice::synchronize() {
  DeviceScope ds(gpu_);
  if (hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream_)); e != hipSuccess) {
    fail(from_hip(e, "synchronize"));
  }
}

dynacore::Result<dynacore::Tensor> DynaqGpuDevice::upload(const dynacore::Tensor& host) {
  const TensorView& v = host.view();
  const int t = dq_type(v.dtype());
  if (t >= 0) {
    // a quantized weight [n, k]: the library's planes; the handle is the data token
    if (v.rank() != 2) return dynacore::InvalidArgument("a quantized weight is an [n, k] tensor");
    dq_weight* h = nullptr;
    {
      DeviceScope ds(gpu_);
      if (int rc = dq_weight_upload(t, v.data(), v.dim(0), v.dim(1), v.stride(0), stream_, &h); rc != DQ_OK) {
        return from_dq(rc, "upload");
      }
    }
    std::shared_ptr<WeightRegistry> reg = weights_;
    {
      std::lock_guard<std::mutex> lock(reg->mu);
      reg->handles[h] = h;
    }
    std::shared_ptr<const void> keep(h, [reg](const void* q) {
      dq_weight* hw = nullptr;
      {
        std::lock_guard<std::mutex> lock(reg->mu);
        auto it = reg->handles.find(q);
        if (it != reg->handles.end()) {
          hw = it->second;
          reg->handles.erase(it);
        }
      }
      if (hw != nullptr) (void)dq_weight_free(hw);
    });
    std::shared_ptr<dynacore::Storage> st =
        dynacore::Storage::borrow(h, (size_t)v.span_bytes(), device(), std::move(keep));
    return dynacore::Tensor::from_storage(std::move(st), TensorView(h, v.layout(), device()));
  }
  // anything else (fp32 / fp16 vectors, norms, biases): the bytes as they are
  const size_t bytes = (size_t)v.span_bytes();
  ENGINE_ASSIGN_OR_RETURN(std::shared_ptr<dynacore::Storage> st, allocate(bytes));
  {
    DeviceScope ds(gpu_);
    if (hipError_t e = hipMemcpy(st->data(), v.data(), bytes, hipMemcpyHostToDevice); e != hipSuccess) {
      return from_hip(e, "upload");
    }
  }
  void* data = st->data();
  return dynacore::Tensor::from_storage(std::move(st), TensorView(data, v.layout(), device()));
}

void DynaqGpuDevice::download(const TensorView& src, std::span<float> dst) {
  if (!fp32_matrix(src) || (int64_t)dst.size() < rows_of(src) * cols_of(src)) {
    fail(dynacore::InvalidArgument("download: an fp32 [rows, cols] tensor into rows * cols floats"));
    return;
  }
  DeviceScope ds(gpu_);
  const size_t width = (size_t)cols_of(src) * 4;
  hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream_));
  if (e == hipSuccess) {
    e = hipMemcpy2D(dst.data(), width, src.data(), (size_t)row_floats(src) * 4, width, (size_t)rows_of(src),
                    hipMemcpyDeviceToHost);
  }
  if (e != hipSuccess) fail(from_hip(e, "download"));
}

void DynaqGpuDevice::set_kernel_plan(const dynacore::KernelPlan& plan) {
  std::lock_guard<std::mutex> lock(mu_);
  plan_ = to_dq_plan(plan);
}

void DynaqGpuDevice::prepack_weight(const TensorView& w, bool int16_activations) {
  // upload() already laid the weight out for every kernel (int16 activations included)
  (void)w;
  (void)int16_activations;
}

dynacore::Device::MemoryStats DynaqGpuDevice::memory_stats() const {
  MemoryStats m;
  {
    std::lock_guard<std::mutex> lock(weights_->mu);
    for (const auto& kv : weights_->handles) {
      int64_t bytes = 0;
      if (dq_weight_info(kv.second, nullptr, nullptr, nullptr, &bytes) == DQ_OK) m.weight_bytes += bytes;
    }
  }
  m.buffer_bytes = weights_->buffer_bytes.load();
  DeviceScope ds(gpu_);
  size_t free_b = 0, total_b = 0;
  if (hipMemGetInfo(&free_b, &total_b) == hipSuccess) m.free_bytes = (int64_t)free_b;
  return m;
}

bool DynaqGpuDevice::supports_weight_type(dynacore::DType type) const { return dq_type(type) >= 0; }

// ---- matmuls -----------------------------------------------------------------

const dq_weight* DynaqGpuDevice::weight_of(const TensorView& w) const {
  std::lock_guard<std::mutex> lock(weights_->mu);
  auto it = weights_->handles.find(w.data());
  return it == weights_->handles.end() ? nullptr : it->second;
}

dq_selection DynaqGpuDevice::select(const TensorView& x, const TensorView& w) const {
  const dq_matmul_shape s{rows_of(x), w.dim(0), cols_of(x), dq_type(w.dtype()),
                          row_floats(x) == cols_of(x) ? 1 : 0};
  dq_plan p;
  {
    std::lock_guard<std::mutex> lock(mu_);
    p = plan_;
  }
  dq_selection sel{-1, -1};
  if (dq_select(&s, &p, &sel) != DQ_OK) sel = dq_selection{-1, -1};
  return sel;
}

void DynaqGpuDevice::matmul(const TensorView& x, const TensorView& w, const TensorView* bias, const TensorView& y) {
  const dq_weight* h = weight_of(w);
  if (h == nullptr) {
    fail(dynacore::InvalidArgument("matmul: w is not a whole weight uploaded by this device"));
    return;
  }
  if (!fp32_matrix(x) || !fp32_matrix(y) || cols_of(x) != w.dim(1) || rows_of(y) != rows_of(x) ||
      cols_of(y) != w.dim(0)) {
    fail(dynacore::InvalidArgument("matmul: x [m, k], w [n, k] and y [m, n] do not match"));
    return;
  }
  dq_plan p;
  {
    std::lock_guard<std::mutex> lock(mu_);
    p = plan_;
  }
  DeviceScope ds(gpu_);
  const int rc = dq_matmul_plan(h, &p, x.data_as<const float>(), rows_of(x), row_floats(x), y.data_as<float>(),
                                row_floats(y), bias != nullptr ? bias->data_as<const float>() : nullptr, stream_);
  if (rc != DQ_OK) fail_dq(rc, "matmul");
}

void DynaqGpuDevice::matmul_many(std::span<const MatmulJob> jobs) {
  // the jobs selected into the class dq_matmul runs (super-block int8 for K-quants,
  // per-32 int8 for Q8_0 / Q4_0) go to one grouped call, which computes exactly that
  // class; every other job runs as matmul() runs it
  std::vector<dq_matmul_job> grouped;
  for (const MatmulJob& j : jobs) {
    const dq_weight* h = weight_of(j.w);
    const dq_selection sel = h != nullptr ? select(j.x, j.w) : dq_selection{-1, -1};
    const bool same_class = (sel.kernel == DQ_KERNEL_INT8_SUPERBLOCK || sel.kernel == DQ_KERNEL_INT8_PER32) &&
                            sel.act == dq_act_format_for(dq_type(j.w.dtype()));
    if (!same_class || !fp32_matrix(j.x) || !fp32_matrix(j.y) || cols_of(j.x) != j.w.dim(1) ||
        rows_of(j.y) != rows_of(j.x) || cols_of(j.y) != j.w.dim(0)) {
      matmul(j.x, j.w, j.bias, j.y);  // checks and reports what does not fit
      continue;
    }
    grouped.push_back(dq_matmul_job{h, j.x.data_as<const float>(), rows_of(j.x), row_floats(j.x),
                                    j.y.data_as<float>(), row_floats(j.y),
                                    j.bias != nullptr ? j.bias->data_as<const float>() : nullptr});
  }
  if (grouped.empty()) return;
  DeviceScope ds(gpu_);
  if (int rc = dq_matmul_many(grouped.data(), (int64_t)grouped.size(), stream_); rc != DQ_OK) {
    fail_dq(rc, "matmul_many");
  }
}

void DynaqGpuDevice::act_mul(dynacore::Activation act, const TensorView& gate, const TensorView& up,
                             const TensorView& out) {
  if (!fp32_matrix(gate) || !fp32_matrix(up) || !fp32_matrix(out) || rows_of(up) != rows_of(gate) ||
      cols_of(up) != cols_of(gate) || rows_of(out) != rows_of(gate) || cols_of(out) != cols_of(gate)) {
    fail(dynacore::InvalidArgument("act_mul: gate, up and out must be fp32 [m, n] alike"));
    return;
  }
  DeviceScope ds(gpu_);
  const int rc = dq_act_mul(static_cast<int>(act), gate.data_as<const float>(), row_floats(gate),
                            up.data_as<const float>(), row_floats(up), rows_of(gate), cols_of(gate),
                            out.data_as<float>(), row_floats(out), stream_);
  if (rc != DQ_OK) fail_dq(rc, "act_mul");
}

void DynaqGpuDevice::matmul_gated(dynacore::Activation act, const TensorView& x, const TensorView& w_gate,
                                  const TensorView& w_up, const TensorView& out, const TensorView& gate_scratch,
                                  const TensorView& up_scratch) {
  const dq_weight* hg = weight_of(w_gate);
  const dq_weight* hu = weight_of(w_up);
  const dq_selection sel = hg != nullptr && hu != nullptr ? select(x, w_gate) : dq_selection{-1, -1};
  // the fused launch computes the super-block class; other selections take the
  // unfused sequence of the default (device.h:194-199) under the plan
  if (sel.kernel != DQ_KERNEL_INT8_SUPERBLOCK || w_up.dtype() != w_gate.dtype() || w_up.dim(0) != w_gate.dim(0) ||
      w_up.dim(1) != w_gate.dim(1) || !fp32_matrix(x) || !fp32_matrix(out) || !fp32_matrix(gate_scratch) ||
      !fp32_matrix(up_scratch) || row_floats(gate_scratch) != row_floats(up_scratch)) {
    matmul(x, w_gate, nullptr, gate_scratch);
    matmul(x, w_up, nullptr, up_scratch);
    act_mul(act, gate_scratch, up_scratch, out);
    return;
  }
  if (cols_of(x) != w_gate.dim(1) || rows_of(out) != rows_of(x) || cols_of(out) != w_gate.dim(0)) {
    fail(dynacore::InvalidArgument("matmul_gated: x [m, k], the weights [n, k] and out [m, n] do not match"));
    return;
  }
  DeviceScope ds(gpu_);
  const int rc = dq_matmul_gated(static_cast<int>(act), x.data_as<const float>(), rows_of(x), row_floats(x), hg, hu,
                                 out.data_as<float>(), row_floats(out), gate_scratch.data_as<float>(),
                                 up_scratch.data_as<float>(), row_floats(gate_scratch), stream_);
  if (rc != DQ_OK) fail_dq(rc, "matmul_gated");
}

// ---- outside the quantized-matmul path ----------------------------------------

void DynaqGpuDevice::embedding(const TensorView&, std::span<const int32_t>, const TensorView&) {
  unsupported("embedding");
}
void DynaqGpuDevice::rms_norm(const TensorView&, const TensorView&, float, const TensorView&) {
  unsupported("rms_norm");
}
void DynaqGpuDevice::layer_norm(const TensorView&, const TensorView&, const TensorView*, float, const TensorView&) {
  unsupported("layer_norm");
}
void DynaqGpuDevice::rope(const TensorView&, int32_t, int32_t, std::span<const int32_t>, const dynacore::RopeConfig&,
                          const float*) {
  unsupported("rope");
}
void DynaqGpuDevice::kv_store(const TensorView&, const TensorView&, std::span<const int32_t>,
                              std::span<const int32_t>, std::span<const dynacore::KvLayerView>) {
  unsupported("kv_store");
}
void DynaqGpuDevice::attention(const dynacore::AttentionParams&) { unsupported("attention"); }
void DynaqGpuDevice::activation(dynacore::Activation, const TensorView&, const TensorView&) {
  unsupported("activation");
}
void DynaqGpuDevice::add(const TensorView&, const TensorView&, const TensorView&) { unsupported("add"); }
void DynaqGpuDevice::scale(const TensorView&, float) { unsupported("scale"); }
void DynaqGpuDevice::softcap(const TensorView&, float) { unsupported("softcap"); }
void DynaqGpuDevice::fill(const TensorView&, float) { unsupported("fill"); }
void DynaqGpuDevice::gather_rows(const TensorView&, std::span<const int32_t>, const TensorView&) {
  unsupported("gather_rows");
}
void DynaqGpuDevice::scatter_add_rows(const TensorView&, std::span<const int32_t>, std::span<const float>,
                                      const TensorView&) {
  unsupported("scatter_add_rows");
}

}  // namespace dynaq_shim
