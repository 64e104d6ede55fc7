// Test infrastructure only: drives dynaq_shim::DynaqGpuDevice
// (dynalm_amd/integration/dynaq_gpu_device.cpp) through the reference's own Tensor,
// Storage, Status and KernelPlan, compiled from the reference's sources into
// _ref/libdqdevice_ref.so by the Makefile here (target `device`). tests/test_gpu_device.py
// calls dqdev_run through ctypes; nothing else loads it.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "dynaq_gpu_device.h"

using dynacore::DType;
using dynacore::KernelPlan;
using dynacore::Status;
using dynacore::Tensor;
using dynacore::TensorLayout;
using dynacore::TensorShape;
using dynacore::TensorView;

namespace {

DType to_dtype(int dq) {
  switch (dq) {
    case DQ_Q4_0: return DType::kQ4_0;
    case DQ_Q8_0: return DType::kQ8_0;
    case DQ_Q4_K: return DType::kQ4_K;
    case DQ_Q6_K: return DType::kQ6_K;
    default: return DType::kCount;
  }
}

int report(const Status& st, char* err, int err_len) {
  if (err != nullptr && err_len > 0) {
    std::strncpy(err, st.message().c_str(), (size_t)err_len - 1);
    err[err_len - 1] = '\0';
  }
  return st.ok() ? 0 : static_cast<int>(st.code());
}

// A device fp32 matrix [rows, cols] with a row stride of `stride` floats.
dynacore::Result<Tensor> device_matrix(dynaq_shim::DynaqGpuDevice& dev, int64_t rows, int64_t cols, int64_t stride) {
  ENGINE_ASSIGN_OR_RETURN(std::shared_ptr<dynacore::Storage> st, dev.allocate((size_t)(rows * stride * 4)));
  TensorLayout layout;
  layout.dtype = DType::kF32;
  layout.shape = TensorShape{rows, cols};
  layout.strides[0] = stride * 4;
  layout.strides[1] = 4;
  void* data = st->data();
  return Tensor::from_storage(std::move(st), TensorView(data, layout, dev.device()));
}

}  // namespace

extern "C" {

// One Device call on GPU `gpu`: weights w1 (and w2) of type dq_dtype [n, k] from host rows of
// row_bytes each, uploaded with Device::upload; x [m, k] fp32 (row stride x_stride floats)
// copied into device memory from the host; the plan KernelPlan's member defaults (plan_kind 0:
// KernelPlan::defaults() without its environment overrides) or the all-integer plan (1: super-block int8 at every m
// without qmm, as dq_matmul); then
//   op 0: matmul(x, w1, bias) -> y [m, n]
//   op 1: matmul_many({x, w1, bias, y0}, {x, w2, null, y1}) -> y [2][m][n]
//   op 2: matmul_gated(SiLU, x, w1, w2) -> y [m, n]
//   op 3: fill(y, 0) (outside the path: take_error must report kUnsupported; returns 0 then)
// and synchronize, download into y_out, take_error. Returns 0 or the StatusCode, with the
// message in err. memory[0..2] (may be NULL): weight_bytes, buffer_bytes, free_bytes seen
// before the tensors are released.
int dqdev_run(int gpu, int op, int plan_kind, int dq_dtype, const void* w1_rows, const void* w2_rows, int64_t n,
              int64_t k, int64_t row_bytes, const float* x, int64_t m, int64_t x_stride, const float* bias,
              float* y_out, int64_t* memory, char* err, int err_len) {
  auto made = dynaq_shim::DynaqGpuDevice::create(gpu);
  if (!made.ok()) return report(made.status(), err, err_len);
  dynaq_shim::DynaqGpuDevice& dev = **made;

  const DType dt = to_dtype(dq_dtype);
  if (!dev.supports_weight_type(dt)) return report(dynacore::InvalidArgument("weight type"), err, err_len);
  auto up = [&](const void* rows) -> dynacore::Result<Tensor> {
    ENGINE_ASSIGN_OR_RETURN(Tensor host, Tensor::empty(dt, TensorShape{n, k}));
    if (host.view().stride(0) != row_bytes) return dynacore::InvalidArgument("row bytes differ from the layout's");
    std::memcpy(host.data(), rows, (size_t)(n * row_bytes));
    return dev.upload(host);
  };
  auto w1 = up(w1_rows);
  if (!w1.ok()) return report(w1.status(), err, err_len);
  dynacore::Result<Tensor> w2 = Tensor();
  if (op == 1 || op == 2) {
    w2 = up(w2_rows);
    if (!w2.ok()) return report(w2.status(), err, err_len);
  }

  auto xd = device_matrix(dev, m, k, x_stride);
  const int64_t outs = op == 1 ? 2 : 1;
  auto yd = device_matrix(dev, outs * m, n, n);
  auto gs = device_matrix(dev, m, n, n);
  auto us = device_matrix(dev, m, n, n);
  if (!xd.ok() || !yd.ok() || !gs.ok() || !us.ok()) return report(dynacore::OutOfMemory("buffers"), err, err_len);
  if (hipMemcpy(xd->data(), x, (size_t)(m * x_stride * 4), hipMemcpyHostToDevice) != hipSuccess) {
    return report(dynacore::Internal("copy x"), err, err_len);
  }
  dynacore::Result<Tensor> bd = Tensor();
  if (bias != nullptr) {
    auto hb = Tensor::empty(DType::kF32, TensorShape{n});
    if (!hb.ok()) return report(hb.status(), err, err_len);
    std::memcpy(hb->data(), bias, (size_t)(n * 4));
    bd = dev.upload(*hb);
    if (!bd.ok()) return report(bd.status(), err, err_len);
  }
  const TensorView* bias_view = bias != nullptr ? &bd->view() : nullptr;

  KernelPlan plan{};
  if (plan_kind == 1) {
    plan.int8_decode_max_rows = 1 << 30;
    plan.int8_superblock_max_rows = 1 << 30;
    plan.int8_superblock_min_rows = 1;
    plan.int8_subscale_min_rows = 0;
    plan.qmm = false;  // dq_matmul's plan selects without qmm
  }
  dev.set_kernel_plan(plan);

  auto y_rows = [&](int64_t i) { return *yd->view().slice(0, i * m, m); };
  switch (op) {
    case 0: dev.matmul(xd->view(), w1->view(), bias_view, yd->view()); break;
    case 1: {
      const dynacore::Device::MatmulJob jobs[2] = {{xd->view(), w1->view(), y_rows(0), bias_view},
                                                   {xd->view(), w2->view(), y_rows(1), nullptr}};
      dev.matmul_many(jobs);
      break;
    }
    case 2:
      dev.matmul_gated(dynacore::Activation::kSilu, xd->view(), w1->view(), w2->view(), yd->view(), gs->view(),
                       us->view());
      break;
    case 3: {
      dev.fill(yd->view(), 0.0f);
      const Status st = dev.take_error();
      return st.code() == dynacore::StatusCode::kUnsupported ? 0 : report(dynacore::Internal("fill"), err, err_len);
    }
    default: return report(dynacore::InvalidArgument("op"), err, err_len);
  }
  dev.synchronize();
  dev.download(yd->view(), std::span<float>(y_out, (size_t)(outs * m * n)));
  if (memory != nullptr) {
    const dynacore::Device::MemoryStats ms = dev.memory_stats();
    memory[0] = ms.weight_bytes;
    memory[1] = ms.buffer_bytes;
    memory[2] = ms.free_bytes;
  }
  return report(dev.take_error(), err, err_len);
}

}  // extern "C"
