// dynaq_gpu_device.h -- a dynacore Device (dynacore/include/dynacore/device/device.h:70-219)
// whose tensors live in MI355X device memory and whose quantized matmuls run on libdynaq.
//
// Not part of libdynaq: a dynacore maintainer compiles dynaq_gpu_device.cpp into the
// engine and links libdynaq.so and the HIP runtime. It includes dynacore's headers,
// include/dynaq.h and <hip/hip_runtime_api.h> only; the tests compile it against the
// reference's headers and drive it through the reference's own Tensor and Storage
// (tests/test_integration_shim.py, tests/test_gpu_device.py).
//
// Scope: the quantized-matmul path of the Device interface -- memory (allocate, copy,
// synchronize, upload, download), set_kernel_plan, prepack_weight, supports_weight_type,
// matmul, matmul_many, matmul_gated, act_mul, memory_stats, take_error. The other ops
// (embedding, norms, RoPE, KV store, attention, elementwise, row gather / scatter, MoE)
// are outside that path: they record kUnsupported, which take_error() reports.
//
// Weights: upload() of a Q4_0 / Q8_0 / Q4_K / Q6_K tensor [n, k] repacks it into the
// library's device planes (dq_weight_upload), so prepack_weight has nothing left to do.
// The returned tensor's data pointer is a token for that handle, not device bytes (the
// runtime never dereferences device memory, device.h:80-86); matmul takes whole
// uploaded weights, as the engine passes them. Other dtypes are copied as they are.
//
// Accuracy class: set_kernel_plan keeps the step's KernelPlan, and every matmul runs
// the kernel dynacore's select_matmul picks under it (dq_select / dq_matmul_plan):
// sub-scaled int8 for K-quant decode rows, per-32 int8 for Q8_0 / Q4_0 up to 4 rows,
// int16 for the FFN down projection's plan, fp32 activations for larger batches; the
// super-block (Q8_K) class only when the plan asks for it. matmul_many and
// matmul_gated take libdynaq's grouped and fused launches for the jobs whose
// selection is that super-block class (the launches compute exactly that class),
// and the per-call route for the others.
#pragma once

#include <cstdint>
#include <memory>
#include <mutex>
#include <span>
#include <string_view>

#include "dynacore/device/device.h"
#include "dynaq.h"
#include "dynaq_convert.h"

namespace dynaq_shim {

struct WeightRegistry;

class DynaqGpuDevice final : public dynacore::Device {
 public:
  // GPU `gpu`; every op enqueues on `stream` (a hipStream_t, nullptr: the default stream).
  static dynacore::Result<std::unique_ptr<DynaqGpuDevice>> create(int gpu, void* stream = nullptr);
  ~DynaqGpuDevice() override;

  std::string_view name() const override { return "dynaq-mi355x"; }
  dynacore::DeviceLoc device() const override { return {dynacore::DeviceType::kHip, gpu_}; }
  bool host_accessible() const override { return false; }

  dynacore::Result<std::shared_ptr<dynacore::Storage>> allocate(size_t bytes) override;
  void copy(void* dst, const void* src, size_t bytes) override;
  void synchronize() override;
  dynacore::Result<dynacore::Tensor> upload(const dynacore::Tensor& host) override;
  void download(const dynacore::TensorView& src, std::span<float> dst) override;

  void set_kernel_plan(const dynacore::KernelPlan& plan) override;
  void prepack_weight(const dynacore::TensorView& w, bool int16_activations = false) override;
  dynacore::Status take_error() override;
  MemoryStats memory_stats() const override;
  bool supports_weight_type(dynacore::DType type) const override;

  void matmul(const dynacore::TensorView& x, const dynacore::TensorView& w, const dynacore::TensorView* bias,
              const dynacore::TensorView& y) override;
  void matmul_many(std::span<const MatmulJob> jobs) override;
  void act_mul(dynacore::Activation act, const dynacore::TensorView& gate, const dynacore::TensorView& up,
               const dynacore::TensorView& out) override;
  void matmul_gated(dynacore::Activation act, const dynacore::TensorView& x, const dynacore::TensorView& w_gate,
                    const dynacore::TensorView& w_up, const dynacore::TensorView& out,
                    const dynacore::TensorView& gate_scratch, const dynacore::TensorView& up_scratch) override;

  // outside the quantized-matmul path: kUnsupported
  void embedding(const dynacore::TensorView& table, std::span<const int32_t> ids,
                 const dynacore::TensorView& out) override;
  void rms_norm(const dynacore::TensorView& x, const dynacore::TensorView& weight, float eps,
                const dynacore::TensorView& y) override;
  void layer_norm(const dynacore::TensorView& x, const dynacore::TensorView& weight, const dynacore::TensorView* bias,
                  float eps, const dynacore::TensorView& y) override;
  void rope(const dynacore::TensorView& x, int32_t num_heads, int32_t head_dim, std::span<const int32_t> positions,
            const dynacore::RopeConfig& rope, const float* freq_factors) override;
  void kv_store(const dynacore::TensorView& k, const dynacore::TensorView& v, std::span<const int32_t> positions,
                std::span<const int32_t> row_seq, std::span<const dynacore::KvLayerView> kv) override;
  void attention(const dynacore::AttentionParams& p) override;
  void activation(dynacore::Activation act, const dynacore::TensorView& x, const dynacore::TensorView& out) override;
  void add(const dynacore::TensorView& a, const dynacore::TensorView& b, const dynacore::TensorView& y) override;
  void scale(const dynacore::TensorView& x, float s) override;
  void softcap(const dynacore::TensorView& x, float cap) override;
  void fill(const dynacore::TensorView& x, float value) override;
  void gather_rows(const dynacore::TensorView& src, std::span<const int32_t> rows,
                   const dynacore::TensorView& dst) override;
  void scatter_add_rows(const dynacore::TensorView& src, std::span<const int32_t> rows,
                        std::span<const float> weights, const dynacore::TensorView& dst) override;

  // The plan every matmul is selected under (the step's KernelPlan as a dq_plan).
  const dq_plan& plan() const { return plan_; }

 private:
  DynaqGpuDevice(int gpu, void* stream);
  // the library handle behind an uploaded weight's view (nullptr: not one of ours)
  const dq_weight* weight_of(const dynacore::TensorView& w) const;
  // the selection dq_select makes for this call under the current plan
  dq_selection select(const dynacore::TensorView& x, const dynacore::TensorView& w) const;
  void fail(dynacore::Status st);
  void fail_dq(int rc, const char* what);
  void unsupported(const char* op);

  int gpu_;
  void* stream_;
  dq_plan plan_{};
  std::shared_ptr<WeightRegistry> weights_;
  mutable std::mutex mu_;
  dynacore::Status first_error_;
  int64_t buffer_bytes_ = 0;
};

}  // namespace dynaq_shim
