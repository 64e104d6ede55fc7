// dynaq_cpu_shim.cpp -- puts libdynaq behind a dynacore CpuDevice through its run-time
// extension point ExternalMatmulKernel {name, eligible, run}
// (dynacore/include/dynacore/cpu/cpu_device.h:22-30; registered with
// CpuDevice::register_external_matmul, cpu_device.cpp:818-826; consulted first when
// KernelPlan::external_matmul is set, matmul_registry.cpp:292-299).
//
// Not part of libdynaq: a dynacore maintainer compiles this file into the engine and
// links libdynaq.so. It includes dynacore's headers and include/dynaq.h only; the
// tests compile it against the reference's headers (tests/test_integration_shim.py).
//
// Accuracy class: on every call run() hands the device's current KernelPlan
// (CpuDevice::kernel_plan, cpu_device.h:54) to the adapter, which selects the kernel
// as dynacore's select_matmul would (dq_select). A default-plan engine therefore gets
// sub-scaled int8 for K-quant decode rows, per-32 int8 for Q8_0 / Q4_0 up to 4 rows,
// int16 for the FFN down projection (the plan the model sets around it,
// dynalm/src/model/transformer.cpp:538-550) and fp32 activations for larger batches,
// as on the CPU; the super-block (Q8_K) class stays opt-in.
#include <cstdlib>
#include <utility>

#include "dynacore/cpu/cpu_device.h"
#include "dynaq.h"
#include "dynaq_convert.h"

namespace dynaq_shim {

// Registers GPU `gpu` as `dev`'s external matmul kernel for calls of at least min_rows
// rows, keeping up to `limit` bytes of weight copies in HBM (0: all). Call before
// serving (cpu_device.h:70-72) and set KernelPlan::external_matmul. *out is the
// adapter: free it with dq_external_free once `dev` no longer runs matmuls.
dynacore::Status register_dynaq(dynacore::CpuDevice& dev, int gpu, int64_t min_rows, int64_t limit,
                                dq_external** out) {
  dq_external* e = nullptr;
  if (int rc = dq_external_create(gpu, min_rows, limit, &e); rc != DQ_OK) {
    return dynacore::Status(static_cast<dynacore::StatusCode>(rc), dq_last_error());
  }
  dynacore::ExternalMatmulKernel k;
  k.name = "dynaq-mi355x";
  k.eligible = [e](const dynacore::MatmulShape& s, const void* w) {  // reads no tensor data
    const dq_matmul_shape q{s.m, s.n, s.k, dq_type(s.weight), s.x_dense ? 1 : 0};
    return dq_external_eligible(e, &q, w) == 1;
  };
  k.run = [e, &dev](const dynacore::TensorView& x, const dynacore::TensorView& w, const dynacore::TensorView* bias,
                    const dynacore::TensorView& y) {
    const dq_plan plan = to_dq_plan(dev.kernel_plan());
    const int64_t m = x.rank() > 1 ? x.dim(0) : 1, kk = x.dim(x.rank() - 1), n = w.dim(0);
    const int64_t x_stride = x.rank() > 1 ? x.stride(0) / 4 : kk, y_stride = y.rank() > 1 ? y.stride(0) / 4 : n;
    int rc = dq_external_set_plan(e, &plan);
    if (rc == DQ_OK) {
      rc = dq_external_run(e, x.data_as<const float>(), m, x_stride, w.data(), dq_type(w.dtype()), n, kk, w.stride(0),
                           bias != nullptr ? bias->data_as<const float>() : nullptr, y.data_as<float>(), y_stride);
    }
    if (rc != DQ_OK) std::abort();  // ops are void and cannot fail on valid shapes (device.h:11-13)
  };
  if (dynacore::Status st = dev.register_external_matmul(std::move(k)); !st.ok()) {
    dq_external_free(e);
    return st;
  }
  *out = e;
  return dynacore::Status::Ok();
}

}  // namespace dynaq_shim
