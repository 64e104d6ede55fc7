// dynaq_convert.h -- the two type conversions the reference-side bindings share
// (dynaq_cpu_shim.cpp, dynaq_gpu_device.cpp): KernelPlan's matmul knobs as a dq_plan
// and dynacore's DType as a dq weight type. Header-only, so both files can be linked
// into one engine.
#pragma once

#include "dynacore/kernel/kernel_plan.h"
#include "dynacore/tensor/dtype.h"
#include "dynaq.h"

namespace dynaq_shim {

// KernelPlan's matmul knobs (kernel_plan.h:34-148) as a dq_plan. MatmulKernelId bits
// are dq_kernel bits, so matmul_disabled carries over.
inline dq_plan to_dq_plan(const dynacore::KernelPlan& p) {
  dq_plan q;
  q.expand_min_rows = p.expand_min_rows;
  q.int8_decode_max_rows = p.int8_decode_max_rows;
  q.int16_decode_max_rows = p.int16_decode_max_rows;
  q.int8_superblock_min_rows = p.int8_superblock_min_rows;
  q.int8_superblock_max_rows = p.int8_superblock_max_rows;
  q.int8_subscale_min_rows = p.int8_subscale_min_rows;
  q.matmul_disabled = p.matmul_disabled;
  q.qmm = p.qmm ? 1 : 0;
  q.qmm_gemm_min_rows = p.qmm_gemm_min_rows;
  return q;
}

// DType values are dq_dtype values for the four weight types (-1: none of them).
inline int dq_type(dynacore::DType t) {
  switch (t) {
    case dynacore::DType::kQ4_0: return DQ_Q4_0;
    case dynacore::DType::kQ8_0: return DQ_Q8_0;
    case dynacore::DType::kQ4_K: return DQ_Q4_K;
    case dynacore::DType::kQ6_K: return DQ_Q6_K;
    default: return -1;
  }
}

}  // namespace dynaq_shim
