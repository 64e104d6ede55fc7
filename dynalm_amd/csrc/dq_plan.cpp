// dq_plan.cpp -- dynacore's per-call kernel selection (accuracy classes) for this
// library's kernels: KernelPlan's matmul knobs (dynacore/include/dynacore/kernel/
// kernel_plan.h:29-192) and select_matmul (dynacore/src/kernel/matmul_registry.cpp:
// 94-191,287-429), restated for the kernels that exist on the GPU.
//
// The GPU offers what dynacore calls, in MatmulCaps (matmul_registry.h:103-123), an
// int8-accelerated backend with the quantizers quantize_act / _sb / _sx / 16, per-32
// row dots for all four weight types, super-block and sub-scaled dots for Q4_K and
// Q6_K, int16 row dots for all four weight types, and qmm (qmm.h's int8 and int16
// contracts for every weight type, with a gemm kernel for Q8_0, Q4_0 and Q4_K). It has
// none of the kernels that read dynacore's interleaved x8 copies, no SME and no
// external kernels of
// its own, so selection passes over those as the reference does when their caps are
// absent. Host code only; no GPU is needed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "../../include/dynaq.h"
#include "dq_internal.h"

namespace {

bool allowed(const dq_plan& p, int id) { return (p.matmul_disabled & (1u << id)) == 0; }

bool kquant(int t) { return t == DQ_Q4_K || t == DQ_Q6_K; }

// MatmulCaps::qmm_gemm of this GPU: the weight types whose qmm rows run on a GEMM kernel
// (dq_gemm_b32.hip, dq_gemm_p32.hip, dq_gemm_q16.hip, dq_gemm_q6x.hip): all four.
bool qmm_gemm(int t) { return t == DQ_Q8_0 || t == DQ_Q4_0 || t == DQ_Q4_K || t == DQ_Q6_K; }

}  // namespace

namespace dq {

dq_plan default_plan() {
  dq_plan p;
  p.expand_min_rows = 2;           // kernel_plan.h:34
  p.int8_decode_max_rows = 4;      // kernel_plan.h:58
  p.int16_decode_max_rows = 0;     // kernel_plan.h:66
  p.int8_superblock_min_rows = 0;  // kernel_plan.h:77 (fails DD-053: off)
  p.int8_superblock_max_rows = 8;  // kernel_plan.h:81
  p.int8_subscale_min_rows = 1;    // kernel_plan.h:92
  p.matmul_disabled = 0;           // kernel_plan.h:148
  p.qmm = 1;                       // kernel_plan.h:156
  p.qmm_gemm_min_rows = 9;         // kernel_plan.h:158
  return p;
}

dq_selection select(const dq_matmul_shape& s, const dq_plan& p) {
  const int64_t m = s.m, k = s.k;
  const int wt = s.dtype;
  // Native qmm kernels (matmul_registry.cpp:313-340): the activation precision the op
  // allows, int8 per-32 up to int8_decode_max_rows rows, else int16 up to
  // int16_decode_max_rows; the gemm from qmm_gemm_min_rows rows where it exists, else
  // the gemv. (No external kernels and no SME precede it here.)
  if (p.qmm && k % 32 == 0) {
    int act = DQ_ACT_F32;
    if (p.int8_decode_max_rows > 0) {
      act = m <= p.int8_decode_max_rows ? DQ_ACT_PER32 : DQ_ACT_F32;
    } else if (p.int16_decode_max_rows > 0) {
      act = m <= p.int16_decode_max_rows ? DQ_ACT_Q16 : DQ_ACT_F32;
    }
    if (act != DQ_ACT_F32) {
      if (m >= p.qmm_gemm_min_rows && qmm_gemm(wt) && allowed(p, DQ_KERNEL_QMM_GEMM)) {
        return dq_selection{DQ_KERNEL_QMM_GEMM, act};
      }
      if (allowed(p, DQ_KERNEL_QMM_GEMV)) return dq_selection{DQ_KERNEL_QMM_GEMV, act};
    }
  }
  // The int8 family (select_int8, matmul_registry.cpp:94-191).
  if (p.int8_decode_max_rows > 0 && k % 32 == 0) {
    const bool sb_rows = k % 256 == 0 && m <= std::max(p.int8_decode_max_rows, p.int8_superblock_max_rows);
    // Sub-scaled activations (DD-077); the interleaved-copy variants need a copy
    // this backend does not keep.
    if (sb_rows && p.int8_subscale_min_rows > 0 && m >= p.int8_subscale_min_rows && kquant(wt) &&
        allowed(p, DQ_KERNEL_INT8_SUBSCALED)) {
      return dq_selection{DQ_KERNEL_INT8_SUBSCALED, DQ_ACT_SX};
    }
    // Super-block activations (DD-075, opt-in).
    if (sb_rows && p.int8_superblock_min_rows > 0 && m >= p.int8_superblock_min_rows && kquant(wt) &&
        allowed(p, DQ_KERNEL_INT8_SUPERBLOCK)) {
      return dq_selection{DQ_KERNEL_INT8_SUPERBLOCK, DQ_ACT_Q8_K};
    }
    // Per-32 activations (DD-053).
    if (m <= p.int8_decode_max_rows && allowed(p, DQ_KERNEL_INT8_PER32)) {
      return dq_selection{DQ_KERNEL_INT8_PER32, DQ_ACT_PER32};
    }
  }
  // int16 prefill and int16 decode tiles read interleaved copies: absent here. The
  // int16 row kernel (DD-076, matmul_registry.cpp:407-416), every weight type.
  if (m <= p.int16_decode_max_rows && k % 32 == 0 && allowed(p, DQ_KERNEL_INT16_ROWS)) {
    return dq_selection{DQ_KERNEL_INT16_ROWS, DQ_ACT_Q16};
  }
  // fp32: expand + GEMM for dense batches, else the row kernel (matmul_registry.cpp:418-428).
  if (m >= p.expand_min_rows && s.x_dense) return dq_selection{DQ_KERNEL_F32_EXPAND_GEMM, DQ_ACT_F32};
  return dq_selection{DQ_KERNEL_F32_ROW_DOT, DQ_ACT_F32};
}

}  // namespace dq

extern "C" {

int dq_plan_defaults(dq_plan* out) {
  if (out == nullptr) return dq::set_error(DQ_INVALID_ARGUMENT, "null plan");
  *out = dq::default_plan();
  return DQ_OK;
}

int dq_plan_ffn_down(const dq_plan* base, dq_plan* out) {
  if (out == nullptr) return dq::set_error(DQ_INVALID_ARGUMENT, "null plan");
  const dq_plan b = base != nullptr ? *base : dq::default_plan();
  dq_plan d = b;
  // transformer.cpp:541-550 with int8_ffn_down == false, int16_ffn_down == true
  if (b.int8_decode_max_rows > 0) d.int16_decode_max_rows = std::max(b.int8_decode_max_rows, b.int8_superblock_max_rows);
  d.int8_decode_max_rows = 0;
  *out = d;
  return DQ_OK;
}

int dq_select(const dq_matmul_shape* s, const dq_plan* plan, dq_selection* out) {
  if (s == nullptr || out == nullptr) return dq::set_error(DQ_INVALID_ARGUMENT, "null argument");
  // validate_matmul_shape (matmul_registry.cpp:264-278) for the four weight types
  if (s->m <= 0 || s->n <= 0 || s->k <= 0) {
    return dq::set_error(DQ_INVALID_ARGUMENT, "matmul dims must be positive (m %lld, n %lld, k %lld)", (long long)s->m,
                         (long long)s->n, (long long)s->k);
  }
  if (dq_row_bytes(s->dtype, s->k) < 0) {
    if (dq_row_bytes(s->dtype, 256) < 0) return dq::set_error(DQ_UNSUPPORTED, "weight type %d is not supported", s->dtype);
    return dq::set_error(DQ_INVALID_ARGUMENT, "k %lld is not a multiple of the block", (long long)s->k);
  }
  *out = dq::select(*s, plan != nullptr ? *plan : dq::default_plan());
  return DQ_OK;
}

}  // extern "C"
