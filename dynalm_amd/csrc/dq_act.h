// dq_act.h -- the activations of the gated MLP projection on the device
// (dynacore Activation: dynacore/include/dynacore/device/ops.h:14), with the
// reference's fp32 steps.
//
// The library is built with -ffp-contract=off and correctly rounded fp32 division,
// so each multiply, add and divide below rounds where it is written, as the
// reference's x86 build does (no FMA in its baseline objects). SiLU is then
// bit-identical to the reference; GELU calls the device erff / tanhf, which agree
// with the host libm to a few ulp only.
#pragma once

#include "dq_device.h"
#include "dq_internal.h"

namespace dq {

// e^x for x <= 0 (dynacore/include/dynacore/base/fast_exp.h:16-35): comparison
// clamp to [-87, 88] (NaN goes to -87), n = round(x / ln 2) by the 1.5 * 2^23
// trick, r = x - n ln 2 with ln 2 in two parts, e^r by Horner's rule on the
// degree-6 Taylor polynomial, times 2^n built in the exponent field.
DQ_DEV float exp_nonpos(float x) {
  x = x > -87.0f ? (x < 88.0f ? x : 88.0f) : -87.0f;
  const float n = (x * 1.44269504088896341f + 12582912.0f) - 12582912.0f;
  const float r = x - n * 0.693145751953125f - n * 1.428606765330187e-06f;
  float p = 1.0f / 720;
  p = p * r + 1.0f / 120;
  p = p * r + 1.0f / 24;
  p = p * r + 1.0f / 6;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  return p * __uint_as_float((u32)((int)n + 127) << 23);
}

// act(x) (dynacore/cpu/cpu_device.cpp:117-134): SiLU x * (x >= 0 ? 1 : e) / (1 + e)
// with e = e^-|x|; GELU 0.5 x (1 + erf(x / sqrt 2)); GELU-tanh
// 0.5 x (1 + tanh(sqrt(2 / pi) (x + 0.044715 x^3))).
DQ_DEV float act_apply(int act, float x) {
  if (act == kActSilu) {
    const float e = exp_nonpos(-fabsf(x));
    return x * (x >= 0.0f ? 1.0f : e) / (1.0f + e);
  }
  if (act == kActGelu) return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
  const float kc = 0.7978845608028654f;
  return 0.5f * x * (1.0f + tanhf(kc * (x + 0.044715f * x * x * x)));
}

}  // namespace dq
