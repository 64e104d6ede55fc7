// dq_quant.h -- device functions of the activation quantizers, shared by the
// standalone quantizer kernels (dq_kernels.hip) and the GEMV's fused decode path
// (dq_gemv.hip), so both write the same code bytes.
//
// Contracts: per-32 ActBlockQ8 dynacore/cpu/generic/kernels_generic.cpp:187-207;
// one scale per 256 values (Q8_K) dynacore/cpu/avx2/kernels_avx2.cpp:638-644;
// sub-scaled ActSuperQ8 dynacore/cpu/avx2/kernels_avx2.cpp:1077-1096;
// int16 ActBlockQ16 dynacore/cpu/avx2/kernels_avx2.cpp:1631-1652.
#pragma once

#include "dq_device.h"

namespace dq {

// ===================================================================== quantizers
// One wave per 256 values of a row; lane l holds values 4l .. 4l+3.

// Loads values [v0, v0 + 4) of a row through a buffer resource (zeros past the end).
DQ_DEV void load4f(__amdgpu_buffer_rsrc_t r, u32 off, float v[4]) {
  const v4u u = ld16(r, off);
  v[0] = as_f(u.x);
  v[1] = as_f(u.y);
  v[2] = as_f(u.z);
  v[3] = as_f(u.w);
}

// The comparison clamp of kernels_generic.cpp:199 (NaN goes to -L).
DQ_DEV float clampl(float v, float l) { return v > -l ? (v < l ? v : l) : -l; }

// 4 codes at inverse scale id, round half to even; returns the packed bytes and adds their sum.
DQ_DEV u32 codes4_rne(const float v[4], float id, int& sum) {
  u32 packed = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int c = (int)__builtin_rintf(clampl(v[i] * id, 127.0f));
    c = c < -127 ? -127 : (c > 127 ? 127 : c);
    sum += c;
    packed |= ((u32)c & 0xFFu) << (8 * i);
  }
  return packed;
}

// Q8_K quantization of one 256-value super-block held 4 values per lane (lane l:
// values 4l .. 4l+3): d = amax/127, codes round half to even at 1/d
// (kernels_avx2.cpp:638-644). Returns the lane's 4 packed codes, d, and in every
// lane the sum of the 16 codes of its 4-lane group (bsums[l / 4]).
DQ_DEV u32 q8k_quant(const float v[4], float& d, int& bsum) {
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = max8f(amax);
  amax = fmaxf(amax, as_f((u32)dpp<kRowRor8>((int)as_u(amax))));  // rows of 16 lanes
  // the four row maxima (wave-uniform reads, no LDS round trip)
  const float r0 = as_f(__builtin_amdgcn_readlane(as_u(amax), 0)), r1 = as_f(__builtin_amdgcn_readlane(as_u(amax), 16));
  const float r2 = as_f(__builtin_amdgcn_readlane(as_u(amax), 32)), r3 = as_f(__builtin_amdgcn_readlane(as_u(amax), 48));
  amax = fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
  d = amax / 127.0f;
  const float id = d > 0 ? 1.0f / d : 0.0f;
  int sum = 0;
  const u32 packed = codes4_rne(v, id, sum);
  sum += dpp<kQuadXor1>(sum);
  sum += dpp<kQuadXor2>(sum);
  bsum = sum;
  return packed;
}

// Per-32 ActBlockQ8 quantization (kernels_generic.cpp:187-207) of 8 blocks held 4
// values per lane (lanes 8i .. 8i+7 hold block i): returns the lane's packed codes,
// the block's d and (in every lane of the block) the block's code sum.
DQ_DEV u32 per32_quant(const float v[4], float& d, int& sum) {
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = max8f(amax);
  d = amax / 127.0f;
  const float id = d > 0 ? 1.0f / d : 0.0f;
  int s = 0;
  const u32 packed = codes4_rne(v, id, s);
  sum = red8(s);
  return packed;
}

// Sub-scaled ActSuperQ8 quantization (kernels_avx2.cpp:1077-1096) of one 256-value
// super-block held 4 values per lane (lanes 8b .. 8b+7 hold 32-value block b):
// u = amax256 / (127 * 128); the block's multiplier m = clamp(ceil(amax32 / (127 u)),
// 1, 128) (1 when u == 0); codes round half to even at scale u * m. Returns the
// lane's packed codes, u, and (in every lane of the block) m and the code sum.
DQ_DEV u32 sx_quant(const float v[4], float& u, int& m, int& sum) {
  const float a32 = max8f(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  float amax = fmaxf(a32, as_f((u32)dpp<kRowRor8>((int)as_u(a32))));  // rows of 16 lanes
  const float r0 = as_f(__builtin_amdgcn_readlane(as_u(amax), 0)), r1 = as_f(__builtin_amdgcn_readlane(as_u(amax), 16));
  const float r2 = as_f(__builtin_amdgcn_readlane(as_u(amax), 32)), r3 = as_f(__builtin_amdgcn_readlane(as_u(amax), 48));
  amax = fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
  u = amax / (127.0f * 128.0f);
  m = 1;
  if (u > 0) {
    const int c = (int)ceilf(a32 / (127.0f * u));
    m = c < 1 ? 1 : (c > 128 ? 128 : c);
  }
  const float s = u * (float)m;
  const float id = s > 0 ? 1.0f / s : 0.0f;
  int cs = 0;
  const u32 packed = codes4_rne(v, id, cs);
  sum = red8(cs);
  return packed;
}

// int16 ActBlockQ16 quantization (kernels_avx2.cpp:1631-1652) of 8 blocks held 4
// values per lane (lanes 8i .. 8i+7 hold block i): d = amax32 / 32767, codes round
// half to even at 1/d as int32 (values that are not finite or outside the int32
// range become INT32_MIN, as cvtps_epi32 makes them); the stored int16 codes
// saturate (packs_epi32) and the sum is that of the int32 codes. Returns the lane's
// 4 int16 codes packed in two dwords, the block's d and (every lane) its sum.
DQ_DEV v2u q16_quant(const float v[4], float& d, int& sum) {
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = max8f(amax);
  d = amax / 32767.0f;
  const float id = d > 0 ? 1.0f / d : 0.0f;
  int s = 0;
  u32 h[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float r = __builtin_rintf(v[i] * id);
    const int c = (r >= -2147483648.0f && r < 2147483648.0f) ? (int)r : (int)0x80000000u;
    s += c;
    h[i] = (u32)(c < -32768 ? -32768 : (c > 32767 ? 32767 : c)) & 0xFFFFu;
  }
  sum = red8(s);
  return v2u{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
}

}  // namespace dq
