// dq_ceiling.hip -- the two hardware ceilings the benchmark quotes its kernels
// against, measured on the same device in the same run (libdqceil.so, loaded by
// bench.py only; not part of the dq_* interface):
//
// - dqc_read_q4k: the decode GEMV's memory traffic and nothing else. Same grid (one
//   workgroup per 64-row group, W waves, each wave a contiguous run of super-blocks),
//   same loads (per super-block: eight 1 KB nontemporal dwordx4 loads of the code
//   plane and one 1 KB load of the header plane, at the GEMV's offsets), and one fp32
//   store per row. Its time is what the GEMV would take if its arithmetic, LDS
//   staging, barrier and in-order chain were free.
// - dqc_mfma_rate: back-to-back MFMAs (int8 v_mfma_i32_16x16x64_i8 or
//   v_mfma_i32_32x32x32_i8, or f16 v_mfma_f32_32x32x16_f16), eight independent
//   accumulators per wave, two waves per SIMD on every CU: the matrix rate a GEMM could
//   reach at the clock the device runs under MFMA load.
// - dqc_read_flat: a plain read of the same bytes at any launch shape, for the bench's
//   launch-shape sweep (the best one-launch read of them).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dq_device.h"
#include "dq_mfma.h"

namespace {

using dq::u32;
using dq::v4i_t;
using dq::v4u;

typedef int v16i_t __attribute__((ext_vector_type(16)));

// Workgroup = row group G, wave w reads super-blocks [w * bpw, (w + 1) * bpw).
__global__ __launch_bounds__(1024) void k_read_q4k(const uint8_t* __restrict__ qs, const uint8_t* __restrict__ hdr,
                                                   int nblk, int bpw, float* __restrict__ out) {
  const int r = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t G = blockIdx.x;
  const auto r0 = dq::rsrc(qs + G * nblk * 8192, (u32)(nblk * 8192));
  const auto r1 = dq::rsrc(hdr + G * nblk * 1024, (u32)(nblk * 1024));
  u32 x = 0;
  for (int i = 0; i < bpw; ++i) {
    const int b = w * bpw + i;
    const v4u h = dq::ld16nt(r1, (u32)((b * 64 + r) * 16));
    v4u q[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) q[c] = dq::ld16nt(r0, (u32)(((b * 8 + c) * 64 + r) * 16));
    x ^= h.x ^ h.y ^ h.z ^ h.w;
#pragma unroll
    for (int c = 0; c < 8; ++c) x ^= q[c].x ^ q[c].y ^ q[c].z ^ q[c].w;
  }
  // one value per row, as the GEMV writes (wave 0; the others fold into it through LDS)
  __shared__ u32 fold[16][64];
  fold[w][r] = x;
  __syncthreads();
  if (w == 0) {
    const int nw = blockDim.x >> 6;
    for (int i = 1; i < nw; ++i) x ^= fold[i][r];
    out[G * 64 + r] = __builtin_bit_cast(float, x & 0x3FFFFFFFu);
  }
}

// A plain read of `bytes` at a given launch shape: workgroups of `waves` waves, wave v of
// the grid reading the contiguous piece [v * per, (v + 1) * per) (per a multiple of 1 KB)
// with nontemporal 16-byte loads, up to eight 1 KB loads in flight per wave, one value per
// wave written; pieces past the end read zeros (the buffer's range check). The bench's
// launch-shape sweep: the best one-launch read of the decode GEMV's bytes.
__global__ __launch_bounds__(1024) void k_read_flat(const uint8_t* __restrict__ p, u32 per, u32 bytes,
                                                   u32* __restrict__ out) {
  const int r = threadIdx.x & 63;
  const int64_t v = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t base = v * per;
  const auto rs = dq::rsrc(p, bytes);
  u32 x = 0;
  for (u32 o = 0; o < per; o += 8 * 1024) {
    v4u q[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      q[c] = o + c * 1024 < per ? dq::ld16nt(rs, (u32)(base + o + c * 1024 + r * 16)) : v4u{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) x ^= q[c].x ^ q[c].y ^ q[c].z ^ q[c].w;
  }
  if (r == 0) out[v] = x;
}

typedef float v16f_t __attribute__((ext_vector_type(16)));
typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(512) void k_mfma_rate_f16(int iters, int* __restrict__ out) {
  const int l = threadIdx.x & 63;
  const v4u a = {(u32)(l * 0x00010001u), (u32)(l + 1), (u32)(l ^ 7), 3u};
  const v4u b = {(u32)(l * 0x00030001u), 5u, (u32)(l + 9), (u32)(l * 3)};
  v16f_t c[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) c[j] = v16f_t{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      c[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h_t, a), __builtin_bit_cast(v8h_t, b), c[j], 0,
                                                    0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += c[j][e];
  out[blockIdx.x * blockDim.x + threadIdx.x] = (int)s;
}

template <bool k32>
__global__ __launch_bounds__(512) void k_mfma_rate(int iters, int* __restrict__ out) {
  const int l = threadIdx.x & 63;
  const v4u a = {(u32)(l * 0x01010101u), (u32)(l + 1), (u32)(l ^ 7), 3u};
  const v4u b = {(u32)(l * 0x00010203u), 5u, (u32)(l + 9), (u32)(l * 3)};
  if constexpr (k32) {
    v16i_t c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = v16i_t{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        c[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i_t, a), __builtin_bit_cast(v4i_t, b), c[j], 0,
                                                     0, 0);
    }
    int s = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) s += c[j][e];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
  } else {
    v4i_t c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = v4i_t{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = dq::mfma(a, b, c[j]);
    }
    int s = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += c[j].x + c[j].y + c[j].z + c[j].w;
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
  }
}

}  // namespace

extern "C" {

// bytes (a multiple of 1 KB) read by wgs workgroups of waves waves, each wave a contiguous
// piece of whole KB; out: one u32 per wave.
__attribute__((visibility("default"))) int dqc_read_flat(const void* p, int64_t bytes, int wgs, int waves, void* out,
                                                         void* stream) {
  const int64_t nw = (int64_t)wgs * waves;
  if (p == nullptr || out == nullptr || wgs <= 0 || waves <= 0 || waves > 16 || bytes <= 0 || bytes % 1024 != 0 ||
      bytes + nw * 1024 >= (1ll << 32)) {
    return 1;
  }
  const int64_t per = (bytes / 1024 + nw - 1) / nw * 1024;
  hipLaunchKernelGGL(k_read_flat, dim3((unsigned)wgs), dim3(64 * waves), 0, (hipStream_t)stream,
                     (const uint8_t*)p, (u32)per, (u32)bytes, (u32*)out);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// groups row groups of nblk super-blocks (planes of groups * nblk * 8192 and
// * 1024 bytes); waves * bpw == nblk; out: groups * 64 floats.
__attribute__((visibility("default"))) int dqc_read_q4k(const void* qs, const void* hdr, int64_t groups, int nblk,
                                                        int waves, float* out, void* stream) {
  if (qs == nullptr || hdr == nullptr || out == nullptr || groups <= 0 || waves <= 0 || waves > 16 || nblk <= 0 ||
      nblk % waves != 0 || (int64_t)nblk * 8192 >= (1ll << 32) || groups >= (1ll << 31)) {
    return 1;
  }
  hipLaunchKernelGGL(k_read_q4k, dim3((unsigned)groups), dim3(64 * waves), 0, (hipStream_t)stream,
                     (const uint8_t*)qs, (const uint8_t*)hdr, nblk, nblk / waves, out);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// workgroups of 8 waves, each wave iters x 8 MFMAs of the kind (0: int8 16x16x64, 1:
// int8 32x32x32, 2: f16 32x32x16); out: workgroups * 512 ints. Returns the operations
// of the launch through ops (2 M N K per MFMA).
__attribute__((visibility("default"))) int dqc_mfma_rate(int workgroups, int iters, int kind, int* out, double* ops,
                                                         void* stream) {
  if (out == nullptr || ops == nullptr || workgroups <= 0 || iters <= 0 || kind < 0 || kind > 2) return 1;
  if (kind == 0) {
    hipLaunchKernelGGL(k_mfma_rate<false>, dim3((unsigned)workgroups), dim3(512), 0, (hipStream_t)stream, iters, out);
  } else if (kind == 1) {
    hipLaunchKernelGGL(k_mfma_rate<true>, dim3((unsigned)workgroups), dim3(512), 0, (hipStream_t)stream, iters, out);
  } else {
    hipLaunchKernelGGL(k_mfma_rate_f16, dim3((unsigned)workgroups), dim3(512), 0, (hipStream_t)stream, iters, out);
  }
  *ops = (double)workgroups * 8 * iters * 8 * 2.0 * (kind == 0 ? 16.0 * 16 * 64 : kind == 1 ? 32.0 * 32 * 32 : 32.0 * 32 * 16);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
