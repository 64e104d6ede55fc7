// dq_kernels.hip -- gfx950 kernels: activation quantizers, weight repack/unpack,
// decode GEMV (M <= 4 per pass, int8 dot products), integer-partial debug
// kernel, and their host launchers. The MFMA GEMM lives in dq_gemm.hip.
//
// Arithmetic contracts (what "bit-exact" means) follow the reference:
//   quantizers   dynacore/cpu/generic/kernels_generic.cpp:187-207 (per-32),
//                dynacore/src/quantization/quant_formats.cpp:60-74 (GGUF Q8_0),
//                dynacore/cpu/avx2/kernels_avx2.cpp:638-644 (one scale per 256, Q8_K)
//   partials     dynacore/cpu/generic/kernels_generic.cpp:210-310,
//                dynacore/cpu/avx2/kernels_avx2.cpp:976-1058
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dq_device.h"
#include "dq_internal.h"

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

__global__ __launch_bounds__(64) void k_quant_q8k(const float* __restrict__ x, int64_t x_stride, int64_t k,
                                                  uint8_t* __restrict__ out, int64_t orb) {
  const int l = threadIdx.x;
  const int64_t sb = blockIdx.x, row = blockIdx.y;
  const auto rx = rsrc(x + row * x_stride, (u32)(k * 4));
  float v[4];
  load4f(rx, (u32)((sb * 256 + 4 * l) * 4), v);
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = max8f(amax);
#pragma unroll
  for (int s = 8; s < 64; s <<= 1) amax = fmaxf(amax, __shfl_xor(amax, s, 64));
  const float d = amax / 127.0f;
  const float id = d > 0 ? 1.0f / d : 0.0f;
  int sum = 0;
  const u32 packed = codes4_rne(v, id, sum);
  uint8_t* o = out + row * orb + sb * 292;
  *reinterpret_cast<u32*>(o + 4 + 4 * l) = packed;
  // bsums: 16 values = 4 lanes
  sum += dpp<kQuadXor1>(sum);
  sum += dpp<kQuadXor2>(sum);
  if ((l & 3) == 0) *reinterpret_cast<int16_t*>(o + 260 + 2 * (l >> 2)) = (int16_t)sum;
  if (l == 0) *reinterpret_cast<float*>(o) = d;
}

// Per-32 blocks (ActBlockQ8 40 B or GGUF Q8_0 34 B): 8 lanes per block.
template <int AF>
__global__ __launch_bounds__(64) void k_quant_b32(const float* __restrict__ x, int64_t x_stride, int64_t k,
                                                  uint8_t* __restrict__ out, int64_t orb) {
  const int l = threadIdx.x;
  const int64_t row = blockIdx.y;
  const int64_t blk = blockIdx.x * 8 + (l >> 3);  // 32-value block of this lane
  const auto rx = rsrc(x + row * x_stride, (u32)(k * 4));
  float v[4];
  load4f(rx, (u32)((blockIdx.x * 256 + 4 * l) * 4), v);
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = max8f(amax);
  const float d = amax / 127.0f;
  const bool valid = blk * 32 < k;
  if (AF == kActPer32) {
    const float id = d > 0 ? 1.0f / d : 0.0f;
    int sum = 0;
    const u32 packed = codes4_rne(v, id, sum);
    sum = red8(sum);
    if (valid) {
      uint8_t* o = out + row * orb + blk * 40;
      *reinterpret_cast<u32*>(o + 8 + 4 * (l & 7)) = packed;
      if ((l & 7) == 0) {
        *reinterpret_cast<float*>(o) = d;
        *reinterpret_cast<int32_t*>(o + 4) = sum;
      }
    }
  } else {
    // GGUF Q8_0: codes round half away from zero at the fp32 d, fp16 d stored.
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    u32 packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = (int)__builtin_roundf(clampl(v[i] * id, 127.0f));
      packed |= ((u32)c & 0xFFu) << (8 * i);
    }
    if (valid) {
      uint8_t* o = out + row * orb + blk * 34;
      uint16_t* oc = reinterpret_cast<uint16_t*>(o + 2 + 4 * (l & 7));
      oc[0] = (uint16_t)(packed & 0xFFFFu);
      oc[1] = (uint16_t)(packed >> 16);
      if ((l & 7) == 0) *reinterpret_cast<uint16_t*>(o) = f2h(d);
    }
  }
}

// ============================================================ repack / unpack
// One thread per GGUF byte: row n, byte o of the row -> plane p, offset.

struct Planes {
  uint8_t* p[kMaxPlanes];
};

DQ_DEV int64_t plane_offset(int t, int64_t n, int64_t blk, int64_t nblk, int unit, int off) {
  const int64_t G = n / kRowGroup, r = n % kRowGroup;
  return ((G * nblk + blk) * kRowGroup + r) * unit + off;
}

template <bool kPack>
__global__ __launch_bounds__(256) void k_repack(int t, const uint8_t* __restrict__ src, uint8_t* __restrict__ dst_rows,
                                                int64_t row_stride, int64_t n, int64_t nblk, Planes planes) {
  const int bb = block_bytes(t);
  const int64_t row_bytes = nblk * bb;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * row_bytes) return;
  const int64_t row = idx / row_bytes, o = idx % row_bytes;
  const int64_t blk = o / bb;
  int p, off;
  plane_of_byte(t, (int)(o % bb), &p, &off);
  const int64_t at = plane_offset(t, row, blk, nblk, plane_unit(t, p), off);
  if (kPack) {
    planes.p[p][at] = src[row * row_stride + o];
  } else {
    dst_rows[row * row_stride + o] = planes.p[p][at];
  }
}

// ===================================================================== GEMV
// One wave (64 lanes) per group of 8 weight rows: lane l -> row r = l / 8 of the
// group, chunk c = l % 8. M activation rows share each weight load. Weights are
// loaded in batches of U blocks (super-blocks) ahead of their use.

// ---- Q4_K: chunk c = bytes 16c .. 16c+15 of the 128 B of qs: low nibbles are
// values 16h .. 16h+15 of sub-block ja = 2*(c/2), high nibbles the same values of
// sub-block jb = ja + 1, with h = c % 2.
template <int AF, int M, int U>
__global__ __launch_bounds__(64) void k_gemv_q4k(const uint8_t* __restrict__ qs_plane,
                                                 const uint8_t* __restrict__ hdr_plane, int nb, int64_t g0,
                                                 int64_t n0, int64_t n1, const uint8_t* __restrict__ acts,
                                                 int64_t arb, float* __restrict__ y, int64_t ys,
                                                 const float* __restrict__ bias, int32_t* __restrict__ dbg,
                                                 int64_t dbg_n) {
  const int lane = threadIdx.x, r = lane >> 3, c = lane & 7, jp = c >> 1, h = c & 1;
  const int ja = 2 * jp, jb = ja + 1;
  const int64_t G = g0 + blockIdx.x;
  const int64_t n = G * kRowGroup + r;
  const auto rq = rsrc(qs_plane + G * nb * 1024, (u32)(nb * 1024));
  const auto rh = rsrc(hdr_plane + G * nb * 128, (u32)(nb * 128));
  const auto ra = rsrc(acts, (u32)(M * arb));
  float acc[M];
#pragma unroll
  for (int mm = 0; mm < M; ++mm) acc[mm] = 0.0f;

  for (int b0 = 0; b0 < nb; b0 += U) {
    v4u q[U], hd[U], alo[U][M], ahi[U][M];
    v2u ma[U][M], mb[U][M];
    u32 da[U][M];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = b0 + u;
      q[u] = ld16(rq, (u32)((b * 8 + r) * 128 + c * 16));
      hd[u] = ld16(rh, (u32)((b * 8 + r) * 16));
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        if (AF == kActQ8_K) {
          const u32 base = (u32)(mm * arb + (int64_t)b * 292);
          alo[u][mm] = ld16(ra, base + 4 + 32 * ja + 16 * h);
          ahi[u][mm] = ld16(ra, base + 4 + 32 * jb + 16 * h);
          ma[u][mm] = ld8(ra, base + 260 + 8 * jp);  // bsums[4jp .. 4jp+3]
          da[u][mm] = ld4(ra, base);
        } else {  // per-32 ActBlockQ8
          const u32 base = (u32)(mm * arb + ((int64_t)b * 8 + ja) * 40);
          alo[u][mm] = ld16(ra, base + 8 + 16 * h);
          ahi[u][mm] = ld16(ra, base + 40 + 8 + 16 * h);
          ma[u][mm] = ld8(ra, base);       // d, sum of block ja
          mb[u][mm] = ld8(ra, base + 40);  // d, sum of block jb
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = b0 + u;
      if (b >= nb) break;
      const float d = h2f(hd[u].x), dmin = h2f(hd[u].x >> 16);
      int sca, mna, scb, mnb;
      scale_min_k4(ja, hd[u].y, hd[u].z, hd[u].w, sca, mna);
      scale_min_k4(jb, hd[u].y, hd[u].z, hd[u].w, scb, mnb);
      const v4u lo = q[u] & 0x0F0F0F0Fu;
      const v4u hi = (q[u] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        const int plo = sdot16(lo, alo[u][mm], 0);
        const int phi = sdot16(hi, ahi[u][mm], 0);
        if (AF == kActQ8_K) {
          // bsums of values 16h.. of sub-blocks ja, jb: indices 4jp + h and 4jp + 2 + h.
          const int bsa = (int)(int16_t)(ma[u][mm].x >> (16 * h));
          const int bsb = (int)(int16_t)(ma[u][mm].y >> (16 * h));
          const int S = red8(sca * plo + scb * phi);
          const int Mn = red8(mna * bsa + mnb * bsb);
          // canonical order: u = d*S; u = fma(-dmin, Mn, u); acc = fma(da, u, acc)
          float t = d * (float)S;
          t = fmaf(-dmin, (float)Mn, t);
          acc[mm] = fmaf(as_f(da[u][mm]), t, acc[mm]);
          if (dbg != nullptr && c == 0 && n < dbg_n) {
            int32_t* o = dbg + ((mm * dbg_n + n) * nb + b) * 2;
            o[0] = S;
            o[1] = Mn;
          }
        } else {
          // Whole sub-block partials (lanes h = 0, 1 hold the two halves); lane h
          // then adds sub-block ja (h = 0) or jb (h = 1) in the generic form
          // a.d * (d*sc*P - dmin*m*a.sum) (kernels_generic.cpp:274).
          const int pa = red2(plo), pb = red2(phi);
          const int P = h ? pb : pa, sc = h ? scb : sca, mn = h ? mnb : mna;
          const v2u meta = h ? mb[u][mm] : ma[u][mm];
          const float ad = as_f(meta.x);
          const float t = (d * (float)sc) * (float)P - (dmin * (float)mn) * (float)(int)meta.y;
          acc[mm] += ad * t;
        }
      }
    }
  }
#pragma unroll
  for (int mm = 0; mm < M; ++mm) {
    const float v = AF == kActQ8_K ? acc[mm] : red8f(acc[mm]);
    if (c == 0 && n >= n0 && n < n1) y[mm * ys + n] = bias ? v + bias[n] : v;
  }
}

// ---- Q6_K: chunk c = ql bytes 16c .. 16c+15 (half p = c/4, Lp0 = 16*(c%4)): low
// nibbles are values 128p + Lp0 + i, high nibbles values 128p + Lp0 + 64 + i; their
// 2 high bits come from qh bytes 32p + 16*(c%2) + i at bit pairs s and s + 2,
// s = (c%4)/2 (quant_formats.cpp:192-216). Scale units u_lo = 8p + c%4, u_hi = u_lo + 4.
template <int AF, int M, int U>
__global__ __launch_bounds__(64) void k_gemv_q6k(const uint8_t* __restrict__ ql_plane,
                                                 const uint8_t* __restrict__ qh_plane,
                                                 const uint8_t* __restrict__ sc_plane,
                                                 const uint8_t* __restrict__ d_plane, int nb, int64_t g0, int64_t n0,
                                                 int64_t n1, const uint8_t* __restrict__ acts, int64_t arb,
                                                 float* __restrict__ y, int64_t ys, const float* __restrict__ bias,
                                                 int32_t* __restrict__ dbg, int64_t dbg_n) {
  const int lane = threadIdx.x, r = lane >> 3, c = lane & 7, p = c >> 2, cc = c & 3, s = cc >> 1;
  const int ulo = 8 * p + cc, uhi = ulo + 4;
  const int64_t G = g0 + blockIdx.x;
  const int64_t n = G * kRowGroup + r;
  const auto rl = rsrc(ql_plane + G * nb * 1024, (u32)(nb * 1024));
  const auto rhh = rsrc(qh_plane + G * nb * 512, (u32)(nb * 512));
  const auto rs = rsrc(sc_plane + G * nb * 128, (u32)(nb * 128));
  const auto rd = rsrc(d_plane + G * nb * 16, (u32)(nb * 16));
  const auto ra = rsrc(acts, (u32)(M * arb));
  float acc[M];
#pragma unroll
  for (int mm = 0; mm < M; ++mm) acc[mm] = 0.0f;

  for (int b0 = 0; b0 < nb; b0 += U) {
    v4u L[U], H[U], alo[U][M], ahi[U][M];
    v2u sc8[U];
    u32 dw[U], m0[U][M], m1[U][M], m2[U][M];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = b0 + u;
      L[u] = ld16(rl, (u32)((b * 8 + r) * 128 + 16 * c));
      H[u] = ld16(rhh, (u32)((b * 8 + r) * 64 + 32 * p + 16 * (cc & 1)));
      sc8[u] = ld8(rs, (u32)((b * 8 + r) * 16 + 8 * p));
      dw[u] = ld2(rd, (u32)((b * 8 + r) * 2));
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        if (AF == kActQ8_K) {
          const u32 base = (u32)(mm * arb + (int64_t)b * 292);
          alo[u][mm] = ld16(ra, base + 4 + 128 * p + 16 * cc);
          ahi[u][mm] = ld16(ra, base + 4 + 128 * p + 64 + 16 * cc);
          m0[u][mm] = ld2(ra, base + 260 + 2 * ulo);
          m1[u][mm] = ld2(ra, base + 260 + 2 * uhi);
          m2[u][mm] = ld4(ra, base);
        } else {
          const int64_t bl = (int64_t)b * 8 + 4 * p + (cc >> 1), bh = bl + 2;
          alo[u][mm] = ld16(ra, (u32)(mm * arb + bl * 40 + 8 + 16 * (cc & 1)));
          ahi[u][mm] = ld16(ra, (u32)(mm * arb + bh * 40 + 8 + 16 * (cc & 1)));
          m0[u][mm] = ld4(ra, (u32)(mm * arb + bl * 40));
          m1[u][mm] = ld4(ra, (u32)(mm * arb + bh * 40));
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = b0 + u;
      if (b >= nb) break;
      const v4u qlo = (L[u] & 0x0F0F0F0Fu) | (((H[u] >> (2 * s)) & 0x03030303u) << 4);
      const v4u qhi = ((L[u] >> 4) & 0x0F0F0F0Fu) | (((H[u] >> (2 * s + 4)) & 0x03030303u) << 4);
      const int sclo = (int)(int8_t)(sc8[u].x >> (8 * cc));
      const int schi = (int)(int8_t)(sc8[u].y >> (8 * cc));
      const float d = h2f(dw[u]);
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        if (AF == kActQ8_K) {
          // sum (q - 32) a = sum q a - 32 * (sum of the 16 codes) = ... - 32 * bsums[u]
          const int plo = sdot16(qlo, alo[u][mm], 0) - 32 * (int)(int16_t)m0[u][mm];
          const int phi = sdot16(qhi, ahi[u][mm], 0) - 32 * (int)(int16_t)m1[u][mm];
          const int S = red8(sclo * plo + schi * phi);
          acc[mm] = fmaf(as_f(m2[u][mm]), d * (float)S, acc[mm]);
          if (dbg != nullptr && c == 0 && n < dbg_n) {
            int32_t* o = dbg + ((mm * dbg_n + n) * nb + b) * 2;
            o[0] = S;
            o[1] = 0;
          }
        } else {
          // signed codes q - 32 as int8 bytes: flip bit 5, then extend its sign.
          v4u slo = qlo ^ 0x20202020u, shi = qhi ^ 0x20202020u;
          slo |= (slo & 0x20202020u) * 6u;
          shi |= (shi & 0x20202020u) * 6u;
          const int plo = sdot16(slo, alo[u][mm], 0);
          const int phi = sdot16(shi, ahi[u][mm], 0);
          // generic order per 16 values: ((a.d * d) * sc) * P (kernels_generic.cpp:304)
          acc[mm] += ((as_f(m0[u][mm]) * d) * (float)sclo) * (float)plo;
          acc[mm] += ((as_f(m1[u][mm]) * d) * (float)schi) * (float)phi;
        }
      }
    }
  }
#pragma unroll
  for (int mm = 0; mm < M; ++mm) {
    const float v = AF == kActQ8_K ? acc[mm] : red8f(acc[mm]);
    if (c == 0 && n >= n0 && n < n1) y[mm * ys + n] = bias ? v + bias[n] : v;
  }
}

// ---- Q8_0 / Q4_0 with per-32 or GGUF Q8_0 activations: lane c takes the whole
// 32-value block 8*it + c of its row.

// 32 activation codes of a GGUF Q8_0 block (34 B; codes at byte 2, so 2-byte aligned).
DQ_DEV void ld_q80_codes(__amdgpu_buffer_rsrc_t ra, u32 base, v4u& a0, v4u& a1) {
  const u32 off = base + 2, al = off & ~3u, sh = off & 3u;  // sh is 0 or 2
  const v4u x0 = ld16(ra, al), x1 = ld16(ra, al + 16);
  const u32 x2 = ld4(ra, al + 32);
  if (sh == 0) {
    a0 = x0;
    a1 = x1;
  } else {
    a0.x = __builtin_amdgcn_alignbyte(x0.y, x0.x, 2);
    a0.y = __builtin_amdgcn_alignbyte(x0.z, x0.y, 2);
    a0.z = __builtin_amdgcn_alignbyte(x0.w, x0.z, 2);
    a0.w = __builtin_amdgcn_alignbyte(x1.x, x0.w, 2);
    a1.x = __builtin_amdgcn_alignbyte(x1.y, x1.x, 2);
    a1.y = __builtin_amdgcn_alignbyte(x1.z, x1.y, 2);
    a1.z = __builtin_amdgcn_alignbyte(x1.w, x1.z, 2);
    a1.w = __builtin_amdgcn_alignbyte(x2, x1.w, 2);
  }
}

template <int WT, int AF, int M, int U>
__global__ __launch_bounds__(64) void k_gemv_b32(const uint8_t* __restrict__ qs_plane,
                                                 const uint8_t* __restrict__ d_plane, int nblk, int64_t g0, int64_t n0,
                                                 int64_t n1, const uint8_t* __restrict__ acts, int64_t arb,
                                                 float* __restrict__ y, int64_t ys, const float* __restrict__ bias) {
  constexpr int kUnit = WT == kQ8_0 ? 32 : 16;  // qs bytes per block
  const int lane = threadIdx.x, r = lane >> 3, c = lane & 7;
  const int64_t G = g0 + blockIdx.x;
  const int64_t n = G * kRowGroup + r;
  const auto rq = rsrc(qs_plane + G * nblk * 8 * kUnit, (u32)(nblk * 8 * kUnit));
  const auto rd = rsrc(d_plane + G * nblk * 16, (u32)(nblk * 16));
  const auto ra = rsrc(acts, (u32)(M * arb));
  const int ab = AF == kActPer32 ? 40 : 34;
  float acc[M];
#pragma unroll
  for (int mm = 0; mm < M; ++mm) acc[mm] = 0.0f;

  for (int i0 = 0; i0 < nblk; i0 += 8 * U) {
    v4u w0[U], w1[U], a0[U][M], a1[U][M];
    u32 dw[U], da[U][M], sa[U][M];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int blk = i0 + 8 * u + c;
      w0[u] = ld16(rq, (u32)((blk * 8 + r) * kUnit));
      if (WT == kQ8_0) w1[u] = ld16(rq, (u32)((blk * 8 + r) * kUnit + 16));
      dw[u] = ld2(rd, (u32)((blk * 8 + r) * 2));
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        const u32 base = (u32)(mm * arb + (int64_t)blk * ab);
        if (AF == kActPer32) {
          a0[u][mm] = ld16(ra, base + 8);
          a1[u][mm] = ld16(ra, base + 24);
          da[u][mm] = ld4(ra, base);
          sa[u][mm] = ld4(ra, base + 4);
        } else {
          ld_q80_codes(ra, base, a0[u][mm], a1[u][mm]);
          da[u][mm] = ld2(ra, base);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int blk = i0 + 8 * u + c;
      if (blk >= nblk) continue;
      const float d = h2f(dw[u]);
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        int P;
        if (WT == kQ8_0) {
          P = sdot16(w1[u], a1[u][mm], sdot16(w0[u], a0[u][mm], 0));
        } else {
          // Q4_0: low nibbles are values 0..15, high nibbles 16..31; code = nibble - 8.
          const v4u lo = w0[u] & 0x0F0F0F0Fu, hi = (w0[u] >> 4) & 0x0F0F0F0Fu;
          int sum;
          if (AF == kActPer32) {
            sum = (int)sa[u][mm];
          } else {
            const v4u ones = {0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};
            sum = sdot16(ones, a1[u][mm], sdot16(ones, a0[u][mm], 0));
          }
          P = sdot16(hi, a1[u][mm], sdot16(lo, a0[u][mm], 0)) - 8 * sum;
        }
        const float dA = AF == kActPer32 ? as_f(da[u][mm]) : h2f(da[u][mm]);
        // generic order: (dw * da) * (float)P (kernels_generic.cpp:220,235)
        acc[mm] += (d * dA) * (float)P;
      }
    }
  }
#pragma unroll
  for (int mm = 0; mm < M; ++mm) {
    const float v = red8f(acc[mm]);
    if (c == 0 && n >= n0 && n < n1) y[mm * ys + n] = bias ? v + bias[n] : v;
  }
}

// ========================================================== integer partials
// One thread per (activation row, weight row, scale unit): the exact integer dot
// of the unit, decoded from the device layout with plain byte arithmetic.

DQ_DEV int act_code(int af, const uint8_t* a, int64_t i) {
  switch (af) {
    case kActPer32: return (int8_t)a[(i / 32) * 40 + 8 + i % 32];
    case kActQ8_0: return (int8_t)a[(i / 32) * 34 + 2 + i % 32];
    default: return (int8_t)a[(i / 256) * 292 + 4 + i % 256];
  }
}

__global__ __launch_bounds__(256) void k_units(int t, int af, const uint8_t* p0, const uint8_t* p1, int64_t nblk,
                                               int64_t n, int64_t k, int64_t m, const uint8_t* __restrict__ acts,
                                               int64_t arb, int32_t* __restrict__ units, int64_t nu) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= m * n * nu) return;
  const int64_t u = idx % nu, row = (idx / nu) % n, mm = idx / (nu * n);
  const uint8_t* a = acts + mm * arb;
  const int64_t G = row / kRowGroup, r = row % kRowGroup;
  int s = 0;
  if (t == kQ8_0 || t == kQ4_0) {
    const int unit = t == kQ8_0 ? 32 : 16;
    const uint8_t* q = p0 + ((G * nblk + u) * kRowGroup + r) * unit;
    for (int i = 0; i < 32; ++i) {
      const int w = t == kQ8_0 ? (int)(int8_t)q[i] : (int)((i < 16 ? (q[i] & 15) : (q[i - 16] >> 4))) - 8;
      s += w * act_code(af, a, u * 32 + i);
    }
  } else if (t == kQ4_K) {
    const int64_t b = u / 8;
    const int j = (int)(u % 8);
    const uint8_t* qs = p0 + ((G * nblk + b) * kRowGroup + r) * 128 + 32 * (j / 2);
    for (int i = 0; i < 32; ++i) {
      const int w = (j & 1) ? (qs[i] >> 4) : (qs[i] & 15);
      s += w * act_code(af, a, b * 256 + 32 * j + i);
    }
  } else {  // Q6_K: unit = 16 values 16*uu .. of super-block b
    const int64_t b = u / 16;
    const int uu = (int)(u % 16);
    const uint8_t* ql = p0 + ((G * nblk + b) * kRowGroup + r) * 128;
    const uint8_t* qh = p1 + ((G * nblk + b) * kRowGroup + r) * 64;
    for (int i = 0; i < 16; ++i) {
      const int v = 16 * uu + i;          // value index in the super-block
      const int half = v / 128, w = v % 128, quarter = w / 32, l = w % 32;
      const int lb = ql[64 * half + l + (quarter & 1) * 32];
      const int nib = quarter < 2 ? (lb & 15) : (lb >> 4);
      const int hb = (qh[32 * half + l] >> (2 * quarter)) & 3;
      s += ((nib | (hb << 4)) - 32) * act_code(af, a, b * 256 + v);
    }
  }
  units[idx] = s;
}

// ================================================================ launchers

static inline dim3 grid1(int64_t total, int block) { return dim3((unsigned)((total + block - 1) / block)); }

hipError_t launch_quantize(int af, const float* x, int64_t m, int64_t k, int64_t x_stride, uint8_t* out,
                           int64_t orb, hipStream_t s) {
  if (m == 0 || k == 0) return hipSuccess;
  if (af == kActQ8_K) {
    hipLaunchKernelGGL(k_quant_q8k, dim3((unsigned)(k / 256), (unsigned)m), dim3(64), 0, s, x, x_stride, k, out, orb);
  } else if (af == kActPer32) {
    hipLaunchKernelGGL(k_quant_b32<kActPer32>, dim3((unsigned)((k + 255) / 256), (unsigned)m), dim3(64), 0, s, x,
                       x_stride, k, out, orb);
  } else {
    hipLaunchKernelGGL(k_quant_b32<kActQ8_0>, dim3((unsigned)((k + 255) / 256), (unsigned)m), dim3(64), 0, s, x,
                       x_stride, k, out, orb);
  }
  return hipGetLastError();
}

hipError_t launch_repack(int t, const uint8_t* src, int64_t row_stride, int64_t n, int64_t nblk, uint8_t* const* planes,
                         hipStream_t s) {
  Planes pl{};
  for (int i = 0; i < num_planes(t); ++i) pl.p[i] = planes[i];
  const int64_t total = n * nblk * block_bytes(t);
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(k_repack<true>, grid1(total, 256), dim3(256), 0, s, t, src, nullptr, row_stride, n, nblk, pl);
  return hipGetLastError();
}

hipError_t launch_unpack(int t, uint8_t* dst, int64_t row_stride, int64_t n, int64_t nblk, uint8_t* const* planes,
                         hipStream_t s) {
  Planes pl{};
  for (int i = 0; i < num_planes(t); ++i) pl.p[i] = planes[i];
  const int64_t total = n * nblk * block_bytes(t);
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(k_repack<false>, grid1(total, 256), dim3(256), 0, s, t, nullptr, dst, row_stride, n, nblk, pl);
  return hipGetLastError();
}

template <int AF, int M>
static void gemv_q4k_m(const WeightDev& w, const uint8_t* acts, int64_t arb, int64_t n0, int64_t n1, float* y,
                       int64_t ys, const float* bias, int32_t* dbg, hipStream_t s) {
  constexpr int U = M == 1 ? 8 : (M == 2 ? 4 : 2);
  const int64_t g0 = n0 / kRowGroup, g1 = (n1 + kRowGroup - 1) / kRowGroup;
  hipLaunchKernelGGL((k_gemv_q4k<AF, M, U>), dim3((unsigned)(g1 - g0)), dim3(64), 0, s, w.plane[0], w.plane[1],
                     (int)w.nblk, g0, n0, n1, acts, arb, y, ys, bias, dbg, w.n);
}

template <int AF, int M>
static void gemv_q6k_m(const WeightDev& w, const uint8_t* acts, int64_t arb, int64_t n0, int64_t n1, float* y,
                       int64_t ys, const float* bias, int32_t* dbg, hipStream_t s) {
  constexpr int U = M == 1 ? 4 : 2;
  const int64_t g0 = n0 / kRowGroup, g1 = (n1 + kRowGroup - 1) / kRowGroup;
  hipLaunchKernelGGL((k_gemv_q6k<AF, M, U>), dim3((unsigned)(g1 - g0)), dim3(64), 0, s, w.plane[0], w.plane[1],
                     w.plane[2], w.plane[3], (int)w.nblk, g0, n0, n1, acts, arb, y, ys, bias, dbg, w.n);
}

template <int WT, int AF, int M>
static void gemv_b32_m(const WeightDev& w, const uint8_t* acts, int64_t arb, int64_t n0, int64_t n1, float* y,
                       int64_t ys, const float* bias, hipStream_t s) {
  constexpr int U = M == 1 ? 4 : 2;
  const int64_t g0 = n0 / kRowGroup, g1 = (n1 + kRowGroup - 1) / kRowGroup;
  hipLaunchKernelGGL((k_gemv_b32<WT, AF, M, U>), dim3((unsigned)(g1 - g0)), dim3(64), 0, s, w.plane[0], w.plane[1],
                     (int)w.nblk, g0, n0, n1, acts, arb, y, ys, bias);
}

// M rows (1..4) of one pass.
template <int M>
static hipError_t gemv_pass(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t n0, int64_t n1,
                            float* y, int64_t ys, const float* bias, int32_t* dbg, hipStream_t s) {
  switch (w.dtype) {
    case kQ4_K:
      if (af == kActQ8_K) gemv_q4k_m<kActQ8_K, M>(w, acts, arb, n0, n1, y, ys, bias, dbg, s);
      else gemv_q4k_m<kActPer32, M>(w, acts, arb, n0, n1, y, ys, bias, dbg, s);
      break;
    case kQ6_K:
      if (af == kActQ8_K) gemv_q6k_m<kActQ8_K, M>(w, acts, arb, n0, n1, y, ys, bias, dbg, s);
      else gemv_q6k_m<kActPer32, M>(w, acts, arb, n0, n1, y, ys, bias, dbg, s);
      break;
    case kQ8_0:
      if (af == kActPer32) gemv_b32_m<kQ8_0, kActPer32, M>(w, acts, arb, n0, n1, y, ys, bias, s);
      else gemv_b32_m<kQ8_0, kActQ8_0, M>(w, acts, arb, n0, n1, y, ys, bias, s);
      break;
    default:
      if (af == kActPer32) gemv_b32_m<kQ4_0, kActPer32, M>(w, acts, arb, n0, n1, y, ys, bias, s);
      else gemv_b32_m<kQ4_0, kActQ8_0, M>(w, acts, arb, n0, n1, y, ys, bias, s);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_gemv(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int64_t n0, int64_t n1,
                       float* y, int64_t ys, const float* bias, int32_t* dbg, hipStream_t s) {
  for (int64_t r0 = 0; r0 < m; r0 += 4) {
    const int rows = (int)(m - r0 < 4 ? m - r0 : 4);
    const uint8_t* a = acts + r0 * arb;
    float* yy = y + r0 * ys;
    int32_t* dd = dbg ? dbg + r0 * w.n * w.nblk * 2 : nullptr;
    hipError_t e;
    switch (rows) {
      case 1: e = gemv_pass<1>(w, af, a, arb, n0, n1, yy, ys, bias, dd, s); break;
      case 2: e = gemv_pass<2>(w, af, a, arb, n0, n1, yy, ys, bias, dd, s); break;
      case 3: e = gemv_pass<3>(w, af, a, arb, n0, n1, yy, ys, bias, dd, s); break;
      default: e = gemv_pass<4>(w, af, a, arb, n0, n1, yy, ys, bias, dd, s); break;
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_units(const WeightDev& w, int af, const uint8_t* acts, int64_t arb, int64_t m, int32_t* units,
                        int64_t nu, hipStream_t s) {
  const int64_t total = m * w.n * nu;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(k_units, grid1(total, 256), dim3(256), 0, s, w.dtype, af, w.plane[0], w.plane[1], w.nblk, w.n,
                     w.k, m, acts, arb, units, nu);
  return hipGetLastError();
}

}  // namespace dq
