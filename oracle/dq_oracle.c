/*
 * dq_oracle.c -- CPU oracle for the block-quantized matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see dq_oracle.h): used by tests/, the smoke check
 * and bench.py's cpu_baseline leg as the checker; never by the product.
 *
 * Build with -ffp-contract=off (oracle/Makefile does): every fp32 operation
 * below rounds where it is written. Where the canonical order uses a fused
 * multiply-add it calls fmaf() explicitly.
 */
#include "dq_oracle.h"

#include <math.h>
#include <string.h>

/* ---------------------------------------------------------------- sizes */

int64_t dqo_block_elems(int dtype) {
  switch (dtype) {
    case DQO_Q4_0: case DQO_Q8_0: return 32;
    case DQO_Q4_K: case DQO_Q6_K: case DQO_Q8_K: return 256;
    default: return -1;
  }
}

/* Block byte sizes: dynacore/src/tensor/dtype.cpp:24-45. */
int64_t dqo_block_bytes(int dtype) {
  switch (dtype) {
    case DQO_Q4_0: return 18;
    case DQO_Q8_0: return 34;
    case DQO_Q4_K: return 144;
    case DQO_Q6_K: return 210;
    case DQO_Q8_K: return 292;
    default: return -1;
  }
}

/* dtype_row_bytes (dtype.cpp:50-54): -1 unless k is a whole number of blocks. */
int64_t dqo_row_bytes(int dtype, int64_t k) {
  const int64_t be = dqo_block_elems(dtype);
  if (be <= 0 || k < 0 || k % be != 0) return -1;
  return k / be * dqo_block_bytes(dtype);
}

int64_t dqo_act_block_elems(int fmt) {
  switch (fmt) {
    case DQO_ACT_PER32: case DQO_ACT_Q8_0: case DQO_ACT_Q16: case DQO_ACT_F32: return 32;
    case DQO_ACT_Q8_K: case DQO_ACT_SX: return 256;
    default: return -1;
  }
}

static int64_t act_block_bytes(int fmt) {
  switch (fmt) {
    case DQO_ACT_PER32: return 40;  /* cpu_kernels.h:31-36 */
    case DQO_ACT_Q8_0: return 34;   /* quant_formats.h:23 */
    case DQO_ACT_Q8_K: return 292;  /* quant_formats.h:30 */
    case DQO_ACT_SX: return 320;    /* cpu_kernels.h:62-69 */
    case DQO_ACT_Q16: return 72;    /* cpu_kernels.h:77-82 */
    case DQO_ACT_F32: return 128;   /* 32 floats */
    default: return -1;
  }
}

int64_t dqo_act_row_bytes(int fmt, int64_t k) {
  const int64_t be = dqo_act_block_elems(fmt);
  if (be <= 0 || k < 0 || k % be != 0) return -1;
  return k / be * act_block_bytes(fmt);
}

/* ----------------------------------------------------------------- fp16 */

static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline uint16_t rd16(const uint8_t* p) { uint16_t v; memcpy(&v, p, 2); return v; }
static inline int16_t rd16s(const uint8_t* p) { int16_t v; memcpy(&v, p, 2); return v; }
static inline float rdf(const uint8_t* p) { float v; memcpy(&v, p, 4); return v; }
static inline int32_t rdi(const uint8_t* p) { int32_t v; memcpy(&v, p, 4); return v; }

/* IEEE binary16 -> binary32, exact (fp16.h:18-40 computes the same function).
 * NaNs keep their payload with the quiet bit set, as the reference's multiply does. */
float dqo_fp16_to_fp32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  if (e == 0x1F) return bits_f(sign | 0x7F800000u | (m << 13) | (m ? 0x00400000u : 0u));
  if (e != 0) return bits_f(sign | ((e + 112u) << 23) | (m << 13));
  /* zero / subnormal: m * 2^-24, exact in fp32 */
  return bits_f(sign | f_bits((float)m * 0x1.0p-24f));
}

/* IEEE binary32 -> binary16, round to nearest even, overflow to infinity,
 * NaN -> 0x7E00 with the sign kept (fp16.h:42-62 computes the same function). */
uint16_t dqo_fp32_to_fp16(float f) {
  const uint32_t w = f_bits(f);
  const uint16_t sign = (uint16_t)((w >> 16) & 0x8000u);
  const uint32_t a = w & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7E00u;
  if (a >= 0x477FF000u) return sign | 0x7C00u; /* >= 65520: rounds to infinity */
  const uint32_t e = a >> 23;
  if (e >= 113) { /* normal half: |f| >= 2^-14 */
    uint32_t h = ((e - 112u) << 10) | ((a >> 13) & 0x3FFu);
    const uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* carry may reach the exponent */
    return sign | (uint16_t)h;
  }
  if (e < 102) return sign; /* below 2^-25: rounds to zero */
  {
    const uint32_t m = (a & 0x7FFFFFu) | 0x800000u; /* value = m * 2^(e-150); half units = m * 2^(e-126) */
    const uint32_t shift = 126u - e;                 /* 14 .. 24 */
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), halfway = 1u << (shift - 1u);
    if (rem > halfway || (rem == halfway && (q & 1u))) q += 1; /* 1024 becomes the smallest normal */
    return sign | (uint16_t)q;
  }
}

void dqo_fp16_to_fp32_n(const uint16_t* h, float* f, int64_t n) {
  for (int64_t i = 0; i < n; ++i) f[i] = dqo_fp16_to_fp32(h[i]);
}
void dqo_fp32_to_fp16_n(const float* f, uint16_t* h, int64_t n) {
  for (int64_t i = 0; i < n; ++i) h[i] = dqo_fp32_to_fp16(f[i]);
}

/* The 6-bit scale and min of Q4_K sub-block j from the 12 packed bytes
 * (quant_formats.h:62-70). */
void dqo_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 15) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* -------------------------------------------------------- code unpacking */

/* The 256 weight codes of a Q4_K super-block, 0..15 in value order
 * (quant_formats.cpp:150-167: 64-value groups, low nibbles first). */
static void q4k_codes(const uint8_t* blk, int8_t* q) {
  const uint8_t* qs = blk + 16;
  for (int g = 0; g < 4; ++g) {
    for (int t = 0; t < 32; ++t) {
      q[64 * g + t] = (int8_t)(qs[32 * g + t] & 15);
      q[64 * g + 32 + t] = (int8_t)(qs[32 * g + t] >> 4);
    }
  }
}

/* The 256 signed codes (q - 32, in -32..31) of a Q6_K super-block
 * (quant_formats.cpp:192-216). */
static void q6k_codes(const uint8_t* blk, int8_t* q) {
  const uint8_t* ql = blk;
  const uint8_t* qh = blk + 128;
  for (int p = 0; p < 2; ++p) {
    for (int l = 0; l < 32; ++l) {
      const int h = qh[32 * p + l];
      q[128 * p + l] = (int8_t)(((ql[64 * p + l] & 15) | (((h >> 0) & 3) << 4)) - 32);
      q[128 * p + l + 32] = (int8_t)(((ql[64 * p + l + 32] & 15) | (((h >> 2) & 3) << 4)) - 32);
      q[128 * p + l + 64] = (int8_t)(((ql[64 * p + l] >> 4) | (((h >> 4) & 3) << 4)) - 32);
      q[128 * p + l + 96] = (int8_t)(((ql[64 * p + l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32);
    }
  }
}

/* The 32 signed codes of a Q4_0 block (nibble - 8; low nibbles = values 0-15,
 * quant_formats.cpp:12-20). */
static void q40_codes(const uint8_t* blk, int8_t* q) {
  for (int j = 0; j < 16; ++j) {
    q[j] = (int8_t)((blk[2 + j] & 15) - 8);
    q[j + 16] = (int8_t)((blk[2 + j] >> 4) - 8);
  }
}

/* ----------------------------------------------------------- dequantize */

int dqo_dequantize(int dtype, const void* blocks, float* y, int64_t n) {
  const int64_t be = dqo_block_elems(dtype), bb = dqo_block_bytes(dtype);
  if (be <= 0 || n % be != 0) return -1;
  const uint8_t* b = (const uint8_t*)blocks;
  int8_t q[256];
  for (int64_t i = 0; i < n / be; ++i, b += bb, y += be) {
    switch (dtype) {
      case DQO_Q8_0: { /* quant_formats.cpp:76-81 */
        const float d = dqo_fp16_to_fp32(rd16(b));
        for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)b[2 + j] * d;
        break;
      }
      case DQO_Q4_0: { /* quant_formats.cpp:12-20 */
        const float d = dqo_fp16_to_fp32(rd16(b));
        q40_codes(b, q);
        for (int j = 0; j < 32; ++j) y[j] = (float)q[j] * d;
        break;
      }
      case DQO_Q4_K: { /* quant_formats.cpp:150-167 */
        const float d = dqo_fp16_to_fp32(rd16(b)), dmin = dqo_fp16_to_fp32(rd16(b + 2));
        q4k_codes(b, q);
        for (int j = 0; j < 8; ++j) {
          uint8_t sc, mn;
          dqo_scale_min_k4(j, b + 4, &sc, &mn);
          const float d1 = d * (float)sc, m1 = dmin * (float)mn;
          for (int t = 0; t < 32; ++t) y[32 * j + t] = d1 * (float)q[32 * j + t] - m1;
        }
        break;
      }
      case DQO_Q6_K: { /* quant_formats.cpp:192-216 */
        const float d = dqo_fp16_to_fp32(rd16(b + 208));
        q6k_codes(b, q);
        for (int e = 0; e < 256; ++e) y[e] = d * (float)(int8_t)b[192 + e / 16] * (float)q[e];
        break;
      }
      case DQO_Q8_K: { /* quant_formats.cpp:218-222 */
        const float d = rdf(b);
        for (int j = 0; j < 256; ++j) y[j] = d * (float)(int8_t)b[4 + j];
        break;
      }
      default: return -1;
    }
  }
  return 0;
}

/* kernels_avx2.cpp:370-466: store_scaled(q, n, d, mn) writes fma(q, d, mn) for each
 * code; Q4_K passes (d * sc_j, -dmin * m_j) per 32 values (low nibbles of 32 qs bytes,
 * then their high nibbles), Q6_K (d * sc_g, 0) per 16, Q8_0 / Q4_0 (d, 0) per block. */
int dqo_expand_x86(int dtype, const void* blocks, float* y, int64_t n) {
  const int64_t be = dqo_block_elems(dtype), bb = dqo_block_bytes(dtype);
  if (be <= 0 || n % be != 0 || dtype == DQO_Q8_K) return -1;
  const uint8_t* b = (const uint8_t*)blocks;
  int8_t q[256];
  for (int64_t i = 0; i < n / be; ++i, b += bb, y += be) {
    switch (dtype) {
      case DQO_Q8_0: { /* :375-378 */
        const float d = dqo_fp16_to_fp32(rd16(b));
        for (int j = 0; j < 32; ++j) y[j] = fmaf((float)(int8_t)b[2 + j], d, 0.0f);
        break;
      }
      case DQO_Q4_0: { /* :380-391 */
        const float d = dqo_fp16_to_fp32(rd16(b));
        q40_codes(b, q);
        for (int j = 0; j < 32; ++j) y[j] = fmaf((float)q[j], d, 0.0f);
        break;
      }
      case DQO_Q4_K: { /* :420-438 */
        const float d = dqo_fp16_to_fp32(rd16(b)), dmin = dqo_fp16_to_fp32(rd16(b + 2));
        q4k_codes(b, q);
        for (int j = 0; j < 8; ++j) {
          uint8_t sc, mn;
          dqo_scale_min_k4(j, b + 4, &sc, &mn);
          const float d1 = d * (float)sc, m1 = -dmin * (float)mn;
          for (int t = 0; t < 32; ++t) y[32 * j + t] = fmaf((float)q[32 * j + t], d1, m1);
        }
        break;
      }
      case DQO_Q6_K: { /* :440-466 */
        const float d = dqo_fp16_to_fp32(rd16(b + 208));
        q6k_codes(b, q);
        for (int e = 0; e < 256; ++e) y[e] = fmaf((float)q[e], d * (float)(int8_t)b[192 + e / 16], 0.0f);
        break;
      }
      default: return -1;
    }
  }
  return 0;
}

int dqo_dequantize_act(int fmt, const void* a, float* y, int64_t n) {
  const int64_t be = dqo_act_block_elems(fmt), bb = act_block_bytes(fmt);
  if (be <= 0 || n % be != 0) return -1;
  const uint8_t* b = (const uint8_t*)a;
  for (int64_t i = 0; i < n / be; ++i, b += bb, y += be) {
    switch (fmt) {
      case DQO_ACT_PER32: {
        const float d = rdf(b);
        for (int j = 0; j < 32; ++j) y[j] = d * (float)(int8_t)b[8 + j];
        break;
      }
      case DQO_ACT_Q8_0: {
        const float d = dqo_fp16_to_fp32(rd16(b));
        for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)b[2 + j] * d;
        break;
      }
      case DQO_ACT_Q8_K: {
        const float d = rdf(b);
        for (int j = 0; j < 256; ++j) y[j] = d * (float)(int8_t)b[4 + j];
        break;
      }
      case DQO_ACT_SX: {
        const float u = rdf(b + 256);
        for (int j = 0; j < 256; ++j) {
          const float s = u * (float)rd16s(b + 260 + 2 * (j / 32));
          y[j] = s * (float)(int8_t)b[j];
        }
        break;
      }
      case DQO_ACT_Q16: {
        const float d = rdf(b);
        for (int j = 0; j < 32; ++j) y[j] = d * (float)rd16s(b + 8 + 2 * j);
        break;
      }
      case DQO_ACT_F32: memcpy(y, b, 128); break;
      default: return -1;
    }
  }
  return 0;
}

/* ------------------------------------------------------------ quantizers */

/* max |x| over n values, NaN never replacing the running maximum
 * (std::max(amax, std::fabs(x)) in kernels_generic.cpp:190). */
static float abs_max(const float* x, int n) {
  float amax = 0.0f;
  for (int i = 0; i < n; ++i) {
    const float a = fabsf(x[i]);
    amax = (amax < a) ? a : amax;
  }
  return amax;
}

/* The comparison clamp of kernels_generic.cpp:199 (NaN goes to -L). */
static inline float clamp_l(float v, float l) { return v > -l ? (v < l ? v : l) : -l; }

/* 32 codes at scale d, round half to even: the inner loop of quantize_act
 * (kernels_generic.cpp:191-203) and of quantize_block (kernels_avx2.cpp:609-631).
 * Returns the code sum. */
static int32_t codes_rne(const float* x, float d, int8_t* q) {
  const float id = d > 0 ? 1.0f / d : 0.0f;
  int32_t sum = 0;
  for (int i = 0; i < 32; ++i) {
    const float v = clamp_l(x[i] * id, 127.0f);
    int32_t c = (int32_t)rintf(v); /* default rounding mode: nearest, ties to even */
    c = c < -127 ? -127 : (c > 127 ? 127 : c);
    q[i] = (int8_t)c;
    sum += c;
  }
  return sum;
}

/* GGUF Q8_0 (quant_formats.cpp:60-74): d = amax/127 in fp32, codes rounded half
 * away from zero (std::lround) at that fp32 d, d stored as fp16. */
static void quantize_q8_0_block(const float* x, uint8_t* out) {
  const float amax = abs_max(x, 32);
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  const uint16_t h = dqo_fp32_to_fp16(d);
  memcpy(out, &h, 2);
  for (int i = 0; i < 32; ++i) {
    const float v = clamp_l(x[i] * id, 127.0f);
    out[2 + i] = (uint8_t)(int8_t)lroundf(v);
  }
}

/* Per-32 ActBlockQ8 (kernels_generic.cpp:187-207): d = amax/127 (fp32), codes
 * round half to even, sum of the codes. */
static void quantize_per32_block(const float* x, uint8_t* out) {
  const float d = abs_max(x, 32) / 127.0f;
  int8_t q[32];
  const int32_t sum = codes_rne(x, d, q);
  memcpy(out, &d, 4);
  memcpy(out + 4, &sum, 4);
  memcpy(out + 8, q, 32);
}

/* Q8_K: one scale per 256 values, d = amax256/127 (fp32), each 32-block's codes
 * as quantize_block at that d (kernels_avx2.cpp:638-644), bsums[g] = sum of
 * codes 16g .. 16g+15 (quant_formats.h:30). */
static void quantize_q8_K_block(const float* x, uint8_t* out) {
  const float d = abs_max(x, 256) / 127.0f;
  int8_t q[256];
  for (int b = 0; b < 8; ++b) (void)codes_rne(x + 32 * b, d, q + 32 * b);
  memcpy(out, &d, 4);
  memcpy(out + 4, q, 256);
  for (int g = 0; g < 16; ++g) {
    int32_t s = 0;
    for (int t = 0; t < 16; ++t) s += q[16 * g + t];
    const int16_t s16 = (int16_t)s;
    memcpy(out + 260 + 2 * g, &s16, 2);
  }
}

/* Sub-scaled ActSuperQ8 (kernels_avx2.cpp:1077-1096): u = amax256/(127*128);
 * per 32-block m = clamp(ceil(amax32/(127u)), 1, 128) (1 when u == 0); codes at
 * scale u*m; ms = (u*m)*sum. */
static void quantize_sx_block(const float* x, uint8_t* out) {
  const float u = abs_max(x, 256) / (127.0f * 128.0f);
  memset(out, 0, 320);
  memcpy(out + 256, &u, 4);
  for (int b = 0; b < 8; ++b) {
    int32_t m = 1;
    if (u > 0) {
      const float need = abs_max(x + 32 * b, 32) / (127.0f * u);
      const int32_t c = (int32_t)ceilf(need);
      m = c < 1 ? 1 : (c > 128 ? 128 : c);
    }
    const float s = u * (float)m;
    const int32_t sum = codes_rne(x + 32 * b, s, (int8_t*)out + 32 * b);
    const int16_t m16 = (int16_t)m;
    const float ms = s * (float)sum;
    memcpy(out + 260 + 2 * b, &m16, 2);
    memcpy(out + 276 + 4 * b, &ms, 4);
  }
}

/* int16 ActBlockQ16 (quantize_act16, kernels_avx2.cpp:1631-1652): d = amax32/32767
 * (fp32), id = 1/d (0 when d == 0), r = x*id rounded half to even; the int32
 * conversion gives INT32_MIN for NaN and out-of-range r (cvtps_epi32); sum = the
 * wrapping int32 sum of those codes; the stored codes saturate to int16
 * (packs_epi32). amax here never takes a NaN (the reference's AVX2 max does,
 * depending on the NaN's lane: NaN inputs are outside this format's parity). */
static void quantize_q16_block(const float* x, uint8_t* out) {
  const float d = abs_max(x, 32) / 32767.0f;
  const float id = d > 0 ? 1.0f / d : 0.0f;
  uint32_t sum = 0;
  for (int i = 0; i < 32; ++i) {
    const float r = rintf(x[i] * id);
    const int32_t c = (r >= -2147483648.0f && r < 2147483648.0f) ? (int32_t)r : INT32_MIN;
    sum += (uint32_t)c;
    const int16_t q = (int16_t)(c < -32768 ? -32768 : (c > 32767 ? 32767 : c));
    memcpy(out + 8 + 2 * i, &q, 2);
  }
  const int32_t s = (int32_t)sum;
  memcpy(out, &d, 4);
  memcpy(out + 4, &s, 4);
}

int dqo_quantize_act(int fmt, const float* x, void* out, int64_t n) {
  const int64_t be = dqo_act_block_elems(fmt), bb = act_block_bytes(fmt);
  if (be <= 0 || n % be != 0) return -1;
  uint8_t* o = (uint8_t*)out;
  for (int64_t b = 0; b < n / be; ++b, x += be, o += bb) {
    switch (fmt) {
      case DQO_ACT_PER32: quantize_per32_block(x, o); break;
      case DQO_ACT_Q8_0: quantize_q8_0_block(x, o); break;
      case DQO_ACT_Q8_K: quantize_q8_K_block(x, o); break;
      case DQO_ACT_SX: quantize_sx_block(x, o); break;
      case DQO_ACT_Q16: quantize_q16_block(x, o); break;
      case DQO_ACT_F32: memcpy(o, x, 128); break;
      default: return -1;
    }
  }
  return 0;
}

int dqo_quantize_act_rows(int fmt, const float* x, int64_t m, int64_t n, int64_t x_stride, void* out) {
  const int64_t rb = dqo_act_row_bytes(fmt, n);
  if (rb < 0) return -1;
  for (int64_t r = 0; r < m; ++r) {
    if (dqo_quantize_act(fmt, x + r * x_stride, (uint8_t*)out + r * rb, n) != 0) return -1;
  }
  return 0;
}

/* ------------------------------------------------------ weight encoders */
/* The reference has no quantizer for Q4_0 / Q4_K / Q6_K (quant_formats.h:41-59
 * declares only quantize_q8_0). These are this project's own deterministic
 * encoders: any valid block bytes serve, because the CPU oracle and the GPU
 * consume the same bytes. */

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* Q4_0: d = (value of largest magnitude) / -8 rounded to fp16, codes
 * clamp(floor(x / d + 8.5), 0, 15). */
static void encode_q4_0_block(const float* x, uint8_t* out) {
  float vmax = 0.0f, amax = 0.0f;
  for (int i = 0; i < 32; ++i) {
    if (fabsf(x[i]) > amax) { amax = fabsf(x[i]); vmax = x[i]; }
  }
  const uint16_t h = dqo_fp32_to_fp16(vmax / -8.0f);
  const float d = dqo_fp16_to_fp32(h);
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  memcpy(out, &h, 2);
  for (int j = 0; j < 16; ++j) {
    const int lo = clampi((int)floorf(x[j] * id + 8.5f), 0, 15);
    const int hi = clampi((int)floorf(x[j + 16] * id + 8.5f), 0, 15);
    out[2 + j] = (uint8_t)(lo | (hi << 4));
  }
}

/* Q4_K: per 32-value sub-block an offset -min(0, min x) and a step
 * (max - min)/15; super-block d = max step / 63 and dmin = max offset / 63 in
 * fp16; 6-bit sc = ceil(step / d), m = ceil(offset / dmin); codes
 * round((x + dmin*m) / (d*sc)) in 0..15. Scales packed as get_scale_min_k4
 * (quant_formats.h:62-70) reads them. */
static void encode_q4_K_block(const float* x, uint8_t* out) {
  float step[8], off[8], max_step = 0.0f, max_off = 0.0f;
  for (int j = 0; j < 8; ++j) {
    float lo = 0.0f, hi = -INFINITY;
    for (int t = 0; t < 32; ++t) {
      const float v = x[32 * j + t];
      lo = v < lo ? v : lo;
      hi = v > hi ? v : hi;
    }
    step[j] = (hi - lo) / 15.0f;
    off[j] = -lo;
    max_step = step[j] > max_step ? step[j] : max_step;
    max_off = off[j] > max_off ? off[j] : max_off;
  }
  const uint16_t hd = dqo_fp32_to_fp16(max_step / 63.0f), hm = dqo_fp32_to_fp16(max_off / 63.0f);
  const float d = dqo_fp16_to_fp32(hd), dmin = dqo_fp16_to_fp32(hm);
  uint8_t sc[8], mn[8];
  for (int j = 0; j < 8; ++j) {
    sc[j] = (uint8_t)(d > 0 ? clampi((int)ceilf(step[j] / d), 0, 63) : 0);
    mn[j] = (uint8_t)(dmin > 0 ? clampi((int)ceilf(off[j] / dmin), 0, 63) : 0);
  }
  memcpy(out, &hd, 2);
  memcpy(out + 2, &hm, 2);
  uint8_t* s = out + 4;
  for (int j = 0; j < 4; ++j) {
    s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    s[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
    s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
  }
  int8_t q[256];
  for (int j = 0; j < 8; ++j) {
    const float st = d * (float)sc[j], o = dmin * (float)mn[j];
    for (int t = 0; t < 32; ++t) {
      q[32 * j + t] = (int8_t)(st > 0 ? clampi((int)lroundf((x[32 * j + t] + o) / st), 0, 15) : 0);
    }
  }
  for (int g = 0; g < 4; ++g) {
    for (int t = 0; t < 32; ++t) out[16 + 32 * g + t] = (uint8_t)(q[64 * g + t] | (q[64 * g + 32 + t] << 4));
  }
}

/* Q6_K: per 16 values a step amax/31; super-block d = max step / 127 in fp16;
 * int8 sc = ceil(step / d); codes round(x / (d*sc)) in -32..31, stored + 32 in
 * the ql / qh bit planes of quant_formats.cpp:192-216. */
static void encode_q6_K_block(const float* x, uint8_t* out) {
  float step[16], max_step = 0.0f;
  for (int u = 0; u < 16; ++u) {
    step[u] = abs_max(x + 16 * u, 16) / 31.0f;
    max_step = step[u] > max_step ? step[u] : max_step;
  }
  const uint16_t hd = dqo_fp32_to_fp16(max_step / 127.0f);
  const float d = dqo_fp16_to_fp32(hd);
  int8_t sc[16];
  uint8_t q[256];
  for (int u = 0; u < 16; ++u) {
    sc[u] = (int8_t)(d > 0 ? clampi((int)ceilf(step[u] / d), 0, 127) : 0);
    const float st = d * (float)sc[u];
    for (int t = 0; t < 16; ++t) {
      const int c = st > 0 ? clampi((int)lroundf(x[16 * u + t] / st), -32, 31) : 0;
      q[16 * u + t] = (uint8_t)(c + 32);
    }
  }
  memset(out, 0, 210);
  for (int p = 0; p < 2; ++p) {
    for (int l = 0; l < 32; ++l) {
      const uint8_t* v = q + 128 * p;
      out[64 * p + l] = (uint8_t)((v[l] & 15) | ((v[l + 64] & 15) << 4));
      out[64 * p + l + 32] = (uint8_t)((v[l + 32] & 15) | ((v[l + 96] & 15) << 4));
      out[128 + 32 * p + l] = (uint8_t)((v[l] >> 4) | ((v[l + 32] >> 4) << 2) | ((v[l + 64] >> 4) << 4) | ((v[l + 96] >> 4) << 6));
    }
  }
  memcpy(out + 192, sc, 16);
  memcpy(out + 208, &hd, 2);
}

int dqo_encode_weight(int dtype, const float* x, void* out, int64_t n) {
  const int64_t be = dqo_block_elems(dtype), bb = dqo_block_bytes(dtype);
  if (be <= 0 || n % be != 0 || dtype == DQO_Q8_K) return -1;
  uint8_t* o = (uint8_t*)out;
  for (int64_t b = 0; b < n / be; ++b, x += be, o += bb) {
    switch (dtype) {
      case DQO_Q8_0: quantize_q8_0_block(x, o); break;
      case DQO_Q4_0: encode_q4_0_block(x, o); break;
      case DQO_Q4_K: encode_q4_K_block(x, o); break;
      case DQO_Q6_K: encode_q6_K_block(x, o); break;
      default: return -1;
    }
  }
  return 0;
}

int dqo_encode_weight_rows(int dtype, const float* x, int64_t rows, int64_t n, void* out) {
  const int64_t rb = dqo_row_bytes(dtype, n);
  if (rb < 0) return -1;
  for (int64_t r = 0; r < rows; ++r) {
    if (dqo_encode_weight(dtype, x + r * n, (uint8_t*)out + r * rb, n) != 0) return -1;
  }
  return 0;
}

/* ------------------------------------------------------------- partials */

static int pair_ok(int wtype, int fmt) {
  if (fmt == DQO_ACT_F32) return 0; /* no integer partials; the dots have their own path */
  if (fmt == DQO_ACT_Q16) return wtype == DQO_Q8_0 || wtype == DQO_Q4_0 || wtype == DQO_Q4_K || wtype == DQO_Q6_K;
  switch (wtype) {
    case DQO_Q8_0: case DQO_Q4_0: return fmt == DQO_ACT_PER32 || fmt == DQO_ACT_Q8_0;
    case DQO_Q4_K: case DQO_Q6_K: return fmt == DQO_ACT_PER32 || fmt == DQO_ACT_Q8_K || fmt == DQO_ACT_SX;
    default: return 0;
  }
}

int dqo_partials_count(int wtype, int fmt, int64_t k, int64_t* units, int64_t* sb_terms) {
  if (!pair_ok(wtype, fmt) || dqo_row_bytes(wtype, k) < 0 || dqo_act_row_bytes(fmt, k) < 0) return -1;
  *units = wtype == DQO_Q6_K ? k / 16 : k / 32;
  *sb_terms = !(wtype == DQO_Q4_K || wtype == DQO_Q6_K) || fmt == DQO_ACT_PER32 || fmt == DQO_ACT_Q16 ? 0
              : fmt == DQO_ACT_SX ? 3 * (k / 256) : 2 * (k / 256);
  return 0;
}

/* Activation codes of value i of a quantized row. */
static int32_t act_code(int fmt, const uint8_t* a, int64_t i) {
  switch (fmt) {
    case DQO_ACT_PER32: return (int8_t)a[(i / 32) * 40 + 8 + i % 32];
    case DQO_ACT_Q8_0: return (int8_t)a[(i / 32) * 34 + 2 + i % 32];
    case DQO_ACT_Q8_K: return (int8_t)a[(i / 256) * 292 + 4 + i % 256];
    case DQO_ACT_SX: return (int8_t)a[(i / 256) * 320 + i % 256];
    case DQO_ACT_Q16: return rd16s(a + (i / 32) * 72 + 8 + 2 * (i % 32));
    default: return 0;
  }
}

/* Code sum of 32-block b of an activation row. */
static int32_t act_sum32(int fmt, const uint8_t* a, int64_t b) {
  switch (fmt) {
    case DQO_ACT_PER32: return rdi(a + b * 40 + 4);
    case DQO_ACT_Q16: return rdi(a + b * 72 + 4);
    case DQO_ACT_Q8_K: {
      const uint8_t* blk = a + (b / 8) * 292;
      const int j = (int)(b % 8);
      return (int32_t)rd16s(blk + 260 + 4 * j) + (int32_t)rd16s(blk + 262 + 4 * j);
    }
    default: {
      int32_t s = 0;
      for (int t = 0; t < 32; ++t) s += act_code(fmt, a, 32 * b + t);
      return s;
    }
  }
}

/* Signed weight codes of super-block / block `b` (values in storage order). */
static void weight_codes(int wtype, const uint8_t* w, int64_t b, int8_t* q) {
  switch (wtype) {
    case DQO_Q8_0: memcpy(q, w + b * 34 + 2, 32); break;
    case DQO_Q4_0: q40_codes(w + b * 18, q); break;
    case DQO_Q4_K: q4k_codes(w + b * 144, q); break;
    case DQO_Q6_K: q6k_codes(w + b * 210, q); break;
    default: break;
  }
}

/* Exact integer partials (Appendix of the arithmetic contract):
 *   Q8_0 / Q4_0 x per-32 | Q8_0: P_b = sum_{i<32} w_i a_i   (kernels_generic.cpp:210-239)
 *   Q4_K: P_j over 32 values (kernels_generic.cpp:261-279)
 *   Q6_K: P_u over 16 values (kernels_generic.cpp:282-310)
 *   Q4_K x Q8_K: S = sum_j sc_j P_j, Mn = sum_j m_j sum_j (kernels_avx2.cpp:976-1014)
 *   Q6_K x Q8_K: S = sum_u sc_u P_u (kernels_avx2.cpp:1019-1058)
 *   x sub-scaled: S = sum sc * m_b * P (kernels_avx2.cpp:1117-1216) in 64 bits (it can
 *     exceed 2^31: 8 * 63 * 128 * 32 * 15 * 127), reported as its low and high
 *     words; Mn = sum_j m_j * (m_b * sum_b of the sub-block's codes), the exact
 *     integer behind the reference's ms_b = u * m_b * sum_b (kernels_avx2.cpp:1087-1092). */
int dqo_partials(int wtype, int fmt, const void* wrow, const void* arow, int64_t k, int32_t* units, int32_t* sb) {
  int64_t nu, ns;
  if (dqo_partials_count(wtype, fmt, k, &nu, &ns) != 0) return -1;
  const uint8_t* w = (const uint8_t*)wrow;
  const uint8_t* a = (const uint8_t*)arow;
  int8_t q[256];
  if (wtype == DQO_Q8_0 || wtype == DQO_Q4_0) {
    for (int64_t b = 0; b < k / 32; ++b) {
      weight_codes(wtype, w, b, q);
      int32_t s = 0;
      for (int t = 0; t < 32; ++t) s += (int32_t)q[t] * act_code(fmt, a, 32 * b + t);
      units[b] = s;
    }
    return 0;
  }
  const int ul = wtype == DQO_Q6_K ? 16 : 32; /* values per unit */
  for (int64_t b = 0; b < k / 256; ++b) {
    weight_codes(wtype, w, b, q);
    const uint8_t* blk = w + b * (wtype == DQO_Q4_K ? 144 : 210);
    int64_t S = 0;
    int32_t Mn = 0;
    for (int u = 0; u < 256 / ul; ++u) {
      int32_t p = 0;
      for (int t = 0; t < ul; ++t) p += (int32_t)q[ul * u + t] * act_code(fmt, a, 256 * b + ul * u + t);
      units[b * (256 / ul) + u] = p;
      int32_t scale;
      if (wtype == DQO_Q4_K) {
        uint8_t sc, mn;
        dqo_scale_min_k4(u, blk + 4, &sc, &mn);
        scale = sc;
        if (ns) {
          const int32_t mb = fmt == DQO_ACT_SX ? rd16s(a + b * 320 + 260 + 2 * u) : 1;
          Mn += (int32_t)mn * (mb * act_sum32(fmt, a, 8 * b + u));
        }
      } else {
        scale = (int8_t)blk[192 + u];
      }
      if (fmt == DQO_ACT_SX) scale *= rd16s(a + b * 320 + 260 + 2 * (u * ul / 32));
      S += (int64_t)scale * p;
    }
    if (ns && fmt == DQO_ACT_SX) {
      sb[3 * b] = (int32_t)(uint32_t)((uint64_t)S & 0xFFFFFFFFu);
      sb[3 * b + 1] = (int32_t)(S >> 32);
      sb[3 * b + 2] = Mn;
    } else if (ns) {
      sb[2 * b] = (int32_t)S;
      sb[2 * b + 1] = Mn;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ dots */

/* fp32 activations: the generic vec_dot_* (kernels_generic.cpp:67-150), every fp32
 * operation rounding where written (the generic tier has no FMA contraction). */
static float vec_dot_f32(int wtype, const uint8_t* w, const float* x, int64_t k) {
  float sum = 0.0f;
  if (wtype == DQO_Q8_0 || wtype == DQO_Q4_0) {
    const int64_t bb = wtype == DQO_Q8_0 ? 34 : 18;
    for (int64_t i = 0; i < k / 32; ++i, x += 32) {
      const uint8_t* b = w + i * bb;
      float s = 0.0f;
      if (wtype == DQO_Q8_0) {
        for (int j = 0; j < 32; ++j) s = s + (float)(int8_t)b[2 + j] * x[j];
      } else {
        for (int j = 0; j < 16; ++j) {
          s = s + (float)((b[2 + j] & 0x0F) - 8) * x[j];
          s = s + (float)((b[2 + j] >> 4) - 8) * x[j + 16];
        }
      }
      sum = sum + dqo_fp16_to_fp32(rd16(b)) * s;
    }
    return sum;
  }
  for (int64_t i = 0; i < k / 256; ++i) {
    if (wtype == DQO_Q4_K) {
      const uint8_t* b = w + i * 144;
      const float d = dqo_fp16_to_fp32(rd16(b)), dmin = dqo_fp16_to_fp32(rd16(b + 2));
      const uint8_t* q = b + 16;
      for (int j = 0, is = 0; j < 256; j += 64, is += 2, q += 32, x += 64) {
        uint8_t sc, m;
        float dot_lo = 0.0f, sum_lo = 0.0f, dot_hi = 0.0f, sum_hi = 0.0f;
        for (int l = 0; l < 32; ++l) {
          dot_lo = dot_lo + (float)(q[l] & 0xF) * x[l];
          sum_lo = sum_lo + x[l];
          dot_hi = dot_hi + (float)(q[l] >> 4) * x[l + 32];
          sum_hi = sum_hi + x[l + 32];
        }
        dqo_scale_min_k4(is, b + 4, &sc, &m);
        sum = sum + ((d * (float)sc) * dot_lo - (dmin * (float)m) * sum_lo);
        dqo_scale_min_k4(is + 1, b + 4, &sc, &m);
        sum = sum + ((d * (float)sc) * dot_hi - (dmin * (float)m) * sum_hi);
      }
    } else { /* Q6_K */
      const uint8_t* b = w + i * 210;
      const float d = dqo_fp16_to_fp32(rd16(b + 208));
      const uint8_t* ql = b;
      const uint8_t* qh = b + 128;
      const int8_t* sc = (const int8_t*)(b + 192);
      for (int part = 0; part < 2; ++part, ql += 64, qh += 32, sc += 8, x += 128) {
        float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int l = 0; l < 32; ++l) {
          const int is = l / 16;
          const int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
          const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
          const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
          const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
          s[is + 0] = s[is + 0] + (float)q1 * x[l];
          s[is + 2] = s[is + 2] + (float)q2 * x[l + 32];
          s[is + 4] = s[is + 4] + (float)q3 * x[l + 64];
          s[is + 6] = s[is + 6] + (float)q4 * x[l + 96];
        }
        for (int g = 0; g < 8; ++g) sum = sum + (d * (float)sc[g]) * s[g];
      }
    }
  }
  return sum;
}

float dqo_dot(int wtype, int fmt, const void* wrow, const void* arow, int64_t k) {
  if (fmt == DQO_ACT_F32) {
    if (dqo_row_bytes(wtype, k) < 0 || k % 32 != 0) return NAN;
    return vec_dot_f32(wtype, (const uint8_t*)wrow, (const float*)arow, k);
  }
  if (!pair_ok(wtype, fmt) || dqo_row_bytes(wtype, k) < 0 || dqo_act_row_bytes(fmt, k) < 0) return NAN;
  const uint8_t* w = (const uint8_t*)wrow;
  const uint8_t* a = (const uint8_t*)arow;
  int32_t units[4096 / 16 + 16];
  int32_t sb[3];
  float acc = 0.0f;

  if (fmt == DQO_ACT_Q16) {
    /* int16 activations: the arithmetic of dot_rows16_* (kernels_avx2.cpp:1662-1765)
     * in one accumulator. Per unit the exact integer P (32 values; Q6_K 16) times
     * the integer sub-block scale, acc = fma((float)(sc*P), d*da, acc); Q4_K's mins
     * term cor += dmin*((m*da)*(float)sum) apart, returned as acc - cor. */
    float cor = 0.0f;
    const int b32 = wtype == DQO_Q8_0 || wtype == DQO_Q4_0;
    for (int64_t b = 0; b < (b32 ? k / 32 : k / 256); ++b) {
      if (wtype == DQO_Q8_0) {
        int32_t p = 0;
        for (int t = 0; t < 32; ++t) p += (int32_t)(int8_t)w[b * 34 + 2 + t] * act_code(fmt, a, 32 * b + t);
        const float dw = dqo_fp16_to_fp32(rd16(w + b * 34));
        acc = fmaf((float)p, dw * rdf(a + b * 72), acc);
        continue;
      }
      if (wtype == DQO_Q4_0) {
        /* no AVX2 kernel: qmm's dot_row_ref (qmm_reference.cpp:68-93) with the codes
         * qmm_unpack.h:61-75 unpacks, acc += (dw * da) * (float)P per block */
        int8_t q[32];
        weight_codes(wtype, w, b, q);
        int32_t p = 0;
        for (int t = 0; t < 32; ++t) p += (int32_t)q[t] * act_code(fmt, a, 32 * b + t);
        const float t1 = dqo_fp16_to_fp32(rd16(w + b * 18)) * rdf(a + b * 72);
        const float t2 = t1 * (float)p;
        acc = acc + t2;
        continue;
      }
      const uint8_t* blk = w + b * (wtype == DQO_Q4_K ? 144 : 210);
      if (dqo_partials(wtype, fmt, blk, a + b * 8 * 72, 256, units, sb) != 0) return NAN;
      if (wtype == DQO_Q4_K) {
        const float d = dqo_fp16_to_fp32(rd16(blk)), dmin = dqo_fp16_to_fp32(rd16(blk + 2));
        for (int j = 0; j < 8; ++j) {
          uint8_t sc, mn;
          dqo_scale_min_k4(j, blk + 4, &sc, &mn);
          const uint8_t* ab = a + (b * 8 + j) * 72;
          const float ad = rdf(ab);
          acc = fmaf((float)((int32_t)sc * units[j]), d * ad, acc);
          const float t1 = (float)mn * ad;
          const float t2 = t1 * (float)rdi(ab + 4);
          cor = cor + dmin * t2;
        }
      } else {
        const float d = dqo_fp16_to_fp32(rd16(blk + 208));
        for (int u = 0; u < 16; ++u) {
          const float ad = rdf(a + (b * 8 + u / 2) * 72);
          acc = fmaf((float)((int32_t)(int8_t)blk[192 + u] * units[u]), d * ad, acc);
        }
      }
    }
    return acc - cor;
  }

  if (wtype == DQO_Q8_0 || wtype == DQO_Q4_0) {
    /* dot_rows_q8_0 / dot_rows_q4_0 (kernels_generic.cpp:216-239):
     * acc += (dw * da) * (float)P_b, blocks in order. */
    const int64_t wb = wtype == DQO_Q8_0 ? 34 : 18;
    for (int64_t b = 0; b < k / 32; ++b) {
      int8_t q[32];
      weight_codes(wtype, w, b, q);
      int32_t p = 0;
      for (int t = 0; t < 32; ++t) p += (int32_t)q[t] * act_code(fmt, a, 32 * b + t);
      const float dw = dqo_fp16_to_fp32(rd16(w + b * wb));
      const float da = fmt == DQO_ACT_PER32 ? rdf(a + b * 40) : dqo_fp16_to_fp32(rd16(a + b * 34));
      const float t1 = dw * da;
      const float t2 = t1 * (float)p;
      acc = acc + t2;
    }
    return acc;
  }

  for (int64_t b = 0; b < k / 256; ++b) {
    const uint8_t* blk = w + b * (wtype == DQO_Q4_K ? 144 : 210);
    /* the partials of this super-block only */
    if (dqo_partials(wtype, fmt, blk, fmt == DQO_ACT_PER32 ? a + b * 8 * 40
                                        : fmt == DQO_ACT_Q8_K ? a + b * 292 : a + b * 320,
                     256, units, sb) != 0) {
      return NAN;
    }
    if (wtype == DQO_Q4_K) {
      const float d = dqo_fp16_to_fp32(rd16(blk)), dmin = dqo_fp16_to_fp32(rd16(blk + 2));
      if (fmt == DQO_ACT_PER32) {
        /* dot_rows_q4_K (kernels_generic.cpp:261-279): per sub-block
         * acc += a.d * (d*sc*(float)P - dmin*m*(float)a.sum). */
        for (int j = 0; j < 8; ++j) {
          uint8_t sc, mn;
          dqo_scale_min_k4(j, blk + 4, &sc, &mn);
          const uint8_t* ab = a + (b * 8 + j) * 40;
          const float ad = rdf(ab);
          const float t1 = d * (float)sc;
          const float t2 = t1 * (float)units[j];
          const float t3 = dmin * (float)mn;
          const float t4 = t3 * (float)rdi(ab + 4);
          const float t5 = t2 - t4;
          const float t6 = ad * t5;
          acc = acc + t6;
        }
      } else if (fmt == DQO_ACT_Q8_K) {
        /* Q8_K: the exact super-block integers S and Mn of kernels_avx2.cpp:976-1014,
         * combined in this library's canonical order
         * u = d*(float)S; u = fma(-dmin, (float)Mn, u); acc = fma(da, u, acc). */
        const float da = rdf(a + b * 292);
        float u = d * (float)sb[0];
        u = fmaf(-dmin, (float)sb[1], u);
        acc = fmaf(da, u, acc);
      } else {
        /* sub-scaled (kernels_avx2.cpp:1117-1163): the exact S and Mn of
         * dqo_partials in the canonical order of the Q8_K pair, u in place of da. */
        const float u = rdf(a + b * 320 + 256);
        const int64_t S = (int64_t)(((uint64_t)(uint32_t)sb[1] << 32) | (uint32_t)sb[0]);
        float t = d * (float)S;
        t = fmaf(-dmin, (float)sb[2], t);
        acc = fmaf(u, t, acc);
      }
    } else { /* Q6_K */
      const float d = dqo_fp16_to_fp32(rd16(blk + 208));
      if (fmt == DQO_ACT_PER32) {
        /* dot_rows_q6_K (kernels_generic.cpp:282-310): per 16 values
         * acc += ((a.d * d) * sc) * (float)P. */
        for (int u = 0; u < 16; ++u) {
          const float ad = rdf(a + (b * 8 + u / 2) * 40);
          const float t1 = ad * d;
          const float t2 = t1 * (float)(int8_t)blk[192 + u];
          const float t3 = t2 * (float)units[u];
          acc = acc + t3;
        }
      } else if (fmt == DQO_ACT_Q8_K) {
        /* S of kernels_avx2.cpp:1019-1058; u = d*(float)S; acc = fma(da, u, acc). */
        const float da = rdf(a + b * 292);
        const float u = d * (float)sb[0];
        acc = fmaf(da, u, acc);
      } else {
        const float u = rdf(a + b * 320 + 256);
        const int64_t S = (int64_t)(((uint64_t)(uint32_t)sb[1] << 32) | (uint32_t)sb[0]);
        acc = fmaf(u, d * (float)S, acc);
      }
    }
  }
  return acc;
}

int dqo_matmul(int wtype, int fmt, const void* w, int64_t w_row_bytes, int64_t n, const void* acts,
               int64_t a_row_bytes, int64_t m, int64_t k, float* y, int64_t y_stride, const float* bias) {
  if ((fmt != DQO_ACT_F32 && !pair_ok(wtype, fmt)) || dqo_row_bytes(wtype, k) < 0 || dqo_act_row_bytes(fmt, k) < 0) return -1;
  for (int64_t r = 0; r < m; ++r) {
    for (int64_t i = 0; i < n; ++i) {
      const float v = dqo_dot(wtype, fmt, (const uint8_t*)w + i * w_row_bytes, (const uint8_t*)acts + r * a_row_bytes, k);
      y[r * y_stride + i] = bias ? v + bias[i] : v;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ PRNG */

uint64_t dqo_splitmix64(uint64_t* state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static double uniform01(uint64_t* s) { return (double)(dqo_splitmix64(s) >> 11) * 0x1.0p-53; }

void dqo_fill_normal(uint64_t seed, float* out, int64_t n, double mean, double std, double outlier_frac,
                     double outlier_sigma) {
  uint64_t s = seed;
  for (int64_t i = 0; i < n; i += 2) {
    const double u1 = 1.0 - uniform01(&s), u2 = uniform01(&s);
    const double r = sqrt(-2.0 * log(u1)), th = 6.283185307179586 * u2;
    out[i] = (float)(mean + std * r * cos(th));
    if (i + 1 < n) out[i + 1] = (float)(mean + std * r * sin(th));
  }
  if (outlier_frac > 0) {
    uint64_t t = seed ^ 0xD1B54A32D192ED03ull;
    for (int64_t i = 0; i < n; ++i) {
      if (uniform01(&t) < outlier_frac) out[i] = (float)(mean + ((dqo_splitmix64(&t) & 1) ? 1.0 : -1.0) * outlier_sigma * std);
    }
  }
}

void dqo_fill_bytes(uint64_t seed, uint8_t* out, int64_t n) {
  uint64_t s = seed;
  for (int64_t i = 0; i < n; i += 8) {
    const uint64_t v = dqo_splitmix64(&s);
    for (int j = 0; j < 8 && i + j < n; ++j) out[i + j] = (uint8_t)(v >> (8 * j));
  }
}

/* ---------------------------------------------------------- activations */

/* fast_exp.h:16-35: the comparison clamp (NaN -> -87), round to nearest through
 * 1.5 * 2^23, r = x - n ln2 in two parts, Horner degree 6, times 2^n. With
 * -ffp-contract=off each product and sum rounds where written. */
float dqo_exp_nonpos(float x) {
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
  const uint32_t bits = (uint32_t)((int32_t)n + 127) << 23;
  float scale;
  memcpy(&scale, &bits, 4);
  return p * scale;
}

/* cpu_device.cpp:117-128: silu(x) = x * (x >= 0 ? 1 : e) / (1 + e), e = e^-|x|;
 * gelu(x) = 0.5 x (1 + erf(x / sqrt 2)); gelu_tanh with sqrt(2 / pi). */
static float act1(int act, float x) {
  switch (act) {
    case DQO_SILU: {
      const float e = dqo_exp_nonpos(-fabsf(x));
      return x * (x >= 0.0f ? 1.0f : e) / (1.0f + e);
    }
    case DQO_GELU:
      return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
    default: {
      const float kc = 0.7978845608028654f;
      return 0.5f * x * (1.0f + tanhf(kc * (x + 0.044715f * x * x * x)));
    }
  }
}

int dqo_activation(int act, const float* x, float* y, int64_t n) {
  if (act != DQO_SILU && act != DQO_GELU && act != DQO_GELU_TANH) return -1;
  for (int64_t i = 0; i < n; ++i) y[i] = act1(act, x[i]);
  return 0;
}

/* ------------------------------------------------- qmm activation buffer */

/* One row of qmm activations: quantize_row_ref, dynacore/cpu/qmm/qmm_reference.cpp:25-51.
   Per 32-value block: amax (NaN ignored, as std::max(amax, |x|) keeps amax), d = amax / qmax,
   id = 1 / d (0 for d == 0), code = nearbyint(clamp(x * id, -qmax, qmax)) with NaN going to
   -qmax, c = d * (float)(code sum). Code i of block b at chunk 4 b + i / 8, byte i % 8,
   chunks cs bytes apart; int16 stores q >> 8 in hi and q & 0xFF in lo. */
static void qmm_row(const float* x, int64_t k, int mode, int8_t* hi, uint8_t* lo, int64_t cs, float* d, float* c,
                    int64_t ds) {
  const float qmax = mode == 0 ? 127.0f : 32767.0f;
  for (int64_t b = 0; b < k / 32; ++b, x += 32) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
      const float a = fabsf(x[i]);
      if (amax < a) amax = a;
    }
    const float db = amax / qmax;
    const float id = db > 0 ? 1.0f / db : 0.0f;
    int32_t sum = 0;
    for (int i = 0; i < 32; ++i) {
      float v = x[i] * id;
      v = v > -qmax ? (v < qmax ? v : qmax) : -qmax;
      const int32_t q = (int32_t)nearbyintf(v);
      sum += q;
      const int64_t at = (b * 4 + i / 8) * cs + i % 8;
      if (mode == 0) {
        hi[at] = (int8_t)q;
      } else {
        hi[at] = (int8_t)(q >> 8);
        lo[at] = (uint8_t)(q & 0xFF);
      }
    }
    d[b * ds] = db;
    c[b * ds] = db * (float)sum;
  }
}

/* All m rows into the layout of ActBuffer::prepare / quantize_rows (qmm_reference.cpp:440-488;
   dynacore/include/dynacore/cpu/qmm.h:57-70): row layout codes at hi + r k, scales at r kb;
   pair layout (paired != 0) rows 2p, 2p + 1 interleaved in 8-byte chunks at hi + p 2k + 16 j
   (+ 8 for the odd row), scales at (p kb + b) 2 + (r & 1), an odd m padded with a zero row.
   hi / lo hold m_pad k bytes, d / c m_pad k / 32 floats (m_pad = m rounded up to even when
   paired). Returns -1 on a bad shape. */
int dqo_qmm_quantize(const float* x, int64_t x_stride, int64_t m, int64_t k, int mode, int paired, int8_t* hi,
                     uint8_t* lo, float* d, float* c) {
  if ((mode != 0 && mode != 1) || m < 0 || k <= 0 || k % 32 != 0 || (mode == 1 && lo == NULL)) return -1;
  const int64_t kb = k / 32;
  for (int64_t r = 0; r < m; ++r) {
    const float* xr = x + r * x_stride;
    if (paired) {
      const int64_t off = (r / 2) * 2 * k + (r & 1) * 8, so = (r / 2) * kb * 2 + (r & 1);
      qmm_row(xr, k, mode, hi + off, mode ? lo + off : NULL, 16, d + so, c + so, 2);
    } else {
      qmm_row(xr, k, mode, hi + r * k, mode ? lo + r * k : NULL, 8, d + r * kb, c + r * kb, 1);
    }
  }
  if (paired && (m & 1)) {
    for (int64_t j = 0; j < k / 8; ++j) {
      memset(hi + (m / 2) * 2 * k + j * 16 + 8, 0, 8);
      if (mode) memset(lo + (m / 2) * 2 * k + j * 16 + 8, 0, 8);
    }
    for (int64_t b = 0; b < kb; ++b) d[((m / 2) * kb + b) * 2 + 1] = c[((m / 2) * kb + b) * 2 + 1] = 0.0f;
  }
  return 0;
}
