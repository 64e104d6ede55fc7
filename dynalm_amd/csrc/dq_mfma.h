// dq_mfma.h -- int8 MFMA helpers shared by the GEMM and the skinny (decode-batch)
// GEMV kernels for gfx950.
#pragma once

#include "dq_device.h"

namespace dq {

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// C + A . B over a 16 x 16 x 64 int8 tile (v_mfma_i32_16x16x64_i8). Lane l supplies
// row (A) / column (B) l % 16 and the 16 K-values 16 (l / 16) .. of it; the result
// lane l holds column l % 16, rows 4 (l / 16) .. 4 (l / 16) + 3.
DQ_DEV v4i_t mfma(v4u a, v4u b, v4i_t c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i_t, a), __builtin_bit_cast(v4i_t, b), c, 0, 0,
                                               0);
}

// Four bytes (each <= 15) times k (<= 7) in two packed 16-bit lanes: bytes stay
// bytes (k * q <= 105), one v_pk_mul_lo_u16.
DQ_DEV u32 mul_bytes(u32 q, u32 kk) {
  return __builtin_bit_cast(u32, __builtin_bit_cast(u16x2, q) * __builtin_bit_cast(u16x2, kk));
}

// v_perm_b32 selectors: bytes (j & 3) of the lane's sub-blocks j = hi, 2 + hi,
// 4 + hi, 6 + hi out of {sc_hi, sc_lo}; and byte s of a word into both 16-bit
// lanes (0x0C selects zero) or into all four bytes.
DQ_DEV u32 sel_subblocks(int hi) { return hi ? 0x07050301u : 0x06040200u; }
DQ_DEV u32 sel_u16x2(int s) { return 0x0C000C00u | ((u32)s << 16) | (u32)s; }
DQ_DEV u32 sel_x4(int s) { return (u32)s * 0x01010101u; }

// Q6_K: w = sc_u (q - 32) (|w| <= 4096) of four codes (bytes of q, 0..63) with the
// unit scale sc (-128..127), split exactly into int8 operands w = 64 wh + wl with
// wh = floor(w / 64) in -64..64 and wl in 0..63; 16-bit lane arithmetic, two codes per
// operation.
DQ_DEV void q6_split(u32 q, int sc, u32& H, u32& L) {
  typedef short s2 __attribute__((ext_vector_type(2)));
  const s2 e = __builtin_bit_cast(s2, __builtin_amdgcn_perm(0u, q, 0x0C010C00u));  // codes 0, 1
  const s2 o = __builtin_bit_cast(s2, __builtin_amdgcn_perm(0u, q, 0x0C030C02u));  // codes 2, 3
  const s2 k = {(short)sc, (short)sc}, c = {(short)(-32 * sc), (short)(-32 * sc)};
  const s2 we = e * k + c, wo = o * k + c;
  const s2 he = we >> (short)6, ho = wo >> (short)6;
  const s2 m63 = {63, 63};
  const s2 le = we & m63, lo = wo & m63;
  H = __builtin_amdgcn_perm(__builtin_bit_cast(u32, ho), __builtin_bit_cast(u32, he), 0x06040200u);
  L = __builtin_amdgcn_perm(__builtin_bit_cast(u32, lo), __builtin_bit_cast(u32, le), 0x06040200u);
}

}  // namespace dq
