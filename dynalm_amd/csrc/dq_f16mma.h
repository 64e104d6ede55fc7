// dq_f16mma.h -- helpers of the f16-matrix-core GEMMs (dq_gemm_h16.hip,
// dq_gemm_p32.hip): the 32 x 32 x 16 f16 MFMA, direct-to-LDS buffer loads, LDS reads
// and the int8 -> f16 operand conversion.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dq_device.h"

namespace dq {

typedef float v16f_t __attribute__((ext_vector_type(16)));
typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));

// C + A . B over a 32 x 32 x 16 f16 tile (v_mfma_f32_32x32x16_f16). Lane l supplies row
// (A) / column (B) l % 32 and K = 8 (l / 32) .. + 7; result register r of lane l is row
// 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
DQ_DEV v16f_t mfma_h(v4u a, v4u b, v16f_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h_t, a), __builtin_bit_cast(v8h_t, b), c, 0, 0,
                                                0);
}
DQ_DEV v4u lds16(const uint8_t* p) { return *reinterpret_cast<const v4u*>(p); }

// Direct-to-LDS buffer loads: lane l's 16 (4) bytes land at dst + 16 l (4 l).
DQ_DEV void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* dst, u32 voff, u32 soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, soff, 0, 0);
}
DQ_DEV void dma4(__amdgpu_buffer_rsrc_t r, uint8_t* dst, u32 voff, u32 soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 4, voff, soff, 0, 0);
}

// LDS reads that stay where they are written: ordered with the other volatile
// accesses and the empty asm statements that pin the results computed before them.
DQ_DEV v4u lds16v(const uint8_t* p) {
  typedef const volatile __attribute__((address_space(3))) v4u lds_v4u;
  return *(lds_v4u*)(p);
}
DQ_DEV u32 lds4v(const uint8_t* p) {
  typedef const volatile __attribute__((address_space(3))) u32 lds_u32;
  return *(lds_u32*)(p);
}
DQ_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Eight int8 codes (two dwords) as f16 in the half order {c0 bytes 0, 2, 1, 3, c1
// bytes 0, 2, 1, 3}: the order in which packed 16-bit lanes take bytes (0, 2) and
// (1, 3) of a dword.
DQ_DEV v4u codes_f16(u32 c0, u32 c1) {
  auto h = [](u32 w, int i) -> u32 {
    return (u32)__builtin_bit_cast(uint16_t, (_Float16)(float)(int8_t)((w >> (8 * i)) & 0xFFu));
  };
  return v4u{h(c0, 0) | (h(c0, 2) << 16), h(c0, 1) | (h(c0, 3) << 16), h(c1, 0) | (h(c1, 2) << 16),
             h(c1, 1) | (h(c1, 3) << 16)};
}
DQ_DEV u32 f16_pair(int a, int b) {
  return (u32)__builtin_bit_cast(uint16_t, (_Float16)(float)a) |
         ((u32)__builtin_bit_cast(uint16_t, (_Float16)(float)b) << 16);
}

}  // namespace dq
