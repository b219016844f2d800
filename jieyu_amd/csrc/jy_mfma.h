// jy_mfma.h — operand types of the matrix-core (MFMA) kernels and the exact int8 -> fp16
// conversion they share.
#pragma once

#include <cstdint>

namespace jy {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef int i4_t __attribute__((ext_vector_type(4)));
typedef int i2_t __attribute__((ext_vector_type(2)));

// 8 int8 values (two dwords, byte e of w0 | w1 << 32 is element e) -> 8 fp16 values, exact:
// each byte biased by 128 into the mantissa of 1024 (0x6400 | u = 1024 + u), then less 1152
__device__ __forceinline__ h8_t q8_to_h8(uint32_t w0, uint32_t w1) {
    w0 ^= 0x80808080u;
    w1 ^= 0x80808080u;
    const uint32_t e = 0x64646464u;
    const uint32_t p0 = __builtin_amdgcn_perm(e, w0, 0x04010400u), p1 = __builtin_amdgcn_perm(e, w0, 0x04030402u);
    const uint32_t p2 = __builtin_amdgcn_perm(e, w1, 0x04010400u), p3 = __builtin_amdgcn_perm(e, w1, 0x04030402u);
    const h2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
    const h2_t r0 = __builtin_bit_cast(h2_t, p0) - off, r1 = __builtin_bit_cast(h2_t, p1) - off;
    const h2_t r2 = __builtin_bit_cast(h2_t, p2) - off, r3 = __builtin_bit_cast(h2_t, p3) - off;
    return h8_t{r0.x, r0.y, r1.x, r1.y, r2.x, r2.y, r3.x, r3.y};
}

}  // namespace jy
