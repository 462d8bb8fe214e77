// Operands of the int8 matrix-core products (gfx950,
// v_mfma_i32_32x32x32_i8), shared by the dense-branch kernels
// (jm_mfma.hip) and the small-batch gate/up kernel (jm_gumx.hip).
//
// Lane layout (checked on the device): A[i][k] at lane i % 32,
// k = 16 (l / 32) + j; B[k][n] at lane n % 32, k = 16 (l / 32) + j; D
// register v of lane l = (i = 8 (v / 4) + 4 (l / 32) + v % 4, n = l % 32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jm {

typedef int int4v __attribute__((ext_vector_type(4)));
typedef int int8v __attribute__((ext_vector_type(8)));
typedef int int16v __attribute__((ext_vector_type(16)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// Two dwords of 8 packed nibbles each (value i in bits 4i..4i+3) as four
// dwords of unsigned int8 q in i8_pos order: of each dword, values 0 2 4 6,
// then 1 3 5 7.  The products take q, not q - 8: the callers add -8 times
// the tokens' group sums, which carries the -8.
__device__ __forceinline__ int4v wdigits(uint32_t w0, uint32_t w1) {
    return int4v{(int)(w0 & 0x0F0F0F0Fu), (int)((w0 >> 4) & 0x0F0F0F0Fu), (int)(w1 & 0x0F0F0F0Fu),
                 (int)((w1 >> 4) & 0x0F0F0F0Fu)};
}

}  // namespace jm
