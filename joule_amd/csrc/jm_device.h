// Device helpers shared by the MoE kernels (gfx950, wave64).
//
// Everything here is compiled with -ffp-contract=off: where the reference's
// arithmetic has a fused multiply-add it is written as __builtin_fmaf, and
// nothing else is fused, so the router reproduces the reference bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define JM_WAVE 64

namespace jm {

// ---------------------------------------------------------------- fp16/bf16

// IEEE binary16 bits -> float (exact for every code; subnormals renormalised,
// Inf/NaN kept).  Same mapping as decode_kernel.c:64-85.
__device__ __forceinline__ float fp16_bits_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t frac = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1Fu) {
        bits = sign | 0x7F800000u | (frac << 13);
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (frac << 13);
    } else if (frac == 0) {
        bits = sign;
    } else {
        const int lz = __clz(frac) - 21;       // leading zeros within the 11-bit field
        frac = (frac << lz) & 0x3FFu;
        bits = sign | ((uint32_t)(113 - lz) << 23) | (frac << 13);
    }
    return __uint_as_float(bits);
}

// Hardware conversion (v_cvt_f32_f16); exact for all codes including
// subnormals.  Used in the hot loops.
__device__ __forceinline__ float fp16_hw(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
    return __uint_as_float(h << 16);
}

// ---------------------------------------------------------------- expf_fast

// The reference's exponential, decode_kernel.c:94-108 (expert_ffn.c:40-54):
// clamp, y = v*log2(e), k = trunc(y +- 0.5), f = y - k, Horner with one
// fused multiply-add per step (clang contracts `c + f*(...)`), times 2^k.
// A NaN argument returns 0: the reference runs on x86, where converting NaN
// to int gives INT_MIN, whose biased exponent is negative (the GPU's own
// conversion would give 0 and let the NaN through).
__device__ __forceinline__ float expf_fast(float v) {
    if (v != v) return 0.0f;
    if (v < -17.0f) return 0.0f;
    if (v > 88.0f) v = 88.0f;
    const float y = __fmul_rn(v, 1.4426950408889634f);
    const int k = (int)(y >= 0.0f ? __fadd_rn(y, 0.5f) : __fsub_rn(y, 0.5f));
    const float f = __fsub_rn(y, (float)k);
    float p = __builtin_fmaf(f, 0.0013330f, 0.0096181f);
    p = __builtin_fmaf(f, p, 0.0555041f);
    p = __builtin_fmaf(f, p, 0.2402265f);
    p = __builtin_fmaf(f, p, 0.6931472f);
    p = __builtin_fmaf(f, p, 1.0f);
    int biased = k + 127;
    if (biased < 0) return 0.0f;
    if (biased > 254) biased = 254;
    return __fmul_rn(p, __uint_as_float((uint32_t)biased << 23));
}

// SiLU(g) * u exactly as the reference writes it: (g / (1 + e^-g)) * u.
__device__ __forceinline__ float swiglu(float g, float u) {
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf_fast(-g))), u);
}

// ------------------------------------------------------- activation digits
//
// The expert GEMV multiplies signed 4-bit weights (q - 8) by activations
// with v_dot8_i32_i4.  An activation group of G values (the columns one
// weight-scale group covers) is written as integers a_j = rint(x_j / s) with
// s = max|x| / R, and each a_j as NDIG signed base-16 digits in [-8, 7]
// (a_j = sum_k d_jk 16^k).  Digit k of the 8 values of one dword-slot is
// packed into one 32-bit word, nibble i = value i, matching the nibble order
// of the packed weights.  R = 7 (16^NDIG - 1) / 15 is the largest magnitude
// whose balanced digits fit.  The group dot sum_j (q_j - 8) a_j is then an
// exact integer; it is converted to float and scaled by s * weight scale.

template <int NDIG>
struct Digits {
    static constexpr int R = NDIG == 4 ? 30583 : NDIG == 5 ? 489335 : 1911;
    static_assert(NDIG >= 3 && NDIG <= 5, "3..5 digits keep the group dot inside int32");
};

// Split integer a (|a| <= R) into NDIG balanced base-16 digits.
template <int NDIG>
__device__ __forceinline__ void split_digits(int a, int* dig) {
#pragma unroll
    for (int k = 0; k < NDIG; k++) {
        const int dk = ((a + 8) & 15) - 8;
        dig[k] = dk;
        a = (a - dk) >> 4;
    }
}

// One group's scale: s = maxabs / R (0 for an all-zero group).  A NaN or Inf
// anywhere in the group makes s NaN so that it propagates to the output.
template <int NDIG>
__device__ __forceinline__ float digit_scale(float maxabs, bool nonfinite) {
    if (nonfinite) return __int_as_float(0x7FC00000);
    return __fdiv_rn(maxabs, (float)Digits<NDIG>::R);
}

// v_dot8_i32_i4: acc + sum_i a.nib[i] * b.nib[i] with signed nibbles.
__device__ __forceinline__ int dot8(uint32_t a, uint32_t b, int acc) {
    return __builtin_amdgcn_sdot8((int)a, (int)b, acc, false);
}

// ------------------------------------------------------------ wave helpers

template <int W>
__device__ __forceinline__ float seg_sum(float v) {
    // Butterfly sum over aligned segments of W lanes (W a power of two <= 64).
#pragma unroll
    for (int o = W / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, JM_WAVE);
    return v;
}

}  // namespace jm
