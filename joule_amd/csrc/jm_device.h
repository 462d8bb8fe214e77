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
    // written without branches: every path is computed and the early-out
    // cases select 0 at the end
    const bool zero = (v != v) || (v < -17.0f);
    v = v > 88.0f ? 88.0f : v;
    const float y = __fmul_rn(v, 1.4426950408889634f);
    const int k = (int)(y >= 0.0f ? __fadd_rn(y, 0.5f) : __fsub_rn(y, 0.5f));
    const float f = __fsub_rn(y, (float)k);
    float p = __builtin_fmaf(f, 0.0013330f, 0.0096181f);
    p = __builtin_fmaf(f, p, 0.0555041f);
    p = __builtin_fmaf(f, p, 0.2402265f);
    p = __builtin_fmaf(f, p, 0.6931472f);
    p = __builtin_fmaf(f, p, 1.0f);
    const int biased = k + 127;
    const int bc = biased < 0 ? 0 : biased > 254 ? 254 : biased;
    const float r = __fmul_rn(p, __uint_as_float((uint32_t)bc << 23));
    return (zero || biased < 0) ? 0.0f : r;
}

// The reference's square root, decode_kernel.c:88-93: a bit-level first
// guess (exponent halved) refined by one Newton step; relative error below
// 2e-3, exact at powers of 4.
__host__ __device__ __forceinline__ float sqrtf_fast(float x) {
    union { float f; uint32_t u; } v = {x};
    v.u = (v.u + 0x3F800000u) >> 1;
#ifdef __HIP_DEVICE_COMPILE__
    return __fmul_rn(0.5f, __fadd_rn(v.f, __fdiv_rn(x, v.f)));
#else
    return 0.5f * (v.f + x / v.f);
#endif
}

// RMSNorm scale of a row with sum of squares ss over n values, as
// rms_norm computes it (decode_kernel.c:224-230): 1 / sqrtf_fast(ss / n + eps).
__device__ __forceinline__ float rms_inv(float ss, int n, float eps) {
    return __fdiv_rn(1.0f, sqrtf_fast(__fadd_rn(__fdiv_rn(ss, (float)n), eps)));
}

// float -> bfloat16 bits, round to nearest even (finite values).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// A device address read from memory (a table of cache addresses) is a
// generic pointer to the compiler, which then emits flat loads: these also
// count against the LDS counter, so that every LDS wait waits for them.  As
// global pointers they become global loads.
template <typename T>
using gptr = T __attribute__((address_space(1)))*;

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// 16 bytes at a global address (16-byte aligned)
__device__ __forceinline__ uint4 load_g16(gptr<const uint16_t> p) {
    const u32x4_t v = *(gptr<const u32x4_t>)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ------------------------------------------------- bf16 matrix-core operands

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Two floats as packed bf16, rounded to nearest even (v_cvt_pk_bf16_f32;
// a and b finite).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const bf16x2_t h = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, h);
}

// The two-term bf16 split of a and b: hi = bf16(v), lo = bf16(v - hi), each
// packed (a in the low half).  hi + lo is within 2^-18 |v| of v, so a product
// taken as hi*w + lo*w with exact bf16 w and fp32 accumulation keeps
// float32-level accuracy.
__device__ __forceinline__ void split_bf16x2(float a, float b, uint32_t& hi, uint32_t& lo) {
    hi = pack_bf16x2(a, b);
    lo = pack_bf16x2(__fsub_rn(a, __uint_as_float(hi << 16)), __fsub_rn(b, __uint_as_float(hi & 0xFFFF0000u)));
}

// 2^p as a float, -126 <= p <= 127
__device__ __forceinline__ float exp2i(int p) { return __uint_as_float((uint32_t)(127 + p) << 23); }

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

// DPP lane moves (CDNA row = 16 lanes).
constexpr int DPP_XOR1 = 0xB1;          // quad_perm(1,0,3,2)
constexpr int DPP_XOR2 = 0x4E;          // quad_perm(2,3,0,1)
constexpr int DPP_ROW_MIRROR = 0x140;   // lane i <- 15 - i within a row
constexpr int DPP_HALF_MIRROR = 0x141;  // lane i <- 7 - i within 8 lanes
constexpr int DPP_ROL4 = 0x12C;         // lane i <- i + 4 (mod 16) within a row (row_ror:12)
constexpr int DPP_ROR8 = 0x128;         // lane i <- i ^ 8 within a row (row_ror:8)

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
// xor 16 within 32 lanes (ds_swizzle bit mode: and 0x1F, or 0, xor 0x10)
__device__ __forceinline__ float swz_xor16_f(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}
__device__ __forceinline__ int swz_xor16_i(int v) { return __builtin_amdgcn_ds_swizzle(v, 0x401F); }

// Sum over aligned segments of W lanes (W = 2..64); every lane of a segment
// ends with the same bits (each step adds a lane to its partner, and fp32
// addition is commutative).
template <int W>
__device__ __forceinline__ float seg_sum(float v) {
    if (W >= 2) v = __fadd_rn(v, dpp_f<DPP_XOR1>(v));
    if (W >= 4) v = __fadd_rn(v, dpp_f<DPP_XOR2>(v));
    if (W >= 8) v = __fadd_rn(v, dpp_f<DPP_HALF_MIRROR>(v));
    if (W >= 16) v = __fadd_rn(v, dpp_f<DPP_ROW_MIRROR>(v));
    if (W >= 32) v = __fadd_rn(v, swz_xor16_f(v));
    if (W >= 64) v = __fadd_rn(v, __shfl_xor(v, 32, JM_WAVE));
    return v;
}

// One level of a transposing butterfly at lane distance D (32, 16, 8, 4):
// the N values of a lane become N/2, each lane keeping the half selected by
// its lane bit D and adding its partner's copy of that half.  Partners are
// l ^ D for D = 32, 16, 8 and 7 - l within 8 lanes for D = 4.
template <int D, int N>
__device__ __forceinline__ void transpose_level(float* v) {
    const bool hi = (threadIdx.x & D) != 0;
#pragma unroll
    for (int j = 0; j < N / 2; j++) {
        const float a = v[j], b = v[j + N / 2];
        if constexpr (D == 32) {
            const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
            v[j] = __fadd_rn(__uint_as_float(p[0]), __uint_as_float(p[1]));
        } else if constexpr (D == 16) {
            const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
            v[j] = __fadd_rn(__uint_as_float(p[0]), __uint_as_float(p[1]));
        } else {
            const float keep = hi ? b : a, send = hi ? a : b;
            v[j] = __fadd_rn(keep, dpp_f<D == 8 ? DPP_ROR8 : DPP_HALF_MIRROR>(send));
        }
    }
}

// Totals of N = W/4 partial sums per lane over aligned segments of W lanes
// (W = 16, 32, 64), all at once: transposing levels at distances W/2 .. 4,
// then plain sums at distances 2 and 1.  Value v (bits of v = lane bits
// log2(W)-1 .. 2) ends in lanes W*seg + 4*v + {0, 1, 2, 3}; returned.
template <int W>
__device__ __forceinline__ float transpose_sum(float (&v)[W / 4]) {
    constexpr int N = W / 4;
    if constexpr (W == 64) {
        transpose_level<32, N>(v);
        transpose_level<16, N / 2>(v);
        transpose_level<8, N / 4>(v);
        transpose_level<4, N / 8>(v);
    } else if constexpr (W == 32) {
        transpose_level<16, N>(v);
        transpose_level<8, N / 2>(v);
        transpose_level<4, N / 4>(v);
    } else {
        static_assert(W == 16, "segments of 16, 32 or 64 lanes");
        transpose_level<8, N>(v);
        transpose_level<4, N / 2>(v);
    }
    float t = v[0];
    t = __fadd_rn(t, dpp_f<DPP_XOR2>(t));
    t = __fadd_rn(t, dpp_f<DPP_XOR1>(t));
    return t;
}

// Totals of N partial sums per lane over aligned segments of W lanes
// (N = 1 .. W/4): transposing levels at distances W/2 .. W/N, then plain sums
// over the W/N lanes that share a value.  Value v ends in the lanes with
// (lane % W) / (W / N) == v; returned.
template <int W, int N>
__device__ __forceinline__ float transpose_reduce(float (&v)[N]) {
    static_assert(N >= 1 && W / N >= 4 && (N & (N - 1)) == 0, "N a power of two, at most W/4");
    if constexpr (N >= 2) transpose_level<W / 2, N>(v);
    if constexpr (N >= 4) transpose_level<W / 4, N / 2>(v);
    if constexpr (N >= 8) transpose_level<W / 8, N / 4>(v);
    if constexpr (N >= 16) transpose_level<W / 16, N / 8>(v);
    return seg_sum<W / N>(v[0]);
}

template <int W>
__device__ __forceinline__ float seg_max(float v) {
    if (W >= 2) v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    if (W >= 4) v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    if (W >= 8) v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    if (W >= 16) v = fmaxf(v, dpp_f<DPP_ROW_MIRROR>(v));
    if (W >= 32) v = fmaxf(v, swz_xor16_f(v));
    if (W >= 64) v = fmaxf(v, __shfl_xor(v, 32, JM_WAVE));
    return v;
}

template <int W>
__device__ __forceinline__ int seg_or(int v) {
    if (W >= 2) v |= dpp_i<DPP_XOR1>(v);
    if (W >= 4) v |= dpp_i<DPP_XOR2>(v);
    if (W >= 8) v |= dpp_i<DPP_HALF_MIRROR>(v);
    if (W >= 16) v |= dpp_i<DPP_ROW_MIRROR>(v);
    if (W >= 32) v |= swz_xor16_i(v);
    if (W >= 64) v |= __shfl_xor(v, 32, JM_WAVE);
    return v;
}

// ------------------------------------------------- wave-level digit encode

// --------------------------------------- int8 digit pairs (MFMA branch)
//
// The MFMA branch multiplies signed int8 weights (q - 8) by activations
// written as two int8 digits per value: over a G-value group (the columns
// one weight-scale group covers), a_j = rint(x_j / s) with s = max|x| / 32639,
// and a_j = 256 hi_j + lo_j with hi_j, lo_j in [-128, 127] (|a_j| <= 32639 =
// 127 * 256 + 127 keeps hi in range).  A group's integer dot with the
// weights is exact: |sum_j a_j (q_j - 8)| <= G * 32639 * 8 < 2^24, so its
// conversion to float is exact as well.
constexpr int I8_R = 32639;

// Position of value u (0..7) within its aligned 8-value run in the int8
// operand order: the even values, then the odd ones.  That is the byte
// order in which one dword of packed nibbles (value i in bits 4i..4i+3)
// unpacks: its low nibbles, then its high nibbles.
__host__ __device__ constexpr int i8_pos(int u) { return (u & 1) ? 4 + (u >> 1) : (u >> 1); }

// Encode one group of G floats, value i held by lane i of an aligned G-lane
// segment (G = 32 or 64): lane i writes its two digits to hi[p] and lo[p],
// p = its value's place in the int8 operand order; lane 0 writes the scale
// (NaN when the group holds a non-finite value, so that it propagates) and
// the sum of the group's integers q = 256 h + l (exact: below 2^24), which
// the matrix-core kernels fold into their products with unsigned weight
// nibbles.  Only when `store`; every lane of the segment must call this.
template <int G>
__device__ __forceinline__ void encode_i8_group_wave(float v, bool store, int8_t* __restrict__ hi,
                                                     int8_t* __restrict__ lo, float* __restrict__ scale,
                                                     int* __restrict__ qsum) {
    const int i = threadIdx.x & (G - 1);
    const float a = fabsf(v);
    const int bad = seg_or<G>(!(a <= 3.4028235e38f) ? 1 : 0);
    const float mx = seg_max<G>(a);
    const float inv = (mx > 0.0f && !bad) ? __fdiv_rn((float)I8_R, mx) : 0.0f;
    const int q = (int)rintf(__fmul_rn(v, inv));
    const int l = ((q + 128) & 255) - 128;
    const int h = (q - l) >> 8;
    const float qs = seg_sum<G>((float)q);
    if (store) {
        const int p = (i & ~7) + i8_pos(i & 7);
        hi[p] = (int8_t)h;
        lo[p] = (int8_t)l;
        if (i == 0) {
            *scale = bad ? __int_as_float(0x7FC00000) : __fdiv_rn(mx, (float)I8_R);
            *qsum = (int)qs;
        }
    }
}

// Both encodings of one G-value group (one value per lane of a G-lane
// segment) from one pair of segment reductions: the NDIG base-16 digits and
// their scale, as encode_group_wave writes them, and with i8 the int8 digit
// pairs, scale and integer sum, as encode_i8_group_wave writes them (the
// same values as the two calls).  Only when `store`; every lane of the
// segment must call this.
template <int G, int NDIG>
__device__ __forceinline__ void encode_group_both(float v, bool store, uint32_t* __restrict__ dig,
                                                  float* __restrict__ scale, bool i8, int8_t* __restrict__ hi,
                                                  int8_t* __restrict__ lo, float* __restrict__ qscale,
                                                  int* __restrict__ qsum) {
    const int i = threadIdx.x & (G - 1);
    const float a = fabsf(v);
    const int bad = seg_or<G>(!(a <= 3.4028235e38f) ? 1 : 0);
    const float mx = seg_max<G>(a);
    {
        const float s = digit_scale<NDIG>(mx, bad != 0);
        const float inv = (mx > 0.0f && !bad) ? __fdiv_rn((float)Digits<NDIG>::R, mx) : 0.0f;
        int dg[NDIG];
        split_digits<NDIG>((int)rintf(__fmul_rn(v, inv)), dg);
#pragma unroll
        for (int k = 0; k < NDIG; k++) {
            const int word = seg_or<8>((dg[k] & 15) << (4 * (i & 7)));
            if (store && (i & 7) == 0) dig[k * (G / 8) + (i >> 3)] = (uint32_t)word;
        }
        if (store && i == 0) *scale = s;
    }
    if (i8) {
        const float inv = (mx > 0.0f && !bad) ? __fdiv_rn((float)I8_R, mx) : 0.0f;
        const int q = (int)rintf(__fmul_rn(v, inv));
        const int l = ((q + 128) & 255) - 128;
        const int h = (q - l) >> 8;
        const float qs = seg_sum<G>((float)q);
        if (store) {
            const int p = (i & ~7) + i8_pos(i & 7);
            hi[p] = (int8_t)h;
            lo[p] = (int8_t)l;
            if (i == 0) {
                *qscale = bad ? __int_as_float(0x7FC00000) : __fdiv_rn(mx, (float)I8_R);
                *qsum = (int)qs;
            }
        }
    }
}

// encode_group_both for NT groups at once, one value of each per lane: the
// groups' reductions, divisions and digits first, with no branch among them,
// then every store.  The NT dependency chains overlap instead of running one
// after another between the stores' branches.  The same values as NT calls
// of encode_group_both (every step is the same per group).
template <int G, int NDIG, int NT>
__device__ __forceinline__ void encode_groups_n(const float* v, const bool* store, uint32_t* const* dig,
                                                float* const* scale, bool i8, int8_t* const* hi, int8_t* const* lo,
                                                float* const* qscale, int* const* qsum) {
    const int i = threadIdx.x & (G - 1);
    int bad[NT];
    float mx[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const float a = fabsf(v[t]);
        bad[t] = seg_or<G>(!(a <= 3.4028235e38f) ? 1 : 0);
        mx[t] = seg_max<G>(a);
    }
    float sc[NT];
    uint32_t word[NT][NDIG];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        sc[t] = digit_scale<NDIG>(mx[t], bad[t] != 0);
        const float inv = (mx[t] > 0.0f && !bad[t]) ? __fdiv_rn((float)Digits<NDIG>::R, mx[t]) : 0.0f;
        int dg[NDIG];
        split_digits<NDIG>((int)rintf(__fmul_rn(v[t], inv)), dg);
#pragma unroll
        for (int k = 0; k < NDIG; k++) word[t][k] = (uint32_t)seg_or<8>((dg[k] & 15) << (4 * (i & 7)));
    }
    int hv[NT], lv[NT], qi[NT];
    float qsc[NT];
    if (i8) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float inv = (mx[t] > 0.0f && !bad[t]) ? __fdiv_rn((float)I8_R, mx[t]) : 0.0f;
            const int q = (int)rintf(__fmul_rn(v[t], inv));
            lv[t] = ((q + 128) & 255) - 128;
            hv[t] = (q - lv[t]) >> 8;
            qi[t] = (int)seg_sum<G>((float)q);
            qsc[t] = bad[t] ? __int_as_float(0x7FC00000) : __fdiv_rn(mx[t], (float)I8_R);
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        if (!store[t]) continue;
        if ((i & 7) == 0) {
#pragma unroll
            for (int k = 0; k < NDIG; k++) dig[t][k * (G / 8) + (i >> 3)] = word[t][k];
        }
        if (i == 0) *scale[t] = sc[t];
        if (i8) {
            const int p = (i & ~7) + i8_pos(i & 7);
            hi[t][p] = (int8_t)hv[t];
            lo[t][p] = (int8_t)lv[t];
            if (i == 0) {
                *qscale[t] = qsc[t];
                *qsum[t] = qi[t];
            }
        }
    }
}

// Encode one group of G floats, value i held by lane i of an aligned G-lane
// segment (G = 32 or 64), into NDIG x G/8 digit words and one scale.
// Lane j*8 of the segment writes word j of every digit k to dig[k*(G/8)+j];
// lane 0 writes the scale (only when `store`).  Every lane of the segment must
// call this (the reductions cross lanes).
template <int G, int NDIG>
__device__ __forceinline__ void encode_group_wave(float v, bool store, uint32_t* __restrict__ dig,
                                                  float* __restrict__ scale) {
    encode_group_both<G, NDIG>(v, store, dig, scale, false, nullptr, nullptr, nullptr, nullptr);
}

// Digits of the 8 values in lanes 0..7 of the wave with the digit scale of
// a larger group, whose max |value| is mx (nf: the group holds a non-finite
// value, whose scale is NaN).  Digit plane k's word of these 8 values goes
// to dig[4 k]: the caller offsets dig by the word's place in the group.
template <int NDIG>
__device__ __forceinline__ void encode_digits_shared(float v, float mx, bool nf, bool store,
                                                     uint32_t* __restrict__ dig) {
    const int i = threadIdx.x & 7;
    const float inv = (mx > 0.0f && !nf) ? __fdiv_rn((float)Digits<NDIG>::R, mx) : 0.0f;
    int dg[NDIG];
    split_digits<NDIG>((int)rintf(__fmul_rn(v, inv)), dg);
#pragma unroll
    for (int k = 0; k < NDIG; k++) {
        const int word = seg_or<8>((dg[k] & 15) << (4 * i));
        if (store && i == 0) dig[4 * k] = (uint32_t)word;
    }
}

// ---------------------------------------------------------- router top-k

// Float max over the whole wave; every lane gets the result (non-NaN
// inputs).  Rows of 16 lanes reduce with DPP, then the four row maxima are
// read as scalars.
__device__ __forceinline__ float wave_max_f(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_MIRROR>(v));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Softmax over the E scores of one token and top-k selection, one wave
// (decode_kernel.c:1425-1448): max (NaN never wins), p = expf_fast(s - max),
// a sequential sum over e = 0..E-1 by lane 0, p /= sum, k rounds of argmax
// with ties to the lowest index, optional renormalisation by the sequential
// sum of the k weights.
// A round takes the largest candidate p (an exact float max; candidates are
// the p >= 0 not taken yet, so NaN never wins) and, among the entries equal
// to it, the lowest index (first set bit of a ballot, lower e first).  A
// round without candidates yields index -1 and weight -1e30, the reference's
// values when nothing beats its -1e30 start.
// p_lds holds 64*EPL floats.  Lane i < k writes top[i] and tw[i].
// topk_vals takes the scores in registers (v[j] = score of expert lane +
// 64 j; entries past E are ignored); topk_wave loads them from s.
template <int EPL>
__device__ __forceinline__ void topk_vals(const float (&v)[EPL], int E, int k, int renorm, float* p_lds,
                                          int* __restrict__ top, float* __restrict__ tw) {
    const int lane = threadIdx.x & 63;
    float mx = -1e30f;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + 64 * j;
        if (e < E && v[j] > mx) mx = v[j];
    }
    mx = wave_max_f(mx);                       // lane values are >= -1e30, never NaN
    float ex[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + 64 * j;
        ex[j] = expf_fast(__fsub_rn(v[j], mx));
        if (e < E) p_lds[e] = ex[j];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float sum = 0.0f;
    if (lane == 0) {
        // the reads of 32 values are issued together, the adds stay in order
        int e = 0;
        for (; e + 32 <= E; e += 32) {
            float4 q[8];
#pragma unroll
            for (int c = 0; c < 8; c++) q[c] = *(const float4*)(p_lds + e + 4 * c);
#pragma unroll
            for (int c = 0; c < 8; c++) {
                sum = __fadd_rn(sum, q[c].x); sum = __fadd_rn(sum, q[c].y);
                sum = __fadd_rn(sum, q[c].z); sum = __fadd_rn(sum, q[c].w);
            }
        }
        for (; e < E; e++) sum = __fadd_rn(sum, p_lds[e]);
    }
    sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sum), 0));
    float cand[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + 64 * j;
        const float p = __fdiv_rn(ex[j], sum);
        cand[j] = (e < E && p >= 0.0f) ? p : -1.0f;
    }
    float my_w = 0.0f, ss = 0.0f;
    int my_e = -1;
    for (int i = 0; i < k; i++) {
        float best = cand[0];
#pragma unroll
        for (int j = 1; j < EPL; j++) best = fmaxf(best, cand[j]);
        best = wave_max_f(best);
        int bi = -1;
        float bv = -1e30f;
        if (best >= 0.0f) {
            bv = best;
#pragma unroll
            for (int j = 0; j < EPL; j++) {
                const unsigned long long m = __ballot(cand[j] == best);
                if (bi < 0 && m) bi = 64 * j + (int)__builtin_ctzll(m);
            }
#pragma unroll
            for (int j = 0; j < EPL; j++)
                if (lane + 64 * j == bi) cand[j] = -2.0f;
        }
        ss = __fadd_rn(ss, bv);
        if (lane == i) { my_w = bv; my_e = bi; }
    }
    if (renorm) my_w = __fdiv_rn(my_w, ss);
    if (lane < k) {
        top[lane] = my_e;
        tw[lane] = my_w;
    }
}

template <int EPL>
__device__ __forceinline__ void topk_wave(const float* __restrict__ s, int E, int k, int renorm,
                                          float* p_lds, int* __restrict__ top, float* __restrict__ tw) {
    const int lane = threadIdx.x & 63;
    float v[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + 64 * j;
        v[j] = e < E ? s[e] : 0.0f;
    }
    topk_vals<EPL>(v, E, k, renorm, p_lds, top, tw);
}

// ------------------------------------------------------------- dispatch


// Work table entry of one active expert for the expert kernels: its
// segment and the byte offsets of its gate/up/down records, so that an
// expert wave needs one load to know everything it streams.
struct ExpertWork {
    int e, s0, n, pad;
    unsigned long long sc[3], pk[3];
};

// Inclusive prefix sum over the wave with DPP: shifts of 1, 2, 4, 8 within
// rows of 16 lanes, then row 0's total into row 1, rows 0-1's into 2-3.
__device__ __forceinline__ unsigned wave_inclusive_scan(unsigned x) {
    x += (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xF, 0xF, true);   // row_shr:1
    x += (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xF, 0xF, true);   // row_shr:2
    x += (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF, true);   // row_shr:4
    x += (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xF, 0xF, true);   // row_shr:8
    x += (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xA, 0xF, false);  // row_bcast:15
    x += (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xC, 0xF, false);  // row_bcast:31
    return x;
}

// Exclusive prefix sums of two 32-bit fields over the block (blockDim.x <=
// 1024); every thread must call it.  wsum is LDS scratch of 32 unsigned;
// tot receives both totals.
// A block barrier whose fences cover LDS only (the LDS accesses before it
// are complete and visible to the block after it), for blocks whose threads
// exchange data through LDS alone: it states that the block's global
// accesses need no ordering among its threads.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ uint2 block_exclusive_scan2(uint2 v, unsigned* wsum, uint2* tot) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const unsigned a = wave_inclusive_scan(v.x), b = wave_inclusive_scan(v.y);
    if (lane == 63) { wsum[w] = a; wsum[16 + w] = b; }
    lds_barrier();
    unsigned offa = 0, offb = 0, alla = 0, allb = 0;
    for (int j = 0; j < nw; j++) {
        const unsigned ta = wsum[j], tb = wsum[16 + j];
        offa += j < w ? ta : 0u;
        offb += j < w ? tb : 0u;
        alla += ta;
        allb += tb;
    }
    *tot = make_uint2(alla, allb);
    lds_barrier();
    return make_uint2(offa + a - v.x, offb + b - v.y);
}

// Where the records of (part p, key l*E+e) lie in the store blob: the
// store's [3][L*E][2] table of (scales, packed) offsets or, when every
// record sits at base + key * stride + a per-part offset (a store written in
// (layer, expert, part) order, as the reference's converter writes it), that
// formula, which costs no load.
struct RecLoc {
    const unsigned long long* table;   // [3][LE][2]
    long long LE;
    int affine;
    unsigned long long base, stride, so[3], po[3];

    __device__ __forceinline__ void get(int p, long long key, unsigned long long& sc,
                                        unsigned long long& pk) const {
        if (affine) {
            const unsigned long long o = base + (unsigned long long)key * stride;
            sc = o + so[p];
            pk = o + po[p];
        } else {
            sc = table[((long long)p * LE + key) * 2 + 0];
            pk = table[((long long)p * LE + key) * 2 + 1];
        }
    }
};

// Record offsets of expert e (one per part: scales, packed) at key0 =
// layer * E; loaded by the expert's own thread at the start of a dispatch so
// that they are in registers when its work entry is written.
struct ExpertRec {
    unsigned long long sc[3], pk[3];
};

__device__ __forceinline__ ExpertRec load_expert_rec(const RecLoc& rl, long long key0, int e) {
    ExpertRec r;
#pragma unroll
    for (int p = 0; p < 3; p++) rl.get(p, key0 + e, r.sc[p], r.pk[p]);
    return r;
}

// The slots of one expert on the decode path (B * topk <= 256 slots): a
// ballot over the top-k table of every slot.  Slots come out in increasing
// order, the order of the reference's slot lists (decode_kernel.c:1459-1485).
struct BallotSlots {
    unsigned long long m0, m1, m2, m3;
    int n;

    // Loads top[0..nslot) (lane l holds slots l, l + 64, ...) and ballots
    // the slots routed to the expert of slot s.  False when slot s has no
    // expert or an earlier slot has the same expert: then another wave item
    // (that of the expert's first slot) covers it.  *e receives the expert.
    __device__ __forceinline__ bool init(const int* __restrict__ top, int nslot, int E, int s, int* e) {
        const int lane = threadIdx.x & 63;
        const int t0 = lane < nslot ? top[lane] : -1;
        const int t1 = nslot > 64 && lane + 64 < nslot ? top[lane + 64] : -1;
        const int t2 = nslot > 128 && lane + 128 < nslot ? top[lane + 128] : -1;
        const int t3 = nslot > 192 && lane + 192 < nslot ? top[lane + 192] : -1;
        const int j = s >> 6;
        const int tj = j == 0 ? t0 : j == 1 ? t1 : j == 2 ? t2 : t3;
        const int ex = __builtin_amdgcn_readlane(tj, s & 63);
        *e = ex;
        if (ex < 0 || ex >= E) return false;
        set(t0, t1, t2, t3, ex);
        const int lowest = m0 ? __builtin_ctzll(m0) : m1 ? 64 + __builtin_ctzll(m1)
                         : m2 ? 128 + __builtin_ctzll(m2) : 192 + __builtin_ctzll(m3);
        return lowest == s;
    }

    // The slots of expert e from a top-k table in LDS.
    __device__ __forceinline__ void init_lds(const int* top_lds, int nslot, int e) {
        const int lane = threadIdx.x & 63;
        const int t0 = lane < nslot ? top_lds[lane] : -1;
        const int t1 = lane + 64 < nslot ? top_lds[lane + 64] : -1;
        const int t2 = lane + 128 < nslot ? top_lds[lane + 128] : -1;
        const int t3 = lane + 192 < nslot ? top_lds[lane + 192] : -1;
        set(t0, t1, t2, t3, e);
    }

    __device__ __forceinline__ void set(int t0, int t1, int t2, int t3, int e) {
        m0 = __ballot(t0 == e);
        m1 = __ballot(t1 == e);
        m2 = __ballot(t2 == e);
        m3 = __ballot(t3 == e);
        n = __popcll(m0) + __popcll(m1) + __popcll(m2) + __popcll(m3);
    }

    // The next slot in increasing order (n calls in all).
    __device__ __forceinline__ int next() {
        if (m0) { const int s = __builtin_ctzll(m0); m0 &= m0 - 1; return s; }
        if (m1) { const int s = __builtin_ctzll(m1); m1 &= m1 - 1; return 64 + s; }
        if (m2) { const int s = __builtin_ctzll(m2); m2 &= m2 - 1; return 128 + s; }
        const int s = __builtin_ctzll(m3);
        m3 &= m3 - 1;
        return 192 + s;
    }
};

// Decode-path routing summary in LDS, computed by a whole block of at least
// JM_DEC_SLOTS threads (nslot <= JM_DEC_SLOTS): the top-k table (top_l),
// each expert's first slot (first_l, INT_MAX for unrouted experts) and the
// union list (ulist: the slots that are their expert's first, in slot order:
// the reference's union order, decode_kernel.c:1449-1485).  wcnt is LDS
// scratch of JM_DEC_SLOTS / 64 ints.  Returns the union length U.  Every
// thread must call it; it ends with a barrier.
template <int NSLOTS>
__device__ __forceinline__ int decode_union(const int* __restrict__ top, int nslot, int E, int* top_l,
                                            int* first_l, int* ulist, int* wcnt, int* e_out = nullptr) {
    constexpr int NSW = NSLOTS / 64;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    if (tid < nslot) top_l[tid] = top[tid];
    for (int i = tid; i < E; i += blockDim.x) first_l[i] = 0x7FFFFFFF;
    __syncthreads();
    int e_me = -1;
    if (tid < nslot) {
        const int e = top_l[tid];
        if (e >= 0 && e < E) {
            e_me = e;
            atomicMin(&first_l[e], tid);
        }
    }
    __syncthreads();
    const bool first = e_me >= 0 && first_l[e_me] == tid;
    const unsigned long long fm = __ballot(first);
    if (w < NSW && lane == 0) wcnt[w] = __popcll(fm);
    __syncthreads();
    int U = 0, before = 0;
#pragma unroll
    for (int j = 0; j < NSW; j++) {
        const int cj = wcnt[j];
        before += j < w ? cj : 0;
        U += cj;
    }
    if (first) ulist[before + __popcll(fm & ((1ull << lane) - 1ull))] = tid;
    if (e_out) *e_out = e_me;
    __syncthreads();
    return U;
}

// The slots of one work-table entry (dispatch path): seg_slot[s0 .. s0+n),
// the first 64 held one per lane.
struct TableSlots {
    const int* seg_slot;
    int s0, n, slotv, t;

    __device__ __forceinline__ void init(const int* __restrict__ ss, int start, int count) {
        const int lane = threadIdx.x & 63;
        seg_slot = ss;
        s0 = start;
        n = count;
        slotv = lane < count ? ss[start + lane] : 0;
        t = 0;
    }

    __device__ __forceinline__ int next() {
        const int i = t++;
        return i < 64 ? __builtin_amdgcn_readlane(slotv, i) : seg_slot[s0 + i];
    }
};

// Dispatch chunks: 64 consecutive slots, one wave's worth.
constexpr int DISP_CHUNK = 64;

// LDS of dispatch_block, in ints: per-expert chunk counts [E][nchunk],
// segment starts [E + 1], first slots [E], scan scratch [32], then 16 bits
// per slot twice: the expert ids, and the in-chunk ranks (later the union
// keys).
__host__ __device__ constexpr int dispatch_lds_ints(int nslot, int E) {
    return (nslot + DISP_CHUNK - 1) / DISP_CHUNK * E + 2 * E + 1 + 32 + 2 * ((nslot + 1) / 2);
}

// Stable counting sort of nslot (< 65536) slots by expert id, run by one
// whole block (decode_kernel.c:1449-1485 builds the same segments in
// first-appearance order; here they are in expert-id order, slots within a
// segment in increasing b*k+i order).  E <= blockDim.x.  Everything between
// the top-k table and the outputs stays in LDS.  Writes seg_off[E+1],
// seg_slot, active[U] (expert-id order), *n_active = U, first_slot[e], and
// comb[b*k + j] = the token's slots in the reference's union order
// (ascending first appearance of their expert), -1 padded.  With `work`,
// also the expert work table for umax entries: the experts with two or more
// slots first, then those with one (each group in expert-id order), so that
// the longest segments start first; entries past U have n = 0.  `rec` holds
// the record offsets of expert tid (tid < E).  A slot's rank among the
// earlier slots of its chunk with the same expert comes from ballots over
// the bits of the expert id (lanes with equal ids agree on every bit).
// STABLE false (the block's own dispatch): the slots of a segment in no
// particular order.  A slot's place in its segment comes from an LDS atomic
// add on its expert's count and each expert's first slot from an atomic
// min, so the chunk counts, ballots and chunk scans drop out.  Nothing the
// block computes depends on that order: a slot's products, act, y and its
// place in the union order (from the first slots) are the same wherever
// it sits in its segment; the work table and tile lists come from the
// counts alone.  The block's threads exchange data through LDS only (its
// global outputs are not read back), so its barriers order LDS alone.
// With wn (STABLE false only: it may
// alias the counts, which are dead once the segment starts are scanned),
// wn[u] = the slot count of work entry u, for u < umax.
template <bool STABLE = true>
__device__ __forceinline__ void dispatch_block(const int* top, int nslot, int E, int k, int* lds,
                                               int* __restrict__ seg_off, int* __restrict__ seg_slot,
                                               int* __restrict__ active, int* __restrict__ n_active,
                                               int* __restrict__ first_slot, int* __restrict__ comb,
                                               ExpertWork* __restrict__ work = nullptr,
                                               int umax = 0, const ExpertRec* rec = nullptr, int* wn = nullptr) {
    constexpr unsigned short NONE = 0xFFFF;
    const int nchunk = STABLE ? (nslot + DISP_CHUNK - 1) / DISP_CHUNK : 1;
    int* cnt = lds;                              // [E][nchunk] (STABLE) or [E]
    int* off = cnt + nchunk * E;                 // [E + 1]
    int* fs = off + E + 1;                       // [E]
    unsigned* wsum = (unsigned*)(fs + E);        // [32]
    unsigned short* te = (unsigned short*)(wsum + 32);   // [nslot] expert id, NONE: no expert
    unsigned short* rk = te + 2 * ((nslot + 1) / 2);     // [nslot] rank (in chunk or segment), then union key
    const int tid = threadIdx.x, nth = blockDim.x, lane = tid & 63, w = tid >> 6, nw = nth >> 6;
    for (int i = tid; i < nchunk * E; i += nth) cnt[i] = 0;
    if (!STABLE)
        for (int i = tid; i < E; i += nth) fs[i] = 0x7FFFFFFF;
    if (!STABLE) lds_barrier();
    // the thread's entries of the top-k table, DISP_PF at a time with every
    // load issued before the first is used (indices past the end read the
    // last entry and are not used)
    constexpr int DISP_PF = 4;
    for (int s0 = tid; s0 < nslot; s0 += DISP_PF * nth) {
        int ev[DISP_PF];
#pragma unroll
        for (int j = 0; j < DISP_PF; j++) ev[j] = top[min(s0 + j * nth, nslot - 1)];
#pragma unroll
        for (int j = 0; j < DISP_PF; j++) {
            const int s = s0 + j * nth;
            const int e = ev[j];
            const bool ok = e >= 0 && e < E;
            if (s < nslot) {
                te[s] = ok ? (unsigned short)e : NONE;
                if (!STABLE) {
                    rk[s] = ok ? (unsigned short)atomicAdd(&cnt[ok ? e : 0], 1) : NONE;
                    if (ok) atomicMin(&fs[e], s);
                }
            }
        }
    }
    lds_barrier();
    if (STABLE) {
    int nbits = 1;
    while ((1 << nbits) < E) nbits++;
    for (int c = w; c < nchunk; c += nw) {
        const int s = c * DISP_CHUNK + lane;
        const unsigned short e0 = s < nslot ? te[s] : NONE;
        const bool ok = e0 != NONE;
        const int e = ok ? e0 : 0;
        unsigned long long same = __ballot(ok);
        for (int b = 0; b < nbits; b++) {
            const unsigned long long bb = __ballot(ok && ((e >> b) & 1));
            same &= ((e >> b) & 1) ? bb : ~bb;
        }
        const int r = __popcll(same & ((1ull << lane) - 1ull));
        if (s < nslot) rk[s] = ok ? (unsigned short)r : NONE;
        if (ok && r == 0) cnt[e * nchunk + c] = __popcll(same);
    }
    lds_barrier();
    // per expert: exclusive prefix over its chunks (one wave per expert, a
    // wave scan per 64 chunks); the expert's total goes to off[e]
    for (int e = w; e < E; e += nw) {
        unsigned carry = 0;
        for (int c0 = 0; c0 < nchunk; c0 += 64) {
            const int c = c0 + lane;
            const unsigned v = c < nchunk ? (unsigned)cnt[e * nchunk + c] : 0u;
            const unsigned incl = wave_inclusive_scan(v);
            if (c < nchunk) cnt[e * nchunk + c] = (int)(carry + incl - v);
            carry += (unsigned)__shfl(incl, 63, JM_WAVE);
        }
        if (lane == 0) off[e] = (int)carry;
    }
    lds_barrier();
    }
    // one block scan of (count, multi << 16 | single) gives segment starts
    // and the work-table positions of both groups
    const int total_e = tid < E ? (STABLE ? off[tid] : cnt[tid]) : 0;
    uint2 tot;
    const uint2 excl = block_exclusive_scan2(
        make_uint2((unsigned)total_e, ((unsigned)(total_e > 1) << 16) | (unsigned)(total_e == 1)), wsum, &tot);
    const int n_multi = (int)(tot.y >> 16), n_single = (int)(tot.y & 0xFFFFu);
    const int U = n_multi + n_single;
    const int my_off = (int)excl.x;
    if (tid < E) {
        off[tid] = my_off;
        seg_off[tid] = my_off;
    }
    if (tid == 0) {
        off[E] = (int)tot.x;
        seg_off[E] = (int)tot.x;
        *n_active = U;
    }
    if (tid < E && total_e > 0) {
        const int im = (int)(excl.y >> 16), is = (int)(excl.y & 0xFFFFu);
        // expert-id order over both groups: experts below tid with any slot
        active[im + is] = tid;
        if (work) {
            ExpertWork wk;
            wk.e = tid;
            wk.s0 = my_off;
            wk.n = total_e;
            wk.pad = 0;
#pragma unroll
            for (int p = 0; p < 3; p++) { wk.sc[p] = rec->sc[p]; wk.pk[p] = rec->pk[p]; }
            const int u = total_e > 1 ? im : n_multi + is;
            if (u < umax) {
                work[u] = wk;
                if (wn) wn[u] = total_e;
            }
        }
    }
    if (work) {
        for (int u = U + tid; u < umax; u += nth) {
            ExpertWork wk;
            wk.e = -1; wk.s0 = 0; wk.n = 0; wk.pad = 0;
#pragma unroll
            for (int p = 0; p < 3; p++) { wk.sc[p] = 0; wk.pk[p] = 0; }
            work[u] = wk;
            if (wn) wn[u] = 0;
        }
    }
    lds_barrier();
    for (int s = tid; s < nslot; s += nth) {
        const unsigned short r = rk[s];
        if (r == NONE) continue;
        const int e = te[s];
        const int pos = off[e] + (STABLE ? cnt[e * nchunk + s / DISP_CHUNK] : 0) + r;
        seg_slot[pos] = s;
        if (STABLE && pos == off[e]) { first_slot[e] = s; fs[e] = s; }
    }
    if (!STABLE && tid < E && total_e > 0) first_slot[tid] = fs[tid];
    lds_barrier();
    // union order per token: its slots ranked by the first slot of their
    // expert (distinct experts -> distinct keys); slots without an expert go
    // last and are stored as -1.  Each slot's key replaces its rank.
    for (int bi = tid; bi < nslot; bi += nth) {
        const unsigned short e = te[bi];
        rk[bi] = e != NONE ? (unsigned short)fs[e] : NONE;
    }
    lds_barrier();
    // bi / k as a multiply-high for k >= 2: exact for bi * k < 2^32
    // (nslot < 65536, k <= 32); the constant wraps to 0 for k = 1
    const unsigned kmagic = 0xFFFFFFFFu / (unsigned)k + 1u;
    for (int bi = tid; bi < nslot; bi += nth) {
        const int b = k == 1 ? bi : (int)__umulhi((unsigned)bi, kmagic), i = bi - b * k;
        const unsigned short key = rk[bi];
        int r = 0;
#pragma unroll 8
        for (int j = 0; j < k; j++) {
            const unsigned short kj = rk[b * k + j];
            r += (kj < key) || (kj == key && j < i);
        }
        comb[b * k + r] = key != NONE ? bi : -1;
    }
}

}  // namespace jm
