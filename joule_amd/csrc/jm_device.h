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

// DPP lane moves (CDNA row = 16 lanes).
constexpr int DPP_XOR1 = 0xB1;          // quad_perm(1,0,3,2)
constexpr int DPP_XOR2 = 0x4E;          // quad_perm(2,3,0,1)
constexpr int DPP_ROW_MIRROR = 0x140;   // lane i <- 15 - i within a row
constexpr int DPP_HALF_MIRROR = 0x141;  // lane i <- 7 - i within 8 lanes

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

// Encode one group of G floats, value i held by lane i of an aligned G-lane
// segment (G = 32 or 64), into NDIG x G/8 digit words and one scale.
// Lane j*8 of the segment writes word j of every digit k to dig[k*(G/8)+j];
// lane 0 writes the scale (only when `store`).  Every lane of the segment must
// call this (the reductions cross lanes).
template <int G, int NDIG>
__device__ __forceinline__ void encode_group_wave(float v, bool store, uint32_t* __restrict__ dig,
                                                  float* __restrict__ scale) {
    const int i = threadIdx.x & (G - 1);
    const float a = fabsf(v);
    const int bad = seg_or<G>(!(a <= 3.4028235e38f) ? 1 : 0);
    const float mx = seg_max<G>(a);
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

// ---------------------------------------------------------- router top-k

// 64-bit max over the whole wave; every lane gets the result.  Rows of 16
// lanes reduce with DPP, then the four row maxima are read as scalars.
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#define JM_STEP(CTRL)                                                            \
    {                                                                            \
        const unsigned lo = (unsigned)__builtin_amdgcn_mov_dpp((int)(unsigned)v, CTRL, 0xF, 0xF, false); \
        const unsigned hi = (unsigned)__builtin_amdgcn_mov_dpp((int)(unsigned)(v >> 32), CTRL, 0xF, 0xF, false); \
        const unsigned long long o = ((unsigned long long)hi << 32) | lo;        \
        v = o > v ? o : v;                                                       \
    }
    JM_STEP(DPP_XOR1)
    JM_STEP(DPP_XOR2)
    JM_STEP(DPP_HALF_MIRROR)
    JM_STEP(DPP_ROW_MIRROR)
#undef JM_STEP
    unsigned long long m = 0;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)v, 16 * r);
        const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(v >> 32), 16 * r);
        const unsigned long long o = ((unsigned long long)hi << 32) | lo;
        m = o > m ? o : m;
    }
    return m;
}

// Softmax over the E scores of one token and top-k selection, one wave
// (decode_kernel.c:1425-1448): max (NaN never wins), p = expf_fast(s - max),
// a sequential sum over e = 0..E-1 by lane 0, p /= sum, k rounds of argmax
// with ties to the lowest index, optional renormalisation by the sequential
// sum of the k weights.
// Argmax key of a candidate: (bits(p) << 32) | ~e.  Probabilities are >= 0,
// so their bit patterns order like their values, and ~e puts the lower index
// first among equal values; NaN and used entries get key 0, i.e. they are
// never chosen, and a round whose maximum is 0 yields index -1 and weight
// -1e30, the reference's values when nothing beats its -1e30 start.
// p_lds holds 64*EPL floats.  Lane i < k writes top[i] and tw[i].
template <int EPL>
__device__ __forceinline__ void topk_wave(const float* __restrict__ s, int E, int k, int renorm,
                                          float* p_lds, int* __restrict__ top, float* __restrict__ tw) {
    const int lane = threadIdx.x & 63;
    float v[EPL];
    float mx = -1e30f;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + 64 * j;
        v[j] = e < E ? s[e] : __int_as_float(0x7FC00000);
        if (v[j] > mx) mx = v[j];
    }
    mx = seg_max<64>(mx);                      // fmaxf ignores NaN, like the strict > scan
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + 64 * j;
        if (e < E) p_lds[e] = expf_fast(__fsub_rn(v[j], mx));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float sum = 0.0f;
    if (lane == 0) {
        int e = 0;
        for (; e + 4 <= E; e += 4) {
            const float4 q = *(const float4*)(p_lds + e);
            sum = __fadd_rn(sum, q.x); sum = __fadd_rn(sum, q.y);
            sum = __fadd_rn(sum, q.z); sum = __fadd_rn(sum, q.w);
        }
        for (; e < E; e++) sum = __fadd_rn(sum, p_lds[e]);
    }
    sum = __shfl(sum, 0, JM_WAVE);
    unsigned long long key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + 64 * j;
        const float p = e < E ? __fdiv_rn(p_lds[e], sum) : __int_as_float(0x7FC00000);
        key[j] = (p >= 0.0f) ? (((unsigned long long)__float_as_uint(p) << 32) | (unsigned)~e) : 0ull;
    }
    float my_w = 0.0f;
    int my_e = -1;
    for (int i = 0; i < k; i++) {
        unsigned long long best = 0;
#pragma unroll
        for (int j = 0; j < EPL; j++) best = key[j] > best ? key[j] : best;
        best = wave_max_u64(best);
        const int bi = best ? (int)~(unsigned)best : -1;
        const float bv = best ? __uint_as_float((unsigned)(best >> 32)) : -1e30f;
#pragma unroll
        for (int j = 0; j < EPL; j++)
            if (key[j] == best) key[j] = 0;
        if (lane == i) { my_w = bv; my_e = bi; }
    }
    if (renorm) {
        float ss = 0.0f;
        for (int i = 0; i < k; i++) ss = __fadd_rn(ss, __shfl(my_w, i, JM_WAVE));
        my_w = __fdiv_rn(my_w, ss);
    }
    if (lane < k) {
        top[lane] = my_e;
        tw[lane] = my_w;
    }
}

// ------------------------------------------------------------- dispatch

constexpr int DISP_CHUNKS_C = 16;

// Exclusive prefix sum over the block (blockDim.x <= 1024); every thread
// must call it.  wsum is LDS scratch of 16 ints; *total receives the sum.
__device__ __forceinline__ int block_exclusive_scan(int v, int* wsum, int* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, JM_WAVE);
        if (lane >= o) x += y;
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    int off = 0, all = 0;
    for (int j = 0; j < nw; j++) {
        const int t = wsum[j];
        off += j < w ? t : 0;
        all += t;
    }
    *total = all;
    __syncthreads();
    return off + x - v;
}

// Work table entry of one active expert for the expert kernels: its
// segment and the byte offsets of its gate/up/down records, so that an
// expert block needs one load to know everything it streams.
struct ExpertWork {
    int e, s0, n, pad;
    unsigned long long sc[3], pk[3];
};

// LDS of dispatch_block, in ints
__host__ __device__ constexpr int dispatch_lds_ints(int E) { return DISP_CHUNKS_C * E + 3 * E + 1 + 16; }

// Stable counting sort of nslot slots by expert id, run by one whole block
// (decode_kernel.c:1449-1485 builds the same segments in first-appearance
// order; here they are in expert-id order, slots within a segment in
// increasing b*k+i order).  `top` should point to LDS.  Writes
// seg_off[E+1], seg_slot, active[U], *n_active = U, first_slot[e], and
// comb[b*k + j] = the token's slots in the reference's union order
// (ascending first appearance of their expert), -1 padded; with `work`,
// also the expert work table for the first umax active experts (n = 0 past
// U), from the store's [3][L*E][2] record offsets at key0 = layer * E.
__device__ __forceinline__ void dispatch_block(const int* top, int nslot, int E, int k, int* lds,
                                               int* __restrict__ seg_off, int* __restrict__ seg_slot,
                                               int* __restrict__ active, int* __restrict__ n_active,
                                               int* __restrict__ first_slot, int* __restrict__ comb,
                                               int* __restrict__ rank_scratch,
                                               ExpertWork* __restrict__ work = nullptr, int umax = 0,
                                               const unsigned long long* __restrict__ rec_off = nullptr,
                                               long long LE = 0, long long key0 = 0) {
    int* cnt = lds;                              // [DISP_CHUNKS][E]
    int* off = cnt + DISP_CHUNKS_C * E;          // [E + 1]
    int* fs = off + E + 1;                       // [E]
    int* act = fs + E;                           // [E]
    int* wsum = act + E;                         // [16]
    const int tid = threadIdx.x, nth = blockDim.x;
    const int chunk = (nslot + DISP_CHUNKS_C - 1) / DISP_CHUNKS_C;
    for (int i = tid; i < DISP_CHUNKS_C * E; i += nth) cnt[i] = 0;
    __syncthreads();
    for (int s = tid; s < nslot; s += nth) {
        const int e = top[s];
        if (e < 0 || e >= E) { rank_scratch[s] = -1; continue; }
        const int c = s / chunk;
        int rank = 0;
        for (int q = c * chunk; q < s; q++) rank += (top[q] == e);
        rank_scratch[s] = rank;
        atomicAdd(&cnt[c * E + e], 1);
    }
    __syncthreads();
    // per expert: exclusive prefix over chunks, then one block scan of
    // (active flag << 20 | count) gives segment starts and active indices
    int total_e = 0;
    for (int e = tid; e < E; e += nth) {
        int run = 0;
        for (int c = 0; c < DISP_CHUNKS_C; c++) {
            const int n = cnt[c * E + e];
            cnt[c * E + e] = run;
            run += n;
        }
        total_e = run;                           // E <= nth: one expert per thread
    }
    const int packed = tid < E ? (((total_e > 0) << 20) | total_e) : 0;
    int tot;
    const int excl = block_exclusive_scan(packed, wsum, &tot);
    const int U = tot >> 20;
    if (tid < E) {
        off[tid] = excl & 0xFFFFF;
        seg_off[tid] = excl & 0xFFFFF;
        if (total_e > 0) {
            active[excl >> 20] = tid;
            act[excl >> 20] = tid;
        }
    }
    if (tid == 0) {
        off[E] = tot & 0xFFFFF;
        seg_off[E] = tot & 0xFFFFF;
        *n_active = U;
    }
    __syncthreads();
    for (int s = tid; s < nslot; s += nth) {
        const int rank = rank_scratch[s];
        if (rank < 0) continue;
        const int e = top[s];
        const int pos = off[e] + cnt[(s / chunk) * E + e] + rank;
        seg_slot[pos] = s;
        if (pos == off[e]) { first_slot[e] = s; fs[e] = s; }
    }
    __syncthreads();
    // union order per token: its slots ranked by the first slot of their
    // expert (distinct experts -> distinct keys); slots without an expert go
    // last and are stored as -1
    for (int bi = tid; bi < nslot; bi += nth) {
        const int b = bi / k, i = bi % k;
        const int e = top[bi];
        const bool ok = e >= 0 && e < E;
        const int key = ok ? fs[e] : 0x7FFFFFFF;
        int rank = 0;
        for (int j = 0; j < k; j++) {
            const int ej = top[b * k + j];
            const int kj = (ej >= 0 && ej < E) ? fs[ej] : 0x7FFFFFFF;
            rank += (kj < key) || (kj == key && j < i);
        }
        comb[b * k + rank] = ok ? bi : -1;
    }
    if (work) {
        for (int u = tid; u < umax; u += nth) {
            ExpertWork wk;
            wk.pad = 0;
            if (u < U) {
                const int e = act[u];
                wk.e = e;
                wk.s0 = off[e];
                wk.n = off[e + 1] - off[e];
                for (int p = 0; p < 3; p++) {
                    wk.sc[p] = rec_off[((long long)p * LE + key0 + e) * 2 + 0];
                    wk.pk[p] = rec_off[((long long)p * LE + key0 + e) * 2 + 1];
                }
            } else {
                wk.e = -1; wk.s0 = 0; wk.n = 0;
                for (int p = 0; p < 3; p++) { wk.sc[p] = 0; wk.pk[p] = 0; }
            }
            work[u] = wk;
        }
    }
}

}  // namespace jm
