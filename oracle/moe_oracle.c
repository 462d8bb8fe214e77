/*
 * moe_oracle.c -- CPU restatement of the reference MoE decode block.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle and the timed CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only as the checker, never as the thing measured on the
 * GPU path or shipped in the product.
 *
 * It restates, operation by operation, the arithmetic of the reference's
 * native MoE block so that router indices and weights come out bit-identical
 * and expert outputs agree to rounding:
 *
 *   fp16_to_f32         src/jouleai/native/decode_kernel.c:64-85
 *   bf16_to_f32         src/jouleai/native/decode_kernel.c:47-53
 *   expf_fast           src/jouleai/native/decode_kernel.c:94-108
 *   router GEMV         src/jouleai/native/decode_kernel.c:234-256, 693-725
 *   softmax/top-k/renorm src/jouleai/native/decode_kernel.c:1425-1448
 *   union dispatch      src/jouleai/native/decode_kernel.c:1449-1485
 *   q4_row_dot_B        src/jouleai/native/decode_kernel.c:770-858
 *   ffn_expert_worker   src/jouleai/native/decode_kernel.c:1251-1275, 1365-1385
 *   combine             src/jouleai/native/decode_kernel.c:1486-1507
 *   spin pool partition src/jouleai/native/decode_kernel.c:597-675
 *   expert_ffn variants src/jouleai/native/expert_ffn.c:57-215
 *   scalar q4 gemv      src/jouleai/native/quant_gemv.c:35-57
 *
 * Floating-point contraction: the reference is built with clang (zig cc),
 * whose default -ffp-contract=on fuses `a + b*c` written in one expression
 * into an FMA.  This file is compiled with -ffp-contract=off and spells every
 * such fusion as an explicit fmaf(), so the arithmetic does not depend on the
 * compiler building the oracle.
 *
 * The AVX2 reference keeps 8 partial sums (one per SIMD lane r, summing the
 * elements j == r mod 8) and reduces them as ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7)).
 * The lane8_* helpers below hold those 8 partials in a plain array.
 *
 * The block driver runs either that scalar form or an AVX2 form of the same
 * operations (jmo_set_simd): the 8 partial sums in one __m256 with
 * _mm256_fmadd_ps per step and the same reduction tree, so both forms give
 * the same bits (tests/test_oracle_simd.py); the AVX2 form is the timed CPU
 * baseline, the scalar one stays the readable statement.
 */
#define _GNU_SOURCE
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define JMO_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------ */
/* scalar conversions                                                  */
/* ------------------------------------------------------------------ */

/* IEEE binary16 -> binary32 by bit manipulation (decode_kernel.c:64-85).
 * Subnormal halves are renormalised, Inf/NaN payloads are carried over. */
JMO_API float jmo_fp16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t frac = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1Fu) {
        bits = sign | 0x7F800000u | (frac << 13);
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (frac << 13);
    } else if (frac == 0) {
        bits = sign;
    } else {
        /* subnormal: shift the leading one up to the implicit position */
        int shift = 0;
        while (!(frac & 0x400u)) { frac <<= 1; shift++; }
        bits = sign | ((uint32_t)(113 - shift) << 23) | ((frac & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* bf16 -> fp32 is a 16-bit left shift (decode_kernel.c:47-53). */
JMO_API float jmo_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* Array forms (bits compared in memory; a float returned through an FFI may
 * be widened to double, which quiets signalling NaNs). */
JMO_API void jmo_fp16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = jmo_fp16_to_f32(in[i]);
}

JMO_API void jmo_bf16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = jmo_bf16_to_f32(in[i]);
}

/* The reference's own exponential (decode_kernel.c:94-108): clamp, split
 * v*log2(e) into integer k (rounded half away from zero by truncating y+-0.5)
 * and fraction f, a degree-5 polynomial for 2^f evaluated by Horner (each
 * step one FMA under clang's default contraction), then scale by 2^k built
 * directly in the exponent field. */
JMO_API float jmo_expf_fast(float v) {
    /* NaN: the reference's (int) conversion on x86 yields INT_MIN, so its
     * biased exponent is negative and it returns 0; spelled out here */
    if (v != v) return 0.0f;
    if (v < -17.0f) return 0.0f;
    if (v > 88.0f) v = 88.0f;
    const float y = v * 1.4426950408889634f;
    const int k = (int)(y >= 0 ? y + 0.5f : y - 0.5f);
    const float f = y - (float)k;
    float p = fmaf(f, 0.0013330f, 0.0096181f);
    p = fmaf(f, p, 0.0555041f);
    p = fmaf(f, p, 0.2402265f);
    p = fmaf(f, p, 0.6931472f);
    p = fmaf(f, p, 1.0f);
    int biased = k + 127;
    if (biased < 0) return 0.0f;
    if (biased > 254) biased = 254;
    uint32_t bits = (uint32_t)biased << 23;
    float two_k;
    memcpy(&two_k, &bits, sizeof two_k);
    return p * two_k;
}

/* ------------------------------------------------------------------ */
/* 8-lane dot products (the AVX2 accumulation order)                   */
/* ------------------------------------------------------------------ */

static inline float lane8_reduce(const float l[8]) {
    return ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7]));
}

/* Router row dot: decode_kernel.c:234-256 (B=1) and :693-718 (B>1) share it.
 * Each lane is an FMA chain over j == r (mod 8) starting from +0, then the
 * lane tree; a scalar tail (d % 8 != 0) continues with FMAs. */
JMO_API void jmo_expf_fast_array(const float* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = jmo_expf_fast(in[i]);
}

JMO_API float jmo_router_dot(const float* w, const float* x, int d) {
    float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int j = 0;
    for (; j + 8 <= d; j += 8)
        for (int r = 0; r < 8; r++) l[r] = fmaf(w[j + r], x[j + r], l[r]);
    float acc = lane8_reduce(l);
    for (; j < d; j++) acc = fmaf(w[j], x[j], acc);
    return acc;
}

/* scores[b][e] for all tokens and experts (the router GEMV of one layer). */
JMO_API void jmo_router_logits(const float* w, const float* x, int B, int E, int d, float* out) {
    for (int b = 0; b < B; b++)
        for (int e = 0; e < E; e++)
            out[(size_t)b * E + e] = jmo_router_dot(w + (size_t)e * d, x + (size_t)b * d, d);
}

/* Unpack one group of `group` Q4 values: byte j holds element 2j in its low
 * nibble and 2j+1 in its high nibble, stored biased by +8. */
static inline void q4_unpack_group(const uint8_t* p, int group, float* vals) {
    for (int j = 0; j < group / 2; j++) {
        vals[2 * j] = (float)((int)(p[j] & 0x0Fu) - 8);
        vals[2 * j + 1] = (float)((int)(p[j] >> 4) - 8);
    }
}

/* Group dot of the AVX2 kernels: 8 lane chains over the group's values,
 * chain r taking elements r, r+8, ..., then the lane tree. */
static inline float q4_group_lane8(const float* vals, const float* x, int group) {
    float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int t = 0; t < group; t += 8)
        for (int r = 0; r < 8; r++) l[r] = fmaf(vals[t + r], x[t + r], l[r]);
    return lane8_reduce(l);
}

/* Batched Q4 row dot, decode_kernel.c:770-858.  For each full group:
 * acc[b] += hsum_b * scale (one FMA under contraction, `acc[b] += ... * s`).
 * `cols` is the row length, `stride` the distance between token vectors. */
JMO_API void jmo_q4_row_dot_B(const uint8_t* row, const uint16_t* sc,
                              const float* x, int B, float* acc,
                              int cols, int group, int stride) {
    float vals[64];
    for (int b = 0; b < B; b++) acc[b] = 0.0f;
    const int ng = cols / group;
    for (int g = 0; g < ng; g++) {
        const float s = jmo_fp16_to_f32(sc[g]);
        q4_unpack_group(row + (size_t)g * (group / 2), group, vals);
        for (int b = 0; b < B; b++) {
            const float h = q4_group_lane8(vals, x + (size_t)b * stride + (size_t)g * group, group);
            acc[b] = fmaf(h, s, acc[b]);
        }
    }
    /* columns past the last full group (never present when cols % group == 0) */
    const int tail0 = ng * group;
    if (tail0 < cols) {
        const float s = jmo_fp16_to_f32(sc[ng]);
        for (int b = 0; b < B; b++) {
            const float* xb = x + (size_t)b * stride;
            float ga = 0.0f;
            for (int c = tail0; c < cols; c += 2) {
                const uint8_t byte = row[c / 2];
                const float lo = (float)((int)(byte & 0x0Fu) - 8);
                const float hi = (float)((int)(byte >> 4) - 8);
                ga = ga + fmaf(lo, xb[c], hi * xb[c + 1]);
            }
            acc[b] = fmaf(ga, s, acc[b]);
        }
    }
}

/* ------------------------------------------------------------------ */
/* AVX2 forms of the router dot and the batched Q4 row dot              */
/* ------------------------------------------------------------------ */

/* ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)) of the 8 lanes, as lane8_reduce. */
static inline float lane8_reduce_v(__m256 v) {
    __m128 h = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));   /* l_i + l_(i+4) */
    h = _mm_add_ps(h, _mm_movehl_ps(h, h));                                           /* (0+4)+(2+6), (1+5)+(3+7) */
    h = _mm_add_ss(h, _mm_shuffle_ps(h, h, 1));
    return _mm_cvtss_f32(h);
}

JMO_API float jmo_router_dot_avx2(const float* w, const float* x, int d) {
    __m256 l = _mm256_setzero_ps();
    int j = 0;
    for (; j + 8 <= d; j += 8) l = _mm256_fmadd_ps(_mm256_loadu_ps(w + j), _mm256_loadu_ps(x + j), l);
    float acc = lane8_reduce_v(l);
    for (; j < d; j++) acc = fmaf(w[j], x[j], acc);
    return acc;
}

/* Values (q - 8) of 8 consecutive elements as floats, from the dword that
 * packs them (element k in bits 4k..4k+3): the dword broadcast, shifted per
 * lane and masked, then 2^23 + q read as a float less 2^23 + 8 (exact). */
static inline __m256 q4_vec8(const uint8_t* p) {
    const __m256i sh = _mm256_setr_epi32(0, 4, 8, 12, 16, 20, 24, 28);
    int w;
    memcpy(&w, p, sizeof w);
    const __m256i q = _mm256_and_si256(_mm256_srlv_epi32(_mm256_set1_epi32(w), sh),
                                       _mm256_set1_epi32(0x0F));
    return _mm256_sub_ps(_mm256_castsi256_ps(_mm256_or_si256(q, _mm256_set1_epi32(0x4B000000))),
                         _mm256_set1_ps(8388616.0f));
}

/* Four groups' lane reductions at once, each the tree of lane8_reduce_v:
 * h_i = l_i + l_(i+4) for both groups of a 256-bit pair, then
 * (h_0 + h_2) and (h_1 + h_3) side by side for all four, then their sum.
 * Returns [r0, r1, r2, r3]. */
static inline __m128 lane8_reduce4_v(__m256 l0, __m256 l1, __m256 l2, __m256 l3) {
    const __m256 h01 = _mm256_add_ps(_mm256_permute2f128_ps(l0, l1, 0x20), _mm256_permute2f128_ps(l0, l1, 0x31));
    const __m256 h23 = _mm256_add_ps(_mm256_permute2f128_ps(l2, l3, 0x20), _mm256_permute2f128_ps(l2, l3, 0x31));
    /* per 128-bit half: [h0+h2, h1+h3] of group 0 (low) / 1 (high), then of 2 / 3 */
    const __m256 t = _mm256_add_ps(_mm256_shuffle_ps(h01, h23, _MM_SHUFFLE(1, 0, 1, 0)),
                                   _mm256_shuffle_ps(h01, h23, _MM_SHUFFLE(3, 2, 3, 2)));
    const __m256 u = _mm256_hadd_ps(t, t);           /* low: r0, r2; high: r1, r3 */
    return _mm_unpacklo_ps(_mm256_castps256_ps128(u), _mm256_extractf128_ps(u, 1));
}

/* Up to 64 packed bytes (128 elements) as signed bytes q - 8 in element order. */
static inline void q4_bytes(const uint8_t* p, int nbytes, int8_t* out) {
    const __m128i m = _mm_set1_epi8(0x0F), k8 = _mm_set1_epi8(8);
    int i = 0;
    for (; i + 16 <= nbytes; i += 16) {
        const __m128i b = _mm_loadu_si128((const __m128i*)(p + i));
        const __m128i lo = _mm_and_si128(b, m), hi = _mm_and_si128(_mm_srli_epi16(b, 4), m);
        _mm_storeu_si128((__m128i*)(out + 2 * i), _mm_sub_epi8(_mm_unpacklo_epi8(lo, hi), k8));
        _mm_storeu_si128((__m128i*)(out + 2 * i + 16), _mm_sub_epi8(_mm_unpackhi_epi8(lo, hi), k8));
    }
    for (; i < nbytes; i++) {
        out[2 * i] = (int8_t)((int)(p[i] & 0x0Fu) - 8);
        out[2 * i + 1] = (int8_t)((int)(p[i] >> 4) - 8);
    }
}

/* 8 values from signed bytes as floats (exact). */
static inline __m256 q4_vec8_b(const int8_t* q) {
    return _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)q)));
}

/* One token's dot with one row (group 32 or 64): the row decoded to bytes
 * in chunks of four groups, each group's 8 lane chains in one register
 * (the fmaf of q4_group_lane8 per lane and step), four groups' chains
 * interleaved, reduced by the lane8 tree, and a = fmaf(r, s, a) in group
 * order. */
static inline __attribute__((always_inline)) float q4_row_dot1_body(const uint8_t* row, const uint16_t* sc,
                                                                   const float* x, int ng, int group) {
    const int nv = group / 8, gb = group / 2;
    int8_t q[256];
    float a = 0.0f;
    int g = 0;
    for (; g + 4 <= ng; g += 4) {
        q4_bytes(row + (size_t)g * gb, 4 * gb, q);
        /* keep q in memory: 8-byte sign-extending loads from it cost one
         * instruction each, extracting them from registers three */
        __asm__ volatile("" : : "r"(q) : "memory");
        const float* xg = x + (size_t)g * group;
        __m256 l0 = _mm256_setzero_ps(), l1 = l0, l2 = l0, l3 = l0;
        for (int t = 0; t < nv; t++) {
            l0 = _mm256_fmadd_ps(q4_vec8_b(q + 8 * t), _mm256_loadu_ps(xg + 8 * t), l0);
            l1 = _mm256_fmadd_ps(q4_vec8_b(q + group + 8 * t), _mm256_loadu_ps(xg + group + 8 * t), l1);
            l2 = _mm256_fmadd_ps(q4_vec8_b(q + 2 * group + 8 * t), _mm256_loadu_ps(xg + 2 * group + 8 * t), l2);
            l3 = _mm256_fmadd_ps(q4_vec8_b(q + 3 * group + 8 * t), _mm256_loadu_ps(xg + 3 * group + 8 * t), l3);
        }
        const __m128 r = lane8_reduce4_v(l0, l1, l2, l3);
        a = fmaf(_mm_cvtss_f32(r), jmo_fp16_to_f32(sc[g]), a);
        a = fmaf(_mm_cvtss_f32(_mm_shuffle_ps(r, r, 1)), jmo_fp16_to_f32(sc[g + 1]), a);
        a = fmaf(_mm_cvtss_f32(_mm_shuffle_ps(r, r, 2)), jmo_fp16_to_f32(sc[g + 2]), a);
        a = fmaf(_mm_cvtss_f32(_mm_shuffle_ps(r, r, 3)), jmo_fp16_to_f32(sc[g + 3]), a);
    }
    for (; g < ng; g++) {
        q4_bytes(row + (size_t)g * gb, gb, q);
        __m256 l = _mm256_setzero_ps();
        for (int t = 0; t < nv; t++)
            l = _mm256_fmadd_ps(q4_vec8_b(q + 8 * t), _mm256_loadu_ps(x + (size_t)g * group + 8 * t), l);
        a = fmaf(lane8_reduce_v(l), jmo_fp16_to_f32(sc[g]), a);
    }
    return a;
}

/* the body with the group size a constant (32 or 64 values) */
static float q4_row_dot1_avx2(const uint8_t* row, const uint16_t* sc, const float* x, int ng, int group) {
    return group == 64 ? q4_row_dot1_body(row, sc, x, ng, 64) : q4_row_dot1_body(row, sc, x, ng, 32);
}

/* jmo_q4_row_dot_B with each group's 8 lane chains in one register: the same
 * fmaf per lane and step as q4_group_lane8, the same tree, the same
 * acc[b] = fmaf(h, s, acc[b]) in group order.  Independent chains are
 * interleaved (four groups of one token, or two tokens of one group) so that
 * the FMA latency overlaps; no lane's order changes. */
JMO_API void jmo_q4_row_dot_B_avx2(const uint8_t* row, const uint16_t* sc,
                                   const float* x, int B, float* acc,
                                   int cols, int group, int stride) {
    if (group != 32 && group != 64) {
        jmo_q4_row_dot_B(row, sc, x, B, acc, cols, group, stride);
        return;
    }
    const int ng = cols / group, nv = group / 8, gb = group / 2;
    int g = ng;
    if (B == 1) {
        acc[0] = q4_row_dot1_avx2(row, sc, x, ng, group);
    } else {
        for (int b = 0; b < B; b++) acc[b] = 0.0f;
        __m256 v[8];
        for (g = 0; g < ng; g++) {
            const float s = jmo_fp16_to_f32(sc[g]);
            for (int t = 0; t < nv; t++) v[t] = q4_vec8(row + (size_t)g * gb + 4 * t);
            int b = 0;
            for (; b + 2 <= B; b += 2) {
                const float* x0 = x + (size_t)b * stride + (size_t)g * group;
                const float* x1 = x0 + stride;
                __m256 l0 = _mm256_setzero_ps(), l1 = l0;
                for (int t = 0; t < nv; t++) {
                    l0 = _mm256_fmadd_ps(v[t], _mm256_loadu_ps(x0 + 8 * t), l0);
                    l1 = _mm256_fmadd_ps(v[t], _mm256_loadu_ps(x1 + 8 * t), l1);
                }
                acc[b] = fmaf(lane8_reduce_v(l0), s, acc[b]);
                acc[b + 1] = fmaf(lane8_reduce_v(l1), s, acc[b + 1]);
            }
            for (; b < B; b++) {
                const float* x0 = x + (size_t)b * stride + (size_t)g * group;
                __m256 l0 = _mm256_setzero_ps();
                for (int t = 0; t < nv; t++) l0 = _mm256_fmadd_ps(v[t], _mm256_loadu_ps(x0 + 8 * t), l0);
                acc[b] = fmaf(lane8_reduce_v(l0), s, acc[b]);
            }
        }
    }
    const int tail0 = ng * group;
    if (tail0 < cols) {
        const float s = jmo_fp16_to_f32(sc[ng]);
        for (int b = 0; b < B; b++) {
            const float* xb = x + (size_t)b * stride;
            float ga = 0.0f;
            for (int c = tail0; c < cols; c += 2) {
                const uint8_t byte = row[c / 2];
                const float lo = (float)((int)(byte & 0x0Fu) - 8);
                const float hi = (float)((int)(byte >> 4) - 8);
                ga = ga + fmaf(lo, xb[c], hi * xb[c + 1]);
            }
            acc[b] = fmaf(ga, s, acc[b]);
        }
    }
}

/* which form the block driver runs: 0 scalar, 1 AVX2 */
static _Atomic int g_simd = 0;

JMO_API void jmo_set_simd(int on) { atomic_store(&g_simd, on ? 1 : 0); }
JMO_API int jmo_get_simd(void) { return atomic_load(&g_simd); }

static inline float router_dot_sel(const float* w, const float* x, int d) {
    return atomic_load_explicit(&g_simd, memory_order_relaxed) ? jmo_router_dot_avx2(w, x, d) : jmo_router_dot(w, x, d);
}

static inline void row_dot_sel(const uint8_t* row, const uint16_t* sc, const float* x, int B, float* acc,
                               int cols, int group, int stride) {
    if (!atomic_load_explicit(&g_simd, memory_order_relaxed))
        jmo_q4_row_dot_B(row, sc, x, B, acc, cols, group, stride);
    else if (B == 1 && (group == 32 || group == 64) && cols % group == 0)
        acc[0] = q4_row_dot1_avx2(row, sc, x, cols / group, group);
    else
        jmo_q4_row_dot_B_avx2(row, sc, x, B, acc, cols, group, stride);
}

/* ------------------------------------------------------------------ */
/* expert_ffn.c / quant_gemv.c variants (pinned against the real code)  */
/* ------------------------------------------------------------------ */

/* expert_ffn.c:99-130 with the AVX2 group body (:59-94): the group partial is
 * returned already multiplied by its scale and then added (two roundings,
 * the multiply sits in another expression). */
static float q4_row_dot_ffn(const uint8_t* row, const uint16_t* sc,
                            const float* x, int cols, int group) {
    float vals[64];
    float acc = 0.0f;
    const int ng = cols / group;
    for (int g = 0; g < ng; g++) {
        q4_unpack_group(row + (size_t)g * (group / 2), group, vals);
        const float h = q4_group_lane8(vals, x + (size_t)g * group, group);
        acc = acc + h * jmo_fp16_to_f32(sc[g]);
    }
    return acc;
}

/* q4_gemv_f32 of expert_ffn.c:132-142. */
JMO_API void jmo_q4_gemv_ffn(float* out, const float* x, const uint8_t* packed,
                             const uint16_t* scales, int m, int d, int group) {
    for (int i = 0; i < m; i++)
        out[i] = q4_row_dot_ffn(packed + (size_t)i * (d / 2),
                                scales + (size_t)i * (d / group), x, d, group);
}

/* q4_gemm_f32 of expert_ffn.c:200-215: out[t][i] for T token rows. */
JMO_API void jmo_q4_gemm_ffn(float* out, const float* X, int T, const uint8_t* packed,
                             const uint16_t* scales, int m, int d, int group) {
    for (int t = 0; t < T; t++)
        jmo_q4_gemv_ffn(out + (size_t)t * m, X + (size_t)t * d, packed, scales, m, d, group);
}

/* Scalar row dot of quant_gemv.c:35-57 and of expert_job's down loop
 * (expert_ffn.c:173-188): per byte `gacc += lo*x0 + hi*x1`, which clang
 * contracts to gacc + fma(lo, x0, hi*x1); then acc = fma(gacc, s, acc). */
static float q4_row_dot_scalar(const uint8_t* row, const uint16_t* sc,
                               const float* x, int cols, int group) {
    float acc = 0.0f;
    for (int g = 0; g < cols / group; g++) {
        const float s = jmo_fp16_to_f32(sc[g]);
        float gacc = 0.0f;
        for (int j = g * group / 2; j < (g + 1) * group / 2; j++) {
            const float lo = (float)((int)(row[j] & 0x0Fu) - 8);
            const float hi = (float)((int)(row[j] >> 4) - 8);
            gacc = gacc + fmaf(lo, x[2 * j], hi * x[2 * j + 1]);
        }
        acc = fmaf(gacc, s, acc);
    }
    return acc;
}

/* q4_gemv_f32 of quant_gemv.c:35-57. */
JMO_API void jmo_q4_gemv_scalar(float* out, const float* x, const uint8_t* packed,
                                const uint16_t* scales, int m, int d, int group) {
    for (int i = 0; i < m; i++)
        out[i] = q4_row_dot_scalar(packed + (size_t)i * (d / 2),
                                   scales + (size_t)i * (d / group), x, d, group);
}

/* expert_job of expert_ffn.c:159-191: gate/up through the AVX2 row dot,
 * act = silu(g)*u with the reference exp, down through the scalar loop, and
 * the routing probability applied last.  scratch = [m][act] ++ [d][out]. */
JMO_API void jmo_expert_job(const uint8_t* pk_g, const uint16_t* sc_g,
                            const uint8_t* pk_u, const uint16_t* sc_u,
                            const uint8_t* pk_d, const uint16_t* sc_d,
                            int m, int d, int group, const float* x,
                            float* scratch, float prob) {
    float* act = scratch;
    float* wout = scratch + m;
    for (int i = 0; i < m; i++) {
        const float g = q4_row_dot_ffn(pk_g + (size_t)i * (d / 2), sc_g + (size_t)i * (d / group), x, d, group);
        const float u = q4_row_dot_ffn(pk_u + (size_t)i * (d / 2), sc_u + (size_t)i * (d / group), x, d, group);
        act[i] = (g / (1.0f + jmo_expf_fast(-g))) * u;
    }
    for (int i = 0; i < d; i++) {
        const float acc = q4_row_dot_scalar(pk_d + (size_t)i * (m / 2), sc_d + (size_t)i * (m / group),
                                            act, m, group);
        wout[i] = acc * prob;
    }
}

/* Exact dequantisation (q - 8) * fp32(scale), q4_store.py:58-67. */
JMO_API void jmo_q4_dequant(float* out, const uint8_t* packed, const uint16_t* scales,
                            int64_t numel, int group) {
    for (int64_t i = 0; i < numel; i++) {
        const uint8_t byte = packed[i >> 1];
        const int q = (i & 1) ? (byte >> 4) : (byte & 0x0F);
        out[i] = (float)(q - 8) * jmo_fp16_to_f32(scales[i / group]);
    }
}

/* ------------------------------------------------------------------ */
/* router: softmax, top-k, renormalisation                              */
/* ------------------------------------------------------------------ */

/* decode_kernel.c:1425-1448 for one token.  probs is overwritten in place
 * with the normalised softmax.  Ties go to the lowest index because the scan
 * keeps the first strictly larger value.  An index of -1 means no remaining
 * candidate beat -1e30 (only possible with NaN scores). */
JMO_API void jmo_softmax_topk(float* probs, int E, int topk, int renorm,
                              int32_t* top, float* tw) {
    float smax = -1e30f;
    for (int e = 0; e < E; e++) if (probs[e] > smax) smax = probs[e];
    float sum = 0.0f;
    for (int e = 0; e < E; e++) { probs[e] = jmo_expf_fast(probs[e] - smax); sum = sum + probs[e]; }
    for (int e = 0; e < E; e++) probs[e] = probs[e] / sum;
    for (int i = 0; i < topk; i++) {
        int bi = -1;
        float bv = -1e30f;
        for (int e = 0; e < E; e++) {
            int used = 0;
            for (int j = 0; j < i; j++) if (top[j] == e) { used = 1; break; }
            if (!used && probs[e] > bv) { bv = probs[e]; bi = e; }
        }
        top[i] = bi;
        tw[i] = bv;
    }
    if (renorm) {
        float ssum = 0.0f;
        for (int i = 0; i < topk; i++) ssum = ssum + tw[i];
        for (int i = 0; i < topk; i++) tw[i] = tw[i] / ssum;
    }
}

/* ------------------------------------------------------------------ */
/* fixed-id spin pool (same static partition as decode_kernel.c:597-675) */
/* ------------------------------------------------------------------ */

typedef void (*jmo_work_fn)(void* ctx, long id, long lo, long hi);

typedef struct {
    int n_workers;              /* helper threads; the caller is participant n_workers */
    pthread_t th[64];
    long ids[64];
    _Atomic long gen;
    _Atomic long arrived;
    _Atomic int shutdown;
    jmo_work_fn fn;
    void* ctx;
    long lo, hi;
} jmo_pool;

static jmo_pool g_pool;
static pthread_mutex_t g_pool_mu = PTHREAD_MUTEX_INITIALIZER;

static inline void cpu_relax(void) { __builtin_ia32_pause(); }

static void pool_chunk(long id, long np, long lo, long hi, long* clo, long* chi) {
    const long span = hi - lo;
    *clo = lo + span * id / np;
    *chi = lo + span * (id + 1) / np;
}

static void* pool_main(void* arg) {
    const long id = *(long*)arg;
    long seen = 0;
    for (;;) {
        long g;
        int spins = 0;
        while ((g = atomic_load_explicit(&g_pool.gen, memory_order_acquire)) == seen) {
            if (atomic_load_explicit(&g_pool.shutdown, memory_order_acquire)) return NULL;
            if (++spins < 4096) cpu_relax(); else { sched_yield(); spins = 0; }
        }
        seen = g;
        if (atomic_load_explicit(&g_pool.shutdown, memory_order_acquire)) return NULL;
        long clo, chi;
        pool_chunk(id, g_pool.n_workers + 1, g_pool.lo, g_pool.hi, &clo, &chi);
        g_pool.fn(g_pool.ctx, id, clo, chi);
        atomic_fetch_add_explicit(&g_pool.arrived, 1, memory_order_acq_rel);
    }
}

static void pool_stop(void) {
    if (g_pool.n_workers == 0) return;
    atomic_store_explicit(&g_pool.shutdown, 1, memory_order_release);
    atomic_fetch_add_explicit(&g_pool.gen, 1, memory_order_acq_rel);
    for (int i = 0; i < g_pool.n_workers; i++) pthread_join(g_pool.th[i], NULL);
    g_pool.n_workers = 0;
    atomic_store(&g_pool.shutdown, 0);
}

/* Start (or resize to) n_workers helper threads.  Returns 0 on failure. */
JMO_API int jmo_pool_init(int n_workers) {
    if (n_workers < 0) n_workers = 0;
    if (n_workers > 64) n_workers = 64;
    pthread_mutex_lock(&g_pool_mu);
    if (g_pool.n_workers == n_workers) { pthread_mutex_unlock(&g_pool_mu); return 1; }
    pool_stop();
    atomic_store(&g_pool.gen, 0);
    atomic_store(&g_pool.arrived, 0);
    for (int i = 0; i < n_workers; i++) {
        g_pool.ids[i] = i;
        if (pthread_create(&g_pool.th[i], NULL, pool_main, &g_pool.ids[i]) != 0) {
            g_pool.n_workers = i;
            pool_stop();
            pthread_mutex_unlock(&g_pool_mu);
            return 0;
        }
        g_pool.n_workers = i + 1;
    }
    pthread_mutex_unlock(&g_pool_mu);
    return 1;
}

JMO_API void jmo_pool_shutdown(void) {
    pthread_mutex_lock(&g_pool_mu);
    pool_stop();
    pthread_mutex_unlock(&g_pool_mu);
}

/* Run fn over [lo, hi) on the helpers plus the calling thread (which takes
 * the last chunk), returning when every participant has finished. */
static void pool_run(jmo_work_fn fn, void* ctx, long lo, long hi) {
    const int nw = g_pool.n_workers;
    if (nw == 0) { fn(ctx, 0, lo, hi); return; }
    g_pool.fn = fn;
    g_pool.ctx = ctx;
    g_pool.lo = lo;
    g_pool.hi = hi;
    atomic_store_explicit(&g_pool.arrived, 0, memory_order_relaxed);
    atomic_fetch_add_explicit(&g_pool.gen, 1, memory_order_acq_rel);
    long clo, chi;
    pool_chunk(nw, nw + 1, lo, hi, &clo, &chi);
    fn(ctx, nw, clo, chi);
    while (atomic_load_explicit(&g_pool.arrived, memory_order_acquire) < nw) cpu_relax();
}

/* ------------------------------------------------------------------ */
/* the MoE block (layer_ffn_batch)                                      */
/* ------------------------------------------------------------------ */

typedef struct {
    int d, m, E, topk, renorm, group;
    const float* gate_w;          /* [E][d] router weights (bf16 values as fp32) */
    const uint8_t* const* pk;     /* [3*E]: packed rows of gate, up, down per expert */
    const uint16_t* const* sc;    /* [3*E]: fp16 scales of gate, up, down per expert */
} jmo_moe;

typedef struct {
    const jmo_moe* p;
    const float* x;
    int B;
    float* scores;                /* [B][E] */
    const int* sel;               /* [U] union experts, first-appearance order */
    const int* uh;                /* [U+1] slot prefix */
    const int* uidx;              /* slot ids b*topk+i grouped by union expert */
    const float* uw;              /* routing weight per grouped slot */
    float* act;                   /* [U][B][m] */
    float* y;                     /* [U][B][d] */
    int all_tokens;               /* 1: dot every token like the reference does */
} jmo_job;

static void router_worker(void* ctx, long id, long lo, long hi) {
    (void)id;
    jmo_job* j = (jmo_job*)ctx;
    const jmo_moe* p = j->p;
    for (long e = lo; e < hi; e++)
        for (int b = 0; b < j->B; b++)
            j->scores[(size_t)b * p->E + e] =
                router_dot_sel(p->gate_w + (size_t)e * p->d, j->x + (size_t)b * p->d, p->d);
}

static void expert_worker(void* ctx, long id, long lo, long hi) {
    (void)id;
    jmo_job* j = (jmo_job*)ctx;
    const jmo_moe* p = j->p;
    const int d = p->d, m = p->m, B = j->B, G = p->group, E = p->E;
    float* gacc = (float*)malloc(sizeof(float) * (size_t)B * 3);
    float* uacc = gacc + B;
    float* dacc = uacc + B;
    int* tok = (int*)malloc(sizeof(int) * (size_t)B);
    for (long ue = lo; ue < hi; ue++) {
        const int e = j->sel[ue];
        const int s0 = j->uh[ue], s1 = j->uh[ue + 1];
        if (s1 <= s0) continue;
        const uint8_t *pkg = p->pk[e], *pku = p->pk[E + e], *pkd = p->pk[2 * E + e];
        const uint16_t *scg = p->sc[e], *scu = p->sc[E + e], *scd = p->sc[2 * E + e];
        float* acte = j->act + (size_t)ue * B * m;
        float* ye = j->y + (size_t)ue * B * d;
        /* tokens routed to this expert; with all_tokens the dots also run for
         * the others and are discarded, which is the reference's cost model */
        int nt = 0;
        for (int s = s0; s < s1; s++) tok[nt++] = j->uidx[s] / p->topk;
        for (int i = 0; i < m; i++) {
            if (j->all_tokens) {
                row_dot_sel(pkg + (size_t)i * (d / 2), scg + (size_t)i * (d / G), j->x, B, gacc, d, G, d);
                row_dot_sel(pku + (size_t)i * (d / 2), scu + (size_t)i * (d / G), j->x, B, uacc, d, G, d);
            } else {
                for (int t = 0; t < nt; t++) {
                    const int b = tok[t];
                    row_dot_sel(pkg + (size_t)i * (d / 2), scg + (size_t)i * (d / G), j->x + (size_t)b * d, 1, gacc + b, d, G, d);
                    row_dot_sel(pku + (size_t)i * (d / 2), scu + (size_t)i * (d / G), j->x + (size_t)b * d, 1, uacc + b, d, G, d);
                }
            }
            for (int t = 0; t < nt; t++) {
                const int b = tok[t];
                const float g = gacc[b], u = uacc[b];
                acte[(size_t)b * m + i] = (g / (1.0f + jmo_expf_fast(-g))) * u;
            }
        }
        for (int i = 0; i < d; i++) {
            if (j->all_tokens) {
                row_dot_sel(pkd + (size_t)i * (m / 2), scd + (size_t)i * (m / G), acte, B, dacc, m, G, m);
            } else {
                for (int t = 0; t < nt; t++) {
                    const int b = tok[t];
                    row_dot_sel(pkd + (size_t)i * (m / 2), scd + (size_t)i * (m / G), acte + (size_t)b * m, 1, dacc + b, m, G, m);
                }
            }
            for (int s = s0; s < s1; s++) {
                const int b = j->uidx[s] / p->topk;
                ye[(size_t)b * d + i] = fmaf(j->uw[s], dacc[b], ye[(size_t)b * d + i]);
            }
        }
    }
    free(tok);
    free(gacc);
}

/*
 * layer_ffn_batch (decode_kernel.c:1387-1508) for one layer.
 *   x [B][d] -> out [B][d]; top/tw [B][topk] receive the router result.
 * n_threads is the number of participants (1 = inline, as the reference does
 * at B == 1; the reference runs 8 workers + the caller at B > 1).
 * Returns 0 on success, a negative code on invalid shapes or allocation.
 */
JMO_API int jmo_layer_ffn_batch(const jmo_moe* p, const float* x, int B, float* out,
                                int32_t* top, float* tw, int n_threads, int all_tokens) {
    if (!p || B < 0 || p->d <= 0 || p->m <= 0 || p->E <= 0 || p->topk <= 0 ||
        p->topk > p->E || (p->group != 32 && p->group != 64) || p->d % p->group ||
        p->m % p->group)
        return -1;
    if (B == 0) return 0;
    const int d = p->d, m = p->m, E = p->E, k = p->topk;
    const int nslot = B * k;
    const int umax = nslot < E ? nslot : E;
    float* scores = (float*)malloc(sizeof(float) * (size_t)B * E);
    int* sel = (int*)malloc(sizeof(int) * (size_t)(umax + 1));
    int* uh = (int*)malloc(sizeof(int) * (size_t)(umax + 1));
    int* cnt = (int*)calloc((size_t)(umax + 1), sizeof(int));
    int* pos = (int*)malloc(sizeof(int) * (size_t)(umax + 1));
    int* uidx = (int*)malloc(sizeof(int) * (size_t)nslot);
    float* uw = (float*)malloc(sizeof(float) * (size_t)nslot);
    int* slot_u = (int*)malloc(sizeof(int) * (size_t)nslot);
    float* act = (float*)calloc((size_t)umax * B * m, sizeof(float));
    float* y = (float*)calloc((size_t)umax * B * d, sizeof(float));
    if (!scores || !sel || !uh || !cnt || !pos || !uidx || !uw || !slot_u || !act || !y) {
        free(scores); free(sel); free(uh); free(cnt); free(pos); free(uidx); free(uw);
        free(slot_u); free(act); free(y);
        return -2;
    }
    const int workers = n_threads > 1 ? n_threads - 1 : 0;
    if (B > 1 && !jmo_pool_init(workers)) {
        free(scores); free(sel); free(uh); free(cnt); free(pos); free(uidx); free(uw);
        free(slot_u); free(act); free(y);
        return -3;
    }

    jmo_job job = {p, x, B, scores, sel, uh, uidx, uw, act, y, all_tokens};
    /* router scores: inline at B <= 1, pooled over experts otherwise */
    if (B <= 1) router_worker(&job, 0, 0, E);
    else pool_run(router_worker, &job, 0, E);
    for (int b = 0; b < B; b++)
        jmo_softmax_topk(scores + (size_t)b * E, E, k, p->renorm, top + (size_t)b * k, tw + (size_t)b * k);

    /* union of selected experts in first-appearance order over (b, i);
     * a slot whose index is -1 (NaN scores) joins no expert */
    int U = 0;
    for (int s = 0; s < nslot; s++) {
        const int e = top[s];
        int u = 0;
        while (u < U && sel[u] != e) u++;
        if (e < 0) { slot_u[s] = -1; continue; }
        if (u == U) sel[U++] = e;
        slot_u[s] = u;
        cnt[u]++;
    }
    int acc = 0;
    for (int u = 0; u < U; u++) { uh[u] = acc; pos[u] = acc; acc += cnt[u]; }
    uh[U] = acc;
    for (int s = 0; s < nslot; s++) {
        const int u = slot_u[s];
        if (u < 0) continue;
        uidx[pos[u]] = s;
        uw[pos[u]] = tw[s];
        pos[u]++;
    }

    if (B == 1) expert_worker(&job, 0, 0, U);
    else pool_run(expert_worker, &job, 0, U);

    /* combine in union order, starting from +0 */
    for (size_t i = 0; i < (size_t)B * d; i++) out[i] = 0.0f;
    for (int u = 0; u < U; u++) {
        const float* ye = y + (size_t)u * B * d;
        for (size_t i = 0; i < (size_t)B * d; i++) out[i] = out[i] + ye[i];
    }
    free(scores); free(sel); free(uh); free(cnt); free(pos); free(uidx); free(uw);
    free(slot_u); free(act); free(y);
    return 0;
}
