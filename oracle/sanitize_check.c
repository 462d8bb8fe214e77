/*
 * sanitize_check.c -- drives every entry point of the C restatement
 * (moe_oracle.c) for the sanitizer builds of oracle/Makefile:
 *
 *   make -C oracle sanitize     AddressSanitizer + UndefinedBehaviorSanitizer
 *                               build of moe_oracle.c with this driver, run;
 *                               then a ThreadSanitizer build, run
 *
 * TEST INFRASTRUCTURE ONLY, like moe_oracle.c.  The driver builds a small
 * random Q4 layer (packed nibbles, fp16 scales of moderate size) and calls
 * the conversions, the router, the softmax/top-k, the Q4 row dots and GEMMs,
 * expert_job, the dequantisation and the whole MoE block at B = 0, 1, 8 and
 * 16 with 1, 3 and 9 participants of the spin pool (so the pool is started,
 * resized and shut down), checking that results do not depend on the
 * thread count.  Exit status 0 when every check passes; a sanitizer report
 * makes it fail (-fno-sanitize-recover).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    int d, m, E, topk, renorm, group;
    const float* gate_w;
    const uint8_t* const* pk;
    const uint16_t* const* sc;
} jmo_moe;

float jmo_fp16_to_f32(uint16_t h);
float jmo_bf16_to_f32(uint16_t h);
void jmo_fp16_to_f32_array(const uint16_t* in, float* out, int64_t n);
void jmo_bf16_to_f32_array(const uint16_t* in, float* out, int64_t n);
float jmo_expf_fast(float v);
void jmo_expf_fast_array(const float* in, float* out, int64_t n);
float jmo_router_dot(const float* w, const float* x, int d);
void jmo_router_logits(const float* w, const float* x, int B, int E, int d, float* out);
void jmo_q4_row_dot_B(const uint8_t* row, const uint16_t* sc, const float* x, int B, float* acc,
                      int cols, int group, int stride);
void jmo_q4_gemv_ffn(float* out, const float* x, const uint8_t* packed, const uint16_t* scales,
                     int m, int d, int group);
void jmo_q4_gemm_ffn(float* out, const float* X, int T, const uint8_t* packed, const uint16_t* scales,
                     int m, int d, int group);
void jmo_q4_gemv_scalar(float* out, const float* x, const uint8_t* packed, const uint16_t* scales,
                        int m, int d, int group);
void jmo_expert_job(const uint8_t* pk_g, const uint16_t* sc_g, const uint8_t* pk_u, const uint16_t* sc_u,
                    const uint8_t* pk_d, const uint16_t* sc_d, int m, int d, int group, const float* x,
                    float* scratch, float prob);
void jmo_q4_dequant(float* out, const uint8_t* packed, const uint16_t* scales, int64_t numel, int group);
void jmo_softmax_topk(float* probs, int E, int topk, int renorm, int32_t* top, float* tw);
void jmo_set_simd(int on);
int jmo_pool_init(int n_workers);
void jmo_pool_shutdown(void);
int jmo_layer_ffn_batch(const jmo_moe* p, const float* x, int B, float* out, int32_t* top, float* tw,
                        int n_threads, int all_tokens);

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint32_t rnd(void) {
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return (uint32_t)(rng_state >> 11);
}
static float unif(void) { return (float)(rnd() & 0xFFFFFF) / 16777216.0f * 2.0f - 1.0f; }

static int fails = 0;
#define CHECK(c, ...) do { if (!(c)) { fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
    fprintf(stderr, __VA_ARGS__); fputc('\n', stderr); fails++; } } while (0)

int main(void) {
    const int d = 256, m = 128, E = 16, k = 4, G = 64;
    /* conversions over every code */
    uint16_t* codes = malloc(65536 * sizeof(uint16_t));
    float* conv = malloc(65536 * sizeof(float));
    for (int i = 0; i < 65536; i++) codes[i] = (uint16_t)i;
    jmo_fp16_to_f32_array(codes, conv, 65536);
    CHECK(conv[0x3C00] == 1.0f && jmo_fp16_to_f32(0xC000) == -2.0f, "fp16");
    jmo_bf16_to_f32_array(codes, conv, 65536);
    CHECK(conv[0x3F80] == 1.0f && jmo_bf16_to_f32(0x4000) == 2.0f, "bf16");
    float ev[5] = {0.0f, -20.0f, 100.0f, NAN, -1.5f}, eo[5];
    jmo_expf_fast_array(ev, eo, 5);
    CHECK(eo[0] == 1.0f && eo[1] == 0.0f && eo[3] == 0.0f && isfinite(eo[2]), "expf_fast");
    CHECK(jmo_expf_fast(-1.5f) == eo[4], "expf_fast scalar");

    /* one random layer: [E][3] records of (scales, packed) */
    const size_t gu_pk = (size_t)m * d / 2, gu_sc = (size_t)m * d / G;
    const size_t dn_pk = (size_t)d * m / 2, dn_sc = (size_t)d * m / G;
    uint8_t** pk = malloc(3 * E * sizeof(uint8_t*));
    uint16_t** sc = malloc(3 * E * sizeof(uint16_t*));
    for (int p = 0; p < 3; p++)
        for (int e = 0; e < E; e++) {
            const size_t np = p < 2 ? gu_pk : dn_pk, ns = p < 2 ? gu_sc : dn_sc;
            uint8_t* a = malloc(np);
            uint16_t* s = malloc(ns * 2);
            for (size_t i = 0; i < np; i++) a[i] = (uint8_t)rnd();
            for (size_t i = 0; i < ns; i++) s[i] = (uint16_t)(0x2000 + (rnd() & 0x3FF));   /* ~2^-7 */
            pk[p * E + e] = a;
            sc[p * E + e] = s;
        }
    float* gate_w = malloc(sizeof(float) * E * d);
    for (int i = 0; i < E * d; i++) gate_w[i] = unif() * 0.05f;
    const int BMAX = 16;
    float* x = malloc(sizeof(float) * BMAX * d);
    for (int i = 0; i < BMAX * d; i++) x[i] = unif() * 2.0f;

    /* router, softmax/top-k */
    float* lg = malloc(sizeof(float) * BMAX * E);
    jmo_router_logits(gate_w, x, BMAX, E, d, lg);
    CHECK(lg[E + 3] == jmo_router_dot(gate_w + 3 * d, x + d, d), "router_logits vs router_dot");
    int32_t top[16];
    float tw[16], probs[16];
    memcpy(probs, lg, sizeof probs);
    jmo_softmax_topk(probs, E, k, 1, top, tw);
    CHECK(top[0] >= 0 && top[0] < E && fabsf(tw[0] + tw[1] + tw[2] + tw[3] - 1.0f) < 1e-5f, "topk");

    /* Q4 products */
    float* o1 = malloc(sizeof(float) * BMAX * m);
    float* o2 = malloc(sizeof(float) * BMAX * m);
    jmo_q4_gemv_ffn(o1, x, pk[0], sc[0], m, d, G);
    jmo_q4_gemm_ffn(o2, x, BMAX, pk[0], sc[0], m, d, G);
    CHECK(memcmp(o1, o2, sizeof(float) * m) == 0, "gemm row 0 == gemv");
    jmo_q4_gemv_scalar(o2, x, pk[0], sc[0], m, d, G);
    CHECK(fabsf(o1[5] - o2[5]) <= 1e-4f * (fabsf(o1[5]) + 1.0f), "scalar vs ffn gemv");
    float acc[16];
    jmo_q4_row_dot_B(pk[0], sc[0], x, BMAX, acc, d, G, d);
    CHECK(fabsf(acc[0] - o1[0]) <= 1e-4f * (fabsf(o1[0]) + 1.0f), "row_dot_B");
    float* scratch = malloc(sizeof(float) * (m + d));
    jmo_expert_job(pk[0], sc[0], pk[E], sc[E], pk[2 * E], sc[2 * E], m, d, G, x, scratch, 0.25f);
    CHECK(isfinite(scratch[m + 7]), "expert_job");
    float* deq = malloc(sizeof(float) * m * d);
    jmo_q4_dequant(deq, pk[0], sc[0], (int64_t)m * d, G);
    CHECK(deq[1] == (float)((pk[0][0] >> 4) - 8) * jmo_fp16_to_f32(sc[0][0]), "dequant");

    /* the MoE block with 1, 3 and 9 participants; pool started, resized,
     * shut down, restarted */
    jmo_moe p = {d, m, E, k, 1, G, gate_w, (const uint8_t* const*)pk, (const uint16_t* const*)sc};
    float* out = malloc(sizeof(float) * BMAX * d);
    float* ref = malloc(sizeof(float) * BMAX * d);
    int32_t topb[16 * 4], topr[16 * 4];
    float twb[16 * 4], twr[16 * 4];
    CHECK(jmo_layer_ffn_batch(&p, x, 0, out, topb, twb, 3, 0) == 0, "B = 0");
    const int Bs[3] = {1, 8, 16}, th[4] = {1, 3, 9, 3};
    for (int bi = 0; bi < 3; bi++) {
        const int B = Bs[bi];
        CHECK(jmo_layer_ffn_batch(&p, x, B, ref, topr, twr, 1, 0) == 0, "block B=%d", B);
        for (int ti = 0; ti < 4; ti++) {
            for (int all = 0; all < 2; all++) {
                CHECK(jmo_layer_ffn_batch(&p, x, B, out, topb, twb, th[ti], all) == 0, "block");
                CHECK(memcmp(topb, topr, sizeof(int32_t) * B * k) == 0, "top B=%d threads=%d", B, th[ti]);
                CHECK(memcmp(out, ref, sizeof(float) * B * d) == 0, "out B=%d threads=%d all=%d", B, th[ti], all);
            }
        }
        /* the AVX2 form of the same block: the same bits */
        jmo_set_simd(1);
        for (int ti = 0; ti < 4; ti++) {
            for (int all = 0; all < 2; all++) {
                CHECK(jmo_layer_ffn_batch(&p, x, B, out, topb, twb, th[ti], all) == 0, "block");
                CHECK(memcmp(topb, topr, sizeof(int32_t) * B * k) == 0, "avx2 top B=%d threads=%d", B, th[ti]);
                CHECK(memcmp(out, ref, sizeof(float) * B * d) == 0, "avx2 out B=%d threads=%d all=%d", B, th[ti], all);
            }
        }
        jmo_set_simd(0);
        if (bi == 1) jmo_pool_shutdown();
    }
    jmo_pool_shutdown();
    for (int i = 0; i < 3 * E; i++) { free(pk[i]); free(sc[i]); }
    free(pk); free(sc); free(gate_w); free(x); free(lg); free(o1); free(o2); free(scratch);
    free(deq); free(out); free(ref); free(codes); free(conv);
    if (fails) {
        fprintf(stderr, "%d checks failed\n", fails);
        return 1;
    }
    printf("sanitize_check: all checks passed\n");
    return 0;
}
