// Internal launch interface between the C ABI (jm_api.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jm_device.h"

// Signed base-16 digits per activation value in the Q4 dot (see jm_device.h).
// base-16 digit planes per activation value on the GEMV kernels: 4 by
// default (15-bit block integers), 5 on request (jm_store_set_act_digits:
// 19-bit); the workspace holds JM_NDIG_MAX
#define JM_NDIG_MAX 5
#ifndef JM_NDIG
#define JM_NDIG 4
#endif

// Limits of the kernels: experts per layer (top-k keeps E/64 values per lane,
// dispatch keeps per-expert counts in LDS) and slots (B*topk) per call.
#define JM_MAX_E 512
#define JM_MAX_SLOTS 65535       // the dispatch keeps slot indices in 16 bits
#define JM_MAX_TOPK 32
// Calls with B*topk up to this many slots take the decode path: three
// launches, the experts' slots found by ballots over the top-k table and the
// combine done in the down kernel.  Larger calls take the dispatch path.
#define JM_DEC_SLOTS 256
// Dispatch path: experts with at least dense_min slots take the MFMA branch,
// in tiles of this many tokens.  Its int8 operands (weights q - 8, and the
// activations' two digits) store each run of 8 columns in the order
// i8_pos gives (jm_device.h): the even columns, then the odd ones.
#define JM_DENSE_TILE 32
#define JM_DENSE_MIN_DEFAULT 8

namespace jm {

struct ExpertArgs {
    const uint8_t* blob;      // HBM copy of experts_q4.bin
    RecLoc rec;               // record offsets within blob
    long long key0;           // layer * E
    int E;
    // dispatch path: the work table and its segments
    const ExpertWork* work;   // [umax] per active expert: segment + record offsets
    int umax;                 // work table entries
    const int* seg_slot;      // [B*k] slot ids (b*k+i) grouped by expert, stable
    // decode path: the top-k table
    const int* top;           // [B*k] expert of each slot (-1: none)
    int nslot;                // B*k
    int B;
    int d, m, topk;
    const float* tw;          // [B*k] routing weight of each slot
    const int8_t* xqh;        // [B][d] tokens as int8 digit pairs (hi, lo) in int8 operand order (MFMA branch)
    const int8_t* xql;
    const float* xqs;         // [B][d/G] their scales
    const int* xqc;           // [B][d/G] sums of their integers 256 h + l per group
    const uint32_t* xdig;     // [B][d/G][NDIG][G/8] token digits
    const float* xscale;      // [B][d/G]
    float* act;               // [B*k][m]   SiLU(gate)*up per slot
    uint32_t* adig;           // [B*k][m/32][NDIG][4] act digits, 32 values per group (word j: values 8j..8j+7)
    float* ascale;            // [B*k][m/32]
    float* y;                 // [B*k][d]   weighted expert output per slot (dispatch path)
    float* out;               // [B][d]     block output
    const float* resid;       // [B][d]     added to the block output (NULL: none); may alias out
    int group;
    // dispatch path, dense branch
    int dense_min;            // experts with at least this many slots take the MFMA kernels
    const int2* tiles;        // [max tiles] (work entry, token tile) of the dense experts
    const int* n_tiles;       // [2] how many tiles; how many experts under dense_min (small)
    const int* small;         // [umax] work-table entries of the experts with 1..dense_min-1 slots
    int8_t* aqh;              // [B*k][m] act as int8 digit pairs for the MFMA down
    int8_t* aql;
    float* aqs;               // [B*k][m/G] their scales
    int* aqc;                 // [B*k][m/G] sums of their integers per group
    // decode path with the top-k in the gate/up kernel (gateup_topk): the
    // router scores, and where the table is written
    const float* logits;      // [B][E]
    int renorm;
    int* top_w;               // [B*k] (the same memory as top)
    float* tw_w;              // [B*k] (the same memory as tw)
    int ndig;                 // digit planes of xdig and adig (4 or 5)
};

// Routing front: router scores, top-k, x digits and (dispatch path) the
// dispatch and work table.
struct RouteArgs {
    const void* wt;           // interleaved router copy of the layer
    int wt_bf16;              // 1: wt holds bf16 bits, 0: float32
    const float* x;           // [B][d]
    const float* xpart;       // [nxpart][B][d] slices added to x first (NULL: none)
    int nxpart;
    float* xmid;              // [B][d] receives x + the slices (NULL: not kept)
    const uint16_t* norm_w;   // [d] bf16 RMSNorm weight applied to x first (NULL: x as given)
    float eps;
    int B, E, d, topk, renorm, group;
    float* logits;            // [B][E]
    uint32_t* xdig;           // [B][d/G][NDIG][G/8]
    float* xscale;            // [B][d/G]
    int8_t* xqh;              // [B][d] tokens as int8 digit pairs for the MFMA branch (NULL: not needed)
    int8_t* xql;
    float* xqs;               // [B][d/G] their scales
    int* xqc;                 // [B][d/G] sums of their integers per group
    int* top;                 // [B*k]
    float* tw;                // [B*k]
    int* seg_off;             // [E+1]
    int* seg_slot;            // [B*k]
    int* active;              // [E]
    int* n_active;            // [1]
    int* first_slot;          // [E]
    int* comb;                // [B*k] each token's slots in union order, -1 padded
    ExpertWork* work;         // [umax] expert work table
    int umax;                 // min(E, B*k)
    RecLoc rec;               // store record offsets
    long long key0;           // layer*E
    int dense_min;            // dispatch path: slots from which an expert takes the MFMA kernels
    int2* tiles;              // dense tiles (work entry, token tile), in work-table order
    int* n_tiles;             // [2] dense tiles; experts under dense_min
    int* small;               // [umax] work-table entries of the experts under dense_min
    int skip_topk;            // 1: the top-k runs in the gate/up kernel
    int ndig;                 // digit planes the router writes to xdig (4 or 5)
    int enc_late;             // 1: the dispatch launch encodes the tokens, not the router (k_router_quad only)
    float* xn;                // [B][d] the router's staged tokens, for that encode (NULL: not written)
    const float* xenc;        // [B][d] the tokens that encode reads (x, or xn)
};
// from this many tokens the router serves 4 tokens per block from one read
// of each group's table (k_router_quad), and on the dispatch path the
// dispatch launch encodes the tokens.  Measured crossover of the Qwen3
// block: below it one wave per (group, token) with its own encode is
// 1.1 us faster at 64 tokens and about even at 128; from 192 tokens the
// 4-token form is 3 us faster (10 us at 512).
#ifndef JM_ROUTER_QUAD_MIN_B
#define JM_ROUTER_QUAD_MIN_B 144
#endif
// router scores + x digits (one wave per expert group and token), then the
// top-k of every token (unless skip_topk)
hipError_t launch_route_tok(const RouteArgs& a, hipStream_t st);
// dispatch + work table from a.top (dispatch path); with enc_late, also the
// tokens' digits from a.xenc, on the launch's blocks past the first
hipError_t launch_dispatch_work(const RouteArgs& a, hipStream_t st);
// experts per layer in the router copy: E rounded up to whole groups of 8
__host__ __device__ constexpr int router_experts_padded(int E) { return (E + 7) / 8 * 8; }
hipError_t launch_router_transpose(const void* in, int in_bf16, void* out, int out_bf16, long long rows,
                                   int E, int d, hipStream_t st);
hipError_t launch_bf16_exact(const float* in, long long n, unsigned* flag, hipStream_t st);

hipError_t launch_router(const void* gate_w, int bf16, const float* x, float* logits,
                         int B, int E, int d, hipStream_t st);
hipError_t launch_prep_digits(const float* src, int stride, int rows, int cols, int group,
                              uint32_t* dig, float* scale, hipStream_t st, int ndig = JM_NDIG);
hipError_t launch_topk(const float* logits, int B, int E, int k, int renorm, int* top, float* tw,
                       hipStream_t st);
// E <= JM_MAX_E, nslot <= JM_MAX_SLOTS
hipError_t launch_dispatch(const int* top, int nslot, int E, int k, int* seg_off, int* seg_slot,
                           int* active, int* n_active, int* first_slot, int* comb, hipStream_t st);
// decode path (nslot <= JM_DEC_SLOTS): gate/up over ballot-found slots, then
// down + combine into a.out.  For gateup_topk(B, E) the gate/up kernel
// computes the top-k itself (from a.logits; no top-k launch before it).
#ifndef JM_GU_TOPK_MAX_B
#define JM_GU_TOPK_MAX_B 4
#endif
bool gateup_topk(int B, int E);
hipError_t launch_gateup_dec(const ExpertArgs& a, hipStream_t st);
hipError_t launch_down_comb(const ExpertArgs& a, hipStream_t st);
// dispatch path: gate/up and down over the work table, then the combine
hipError_t launch_gateup(const ExpertArgs& a, int umax, hipStream_t st);
hipError_t launch_down(const ExpertArgs& a, int umax, hipStream_t st);
// dense branch: 1-D grids of (max_tiles + 1) x (row blocks); the blocks past
// n_tiles[0] x (row blocks) run the wave items of the n_tiles[1] experts under
// dense_min (the small list), so no other launch is needed for them.
// mfma_shape_ok: d and the intermediate multiples of 256, up to 2048, and at
// most 1024 or a multiple of 1024 (the tile's token digits stay in LDS one
// 1024-column phase at a time); otherwise the GEMV kernels take every expert
bool mfma_shape_ok(int d, int m);
hipError_t launch_gateup_mfma(const ExpertArgs& a, int max_tiles, hipStream_t st);
hipError_t launch_down_mfma(const ExpertArgs& a, int max_tiles, hipStream_t st);
// The plain Q4 product out[T][m] = X . dequant(W)^T on the matrix cores:
// m a multiple of 256, d as the MFMA contraction, group 32 or 64 with each
// row's scales a multiple of 16 (G = 32) or 8 bytes (G = 64); ws holds
// q4_gemm_mfma_ws bytes
bool q4_gemm_mfma_ok(int m, int d, int group);
// default token count from which jm_q4_gemm_f32 takes the matrix cores
// (jm_set_q4_gemm_min_tokens changes it): the measured crossover
#ifndef JM_Q4_GEMM_MIN_T
#define JM_Q4_GEMM_MIN_T 7
#endif
// K splits the product takes at this shape (1: none); their partial sums
// are part of the workspace
int q4_gemm_splits(int T, int m, int d);
size_t q4_gemm_mfma_ws(int T, int m, int d, int group);
hipError_t launch_q4_gemm_mfma(const uint8_t* packed, const uint16_t* scales, const float* X, int T, int m, int d,
                               int group, void* ws, float* out, hipStream_t st);
// out[b] = (resid[b] +) sum of the token's slots of y in the order comb gives
hipError_t launch_combine(const float* y, const int* comb, int B, int k, int d, const float* resid,
                          float* out, hipStream_t st);
// ---- decoder layer around the MoE block (jm_attn.hip)

// part[s][b][row] = sum over the columns k of column slice s of
// W[row][k] * x[b][k] (* norm_w[k]), rows of up to three stacked bf16
// matrices [rows_i][K]; the consumer sums the K / gemv_slice_cols(K) slices.
struct GemvArgs {
    const float* x;           // [B][K]
    const uint16_t* norm_w;   // [K] bf16 weight multiplied into x, or NULL
    const uint16_t* w[3];     // bf16 [rows[i]][K]
    int rows[3];
    int K, N, B;              // N = rows[0] + rows[1] + rows[2]
    float* part;              // [K / gemv_slice_cols(K)][B][N]
    float* rss;               // [slices][B] receives the sums of x[b][k]^2 over each slice's columns
                              // (the GEMM: one slice of all K), or NULL: not wanted
};
// the decoder's projections take K a multiple of 1024 up to 8192; the
// kernel takes any multiple of its slice width: 512 columns, 1024 from
// K = 4096 when K is a multiple of 1024
bool gemv_shape_ok(int K);
int gemv_slice_cols(int K);
hipError_t launch_gemv_part(const GemvArgs& a, hipStream_t st);
// many tokens (a prefill chunk): the whole sum into part[0] (one slice);
// every row count a multiple of 128, K a multiple of 128
bool gemm_shape_ok(const GemvArgs& a);
// the K slices the GEMM writes for a (1, 2 or 4; the consumer sums them)
int gemm_slices(const GemvArgs& a);
hipError_t launch_gemm_bf16(const GemvArgs& a, hipStream_t st);
// from this many tokens the projections take the GEMM
#define JM_GEMM_MIN_B 33

// Decode attention of one layer for B tokens, head dim 128, H / KH query
// heads per KV head (1, 2, 4 or 8), in splits of 128 positions.
struct AttnArgs {
    const float* qkv;         // [nslice][B][nqkv] slices of the projections of h * norm1 weight:
                              // H q heads, KH k heads, KH v heads
    int nslice;
    int d;                    // width of the layer input h
    const float* rss;         // [nslice][B] sums of h^2 over the slices' columns (the RMSNorm row scale)
    const float* bq;          // [H*128] / [KH*128] biases of the layer, or NULL
    const float* bk;
    const float* bv;
    int nqkv, H, KH, B;
    const uint16_t* qn;       // bf16 q norm weight of the layer, or NULL: [128] per head (qk_norm 1),
                              // [H*128] over the whole vector (qk_norm 2)
    const uint16_t* kn;       // the k norm weight likewise: [128] or [KH*128]
    int qk_norm;              // 0: none, 1: per head, 2: whole vector
    float* qkss;              // qk_norm 2: [B][2] each token's sums of squares of q and of k before the norm
    float eps;
    float rsdiv;              // 1 / the score divisor sqrtf_fast(128)
    const float* cos;         // [maxT][128]
    const float* sin;
    const int* pos;           // [B] position each token writes (T = pos + 1)
    const unsigned long long* kv;   // [B*L][2] k, v caches [maxT][KH][128], bf16 or (kv_f32) float32
    int kv_f32;               // 1: the caches hold float32 (the reference's KVCache), 0: bf16
    int L, layer;
    int append;               // 1: every token has its own cache; the attention appends its k and v
                              // rows itself.  0: k_kv_append appends every row first
    int S;                    // splits the partial buffers hold per (token, KV head)
    float* part_o;            // [B][KH][S][H/KH][128]
    float* part_ml;           // [B][KH][S][H/KH][2]
};
// the projections finished (q out, k and v appended), partial attention,
// then the merge into att [B][H*128]
hipError_t launch_attn(const AttnArgs& a, int qpk, float* att, hipStream_t st);
// lm_head: logits[b][v] = w[v] . x[b] (bf16 rows of d columns), with the
// per-block best row of each token for the argmax.
struct LmArgs {
    const uint16_t* w;        // [V][d] bf16
    const float* x;           // [B][d]
    int V, d, B;
    float* logits;            // [B][V] or NULL
    float* best_v;            // [lm_blocks(V)][B] or NULL (no argmax)
    int* best_i;
};
int lm_blocks(int V);
bool lm_shape_ok(int d);      // d in {1024, 2048, 4096}
// the lm_head, then (out_tok non-NULL) the argmax merge into out_tok [B]
hipError_t launch_lm_head(const LmArgs& a, int* out_tok, hipStream_t st);
hipError_t launch_embed(const uint16_t* embed, int V, int d, const int* tokens, int B, float* out,
                        hipStream_t st);
hipError_t launch_f32_bf16_bits(const float* in, long long n, uint16_t* out, hipStream_t st);
// The dense FFN of one layer (layer_ffn_batch with E == 0): out = resid +
// (silu(x' W1^T) * (x' W2^T)) W3^T, x' = RMSNorm(x) with norm_w (or x).
#ifndef JM_DENSE_MAX_M
#define JM_DENSE_MAX_M 32768
#endif
struct DenseFfn {
    const uint16_t* w1;       // [m][d] bf16 gate rows of the layer
    const uint16_t* w2;       // [m][d] up rows
    const uint16_t* w3;       // [d][m] down rows
    int d, m, B;
    const float* x;           // [B][d]
    const uint16_t* norm_w;   // [d] RMSNorm weight applied to x first, or NULL
    float eps;
    float* rss;               // [d/512][B] the norm's sums of squares (with norm_w)
    float* gu;                // [dense_gu_slices][B][2m] gate and up slices
    float* act;               // [B][m]
    float* dn;                // [dense_dn_slices][B][d] down slices
    const float* resid;       // [B][d] added to the result, or NULL
    float* out;               // [B][d]
};
// d as the projections take it (a multiple of 1024 up to 8192), m a
// multiple of 512 up to JM_DENSE_MAX_M
bool dense_shape_ok(int d, int m);
int dense_gu_slices(int d, int m, int B);
int dense_dn_slices(int d, int m, int B);
hipError_t launch_dense_ffn(const DenseFfn& f, hipStream_t st);
// out [B][n] = resid (or 0) + the ns slices of part [ns][B][n], in order
hipError_t launch_sum_slices(const float* resid, const float* part, int ns, int B, int n, float* out,
                             hipStream_t st);
hipError_t launch_rms_rows(const float* x, const uint16_t* w, int B, int d, float eps, float* out,
                           hipStream_t st);

hipError_t launch_dequant(const uint8_t* packed, const uint16_t* scales, long long numel, int group,
                          float* out, hipStream_t st);
// one expert for one token (expert_job): act = SiLU(g) * u from gu = [g; u],
// then the down output scaled by the routing weight
hipError_t launch_swiglu_vec(const float* gu, int m, float* act, hipStream_t st);
hipError_t launch_scale_vec(float* v, int n, float s, hipStream_t st);
hipError_t launch_q4_rows(const uint8_t* packed, const uint16_t* scales, int rows, int cols, int group,
                          const uint32_t* dig, const float* dscale, int T, float* out, int ostride,
                          hipStream_t st);

}  // namespace jm
