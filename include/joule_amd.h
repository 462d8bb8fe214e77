/*
 * joule_amd.h -- C ABI of the MI355X (gfx950) MoE decode block.
 *
 * Drop-in boundary for the reference's MoE hot path.  Citations are to the
 * reference repository (SatPaingOo/joule):
 *
 *   layer_ffn_batch        src/jouleai/native/decode_kernel.c:1387-1508
 *   KernelCfg              src/jouleai/native/decode_kernel.c:269-286
 *                          (ctypes mirror src/jouleai/native/decoder3.py:35-46)
 *   KernelW expert tables  src/jouleai/native/decode_kernel.c:303, 318-321
 *                          (built by decoder3.py:329-367 _load_experts)
 *   q4_gemv_f32            src/jouleai/native/quant_gemv.c:35, expert_ffn.c:132
 *   q4_gemm_f32            src/jouleai/native/expert_ffn.c:200-215
 *   KernelBackend API      src/jouleai/native/backend.py:45-69
 *
 * Conventions
 *   - Every function returns int: 0 on success, a negative JM_ERR_* code on
 *     failure; jm_last_error() then holds a message (per calling thread).
 *     The reference's functions return void and clamp or ignore bad shapes
 *     (decode_kernel.c:1390, 1522); here bad shapes are errors.
 *   - Tensor pointers are DEVICE pointers (HIP), caller-owned.  The library
 *     allocates only its own workspace and offset table.
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream).
 *     Work is stream-ordered; calls return before the GPU finishes.
 *   - A jm_store is used by one stream at a time (its workspace is shared
 *     by the calls made through it), the per-handle counterpart of the
 *     reference's process-global workspace g_ws (decode_kernel.c:356).
 */
#ifndef JOULE_AMD_H
#define JOULE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JM_ABI_VERSION 1

#define JM_OK 0
#define JM_ERR_ARG (-1)
#define JM_ERR_SHAPE (-2)
#define JM_ERR_HIP (-3)

#define JM_DTYPE_F32 0
#define JM_DTYPE_BF16 1

/* Byte-identical to the reference's KernelCfg (decode_kernel.c:269-286), so
 * a host that already fills one (decoder3.py:95-119) passes it unchanged.
 * Fields read here: L, d, E, topk, intermediate, norm_topk_prob, expert_i8,
 * expert_bf16 (the last two must be 0: the Q4 store). */
typedef struct jm_kernel_cfg {
    int L, d, n_heads, n_kv, hd, E, topk, V;
    float eps;
    int maxT;
    int intermediate;
    int qk_norm_type;
    int bias_qkv;
    int norm_topk_prob;
    int expert_i8;
    int expert_bf16;
} jm_kernel_cfg;

typedef struct jm_store jm_store;

/* ABI version (JM_ABI_VERSION) and the last error message of this thread. */
int jm_version(void);
const char* jm_last_error(void);

/* sizeof(jm_kernel_cfg) and the compile-time kernel parameters: digits per
 * activation value in the Q4 dot, and rows per gate/up work item (the
 * number of act values that share one digit scale). */
int jm_abi_sizes(int* kernel_cfg_bytes, int* ndig, int* nt);

/*
 * HBM-resident expert store.  Replaces the KernelW expert pointer tables
 * expert_pk[3][L*E] / expert_sc[3][L*E] (decode_kernel.c:318-321) that
 * _load_experts (decoder3.py:329-367) builds over an mmap of experts_q4.bin.
 *   blob     device copy of experts_q4.bin, byte for byte (16-byte aligned)
 *   offsets  host uint64 [3][L*E][2]: for part p in (gate, up, down) and
 *            key l*E+e, the byte offsets of the scales and of the packed
 *            nibbles of that record within blob (the index's offset and
 *            offset + scales_bytes)
 *   group    Q4 group size, 64 (the reference store) or 32
 * Checks that every record lies inside the blob.  The blob stays owned by
 * the caller and must outlive the store.  With cfg->E == 0 it makes a dense
 * store instead (no experts; see jm_store_set_dense_ffn).
 */
int jm_store_create(const jm_kernel_cfg* cfg, int group, const void* blob, uint64_t blob_bytes,
                    const uint64_t* offsets, jm_store** out);
int jm_store_destroy(jm_store* s);

/* Router weights, the reference's KernelW.gate_w [L][E][d]
 * (decode_kernel.c:303).  dtype JM_DTYPE_BF16 takes the reference's bf16
 * table as is; JM_DTYPE_F32 takes float32.  The store keeps its own copy,
 * in bf16 when every weight is exactly a bf16 value and in float32
 * otherwise, with the 8 FMA chains of 8 experts interleaved for coalesced
 * loads; the caller's table may be freed after the call.  Synchronises the
 * device. */
int jm_store_set_router(jm_store* s, const void* gate_w, int dtype);

/* The element type the store's router copy holds: JM_DTYPE_BF16 when every
 * weight is exactly a bf16 value (always for a bf16 table), else
 * JM_DTYPE_F32.  Each call reads E*d elements of it. */
int jm_store_router_dtype(const jm_store* s, int* dtype);

/* Size the workspace for batches of up to max_B tokens now, so that later
 * calls with B <= max_B allocate nothing. */
int jm_store_reserve(jm_store* s, int max_B);

int jm_store_info(const jm_store* s, int* L, int* E, int* d, int* m, int* topk, int* group);

/* Batches with B * topk > 256 slots: an expert routed at least min_tokens
 * slots takes the MFMA branch (32-token tiles on the int8 matrix cores:
 * weights q - 8 against each activation's two int8 digits), the others the
 * wave-item GEMV kernels.  0 restores the default (8); a value above
 * B * topk keeps every expert on the GEMV kernels.  No counterpart in the
 * reference, whose batch is at most 16 tokens (decode_kernel.c:1522). */
int jm_store_set_dense_min(jm_store* s, int min_tokens);

/* Base-16 digit planes per activation value on the GEMV (wave-item)
 * kernels: each Q4 group of x, and each 32-value chunk of the SwiGLU act, is
 * carried as block integers of ndig signed digits under one scale (the
 * group's largest magnitude / R, R = 30583 for 4 digits, 489335 for 5).  4
 * (the default; 0 restores it) keeps about 15 bits per group, 5 about 19 bits
 * at more dot products per row.  Router indices and weights do not depend on
 * it.  The MFMA branch's int8 digit pairs are not affected.  No counterpart in
 * the reference, whose activations are float32. */
int jm_store_set_act_digits(jm_store* s, int ndig);
/* The store's digit planes (4 or 5), -1 for a NULL store. */
int jm_store_act_digits(const jm_store* s);

/*
 * The MoE block of one layer: layer_ffn_batch(cfg, W, l, x, B, out)
 * (decode_kernel.c:1387-1508), for any B >= 0 (the reference clamps B to 16
 * at decode_kernel.c:1522).
 *   x        [B][d] float32, out [B][d] float32 (16-byte aligned)
 *   topk_idx optional [B][topk] int32 receives the selected experts
 *   topk_w   optional [B][topk] float32 receives their routing weights
 * Router indices and weights are bit-identical to the reference arithmetic.
 */
int jm_layer_ffn_batch(jm_store* s, int layer, const float* x, int B, float* out,
                       int32_t* topk_idx, float* topk_w, void* stream);

/* jm_layer_ffn_batch for callers that cannot allocate device memory: code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  No counterpart in the reference.  The same kernels and
 * results as jm_layer_ffn_batch, with the workspace in a fixed array of
 * JM_NOALLOC_SCRATCH_BYTES on each device (reserved when the library first
 * creates a store on that device, kept until the process ends) instead of
 * the store's own: the call allocates nothing and fails with JM_ERR_SHAPE
 * when B tokens of the store's shape need more workspace than the array
 * holds (about 140 KB per token for the Qwen3-30B-A3B block: up to ~110
 * tokens).  Every call on a device shares that device's array: calls that
 * overlap on one GPU (other streams, other stores, other threads) race and
 * must be serialised by the caller.  jm_store_copy_workspace does not see
 * this workspace. */
#define JM_NOALLOC_SCRATCH_BYTES (16u << 20)
int jm_layer_ffn_batch_noalloc(jm_store* s, int layer, const float* x, int B, float* out,
                               int32_t* topk_idx, float* topk_w, void* stream);

/* Per-stage timing.  With profiling on, jm_layer_ffn_batch records a HIP
 * event around each of its JM_STAGES stages (route: router scores, top-k and
 * x digits, plus the dispatch when B * topk > 256; gate/up; down with the
 * combine); jm_store_stage_ms waits for the last call and returns the
 * elapsed milliseconds of each stage. */
#define JM_STAGES 3
int jm_store_profile(jm_store* s, int enable);
int jm_store_stage_ms(jm_store* s, float* ms, int n);

/* Copy an intermediate of the last jm_layer_ffn_batch call out of the
 * store's workspace into caller device memory (stream-ordered), for tests and
 * profiling.  `bytes` must not exceed the field's size at the last call's B.
 * Calls with B * topk <= 256 write only JM_WS_LOGITS and JM_WS_ACT (their
 * dispatch is a ballot inside the expert kernels and their combine runs in
 * the down kernel); the other fields are then an error:
 *   JM_WS_LOGITS     float [B][E] router scores
 *   JM_WS_SEG_OFF    int32 [E+1] segment starts (slots grouped by expert)
 *   JM_WS_SEG_SLOT   int32 [B*topk] slot ids b*topk+i grouped by expert
 *   JM_WS_ACTIVE     int32 [E] expert ids with tokens, ascending
 *   JM_WS_N_ACTIVE   int32 [1] how many of them
 *   JM_WS_FIRST_SLOT int32 [E] first slot of each active expert
 *   JM_WS_ACT        float [B*topk][intermediate] SiLU(gate)*up per slot
 *   JM_WS_Y          float [B*topk][d] weighted expert output per slot
 *   JM_WS_N_DENSE_TILES int32 [1] 32-token tiles the MFMA branch computed */
#define JM_WS_LOGITS 0
#define JM_WS_SEG_OFF 1
#define JM_WS_SEG_SLOT 2
#define JM_WS_ACTIVE 3
#define JM_WS_N_ACTIVE 4
#define JM_WS_FIRST_SLOT 5
#define JM_WS_ACT 6
#define JM_WS_Y 7
#define JM_WS_N_DENSE_TILES 8
int jm_store_copy_workspace(const jm_store* s, int field, void* dst, uint64_t bytes, void* stream);

/* ---- batch decode over all layers (decode_layers_batch) ---- */

/* One sequence's cache of one layer, the reference's KVCache
 * (decode_kernel.c:328-331): k and v [maxT][n_kv][hd] in device memory,
 * bfloat16 by default; float32, the reference's own type, after
 * jm_store_set_kv_dtype(store, JM_DTYPE_F32). */
typedef struct jm_kv_cache {
    void* k;
    void* v;
} jm_kv_cache;

/* The reference's KernelW (decode_kernel.c:288-325; ctypes mirror
 * decoder3.py:49-69) field for field, with device pointers.  Read here:
 * final_norm, norm1, norm2 [L][d], wq [L][H*hd][d], wk/wv [L][KH*hd][d],
 * wo [L][d][H*hd] (all bf16), bq/bk/bv (float32, when bias_qkv), qn/kn
 * (bf16: [L][hd] when qk_norm_type = 1, [L][H*hd] / [L][KH*hd] when it is 2),
 * cos/sin [maxT][hd] (float32).
 * gate_w and the expert tables are the store's (jm_store_set_router, the
 * blob); embed and lm_head are not read by jm_decode_layers_batch; w1/w2/w3
 * are the dense FFN's (bf16 [L][m][d], [L][m][d], [L][d][m]), set for a
 * dense store (E = 0) and NULL for an expert store; the int8 fields must be
 * NULL and use_i8 0. */
typedef struct jm_kernel_w {
    const uint16_t* embed;
    const void* lm_head;
    const uint16_t* final_norm;
    const uint16_t* norm1;
    const uint16_t* norm2;
    const uint16_t* wq;
    const uint16_t* wk;
    const uint16_t* wv;
    const uint16_t* wo;
    const float* bq;
    const float* bk;
    const float* bv;
    const uint16_t* qn;
    const uint16_t* kn;
    const uint16_t* gate_w;
    const uint16_t* w1;
    const uint16_t* w2;
    const uint16_t* w3;
    const uint8_t* wq_i8;
    const float* wq_i8s;
    const uint8_t* wk_i8;
    const float* wk_i8s;
    const uint8_t* wv_i8;
    const float* wv_i8s;
    const uint8_t* wo_i8;
    const float* wo_i8s;
    const uint8_t* lm_i8;
    const float* lm_i8s;
    const uint8_t* const* expert_pk[3];
    const uint16_t* const* expert_sc[3];
    const float* cos;
    const float* sin;
    int use_i8;
} jm_kernel_w;

/*
 * decode_layers_batch(cfg, W, kv, positions, xin, B, logits)
 * (decode_kernel.c:1518-1556) over the store's layers: per layer RMSNorm,
 * attention (QKV, per-head QK-norm, RoPE, KV append at positions[b], SDPA,
 * o_proj) and residual, RMSNorm, the store's MoE block and residual; then
 * the final RMSNorm into hidden [B][d] float32, and the lm_head into logits.
 *   cfg        L, d, E, topk, intermediate, norm_topk_prob as the store's;
 *              n_heads, n_kv (n_heads / n_kv in 1, 2, 4, 8), hd = 128, eps,
 *              maxT, qk_norm_type (0: none, 1: per head, 2: whole
 *              vector, :1155-1189), bias_qkv
 *   kv         HOST array of B * L caches, entry b * L + l (as the reference)
 *   positions  HOST int32 [B]: the cache row each token writes; attention
 *              covers rows 0 .. positions[b] (the others must be filled)
 *   xin        [B][d] float32 (device)
 *   logits     optional [B][V] float32 (device): lm_head(hidden), as
 *              lm_head_B (:964-1000); needs jm_store_set_lm_head
 *   hidden     optional [B][d] float32 (device): the final-normed state
 * Any B >= 0 (the reference clamps B to 16, decode_kernel.c:1522).  With
 * jm_store_profile on, jm_store_decode_ms splits the call's time.
 */
int jm_decode_layers_batch(jm_store* s, const jm_kernel_cfg* cfg, const jm_kernel_w* W, const jm_kv_cache* kv,
                           const int32_t* positions, const float* xin, int B, float* logits, float* hidden,
                           void* stream);

/* decode_layers_batch_argmax (decode_kernel.c:1560-1590): the same step,
 * then out_tok[b] = the row of the largest logit of token b, as lm_head_A
 * (:1008-1062) picks it: a row wins only with a strictly larger value
 * (initial -1e30 at row 0), so ties go to the lowest row and NaN never wins.
 * out_tok is int32 [B] in DEVICE memory (the reference's is host memory);
 * no [B][V] logits are written.  hidden is optional as above. */
int jm_decode_layers_batch_argmax(jm_store* s, const jm_kernel_cfg* cfg, const jm_kernel_w* W, const jm_kv_cache* kv,
                                  const int32_t* positions, const float* xin, int B, int32_t* out_tok,
                                  float* hidden, void* stream);

/* prefill_layers(cfg, W, kv, tokens, T, logits) (decode_kernel.c:1606-1615):
 * a prompt of T tokens through every layer.  The reference runs
 * decode_layers_batch once per position; here all T positions go through
 * each layer together, as one batch whose token t sits at position t (the
 * attention of position t covers cache rows 0..t, so the result is the same
 * computation).  Writes cache rows 0..T-1 of the one sequence and, with
 * logits non-NULL, the last position's logits [V] (device).
 *   kv      HOST array of the sequence's L caches (entry l)
 *   tokens  DEVICE int32 [T]; needs W->embed (and the lm_head for logits)
 * T <= cfg->maxT; prompts longer than 512 positions go through in chunks
 * of 512 (each chunk's attention reads the rows the earlier chunks wrote).
 * Runs eagerly (no graph replay). */
int jm_prefill_layers(jm_store* s, const jm_kernel_cfg* cfg, const jm_kernel_w* W, const jm_kv_cache* kv,
                      const int32_t* tokens, int T, float* logits, void* stream);

/* The lm_head, KernelW.lm_head (decode_kernel.c:291; float32 [V][d] in the
 * reference, widened from the checkpoint's bf16 by decoder3.py:226-230).
 * JM_DTYPE_F32 values must be exactly bf16 (an error otherwise);
 * JM_DTYPE_BF16 is taken as is.  The store keeps a bf16 copy [V][d]; d must
 * be 1024, 2048 or 4096.  Synchronises the device. */
int jm_store_set_lm_head(jm_store* s, const void* lm_head, int dtype, int V);

/* The store's lm_head on x [B][d] (device float32): logits [B][V] and/or
 * out_tok [B] (the argmax of jm_decode_layers_batch_argmax); either may be
 * NULL but not both.  The stage entry point of the decode's last step. */
int jm_lm_head(jm_store* s, const float* x, int B, float* logits, int32_t* out_tok, void* stream);

/* embed_lookup (decode_kernel.c:1597-1600) for B tokens: out[b][i] =
 * bf16 embed[tokens[b]][i] (W->embed [V][d], device).  tokens is int32 [B]
 * in DEVICE memory; a token outside [0, V) gives a row of NaN. */
int jm_embed_lookup(const jm_kernel_w* W, const jm_kernel_cfg* cfg, const int32_t* tokens, int B, float* out,
                    void* stream);

/* With enable set, jm_decode_layers_batch records its launches once into a
 * HIP graph and replays it, re-recording when the arguments, the batch size
 * or the number of 128-position attention splits change; calls with
 * profiling on run eagerly.  The KV table and positions are still copied
 * from the host on every call.  Off by default.  No counterpart in the
 * reference. */
int jm_store_decode_graph(jm_store* s, int enable);

/* set_max_layers(n) (decode_kernel.c:1617): later jm_decode_layers_batch,
 * jm_decode_layers_batch_argmax and jm_prefill_layers calls of this store
 * run only layers 0 .. n-1 before the final norm (and lm_head); n < 0 (the
 * default) runs all.  The reference's setting is process-global
 * (g_max_layers); here it is per store. */
int jm_store_set_max_layers(jm_store* s, int n);

/* The element type of the caches (jm_kv_cache) that later
 * jm_decode_layers_batch, jm_decode_layers_batch_argmax and
 * jm_prefill_layers calls of this store read and append to:
 * JM_DTYPE_BF16 (the default: half the bytes per attention read) or
 * JM_DTYPE_F32, the reference's KVCache (decode_kernel.c:328-331), whose
 * appended rows then keep float32 values and whose attention runs in
 * float32 arithmetic throughout. */
int jm_store_set_kv_dtype(jm_store* s, int dtype);

/* A dense model's FFN (layer_ffn_batch with E == 0, decode_kernel.c:
 * 1393-1422): act = silu(x W1^T) * (x W2^T), out = act W3^T with bf16
 * weights shared by the batch.  jm_store_create with cfg->E == 0 (topk 0,
 * blob and offsets NULL) makes a dense store: d a multiple of 1024 up to
 * 8192, intermediate a multiple of 512 up to 32768.  The decoder entry
 * points take the FFN weights from W->w1, w2, w3 ([L][m][d], [L][m][d],
 * [L][d][m], the reference's KernelW fields); jm_layer_ffn_batch on a
 * dense store (with topk_idx and topk_w NULL) uses the ones registered
 * here.  The expert-store entry points (router, stages, workspace copy,
 * the no-allocation block) refuse a dense store. */
int jm_store_set_dense_ffn(jm_store* s, const uint16_t* w1, const uint16_t* w2, const uint16_t* w3);

/* With buf set (device int32, `bytes` long), each later
 * jm_decode_layers_batch also copies every layer's selected experts into
 * buf[l][B][topk], for accounting and tests; NULL turns it off.  No
 * counterpart in the reference. */
int jm_store_trace_topk(jm_store* s, int32_t* buf, uint64_t bytes);

/* Milliseconds of the last profiled jm_decode_layers_batch call: its
 * attention parts (norm1 to the o_proj residual, summed over layers), its
 * MoE blocks (norm2 to the residual) and the whole call (waits for it). */
int jm_store_decode_ms(jm_store* s, float* attn_ms, float* moe_ms, float* total_ms);

/* ---- stage entry points (the steps of layer_ffn_batch, for tests) ---- */

/* Router scores, softmax, top-k and renormalisation
 * (decode_kernel.c:1424-1448): logits [B][E], top [B][topk], tw [B][topk]. */
int jm_router(const void* gate_w, int dtype, const float* x, int B, int E, int d, int topk,
              int renorm, float* logits, int32_t* top, float* tw, void* stream);

/* Token-to-expert dispatch (decode_kernel.c:1449-1485) as a stable counting
 * sort by expert id: seg_off [E+1], seg_slot [nslot], active [E],
 * n_active [1], first_slot [E], and comb [nslot]: each token's slots in the
 * reference's union order (first appearance of their expert), -1 padded. */
int jm_dispatch(const int32_t* top, int nslot, int E, int topk, int32_t* seg_off, int32_t* seg_slot,
                int32_t* active, int32_t* n_active, int32_t* first_slot, int32_t* comb, void* stream);

/* The expert stages of layer_ffn_batch for a given top-k table top [B][topk]
 * (experts outside [0, E) leave their slots' rows untouched), run by the
 * store's wave-item kernels on its workspace; slot = b * topk + i.
 *   jm_expert_gateup: act [B*topk][m] = SwiGLU of the slot's expert's gate
 *     and up rows against x [B][d]: (g / (1 + expf_fast(-g))) * u, the first
 *     half of ffn_expert_worker (decode_kernel.c:1365-1375).
 *   jm_expert_down: y [B*topk][d] = tw[slot] * (down rows . act[slot]), its
 *     second half (:1376-1383).
 *   jm_combine: out [B][d] = each token's y rows summed in the reference's
 *     union order (:1502-1507). */
int jm_expert_gateup(jm_store* s, int layer, const float* x, const int32_t* top, int B, float* act, void* stream);
int jm_expert_down(jm_store* s, int layer, const float* act, const int32_t* top, const float* tw, int B, float* y,
                   void* stream);
int jm_combine(jm_store* s, const float* y, const int32_t* top, int B, float* out, void* stream);

/* Exact dequantisation (q - 8) * float(scale) of one record
 * (q4_store.py:58-67 _dequantize). */
int jm_q4_dequant(float* out, const uint8_t* packed, const uint16_t* scales, int64_t numel, int group,
                  void* stream);

/* ---- the KernelBackend products (backend.py:45-69), device pointers ---- */

/* One expert for one token, the reference's ExpertJob / expert_job
 * (expert_ffn.c:145-191) with the same field order and meaning, on device
 * pointers: scratch[0..m_gg) = act = SiLU(gate . x) * (up . x), then
 * scratch[m_gg..m_gg+d_in) = prob * (down . act).  m_d must equal d_in and
 * d_m must equal m_gg, as in the reference's callers (moe.py:32-42). */
typedef struct jm_expert_job_t {
    const uint8_t* pk_g;
    const uint16_t* sc_g;
    const uint8_t* pk_u;
    const uint16_t* sc_u;
    const uint8_t* pk_d;
    const uint16_t* sc_d;
    int m_gg;
    int d_in;
    int m_d;
    int d_m;
    int group;
    const float* x;
    float* scratch;
    float prob;
} jm_expert_job_t;

int jm_expert_job(const jm_expert_job_t* job, void* stream);

/* out[m] = dequant(W[m][d]) . x[d]; argument order of q4_gemv_f32
 * (quant_gemv.c:35) plus the stream. */
int jm_q4_gemv_f32(float* out, const float* x, const uint8_t* packed, const uint16_t* scales,
                   int m, int d, int group, void* stream);

/* out[T][m] = X[T][d] . dequant(W[m][d])^T; argument order of q4_gemm_f32
 * (expert_ffn.c:201) plus the stream.  From jm_get_q4_gemm_min_tokens()
 * tokens the product runs on the int8 matrix cores (when m, d and group
 * allow it and scales is 16-byte aligned; when its 32-token tiles x 256-row
 * blocks are fewer than 256, the contraction is split over up to 8 blocks
 * and the partial sums are added in split order), below on the v_dot8 digit
 * kernel.  Workspace: one buffer per (device, stream), kept and grown; a
 * call under stream capture takes a stream-ordered allocation instead. */
int jm_q4_gemm_f32(float* out, const float* X, int T, const uint8_t* packed, const uint16_t* scales,
                   int m, int d, int group, void* stream);

/* The token count from which jm_q4_gemm_f32 takes the matrix cores, for the
 * whole process (0 restores the default, the measured crossover of the two
 * kernels).  No counterpart in the reference (a switch between this build's
 * kernels). */
int jm_set_q4_gemm_min_tokens(int tokens);
int jm_get_q4_gemm_min_tokens(void);

#ifdef __cplusplus
}
#endif

#endif /* JOULE_AMD_H */
