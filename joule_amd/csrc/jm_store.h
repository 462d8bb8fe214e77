// The store handle behind the C ABI and the helpers its entry points share
// (jm_api.hip: the MoE block and the stage entry points; jm_decode.hip: the
// batch-decode driver around it).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/joule_amd.h"
#include "jm_kernels.h"

namespace jm {

// The MoE block's workspace for B tokens: one device region, each field
// 256-byte aligned, in this order (ws_layout).
struct Ws {
    float* logits;              // [B][E]
    int* top;                   // [B*k]
    float* tw;                  // [B*k]
    uint32_t* xdig;             // [B][d/G][NDIG][G/8] token digits
    float* xscale;              // [B][d/G]
    int* seg_off;               // [E+1]
    int* seg_slot;              // [B*k]
    int* active;                // [E]
    int* n_active;              // [1]
    int* first_slot;            // [E]
    int* comb;                  // [B*k]
    ExpertWork* work;           // [E]
    int2* tiles;                // [B*k/32 + E] dense tiles (dispatch path)
    int* n_tiles;               // [2] dense tiles, experts under dense_min
    int* small;                 // [E] work-table entries of the experts under dense_min
    float* act;                 // [B*k][m]
    uint32_t* adig;             // [B*k][m/8][NDIG] act digits
    float* ascale;              // [B*k][m/32]
    float* y;                   // [B*k][d]
    int8_t* aqh;                // [B*k][m] act as int8 digit pairs for the MFMA down
    int8_t* aql;
    int8_t* xqh;                // [B][d] tokens as int8 digit pairs for the MFMA gate/up
    int8_t* xql;
    float* xqs;                 // [B][d/G] scales of the token digit pairs
    float* aqs;                 // [B*k][m/G] scales of the act digit pairs
    int* xqc;                   // [B][d/G] sums of the token digit pairs' integers per group
    int* aqc;                   // [B*k][m/G] the same for act
};

}  // namespace jm

// What a captured decode step depends on (the graph bakes in kernel
// arguments): compared bytewise, built from a zeroed struct.
struct DecKey {
    jm_kernel_cfg cfg;
    jm_kernel_w W;
    const float* xin;
    float* hidden;
    float* logits;
    int* out_tok;
    const void* lm;
    int B, S;
    int32_t* trace;
    uint64_t trace_bytes;
    void* ws;
    void* dws;
    void* wt;
    int wt_bf16;                // element type of the router copy: a reallocation may return the same address
    int lm_V;
    int nl;                     // layers the step runs (jm_store_set_max_layers)
    int kv_f32;                 // element type of the caches (jm_store_set_kv_dtype)
    int dense_min;
    int ndig;
    int append;                 // the attention appends the k and v rows itself (no cache shared by two tokens)
};

struct jm_store {
    int L, E, d, m, topk, renorm, group;
    const uint8_t* blob;
    uint64_t blob_bytes;
    uint64_t* off_dev;          // [3][L*E][2]
    jm::RecLoc rec;             // record locator (the table, or the affine formula)
    int dec_last;               // the last call took the decode path
    int n_cu;                   // compute units of the device (persistent grids)
    int lds_max;                // LDS bytes one block may use
    void* wt;                   // [L][Ep/8][d/8/P][64][P] interleaved copy of the router table
    int wt_bf16;                // the copy holds bf16 (the table is exactly bf16-valued)
    int device;
    // workspace, sized for cap_B tokens; last_B = B of the last call
    int cap_B;
    int last_B;
    void* ws;
    jm::Ws w;                   // the fields of ws for cap_B tokens
    // optional per-stage events (jm_store_profile)
    int prof;
    hipEvent_t ev[JM_STAGES + 1];
    int dense_min;              // segment size from which an expert takes the MFMA branch
    int ndig;                   // activation digit planes of the GEMV kernels (jm_store_set_act_digits)
    bool mfma_ok;               // the shape and the records' alignment allow the MFMA branch
    // ---- batch decode (jm_decode_layers_batch) ----
    int max_layers;             // jm_store_set_max_layers: < 0 runs every layer
    int dec_B, dec_S, dec_nqkv, dec_hq, dec_V;   // sizes the decode workspace holds
    uint16_t* lm;               // [V][d] bf16 copy of the lm_head (jm_store_set_lm_head)
    int lm_V;
    void* dws;                  // decode workspace
    float* h;                   // [B][d] residual stream
    float* h2;                  // [B][d] residual stream after attention
    float* qkv;                 // [d/512][B][(H + 2 KH) hd] projection slices
    float* opart;               // [H hd/512][B][d] o_proj slices
    float* part_o;              // [B][KH][S][H/KH][hd] attention partials per position split
    float* part_ml;             // [B][KH][S][H/KH][2] their (max, sum)
    float* att;                 // [B][H hd] attention output
    float* hid;                 // [B][d] final-normed hidden state (when the caller passes none)
    float* xemb;                // [B][d] embedded prompt tokens (jm_prefill_layers)
    float* lmv;                 // [lm blocks][B] per-block best logit (argmax)
    int* lmi;                   // [lm blocks][B] its row
    float* rss;                 // [B] sums of squares of h from the projection GEMM (prefill chunks)
    float* qkss;                // [B][2] sums of squares of q and k (whole-vector QK-norm)
    float* dgu;                 // dense FFN (E = 0): gate/up slices, act, down slices
    float* dact;
    float* ddn;
    const uint16_t* dw[3];      // a dense store's FFN weights for jm_layer_ffn_batch (jm_store_set_dense_ffn)
    int kv_f32;                 // the caches the decoder reads and writes hold float32 (else bf16)
    unsigned long long* tab;    // [B*L][2] KV pointers, then [B] positions (device)
    unsigned long long* tab_host;   // pinned staging of tab
    size_t tab_cap;             // bytes of tab / tab_host
    hipEvent_t tab_ev;          // the last staging copy
    int tab_pending;
    int32_t* trace;             // [L][B][topk] selected experts per layer (jm_store_trace_topk)
    uint64_t trace_bytes;
    // decode step replayed from a captured HIP graph (jm_store_decode_graph)
    int dgraph;
    hipStream_t cap_st;
    hipGraphExec_t gexec;
    DecKey gkey;
    // per-layer attention / MoE split of the last decode call (jm_store_profile)
    int dprof_n;
    hipEvent_t* dev_marks;      // [2 L + 2]
};

namespace jm {

// Record a message for jm_last_error() (per calling thread) and return code.
int fail(int code, const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);

inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// MoE workspace for batches of up to B tokens.
int store_reserve(jm_store* s, int B);
// Bytes of the workspace layout for B tokens of the store's shape, and the
// fields laid out from base (256-byte aligned).
size_t ws_bytes(const jm_store* s, int B);
void ws_layout(const jm_store* s, int B, char* base, Ws* w);

// Decoder-layer extras of the MoE block around its input and output.
struct FfnIo {
    const float* xpart = nullptr;   // [nxpart][B][d] added to x first (the o_proj slices)
    int nxpart = 0;
    float* xmid = nullptr;          // receives x + the slices
    const uint16_t* norm_w = nullptr;   // RMSNorm weight applied next (in the router)
    float eps = 0.0f;
    const float* resid = nullptr;   // out = resid + block (resid may alias out)
};

// Enqueue the MoE block of one layer on x [B][d] into out [B][d], with the
// workspace w (nullptr: the store's own, grown to B tokens first).
// stage_marks: record the store's stage events.
int ffn_enqueue(jm_store* s, int layer, const float* x, int B, float* out, const FfnIo& io,
                bool stage_marks, hipStream_t st, const Ws* w = nullptr);

// Release the batch-decode workspace, staging and events.
void decode_free_all(jm_store* s);
int dense_block(jm_store* s, int layer, const float* x, int B, float* out, hipStream_t st);

}  // namespace jm

#define JM_HIP(expr, what)                                  \
    do {                                                    \
        hipError_t _e = (expr);                             \
        if (_e != hipSuccess) return jm::hip_fail(_e, what); \
    } while (0)
