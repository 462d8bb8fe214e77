// Batch decode over all layers: decode_layers_batch(cfg, W, kv, positions,
// xin, B, logits) (decode_kernel.c:1518-1556) on the GPU, with the MoE block
// of each layer from the store.  Per layer, four launches around the MoE
// block's own:
//
//   qkv      = [Wq; Wk; Wv] . (h * norm1 w), per column slice  k_gemv_part
//   partials = RMSNorm row scale + bias, QK-norm, RoPE, KV append,
//              attention over 128-position splits of the cache  k_attn_part
//              (a prefill chunk, whose positions share one cache: the KV
//              append first, by a launch of its own         k_kv_append)
//   att      = the splits merged                               k_attn_comb
//   opart    = Wo . att, per column slice                      k_gemv_part
//   h2 = h + sum(opart); h = h2 + MoE(RMSNorm2(h2))   the sum and the norm
//              inside the router, the add inside the down/combine kernel
//              (a dense store, E = 0: the slices summed by k_sum_slices and
//              the dense FFN of jm_dense.hip)
//
// then hidden = RMSNorm_final(h).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstring>
#include <vector>

#include "jm_store.h"

using jm::align256;
using jm::aligned;
using jm::fail;
using jm::hip_fail;

namespace {

constexpr int HD = 128;     // head dimension the attention kernels take
constexpr int PSPLIT = 128; // positions per attention split
constexpr int PREFILL_CHUNK = 512;  // prompt positions per pass of jm_prefill_layers

void free_decode(jm_store* s) {
    if (s->gexec) (void)hipGraphExecDestroy(s->gexec);
    s->gexec = nullptr;
    if (s->dws) (void)hipFree(s->dws);
    s->dws = nullptr;
    s->dec_B = s->dec_S = s->dec_nqkv = s->dec_hq = s->dec_V = 0;
}

int decode_reserve(jm_store* s, int B, int S, int nqkv, int hq, int V) {
    const size_t tab_bytes = align256((size_t)B * s->L * 16 + (size_t)B * 4);
    if (tab_bytes > s->tab_cap) {
        if (s->tab_pending) JM_HIP(hipEventSynchronize(s->tab_ev), "hipEventSynchronize staging");
        s->tab_pending = 0;
        if (s->tab_host) (void)hipHostFree(s->tab_host);
        s->tab_host = nullptr;
        JM_HIP(hipHostMalloc((void**)&s->tab_host, tab_bytes, hipHostMallocDefault), "hipHostMalloc staging");
        s->tab_cap = tab_bytes;
        s->dec_B = 0;   // the device table lives in the workspace: regrow it too
    }
    if (!s->tab_ev) JM_HIP(hipEventCreateWithFlags(&s->tab_ev, hipEventDisableTiming), "hipEventCreate");
    if (B <= s->dec_B && S <= s->dec_S && nqkv <= s->dec_nqkv && hq <= s->dec_hq && V <= s->dec_V) return 0;
    B = std::max(B, s->dec_B);
    S = std::max(S, s->dec_S);
    nqkv = std::max(nqkv, s->dec_nqkv);
    hq = std::max(hq, s->dec_hq);
    V = std::max(V, s->dec_V);
    const int d = s->d, m = s->m;
    const bool dense = s->E == 0;
    // slices of a projection's output: the GEMV's K / 512 at most up to 32
    // tokens, the GEMM's K slices (at most 4) from there
    const int gmax = B >= JM_GEMM_MIN_B ? 4 : 0;
    const size_t qkv_sl = (size_t)std::max(d / 512, gmax), op_sl = (size_t)std::max(hq / 512, gmax);
    // (the dense FFN's products: the most slices over every batch up to B)
    const size_t gu_rows = dense ? (size_t)std::max(jm::dense_gu_slices(d, m, 1) * std::min(B, JM_GEMM_MIN_B - 1),
                                                    jm::dense_gu_slices(d, m, B) * B) : 0;
    const size_t dn_rows = dense ? (size_t)std::max(jm::dense_dn_slices(d, m, 1) * std::min(B, JM_GEMM_MIN_B - 1),
                                                    jm::dense_dn_slices(d, m, B) * B) : 0;
    const size_t sz[] = {
        (size_t)B * d * 4,                        // h
        (size_t)B * d * 4,                        // h2
        qkv_sl * B * nqkv * 4,                    // qkv slices
        op_sl * B * d * 4,                        // o_proj slices
        (size_t)B * S * hq * 4,                   // part_o: H heads x hd per split
        (size_t)B * S * (hq / HD) * 2 * 4,        // part_ml
        (size_t)B * hq * 4,                       // att
        (size_t)B * d * 4,                        // hid
        (size_t)B * d * 4,                        // xemb: embedded prompt tokens (prefill)
        (size_t)jm::lm_blocks(V) * B * 4,         // lmv
        (size_t)jm::lm_blocks(V) * B * 4,         // lmi
        qkv_sl * B * 4,                           // rss: sums of squares of h per qkv slice
        (size_t)B * 2 * 4,                        // qkss: sums of squares of q and k (whole-vector QK-norm)
        gu_rows * 2 * m * 4,                      // dgu: dense FFN gate/up slices
        dense ? (size_t)B * m * 4 : 0,            // dact
        dn_rows * d * 4,                          // ddn: dense FFN down slices
        s->tab_cap,                               // KV pointers + positions
    };
    size_t total = 0;
    for (size_t v : sz) total += align256(v);
    JM_HIP(hipSetDevice(s->device), "hipSetDevice");
    JM_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize before decode workspace growth");
    free_decode(s);
    JM_HIP(hipMalloc(&s->dws, total), "hipMalloc decode workspace");
    char* p = (char*)s->dws;
    void** slots[] = {(void**)&s->h, (void**)&s->h2, (void**)&s->qkv, (void**)&s->opart, (void**)&s->part_o,
                      (void**)&s->part_ml, (void**)&s->att, (void**)&s->hid, (void**)&s->xemb, (void**)&s->lmv,
                      (void**)&s->lmi, (void**)&s->rss, (void**)&s->qkss, (void**)&s->dgu, (void**)&s->dact,
                      (void**)&s->ddn, (void**)&s->tab};
    for (size_t i = 0; i < sizeof sz / sizeof sz[0]; i++) {
        *slots[i] = p;
        p += align256(sz[i]);
    }
    JM_HIP(hipMemset(s->dws, 0, total), "hipMemset decode workspace");
    JM_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize after decode workspace clear");
    s->dec_B = B; s->dec_S = S; s->dec_nqkv = nqkv; s->dec_hq = hq; s->dec_V = V;
    return 0;
}

int check_decode_args(const jm_store* s, const jm_kernel_cfg* c, const jm_kernel_w* W, int* qpk) {
    if (c->L != s->L || c->d != s->d || c->E != s->E || c->topk != s->topk || c->intermediate != s->m)
        return fail(JM_ERR_SHAPE, "cfg (L=%d d=%d E=%d topk=%d m=%d) does not match the store (L=%d d=%d E=%d topk=%d m=%d)",
                    c->L, c->d, c->E, c->topk, c->intermediate, s->L, s->d, s->E, s->topk, s->m);
    if ((c->norm_topk_prob ? 1 : 0) != s->renorm) return fail(JM_ERR_SHAPE, "cfg norm_topk_prob differs from the store's");
    if (c->hd != HD) return fail(JM_ERR_SHAPE, "head dim must be %d (got %d)", HD, c->hd);
    if (c->n_heads <= 0 || c->n_kv <= 0 || c->n_heads % c->n_kv)
        return fail(JM_ERR_SHAPE, "n_heads=%d must be a positive multiple of n_kv=%d", c->n_heads, c->n_kv);
    *qpk = c->n_heads / c->n_kv;
    if (*qpk != 1 && *qpk != 2 && *qpk != 4 && *qpk != 8)
        return fail(JM_ERR_SHAPE, "n_heads / n_kv must be 1, 2, 4 or 8 (got %d)", *qpk);
    if (!jm::gemv_shape_ok(c->d) || !jm::gemv_shape_ok(c->n_heads * HD))
        return fail(JM_ERR_SHAPE, "d=%d and n_heads*hd=%d must be multiples of 1024 up to 8192", c->d, c->n_heads * HD);
    if (c->qk_norm_type < 0 || c->qk_norm_type > 2)
        return fail(JM_ERR_SHAPE, "qk_norm_type %d: 0 (none), 1 (per head) or 2 (whole vector)", c->qk_norm_type);
    if (c->maxT <= 0) return fail(JM_ERR_SHAPE, "maxT must be positive");
    if (!(c->eps >= 0.0f)) return fail(JM_ERR_SHAPE, "eps must be >= 0");
    if (!W) return fail(JM_ERR_ARG, "weights are NULL");
    if (!W->final_norm || !W->norm1 || !W->norm2 || !W->wq || !W->wk || !W->wv || !W->wo || !W->cos || !W->sin)
        return fail(JM_ERR_ARG, "final_norm, norm1, norm2, wq, wk, wv, wo, cos and sin must be set");
    if (c->qk_norm_type != 0 && (!W->qn || !W->kn))
        return fail(JM_ERR_ARG, "qk_norm_type %d needs qn and kn", c->qk_norm_type);
    if (c->bias_qkv && (!W->bq || !W->bk || !W->bv)) return fail(JM_ERR_ARG, "bias_qkv needs bq, bk and bv");
    if (W->use_i8 || W->wq_i8 || W->wk_i8 || W->wv_i8 || W->wo_i8 || W->lm_i8)
        return fail(JM_ERR_ARG, "the int8 attention weights are not supported (use_i8 = 0, *_i8 = NULL)");
    if (s->E == 0) {
        // a dense model (decode_kernel.c:1393-1422): the FFN weights come with W
        if (!W->w1 || !W->w2 || !W->w3) return fail(JM_ERR_ARG, "a dense store (E = 0) needs W->w1, w2 and w3");
        if (!aligned(W->w1, 16) || !aligned(W->w2, 16) || !aligned(W->w3, 16))
            return fail(JM_ERR_ARG, "w1, w2 and w3 must be 16-byte aligned");
    } else if (W->w1 || W->w2 || W->w3) {
        return fail(JM_ERR_ARG, "w1/w2/w3 are the dense FFN's: a MoE store (E > 0) takes its FFN from the store");
    }
    const void* al[] = {W->final_norm, W->norm1, W->norm2, W->wq, W->wk, W->wv, W->wo, W->cos, W->sin,
                        c->qk_norm_type != 0 ? (const void*)W->qn : nullptr,
                        c->qk_norm_type != 0 ? (const void*)W->kn : nullptr,
                        c->bias_qkv ? (const void*)W->bq : nullptr, c->bias_qkv ? (const void*)W->bk : nullptr,
                        c->bias_qkv ? (const void*)W->bv : nullptr};
    for (const void* p : al)
        if (p && !aligned(p, 16)) return fail(JM_ERR_ARG, "weight and bias tensors must be 16-byte aligned");
    return 0;
}

// Layers a step runs: all L, or the first max_layers (set_max_layers,
// decode_kernel.c:1617; the loop bound at :1527 and :1568).
int run_layers(const jm_store* s, int L) { return s->max_layers < 0 ? L : std::min(L, s->max_layers); }

// Every launch of one decode step on st (after the staging copy).
int enqueue_step(jm_store* s, const jm_kernel_cfg* c, const jm_kernel_w* W, const float* xin, int B,
                 float* hidden, float* logits, int* out_tok, int S, int qpk, bool append, bool capturing,
                 hipStream_t st) {
    const int L = c->L, d = c->d, H = c->n_heads, KH = c->n_kv;
    const int nl = run_layers(s, L);
    const int nqkv = (H + 2 * KH) * HD;
    const int* pos_dev = (const int*)(s->tab + (size_t)2 * B * L);
    const bool marks = s->prof && !capturing;
#define JM_DMARK(i) if (marks) JM_HIP(hipEventRecord(s->dev_marks[i], st), "hipEventRecord")
    JM_DMARK(0);
    JM_HIP(hipMemcpyAsync(s->h, xin, (size_t)B * d * 4, hipMemcpyDeviceToDevice, st), "copy xin");
    const float sdiv = jm::sqrtf_fast((float)HD);
    for (int l = 0; l < nl; l++) {
        JM_DMARK(2 * l + 1);
        jm::GemvArgs g{};
        g.x = s->h;
        g.norm_w = W->norm1 + (size_t)l * d;
        g.w[0] = W->wq + (size_t)l * H * HD * d;
        g.w[1] = W->wk + (size_t)l * KH * HD * d;
        g.w[2] = W->wv + (size_t)l * KH * HD * d;
        g.rows[0] = H * HD; g.rows[1] = KH * HD; g.rows[2] = KH * HD;
        g.K = d; g.N = nqkv; g.B = B;
        g.part = s->qkv;
        // a prefill chunk takes the GEMM: one slice instead of d / 512; both
        // also give the sums of squares of h per slice for the RMSNorm scale
        const bool gq = B >= JM_GEMM_MIN_B && jm::gemm_shape_ok(g);
        g.rss = s->rss;
        if (gq) JM_HIP(jm::launch_gemm_bf16(g, st), "qkv GEMM launch");
        else JM_HIP(jm::launch_gemv_part(g, st), "qkv launch");

        jm::AttnArgs at{};
        at.qkv = s->qkv; at.nslice = gq ? jm::gemm_slices(g) : d / jm::gemv_slice_cols(d); at.d = d;
        at.rss = g.rss;
        if (c->bias_qkv) {
            at.bq = W->bq + (size_t)l * H * HD;
            at.bk = W->bk + (size_t)l * KH * HD;
            at.bv = W->bv + (size_t)l * KH * HD;
        }
        at.nqkv = nqkv; at.H = H; at.KH = KH; at.B = B;
        // per head: [L][hd] weights; whole vector (decode_kernel.c:1156-1157):
        // [L][H*hd] and [L][KH*hd]
        at.qk_norm = c->qk_norm_type;
        at.qn = c->qk_norm_type == 1 ? W->qn + (size_t)l * HD
              : c->qk_norm_type == 2 ? W->qn + (size_t)l * H * HD : nullptr;
        at.kn = c->qk_norm_type == 1 ? W->kn + (size_t)l * HD
              : c->qk_norm_type == 2 ? W->kn + (size_t)l * KH * HD : nullptr;
        at.qkss = s->qkss;
        at.eps = c->eps; at.rsdiv = 1.0f / sdiv;
        at.cos = W->cos; at.sin = W->sin;
        at.pos = pos_dev; at.kv = s->tab; at.kv_f32 = s->kv_f32; at.L = L; at.layer = l;
        at.S = S; at.part_o = s->part_o; at.part_ml = s->part_ml;
        at.append = append ? 1 : 0;
        // the grid covers the longest token's splits; the buffers hold S_cap
        // per (token, KV head), indexed with the call's S
        JM_HIP(jm::launch_attn(at, qpk, s->att, st), "attention launch");

        jm::GemvArgs o{};
        o.x = s->att;
        o.w[0] = W->wo + (size_t)l * d * H * HD;
        o.rows[0] = d;
        o.K = H * HD; o.N = d; o.B = B;
        o.part = s->opart;
        const bool go = B >= JM_GEMM_MIN_B && jm::gemm_shape_ok(o);
        if (go) JM_HIP(jm::launch_gemm_bf16(o, st), "o_proj GEMM launch");
        else JM_HIP(jm::launch_gemv_part(o, st), "o_proj launch");

        JM_DMARK(2 * l + 2);
        // h2 = h + attention (summed from the o_proj slices in the router),
        // then h = h2 + MoE(RMSNorm(h2))
        const int nop = go ? jm::gemm_slices(o) : H * HD / jm::gemv_slice_cols(H * HD);
        if (s->E == 0) {
            // dense FFN (decode_kernel.c:1393-1422): h2 = h + the o_proj
            // slices, then h = h2 + FFN(RMSNorm(h2))
            JM_HIP(jm::launch_sum_slices(s->h, s->opart, nop, B, d, s->h2, st), "residual launch");
            jm::DenseFfn f{};
            const size_t md = (size_t)s->m * d;
            f.w1 = W->w1 + l * md; f.w2 = W->w2 + l * md; f.w3 = W->w3 + l * md;
            f.d = d; f.m = s->m; f.B = B;
            f.x = s->h2; f.norm_w = W->norm2 + (size_t)l * d; f.eps = c->eps; f.rss = s->rss;
            f.gu = s->dgu; f.act = s->dact; f.dn = s->ddn;
            f.resid = s->h2; f.out = s->h;
            JM_HIP(jm::launch_dense_ffn(f, st), "dense FFN launch");
            continue;
        }
        jm::FfnIo io;
        io.xpart = s->opart; io.nxpart = nop; io.xmid = s->h2;
        io.norm_w = W->norm2 + (size_t)l * d; io.eps = c->eps;
        io.resid = s->h2;
        if (int rc = jm::ffn_enqueue(s, l, s->h, B, s->h, io, false, st)) return rc;
        const size_t tk = (size_t)B * c->topk * 4;
        if (s->trace && (l + 1) * tk <= s->trace_bytes)
            JM_HIP(hipMemcpyAsync((char*)s->trace + l * tk, s->w.top, tk, hipMemcpyDeviceToDevice, st), "top-k trace");
    }
    JM_DMARK(2 * nl + 1);
    JM_HIP(jm::launch_rms_rows(s->h, W->final_norm, B, d, c->eps, hidden, st), "final norm launch");
    if (logits || out_tok) {
        jm::LmArgs la{};
        la.w = s->lm; la.x = hidden; la.V = s->lm_V; la.d = d; la.B = B;
        la.logits = logits;
        la.best_v = out_tok ? s->lmv : nullptr;
        la.best_i = s->lmi;
        JM_HIP(jm::launch_lm_head(la, out_tok, st), "lm_head launch");
    }
    JM_DMARK(2 * nl + 2);
#undef JM_DMARK
    return 0;
}

}  // namespace

namespace jm {

// jm_layer_ffn_batch on a dense store: out = the dense FFN of layer on x,
// with the weights jm_store_set_dense_ffn registered, in the decode
// workspace's buffers.
int dense_block(jm_store* s, int layer, const float* x, int B, float* out, hipStream_t st) {
    if (!s->dw[0]) return fail(JM_ERR_ARG, "dense FFN weights not set (jm_store_set_dense_ffn)");
    if (int rc = decode_reserve(s, B, 0, 0, 0, 0)) return rc;
    JM_HIP(hipSetDevice(s->device), "hipSetDevice");
    DenseFfn f{};
    const size_t md = (size_t)s->m * s->d;
    f.w1 = s->dw[0] + layer * md; f.w2 = s->dw[1] + layer * md; f.w3 = s->dw[2] + layer * md;
    f.d = s->d; f.m = s->m; f.B = B;
    f.x = x; f.gu = s->dgu; f.act = s->dact; f.dn = s->ddn; f.out = out;
    JM_HIP(launch_dense_ffn(f, st), "dense FFN launch");
    return 0;
}

void decode_free_all(jm_store* s) {
    if (s->gexec) (void)hipGraphExecDestroy(s->gexec);
    if (s->cap_st) (void)hipStreamDestroy(s->cap_st);
    s->gexec = nullptr;
    s->cap_st = nullptr;
    free_decode(s);
    if (s->tab_pending) (void)hipEventSynchronize(s->tab_ev);
    if (s->tab_host) (void)hipHostFree(s->tab_host);
    if (s->tab_ev) (void)hipEventDestroy(s->tab_ev);
    if (s->dev_marks) {
        for (int i = 0; i < s->dprof_n; i++) (void)hipEventDestroy(s->dev_marks[i]);
        delete[] s->dev_marks;
    }
    if (s->lm) (void)hipFree(s->lm);
    s->lm = nullptr;
    s->tab_host = nullptr;
    s->tab_ev = nullptr;
    s->dev_marks = nullptr;
    s->dprof_n = 0;
}

}  // namespace jm

namespace {

// True when the n pointers are pairwise different (open addressing over a
// power-of-two table at most half full; pointers are nonzero).
bool cache_pointers_distinct(const unsigned long long* p, size_t n) {
    thread_local std::vector<unsigned long long> set;
    size_t cap = 16;
    while (cap < 2 * n) cap <<= 1;
    set.assign(cap, 0ull);
    for (size_t i = 0; i < n; i++) {
        const unsigned long long v = p[i];
        size_t h = (size_t)((v >> 4) * 0x9E3779B97F4A7C15ull >> 20) & (cap - 1);
        while (set[h]) {
            if (set[h] == v) return false;
            h = (h + 1) & (cap - 1);
        }
        set[h] = v;
    }
    return true;
}

int decode_impl(jm_store* s, const jm_kernel_cfg* c, const jm_kernel_w* W, const jm_kv_cache* kv,
                const int32_t* positions, const float* xin, int B, float* logits, int32_t* out_tok,
                float* hidden, void* stream, bool allow_graph = true) {
    if (!s || !c) return fail(JM_ERR_ARG, "store and cfg must be non-NULL");
    if (s->E > 0 && !s->wt) return fail(JM_ERR_ARG, "router weights not set (jm_store_set_router)");
    int qpk = 0;
    if (int rc = check_decode_args(s, c, W, &qpk)) return rc;
    if (B < 0) return fail(JM_ERR_ARG, "B must be >= 0");
    if (B == 0) return 0;
    if (!kv || !positions || !xin) return fail(JM_ERR_ARG, "kv, positions and xin must be non-NULL");
    if (!aligned(xin, 16) || (hidden && !aligned(hidden, 16))) return fail(JM_ERR_ARG, "xin and hidden must be 16-byte aligned");
    if (logits || out_tok) {
        if (!s->lm) return fail(JM_ERR_ARG, "lm_head not set (jm_store_set_lm_head)");
        if (s->lm_V != c->V) return fail(JM_ERR_SHAPE, "cfg V=%d differs from the lm_head's %d rows", c->V, s->lm_V);
        if (!jm::lm_shape_ok(c->d)) return fail(JM_ERR_SHAPE, "the lm_head takes d = 1024, 2048 or 4096 (got %d)", c->d);
        if (out_tok && !aligned(out_tok, 4)) return fail(JM_ERR_ARG, "out_tok must be 4-byte aligned");
    }
    const int L = c->L, d = c->d, H = c->n_heads, KH = c->n_kv;
    int maxT = 0;
    for (int b = 0; b < B; b++) {
        if (positions[b] < 0 || positions[b] >= c->maxT)
            return fail(JM_ERR_ARG, "positions[%d] = %d outside [0, maxT=%d)", b, positions[b], c->maxT);
        maxT = std::max(maxT, positions[b] + 1);
    }
    for (long long i = 0; i < (long long)B * L; i++)
        if (!kv[i].k || !kv[i].v || !aligned(kv[i].k, 16) || !aligned(kv[i].v, 16))
            return fail(JM_ERR_ARG, "kv[%lld]: k and v must be non-NULL and 16-byte aligned", i);
    const int nqkv = (H + 2 * KH) * HD;
    const int S = (maxT + PSPLIT - 1) / PSPLIT;
    const int S_cap = (c->maxT + PSPLIT - 1) / PSPLIT;
    if (int rc = jm::store_reserve(s, B)) return rc;
    if (int rc = decode_reserve(s, B, S_cap, nqkv, H * HD, (logits || out_tok) ? c->V : 0)) return rc;
    if (!hidden) hidden = s->hid;
    hipStream_t st = (hipStream_t)stream;
    JM_HIP(hipSetDevice(s->device), "hipSetDevice");

    // KV pointer table and positions to the device through pinned staging
    if (s->tab_pending) JM_HIP(hipEventSynchronize(s->tab_ev), "hipEventSynchronize staging");
    for (long long i = 0; i < (long long)B * L; i++) {
        s->tab_host[2 * i] = (unsigned long long)(uintptr_t)kv[i].k;
        s->tab_host[2 * i + 1] = (unsigned long long)(uintptr_t)kv[i].v;
    }
    // The attention kernel may append each token's k and v rows itself
    // (inside the launch that reads the caches) only when no cache is shared
    // by two tokens: a prompt's positions run as one batch over one cache
    // (jm_prefill_layers), and there every row is appended by a launch of
    // its own first.  Checked over every k and v pointer of the call.
    const bool append = cache_pointers_distinct(s->tab_host, (size_t)2 * B * L);
    int* pos_host = (int*)(s->tab_host + (size_t)2 * B * L);
    memcpy(pos_host, positions, (size_t)B * 4);
    const size_t tab_bytes = (size_t)B * L * 16 + (size_t)B * 4;
    JM_HIP(hipMemcpyAsync(s->tab, s->tab_host, tab_bytes, hipMemcpyHostToDevice, st), "staging copy");
    JM_HIP(hipEventRecord(s->tab_ev, st), "hipEventRecord staging");
    s->tab_pending = 1;
    // per-layer split of the time (jm_store_profile): eager calls only
    const int nmarks = 2 * run_layers(s, L) + 3;
    if (s->prof && s->dprof_n != nmarks) {
        if (s->dev_marks) {
            JM_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
            for (int i = 0; i < s->dprof_n; i++) (void)hipEventDestroy(s->dev_marks[i]);
            delete[] s->dev_marks;
        }
        s->dev_marks = new hipEvent_t[nmarks];
        s->dprof_n = 0;
        for (int i = 0; i < nmarks; i++) {
            JM_HIP(hipEventCreateWithFlags(&s->dev_marks[i], hipEventDisableSystemFence), "hipEventCreate");
            s->dprof_n = i + 1;
        }
    }

    if (s->dgraph && !s->prof && allow_graph) {
        // replay the step from a captured graph: kernel arguments are baked
        // in, so the capture is keyed by everything they depend on
        DecKey key;
        memset(&key, 0, sizeof key);
        memcpy(&key.cfg, c, sizeof *c);
        memcpy(&key.W, W, sizeof *W);
        key.xin = xin; key.hidden = hidden; key.logits = logits; key.out_tok = out_tok; key.lm = s->lm;
        key.B = B; key.S = S;
        key.trace = s->trace; key.trace_bytes = s->trace_bytes; key.ws = s->ws; key.dws = s->dws;
        key.wt = s->wt; key.wt_bf16 = s->wt_bf16; key.lm_V = s->lm_V; key.nl = run_layers(s, c->L);
        key.dense_min = s->dense_min;
        key.ndig = s->ndig;
        key.append = append ? 1 : 0;
        key.kv_f32 = s->kv_f32;
        if (!s->gexec || memcmp(&key, &s->gkey, sizeof key) != 0) {
            if (s->gexec) {
                JM_HIP(hipStreamSynchronize(st), "hipStreamSynchronize before recapture");
                (void)hipGraphExecDestroy(s->gexec);
                s->gexec = nullptr;
            }
            if (!s->cap_st) JM_HIP(hipStreamCreateWithFlags(&s->cap_st, hipStreamNonBlocking), "hipStreamCreate");
            JM_HIP(hipStreamBeginCapture(s->cap_st, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
            const int rc = enqueue_step(s, c, W, xin, B, hidden, logits, out_tok, S, qpk, append, true, s->cap_st);
            hipGraph_t graph = nullptr;
            const hipError_t ec = hipStreamEndCapture(s->cap_st, &graph);
            if (rc) {
                if (graph) (void)hipGraphDestroy(graph);
                return rc;
            }
            if (ec != hipSuccess) return hip_fail(ec, "hipStreamEndCapture");
            const hipError_t ei = hipGraphInstantiate(&s->gexec, graph, nullptr, nullptr, 0);
            (void)hipGraphDestroy(graph);
            if (ei != hipSuccess) {
                s->gexec = nullptr;
                return hip_fail(ei, "hipGraphInstantiate");
            }
            memcpy(&s->gkey, &key, sizeof key);
        }
        JM_HIP(hipGraphLaunch(s->gexec, st), "hipGraphLaunch");
        return 0;
    }
    return enqueue_step(s, c, W, xin, B, hidden, logits, out_tok, S, qpk, append, false, st);
}

}  // namespace

extern "C" {

int jm_decode_layers_batch(jm_store* s, const jm_kernel_cfg* c, const jm_kernel_w* W, const jm_kv_cache* kv,
                           const int32_t* positions, const float* xin, int B, float* logits, float* hidden,
                           void* stream) {
    return decode_impl(s, c, W, kv, positions, xin, B, logits, nullptr, hidden, stream);
}

int jm_decode_layers_batch_argmax(jm_store* s, const jm_kernel_cfg* c, const jm_kernel_w* W, const jm_kv_cache* kv,
                                  const int32_t* positions, const float* xin, int B, int32_t* out_tok,
                                  float* hidden, void* stream) {
    if (!out_tok && B > 0) return fail(JM_ERR_ARG, "out_tok must be non-NULL");
    return decode_impl(s, c, W, kv, positions, xin, B, nullptr, out_tok, hidden, stream);
}

int jm_prefill_layers(jm_store* s, const jm_kernel_cfg* c, const jm_kernel_w* W, const jm_kv_cache* kv,
                      const int32_t* tokens, int T, float* logits, void* stream) {
    if (!s || !c || !W) return fail(JM_ERR_ARG, "store, cfg and weights must be non-NULL");
    if (T <= 0) return fail(JM_ERR_ARG, "T must be positive");
    if (T > c->maxT) return fail(JM_ERR_ARG, "T=%d exceeds maxT=%d", T, c->maxT);
    if (!kv || !tokens) return fail(JM_ERR_ARG, "kv and tokens must be non-NULL");
    if (!W->embed) return fail(JM_ERR_ARG, "the embedding (W->embed) must be set");
    if (logits && !s->lm) return fail(JM_ERR_ARG, "lm_head not set (jm_store_set_lm_head)");
    if (logits && s->lm_V != c->V) return fail(JM_ERR_SHAPE, "cfg V=%d differs from the lm_head's %d rows", c->V, s->lm_V);
    // every position of the prompt is one token of the batch: position t,
    // the sequence's caches for each of them; in chunks of PREFILL_CHUNK
    // positions (each chunk's attention reads the rows the earlier chunks
    // wrote), which bounds the MoE dispatch and the workspace
    const int TC = T < PREFILL_CHUNK ? T : PREFILL_CHUNK;
    std::vector<int32_t> pos((size_t)TC);
    std::vector<jm_kv_cache> tab((size_t)TC * c->L);
    for (int t = 0; t < TC; t++)
        for (int l = 0; l < c->L; l++) tab[(size_t)t * c->L + l] = kv[l];
    int qpk = 0;
    if (int rc = check_decode_args(s, c, W, &qpk)) return rc;
    if (int rc = jm::store_reserve(s, TC)) return rc;
    const int nqkv = (c->n_heads + 2 * c->n_kv) * HD;
    if (int rc = decode_reserve(s, TC, (c->maxT + PSPLIT - 1) / PSPLIT, nqkv, c->n_heads * HD, logits ? c->V : 0))
        return rc;
    hipStream_t st = (hipStream_t)stream;
    JM_HIP(hipSetDevice(s->device), "hipSetDevice");
    int n = 0;
    for (int t0 = 0; t0 < T; t0 += n) {
        n = T - t0 < TC ? T - t0 : TC;
        for (int t = 0; t < n; t++) pos[t] = t0 + t;
        JM_HIP(jm::launch_embed(W->embed, c->V, c->d, tokens + t0, n, s->xemb, st), "embedding launch");
        if (int rc = decode_impl(s, c, W, tab.data(), pos.data(), s->xemb, n, nullptr, nullptr, s->hid, stream, false))
            return rc;
    }
    if (logits) {
        // the lm_head at the last position only (prefill_layers, :1606-1615)
        jm::LmArgs la{};
        la.w = s->lm; la.x = s->hid + (size_t)(n - 1) * c->d; la.V = s->lm_V; la.d = c->d; la.B = 1;
        la.logits = logits;
        la.best_i = s->lmi;
        JM_HIP(jm::launch_lm_head(la, nullptr, st), "lm_head launch");
    }
    return 0;
}

int jm_store_set_lm_head(jm_store* s, const void* w, int dtype, int V) {
    if (!s) return fail(JM_ERR_ARG, "store is NULL");
    if (!w) return fail(JM_ERR_ARG, "lm_head is NULL");
    if (V <= 0) return fail(JM_ERR_SHAPE, "V must be positive");
    if (dtype != JM_DTYPE_F32 && dtype != JM_DTYPE_BF16) return fail(JM_ERR_ARG, "lm_head dtype must be f32 or bf16");
    if (!aligned(w, 4)) return fail(JM_ERR_ARG, "lm_head must be 4-byte aligned");
    if (!jm::lm_shape_ok(s->d)) return fail(JM_ERR_SHAPE, "the lm_head takes d = 1024, 2048 or 4096 (got %d)", s->d);
    JM_HIP(hipSetDevice(s->device), "hipSetDevice");
    const long long n = (long long)V * s->d;
    if (dtype == JM_DTYPE_F32) {
        // the reference's lm_head is float32 widened from the checkpoint's
        // bf16 (decoder3.py:226-230): keep it as bf16 when it is exactly that
        unsigned* flag = nullptr;
        JM_HIP(hipMalloc(&flag, sizeof(unsigned)), "hipMalloc flag");
        unsigned h = 0;
        hipError_t e = hipMemset(flag, 0, sizeof(unsigned));
        if (e == hipSuccess) e = jm::launch_bf16_exact((const float*)w, n, flag, nullptr);
        if (e == hipSuccess) e = hipMemcpy(&h, flag, sizeof(unsigned), hipMemcpyDeviceToHost);
        (void)hipFree(flag);
        if (e != hipSuccess) return hip_fail(e, "lm_head bf16 check");
        if (h) return fail(JM_ERR_ARG, "lm_head values must be bf16-representable (float32 widened from bf16)");
    }
    JM_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
    if (s->lm && s->lm_V != V) {
        (void)hipFree(s->lm);
        s->lm = nullptr;
    }
    if (!s->lm) JM_HIP(hipMalloc((void**)&s->lm, (size_t)n * 2), "hipMalloc lm_head copy");
    s->lm_V = V;
    if (dtype == JM_DTYPE_BF16)
        JM_HIP(hipMemcpy(s->lm, w, (size_t)n * 2, hipMemcpyDeviceToDevice), "lm_head copy");
    else
        JM_HIP(jm::launch_f32_bf16_bits((const float*)w, n, s->lm, nullptr), "lm_head conversion");
    JM_HIP(hipDeviceSynchronize(), "lm_head copy");
    return 0;
}

int jm_lm_head(jm_store* s, const float* x, int B, float* logits, int32_t* out_tok, void* stream) {
    if (!s) return fail(JM_ERR_ARG, "store is NULL");
    if (!s->lm) return fail(JM_ERR_ARG, "lm_head not set (jm_store_set_lm_head)");
    if (B < 0) return fail(JM_ERR_ARG, "B must be >= 0");
    if (B == 0) return 0;
    if (!x || (!logits && !out_tok)) return fail(JM_ERR_ARG, "x and one of logits, out_tok must be non-NULL");
    if (!aligned(x, 16)) return fail(JM_ERR_ARG, "x must be 16-byte aligned");
    if (int rc = decode_reserve(s, B, std::max(s->dec_S, 1), std::max(s->dec_nqkv, 512), std::max(s->dec_hq, 512), s->lm_V))
        return rc;
    JM_HIP(hipSetDevice(s->device), "hipSetDevice");
    jm::LmArgs la{};
    la.w = s->lm; la.x = x; la.V = s->lm_V; la.d = s->d; la.B = B;
    la.logits = logits;
    la.best_v = out_tok ? s->lmv : nullptr;
    la.best_i = s->lmi;
    JM_HIP(jm::launch_lm_head(la, out_tok, (hipStream_t)stream), "lm_head launch");
    return 0;
}

int jm_embed_lookup(const jm_kernel_w* W, const jm_kernel_cfg* c, const int32_t* tokens, int B, float* out,
                    void* stream) {
    if (!W || !c || !W->embed) return fail(JM_ERR_ARG, "weights, cfg and embed must be non-NULL");
    if (c->V <= 0 || c->d <= 0) return fail(JM_ERR_SHAPE, "cfg V and d must be positive");
    if (B < 0) return fail(JM_ERR_ARG, "B must be >= 0");
    if (B == 0) return 0;
    if (!tokens || !out) return fail(JM_ERR_ARG, "tokens and out must be non-NULL");
    JM_HIP(jm::launch_embed(W->embed, c->V, c->d, tokens, B, out, (hipStream_t)stream), "embedding launch");
    return 0;
}

int jm_store_decode_graph(jm_store* s, int enable) {
    if (!s) return fail(JM_ERR_ARG, "store is NULL");
    s->dgraph = enable ? 1 : 0;      // a recorded step is kept for later replays
    return 0;
}

int jm_store_set_dense_ffn(jm_store* s, const uint16_t* w1, const uint16_t* w2, const uint16_t* w3) {
    if (!s) return fail(JM_ERR_ARG, "store is NULL");
    if (s->E != 0) return fail(JM_ERR_ARG, "dense FFN weights are for a dense store (E = 0)");
    if (!w1 || !w2 || !w3) return fail(JM_ERR_ARG, "w1, w2 and w3 must be non-NULL");
    if (!aligned(w1, 16) || !aligned(w2, 16) || !aligned(w3, 16))
        return fail(JM_ERR_ARG, "w1, w2 and w3 must be 16-byte aligned");
    s->dw[0] = w1; s->dw[1] = w2; s->dw[2] = w3;
    return 0;
}

int jm_store_set_kv_dtype(jm_store* s, int dtype) {
    if (!s) return fail(JM_ERR_ARG, "store is NULL");
    if (dtype != JM_DTYPE_BF16 && dtype != JM_DTYPE_F32)
        return fail(JM_ERR_ARG, "dtype must be JM_DTYPE_BF16 or JM_DTYPE_F32 (got %d)", dtype);
    s->kv_f32 = dtype == JM_DTYPE_F32 ? 1 : 0;
    return 0;
}

int jm_store_set_max_layers(jm_store* s, int n) {
    if (!s) return fail(JM_ERR_ARG, "store is NULL");
    s->max_layers = n < 0 ? -1 : n;
    return 0;
}

int jm_store_trace_topk(jm_store* s, int32_t* buf, uint64_t bytes) {
    if (!s) return fail(JM_ERR_ARG, "store is NULL");
    if (buf && !aligned(buf, 4)) return fail(JM_ERR_ARG, "trace buffer must be 4-byte aligned");
    s->trace = buf;
    s->trace_bytes = buf ? bytes : 0;
    return 0;
}

int jm_store_decode_ms(jm_store* s, float* attn_ms, float* moe_ms, float* total_ms) {
    if (!s) return fail(JM_ERR_ARG, "store is NULL");
    if (!s->prof || !s->dev_marks) return fail(JM_ERR_ARG, "no profiled decode call (jm_store_profile, then jm_decode_layers_batch)");
    const int L = (s->dprof_n - 3) / 2;
    JM_HIP(hipEventSynchronize(s->dev_marks[s->dprof_n - 1]), "hipEventSynchronize");
    float at = 0.0f, mo = 0.0f, tot = 0.0f, v = 0.0f;
    for (int l = 0; l < L; l++) {
        JM_HIP(hipEventElapsedTime(&v, s->dev_marks[2 * l + 1], s->dev_marks[2 * l + 2]), "hipEventElapsedTime");
        at += v;
        JM_HIP(hipEventElapsedTime(&v, s->dev_marks[2 * l + 2], s->dev_marks[2 * l + 3]), "hipEventElapsedTime");
        mo += v;
    }
    JM_HIP(hipEventElapsedTime(&tot, s->dev_marks[0], s->dev_marks[s->dprof_n - 1]), "hipEventElapsedTime");
    if (attn_ms) *attn_ms = at;
    if (moe_ms) *moe_ms = mo;
    if (total_ms) *total_ms = tot;
    return 0;
}

}  // extern "C"
