// C ABI of the MI355X MoE decode block (declared in include/joule_amd.h).
//
// Every entry point returns an int status (0 = ok, negative = error) and
// records a message readable with jm_last_error().  Pointers to tensors are
// device pointers; the library never frees caller memory.  Work is enqueued
// on the caller's stream (NULL = the default stream); nothing synchronises
// except workspace growth, which the caller can do ahead of time with
// jm_store_reserve().
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <atomic>
#include <cstring>
#include <mutex>
#include <vector>

#include "jm_plugin_ws.h"
#include "jm_store.h"

namespace jm {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(JM_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace jm

namespace {

// Workspace of the plugin products (jm_q4_gemm_f32 / jm_q4_gemv_f32): one
// buffer per (device, stream), the policy of jm_plugin_ws.h (reuse, grow
// with the old buffer retired, or a stream-ordered allocation under
// capture, freed after the call).
struct PluginWs {
    void* p = nullptr;
    bool async = false;
};

struct PluginBuf {
    int dev;
    hipStream_t st;
    void* p;
    size_t bytes;
};

std::mutex g_pws_mu;
std::vector<PluginBuf> g_pws;
std::vector<void*> g_pws_retired;           // replaced buffers, kept until the process ends

int plugin_ws(hipStream_t st, size_t bytes, PluginWs* out) {
    int dev = 0;
    JM_HIP(hipGetDevice(&dev), "hipGetDevice");
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    JM_HIP(hipStreamIsCapturing(st, &cs), "hipStreamIsCapturing");
    std::lock_guard<std::mutex> lk(g_pws_mu);
    PluginBuf* b = nullptr;
    for (auto& x : g_pws)
        if (x.dev == dev && x.st == st) b = &x;
    switch (jm::plugin_ws_action(b ? b->bytes : 0, bytes, cs != hipStreamCaptureStatusNone)) {
        case jm::WsAction::StreamOrdered:
            JM_HIP(hipMallocAsync(&out->p, bytes, st), "hipMallocAsync plugin workspace");
            out->async = true;
            return 0;
        case jm::WsAction::Reuse:
            out->p = b->p;
            return 0;
        case jm::WsAction::Grow:
            break;
    }
    const size_t grow = jm::plugin_ws_grow(b ? b->bytes : 0, bytes);
    void* p = nullptr;
    JM_HIP(hipMalloc(&p, grow), "hipMalloc plugin workspace");
    if (b) {
        if (b->p) g_pws_retired.push_back(b->p);
        b->p = p;
        b->bytes = grow;
    } else {
        g_pws.push_back(PluginBuf{dev, st, p, grow});
    }
    out->p = p;
    return 0;
}

// token count from which jm_q4_gemm_f32 takes the matrix cores
std::atomic<int> g_q4_gemm_min_t{JM_Q4_GEMM_MIN_T};

}  // namespace

// Workspace of jm_layer_ffn_batch_noalloc: one fixed array on each device
// the library runs on, held until the process ends.  Host code never uses
// the array's name as an address: jm_store_create resolves the device
// address once per device (hipGetSymbolAddress with that device current)
// into scratch_ptr, and the calls lay the workspace out from there.
static __device__ __align__(256) unsigned char scratch[JM_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_ptr[MAX_DEVICES];

// Resolve the scratch array's address on `device` (current) once.
int resolve_scratch(int device) {
    if (device < 0 || device >= MAX_DEVICES)
        return jm::fail(JM_ERR_ARG, "device %d beyond the %d the no-allocation workspace tracks", device, MAX_DEVICES);
    std::lock_guard<std::mutex> lk(scratch_mu);
    if (scratch_ptr[device]) return 0;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return jm::hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
    scratch_ptr[device] = p;
    return 0;
}

}  // namespace

namespace {

using jm::aligned;
using jm::align256;
using jm::fail;
using jm::hip_fail;

int check_group_shape(int d, int m, int group) {
    if (group != 32 && group != 64) return fail(JM_ERR_SHAPE, "group must be 32 or 64, got %d", group);
    if (d <= 0 || m <= 0) return fail(JM_ERR_SHAPE, "d and intermediate must be positive");
    if (d % group || m % group) return fail(JM_ERR_SHAPE, "d=%d and intermediate=%d must be multiples of the group %d", d, m, group);
    const int lpr = d / group;
    if (lpr != 16 && lpr != 32 && lpr != 64)
        return fail(JM_ERR_SHAPE, "d / group must be 16, 32 or 64 (got %d)", lpr);
    if (d % 512 || (d / 512 != 1 && d / 512 != 2 && d / 512 != 3 && d / 512 != 4 && d / 512 != 6 && d / 512 != 8))
        return fail(JM_ERR_SHAPE, "d must be 512, 1024, 1536, 2048, 3072 or 4096 (got %d)", d);
    if (m / group > 64) return fail(JM_ERR_SHAPE, "intermediate / group must be <= 64 (got %d)", m / group);
    if (m % 64) return fail(JM_ERR_SHAPE, "intermediate must be a multiple of 64 (got %d)", m);
    if (d % 128) return fail(JM_ERR_SHAPE, "d must be a multiple of 128 (got %d)", d);
    return 0;
}

}  // namespace

namespace {

// Sizes of the Ws fields for B tokens, in field order.
constexpr int WS_NF = 27;
void ws_sizes(const jm_store* s, int B, size_t (&sz)[WS_NF]) {
    const int E = s->E, d = s->d, m = s->m, k = s->topk, G = s->group;
    const size_t nslot = (size_t)B * k;
    // digit planes: room for the most (jm_store_set_act_digits)
    const size_t words_d = (size_t)(d / G) * JM_NDIG_MAX * (G / 8);
    const size_t words_m = (size_t)(m / 8) * JM_NDIG_MAX;
    const size_t max_tiles = nslot / JM_DENSE_TILE + E;
    const size_t v[WS_NF] = {
        (size_t)B * E * 4,            // logits
        nslot * 4,                    // top
        nslot * 4,                    // tw
        (size_t)B * words_d * 4,      // xdig
        (size_t)B * (d / G) * 4,      // xscale
        (size_t)(E + 1) * 4,          // seg_off
        nslot * 4,                    // seg_slot
        (size_t)E * 4,                // active
        4,                            // n_active
        (size_t)E * 4,                // first_slot
        nslot * 4,                    // comb
        (size_t)E * sizeof(jm::ExpertWork),   // work table
        max_tiles * 8,                // dense tiles
        8,                            // n_tiles (tiles, small experts)
        (size_t)E * 4,                // small
        nslot * m * 4,                // act
        nslot * words_m * 4,          // adig
        nslot * (m / 32) * 4,         // ascale
        nslot * d * 4,                // y
        nslot * m,                    // aqh
        nslot * m,                    // aql
        (size_t)B * d,                // xqh
        (size_t)B * d,                // xql
        (size_t)B * (d / G) * 4,      // xqs
        nslot * (m / G) * 4,          // aqs
        (size_t)B * (d / G) * 4,      // xqc
        nslot * (m / G) * 4,          // aqc
    };
    for (int i = 0; i < WS_NF; i++) sz[i] = v[i];
}

}  // namespace

size_t jm::ws_bytes(const jm_store* s, int B) {
    size_t sz[WS_NF];
    ws_sizes(s, B, sz);
    size_t total = 0;
    for (size_t v : sz) total += align256(v);
    return total;
}

void jm::ws_layout(const jm_store* s, int B, char* base, Ws* w) {
    size_t sz[WS_NF];
    ws_sizes(s, B, sz);
    void** slots[WS_NF] = {(void**)&w->logits, (void**)&w->top, (void**)&w->tw, (void**)&w->xdig,
                           (void**)&w->xscale, (void**)&w->seg_off, (void**)&w->seg_slot,
                           (void**)&w->active, (void**)&w->n_active, (void**)&w->first_slot,
                           (void**)&w->comb, (void**)&w->work, (void**)&w->tiles,
                           (void**)&w->n_tiles, (void**)&w->small, (void**)&w->act, (void**)&w->adig,
                           (void**)&w->ascale, (void**)&w->y, (void**)&w->aqh, (void**)&w->aql,
                           (void**)&w->xqh, (void**)&w->xql, (void**)&w->xqs, (void**)&w->aqs,
                           (void**)&w->xqc, (void**)&w->aqc};
    static_assert(sizeof(Ws) == WS_NF * sizeof(void*), "a size for every workspace field");
    for (int i = 0; i < WS_NF; i++) {
        *slots[i] = base;
        base += align256(sz[i]);
    }
}

int jm::store_reserve(jm_store* s, int B) {
    if (B <= s->cap_B || s->E == 0) return 0;      // a dense store has no MoE workspace
    const size_t total = ws_bytes(s, B);
    void* mem = nullptr;
    JM_HIP(hipSetDevice(s->device), "hipSetDevice");
    JM_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize before workspace growth");
    JM_HIP(hipMalloc(&mem, total), "hipMalloc workspace");
    if (s->ws) (void)hipFree(s->ws);
    s->ws = mem;
    ws_layout(s, B, (char*)mem, &s->w);
    JM_HIP(hipMemset(mem, 0, total), "hipMemset workspace");
    JM_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize after workspace clear");
    s->cap_B = B;
    return 0;
}

namespace {

int check_store(const jm_store* s) {
    if (!s) return fail(JM_ERR_ARG, "store is NULL");
    return 0;
}

// the entry points of the expert store (router, experts, MoE workspace)
int check_moe_store(const jm_store* s, const char* what) {
    if (!s) return fail(JM_ERR_ARG, "store is NULL");
    if (s->E == 0) return fail(JM_ERR_ARG, "%s: a dense store (E = 0) has no router or experts", what);
    return 0;
}

// A dense store (E = 0, decode_kernel.c:1393-1422): no expert records; the
// FFN weights come with the decoder's KernelW or jm_store_set_dense_ffn.
int create_dense_store(const jm_kernel_cfg* cfg, jm_store** out) {
    const int L = cfg->L, d = cfg->d, m = cfg->intermediate;
    if (L <= 0) return fail(JM_ERR_SHAPE, "need 0 < L (L=%d)", L);
    if (cfg->topk != 0) return fail(JM_ERR_SHAPE, "a dense store (E = 0) has topk 0 (got %d)", cfg->topk);
    if (cfg->expert_i8 || cfg->expert_bf16) return fail(JM_ERR_SHAPE, "expert_i8/expert_bf16 set on a dense store");
    if (!jm::dense_shape_ok(d, m))
        return fail(JM_ERR_SHAPE, "dense FFN: d=%d must be a multiple of 1024 up to 8192 and intermediate=%d a "
                    "multiple of 512 up to %d", d, m, JM_DENSE_MAX_M);
    int dev = 0;
    JM_HIP(hipGetDevice(&dev), "hipGetDevice");
    jm_store* s = new jm_store();
    memset(s, 0, sizeof *s);
    s->L = L; s->E = 0; s->d = d; s->m = m; s->topk = 0;
    s->dense_min = JM_DENSE_MIN_DEFAULT;
    s->ndig = JM_NDIG;
    s->max_layers = -1;
    s->device = dev;
    hipError_t e = hipDeviceGetAttribute(&s->n_cu, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&s->lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    if (e != hipSuccess) {
        delete s;
        return hip_fail(e, "jm_store_create device attributes");
    }
    if (int rc = resolve_scratch(dev)) {
        delete s;
        return rc;
    }
    *out = s;
    return 0;
}

// Common part of the stage entry points: checks, the workspace for B
// tokens, and the dispatch of the caller's top-k table (the counting sort,
// the expert work table and the union order of the dispatch path) on st.
// The stages run the dispatch path's wave-item kernels at every B.
int stage_setup(jm_store* s, int layer, const int32_t* top, int B, const char* who, hipStream_t st,
                jm::RouteArgs* r, jm::ExpertArgs* a) {
    if (int rc = check_moe_store(s, who)) return rc;
    if (layer < 0 || layer >= s->L) return fail(JM_ERR_ARG, "%s: layer %d outside [0, %d)", who, layer, s->L);
    if (B < 0 || (long long)B * s->topk > JM_MAX_SLOTS)
        return fail(JM_ERR_SHAPE, "%s: need 0 <= B and B * topk <= %d", who, JM_MAX_SLOTS);
    if (B == 0) return 0;
    if (!top) return fail(JM_ERR_ARG, "%s: top is NULL", who);
    const int E = s->E, k = s->topk, nslot = B * k;
    if ((size_t)jm::dispatch_lds_ints(nslot, E) * 4 > (size_t)s->lds_max)
        return fail(JM_ERR_SHAPE, "%s: %d slots over %d experts exceed the dispatch's LDS", who, nslot, E);
    if (int rc = jm::store_reserve(s, B)) return rc;
    JM_HIP(hipSetDevice(s->device), "hipSetDevice");
    const jm::Ws& w = s->w;
    r->B = B; r->E = E; r->d = s->d; r->topk = k; r->group = s->group;
    r->top = const_cast<int*>(top);             // read only
    r->seg_off = w.seg_off; r->seg_slot = w.seg_slot; r->active = w.active; r->n_active = w.n_active;
    r->first_slot = w.first_slot; r->comb = w.comb;
    r->work = w.work; r->umax = std::min(E, nslot); r->rec = s->rec;
    r->key0 = (long long)layer * E;
    r->dense_min = 0x7FFFFFFF;                  // no MFMA tiles
    r->ndig = s->ndig;
    r->tiles = w.tiles; r->n_tiles = w.n_tiles; r->small = w.small;
    JM_HIP(jm::launch_dispatch_work(*r, st), "dispatch launch");
    a->blob = s->blob; a->rec = s->rec; a->key0 = r->key0; a->E = E;
    a->work = w.work; a->umax = r->umax; a->seg_slot = w.seg_slot;
    a->top = r->top; a->nslot = nslot; a->B = B;
    a->d = s->d; a->m = s->m; a->topk = k; a->group = s->group;
    a->xdig = w.xdig; a->xscale = w.xscale;
    a->adig = w.adig; a->ascale = w.ascale;
    a->dense_min = 0x7FFFFFFF;
    a->tiles = w.tiles; a->n_tiles = w.n_tiles; a->small = w.small;
    a->ndig = s->ndig;
    return 0;
}

}  // namespace

namespace jm {

int ffn_enqueue(jm_store* s, int layer, const float* x, int B, float* out, const FfnIo& io,
                bool stage_marks, hipStream_t st, const Ws* wsp) {
    if ((long long)B * s->topk > JM_MAX_SLOTS) return fail(JM_ERR_SHAPE, "B * topk must be <= %d", JM_MAX_SLOTS);
    if (B * s->topk > JM_DEC_SLOTS && (size_t)jm::dispatch_lds_ints(B * s->topk, s->E) * 4 > (size_t)s->lds_max)
        return fail(JM_ERR_SHAPE, "B * topk = %d slots over %d experts exceed the dispatch's LDS", B * s->topk, s->E);
    if (!wsp) {
        if (int rc = store_reserve(s, B)) return rc;
    }
    const Ws& w = wsp ? *wsp : s->w;
    const int E = s->E, d = s->d, k = s->topk, G = s->group;
    JM_HIP(hipSetDevice(s->device), "hipSetDevice");
    const int umax = std::min(E, B * k);
    const int nslot = B * k;
    const bool dec = nslot <= JM_DEC_SLOTS;
    jm::RouteArgs r;
    r.wt = (const char*)s->wt + (size_t)layer * jm::router_experts_padded(E) * d * (s->wt_bf16 ? 2 : 4);
    r.wt_bf16 = s->wt_bf16;
    r.x = x; r.xpart = io.xpart; r.nxpart = io.nxpart; r.xmid = io.xmid;
    r.norm_w = io.norm_w; r.eps = io.eps; r.B = B; r.E = E; r.d = d; r.topk = k; r.renorm = s->renorm; r.group = G;
    r.logits = w.logits; r.xdig = w.xdig; r.xscale = w.xscale; r.top = w.top; r.tw = w.tw;
    r.seg_off = w.seg_off; r.seg_slot = w.seg_slot; r.active = w.active; r.n_active = w.n_active;
    r.first_slot = w.first_slot; r.comb = w.comb;
    r.work = w.work; r.umax = umax; r.rec = s->rec;
    r.key0 = (long long)layer * E;
    r.dense_min = s->dense_min; r.tiles = w.tiles; r.n_tiles = w.n_tiles; r.small = w.small;
    r.skip_topk = dec && jm::gateup_topk(B, E);
    r.ndig = s->ndig;
    // From the quad router's batch sizes on the dispatch path, the tokens'
    // digits are encoded by the dispatch launch, on the CUs its dispatch
    // block leaves idle, instead of by the router.  The decoder layer's
    // normalised tokens reach it through y, which the down stage writes
    // only later.
    r.enc_late = !dec && B >= JM_ROUTER_QUAD_MIN_B;
    const bool layer_in = io.xpart || io.norm_w;
    r.xn = r.enc_late && layer_in ? w.y : nullptr;
    r.xenc = layer_in ? w.y : x;
    jm::ExpertArgs a;
    a.blob = s->blob; a.rec = s->rec; a.key0 = (long long)layer * E; a.E = E;
    a.work = w.work; a.umax = umax; a.seg_slot = w.seg_slot;
    a.top = w.top; a.nslot = nslot; a.B = B;
    a.d = d; a.m = s->m; a.topk = k; a.group = G;
    a.tw = w.tw; a.xdig = w.xdig; a.xscale = w.xscale;
    a.act = w.act; a.adig = w.adig; a.ascale = w.ascale; a.y = w.y; a.out = out; a.resid = io.resid;
    a.dense_min = s->mfma_ok ? s->dense_min : 0x7FFFFFFF;
    r.dense_min = a.dense_min;
    a.tiles = w.tiles; a.n_tiles = w.n_tiles; a.small = w.small;
    const bool mfma = !dec && a.dense_min <= nslot;
    r.xqh = mfma ? w.xqh : nullptr; r.xql = w.xql; r.xqs = w.xqs; r.xqc = w.xqc;
    a.xqh = w.xqh; a.xql = w.xql; a.xqs = w.xqs; a.xqc = w.xqc;
    a.aqh = w.aqh; a.aql = w.aql; a.aqs = w.aqs; a.aqc = w.aqc;
    a.logits = w.logits; a.renorm = s->renorm; a.top_w = w.top; a.tw_w = w.tw;
    a.ndig = s->ndig;
    const int max_tiles = nslot / JM_DENSE_TILE + E;
#define JM_MARK(i) if (s->prof && stage_marks) JM_HIP(hipEventRecord(s->ev[i], st), "hipEventRecord")
    JM_MARK(0);
    JM_HIP(jm::launch_route_tok(r, st), "route launch");
    if (!dec) JM_HIP(jm::launch_dispatch_work(r, st), "dispatch launch");
    JM_MARK(1);
    if (dec) {
        JM_HIP(jm::launch_gateup_dec(a, st), "gate/up launch");
    } else {
        if (mfma) {
            // the MFMA kernels also run the experts under dense_min, as wave
            // items on the blocks past their tiles (the grids' last round)
            JM_HIP(jm::launch_gateup_mfma(a, max_tiles, st), "gate/up MFMA launch");
        } else {
            JM_HIP(jm::launch_gateup(a, umax, st), "gate/up launch");
        }
    }
    JM_MARK(2);
    if (dec) {
        JM_HIP(jm::launch_down_comb(a, st), "down/combine launch");
    } else {
        if (mfma) JM_HIP(jm::launch_down_mfma(a, max_tiles, st), "down MFMA launch");
        else JM_HIP(jm::launch_down(a, umax, st), "down launch");
        JM_HIP(jm::launch_combine(w.y, w.comb, B, k, d, io.resid, out, st), "combine launch");
    }
    JM_MARK(3);
#undef JM_MARK
    if (!wsp) {
        s->dec_last = dec;
        s->last_B = B;
    }
    return 0;
}

}  // namespace jm

extern "C" {

int jm_version(void) { return JM_ABI_VERSION; }

const char* jm_last_error(void) { return jm::g_err; }

int jm_abi_sizes(int* kernel_cfg_bytes, int* ndig, int* nt) {
    if (kernel_cfg_bytes) *kernel_cfg_bytes = (int)sizeof(jm_kernel_cfg);
    if (ndig) *ndig = JM_NDIG;
    if (nt) *nt = 8;
    return 0;
}

int jm_store_create(const jm_kernel_cfg* cfg, int group, const void* blob, uint64_t blob_bytes,
                    const uint64_t* offsets, jm_store** out) {
    if (!cfg || !out) return fail(JM_ERR_ARG, "NULL argument to jm_store_create");
    *out = nullptr;
    if (cfg->E == 0) return create_dense_store(cfg, out);
    if (!blob || !offsets) return fail(JM_ERR_ARG, "NULL argument to jm_store_create");
    const int L = cfg->L, E = cfg->E, d = cfg->d, m = cfg->intermediate, k = cfg->topk;
    if (L <= 0 || E <= 0 || E > JM_MAX_E) return fail(JM_ERR_SHAPE, "need 0 < L and 0 < E <= %d (L=%d E=%d)", JM_MAX_E, L, E);
    if (k <= 0 || k > E || k > JM_MAX_TOPK) return fail(JM_ERR_SHAPE, "need 0 < topk <= min(E, %d) (topk=%d)", JM_MAX_TOPK, k);
    if (cfg->expert_i8 || cfg->expert_bf16)
        return fail(JM_ERR_SHAPE, "only the Q4 expert store is supported (expert_i8/expert_bf16 set)");
    if (int rc = check_group_shape(d, m, group)) return rc;
    if (!aligned(blob, 16)) return fail(JM_ERR_ARG, "store blob must be 16-byte aligned");
    // every record must lie inside the blob, with packed rows 16-byte aligned
    const uint64_t sg = (uint64_t)m * d / group * 2, pg = (uint64_t)m * d / 2;
    bool sc16 = true;                           // the MFMA branch reads scales in 8- and 16-byte pieces
    for (int p = 0; p < 3; p++)
        for (int i = 0; i < L * E; i++) {
            const uint64_t so = offsets[((size_t)p * L * E + i) * 2 + 0];
            const uint64_t po = offsets[((size_t)p * L * E + i) * 2 + 1];
            if (so % 2 || po % 16)
                return fail(JM_ERR_ARG, "record %d of part %d is misaligned (scales %llu, packed %llu)",
                            i, p, (unsigned long long)so, (unsigned long long)po);
            if (so + sg > blob_bytes || po + pg > blob_bytes || so + sg < so || po + pg < po)
                return fail(JM_ERR_ARG, "record %d of part %d lies outside the %llu-byte blob", i, p,
                            (unsigned long long)blob_bytes);
            sc16 = sc16 && so % 16 == 0;
        }
    hipPointerAttribute_t attr;
    hipError_t pe = hipPointerGetAttributes(&attr, blob);
    if (pe != hipSuccess || attr.type != hipMemoryTypeDevice) {
        (void)hipGetLastError();
        return fail(JM_ERR_ARG, "store blob must be device memory");
    }
    jm_store* s = new jm_store();
    memset(s, 0, sizeof *s);
    s->L = L; s->E = E; s->d = d; s->m = m; s->topk = k;
    s->renorm = cfg->norm_topk_prob ? 1 : 0;
    s->group = group;
    s->dense_min = JM_DENSE_MIN_DEFAULT;
    s->ndig = JM_NDIG;
    s->mfma_ok = jm::mfma_shape_ok(d, m) && sc16;
    s->max_layers = -1;
    s->blob = (const uint8_t*)blob;
    s->blob_bytes = blob_bytes;
    s->device = attr.device;
    const size_t ob = (size_t)3 * L * E * 2 * sizeof(uint64_t);
    hipError_t e = hipSetDevice(s->device);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&s->n_cu, hipDeviceAttributeMultiprocessorCount, s->device);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&s->lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, s->device);
    if (e == hipSuccess) e = hipMalloc(&s->off_dev, ob);
    if (e == hipSuccess) e = hipMemcpy(s->off_dev, offsets, ob, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (s->off_dev) (void)hipFree(s->off_dev);
        delete s;
        return hip_fail(e, "jm_store_create offset table");
    }
    // records at base + key * stride + a per-part offset (the reference's
    // converter writes (layer, expert, part) in order): locate them by formula
    s->rec.table = (const unsigned long long*)s->off_dev;
    s->rec.LE = (long long)L * E;
    s->rec.affine = 0;
    {
        const uint64_t* o = offsets;
        const size_t LE = (size_t)L * E;
        const uint64_t base = o[0];
        const uint64_t stride = LE > 1 ? o[2] - o[0] : 0;
        bool affine = LE == 1 || o[2] > o[0];
        uint64_t so[3], po[3];
        for (int p = 0; p < 3 && affine; p++) {
            so[p] = o[(size_t)p * LE * 2 + 0] - base;
            po[p] = o[(size_t)p * LE * 2 + 1] - base;
            for (size_t i = 0; i < LE && affine; i++) {
                const uint64_t b = base + i * stride;
                affine = o[((size_t)p * LE + i) * 2 + 0] == b + so[p] && o[((size_t)p * LE + i) * 2 + 1] == b + po[p];
            }
        }
        if (affine) {
            s->rec.affine = 1;
            s->rec.base = base;
            s->rec.stride = stride;
            for (int p = 0; p < 3; p++) { s->rec.so[p] = so[p]; s->rec.po[p] = po[p]; }
        }
    }
    if (int rc = resolve_scratch(s->device)) {
        (void)hipFree(s->off_dev);
        delete s;
        return rc;
    }
    *out = s;
    return 0;
}

int jm_store_destroy(jm_store* s) {
    if (!s) return 0;
    (void)hipSetDevice(s->device);
    (void)hipDeviceSynchronize();
    if (s->off_dev) (void)hipFree(s->off_dev);
    if (s->wt) (void)hipFree(s->wt);
    if (s->ws) (void)hipFree(s->ws);
    if (s->prof)
        for (int i = 0; i <= JM_STAGES; i++) (void)hipEventDestroy(s->ev[i]);
    jm::decode_free_all(s);
    delete s;
    return 0;
}

int jm_store_set_router(jm_store* s, const void* gate_w, int dtype) {
    if (int rc = check_moe_store(s, "jm_store_set_router")) return rc;
    if (!gate_w) return fail(JM_ERR_ARG, "router weights are NULL");
    if (dtype != JM_DTYPE_F32 && dtype != JM_DTYPE_BF16) return fail(JM_ERR_ARG, "router dtype must be f32 or bf16");
    if (!aligned(gate_w, 4)) return fail(JM_ERR_ARG, "router weights must be 4-byte aligned");
    JM_HIP(hipSetDevice(s->device), "hipSetDevice");
    const size_t n = (size_t)s->L * s->E * s->d;
    int exact = 1;
    if (dtype == JM_DTYPE_F32) {
        unsigned* flag = nullptr;
        JM_HIP(hipMalloc(&flag, sizeof(unsigned)), "hipMalloc flag");
        unsigned h = 0;
        hipError_t e = hipMemset(flag, 0, sizeof(unsigned));
        if (e == hipSuccess) e = jm::launch_bf16_exact((const float*)gate_w, (long long)n, flag, nullptr);
        if (e == hipSuccess) e = hipMemcpy(&h, flag, sizeof(unsigned), hipMemcpyDeviceToHost);
        (void)hipFree(flag);
        if (e != hipSuccess) return hip_fail(e, "router bf16 check");
        exact = h == 0;
    }
    if (s->wt && s->wt_bf16 != exact) {
        (void)hipFree(s->wt);
        s->wt = nullptr;
    }
    const size_t ncopy = (size_t)s->L * jm::router_experts_padded(s->E) * s->d;
    if (!s->wt) JM_HIP(hipMalloc(&s->wt, ncopy * (exact ? 2 : 4)), "hipMalloc router copy");
    s->wt_bf16 = exact;
    JM_HIP(hipMemset(s->wt, 0, ncopy * (exact ? 2 : 4)), "router copy clear");
    JM_HIP(jm::launch_router_transpose(gate_w, dtype == JM_DTYPE_BF16, s->wt, exact, (long long)s->L * s->E,
                                       s->E, s->d, nullptr), "router transpose launch");
    JM_HIP(hipDeviceSynchronize(), "router transpose");
    return 0;
}

int jm_store_reserve(jm_store* s, int max_B) {
    if (int rc = check_store(s)) return rc;
    if (max_B < 0) return fail(JM_ERR_ARG, "max_B must be >= 0");
    return jm::store_reserve(s, max_B);
}

int jm_store_set_dense_min(jm_store* s, int min_tokens) {
    if (int rc = check_store(s)) return rc;
    if (min_tokens < 0) return fail(JM_ERR_ARG, "min_tokens must be >= 0 (0 = default)");
    s->dense_min = min_tokens == 0 ? JM_DENSE_MIN_DEFAULT : min_tokens;
    return 0;
}

int jm_store_set_act_digits(jm_store* s, int ndig) {
    if (int rc = check_store(s)) return rc;
    if (ndig != 0 && ndig != 4 && ndig != 5) return fail(JM_ERR_ARG, "ndig must be 4, 5 or 0 (the default, %d)", JM_NDIG);
    s->ndig = ndig == 0 ? JM_NDIG : ndig;
    return 0;
}

int jm_store_act_digits(const jm_store* s) { return s ? s->ndig : -1; }

int jm_store_info(const jm_store* s, int* L, int* E, int* d, int* m, int* topk, int* group) {
    if (int rc = check_store(s)) return rc;
    if (L) *L = s->L;
    if (E) *E = s->E;
    if (d) *d = s->d;
    if (m) *m = s->m;
    if (topk) *topk = s->topk;
    if (group) *group = s->group;
    return 0;
}

int jm_store_router_dtype(const jm_store* s, int* dtype) {
    if (int rc = check_moe_store(s, "jm_store_router_dtype")) return rc;
    if (!s->wt) return fail(JM_ERR_ARG, "router weights not set (jm_store_set_router)");
    if (dtype) *dtype = s->wt_bf16 ? JM_DTYPE_BF16 : JM_DTYPE_F32;
    return 0;
}

int jm_layer_ffn_batch(jm_store* s, int layer, const float* x, int B, float* out,
                       int32_t* topk_idx, float* topk_w, void* stream) {
    if (int rc = check_store(s)) return rc;
    if (s->E == 0) {
        // the dense FFN (decode_kernel.c:1393-1422): no routing
        if (topk_idx || topk_w) return fail(JM_ERR_ARG, "a dense store (E = 0) has no top-k: pass NULL");
        if (layer < 0 || layer >= s->L) return fail(JM_ERR_ARG, "layer %d outside [0, %d)", layer, s->L);
        if (B < 0) return fail(JM_ERR_ARG, "B must be >= 0");
        if (B == 0) return 0;
        if (!x || !out) return fail(JM_ERR_ARG, "x and out must be non-NULL");
        if (!aligned(x, 16) || !aligned(out, 16)) return fail(JM_ERR_ARG, "x and out must be 16-byte aligned");
        return jm::dense_block(s, layer, x, B, out, (hipStream_t)stream);
    }
    if (!s->wt) return fail(JM_ERR_ARG, "router weights not set (jm_store_set_router)");
    if (layer < 0 || layer >= s->L) return fail(JM_ERR_ARG, "layer %d outside [0, %d)", layer, s->L);
    if (B < 0) return fail(JM_ERR_ARG, "B must be >= 0");
    if (B == 0) return 0;
    if (!x || !out) return fail(JM_ERR_ARG, "x and out must be non-NULL");
    if (!aligned(x, 16) || !aligned(out, 16)) return fail(JM_ERR_ARG, "x and out must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    if (int rc = jm::ffn_enqueue(s, layer, x, B, out, jm::FfnIo{}, true, st)) return rc;
    const int k = s->topk;
    if (topk_idx) JM_HIP(hipMemcpyAsync(topk_idx, s->w.top, (size_t)B * k * 4, hipMemcpyDeviceToDevice, st), "copy top-k");
    if (topk_w) JM_HIP(hipMemcpyAsync(topk_w, s->w.tw, (size_t)B * k * 4, hipMemcpyDeviceToDevice, st), "copy top-k weights");
    return 0;
}

int jm_layer_ffn_batch_noalloc(jm_store* s, int layer, const float* x, int B, float* out,
                               int32_t* topk_idx, float* topk_w, void* stream) {
    if (int rc = check_moe_store(s, "jm_layer_ffn_batch_noalloc")) return rc;
    if (!s->wt) return fail(JM_ERR_ARG, "router weights not set (jm_store_set_router)");
    if (layer < 0 || layer >= s->L) return fail(JM_ERR_ARG, "layer %d outside [0, %d)", layer, s->L);
    if (B < 0) return fail(JM_ERR_ARG, "B must be >= 0");
    if (B == 0) return 0;
    if (!x || !out) return fail(JM_ERR_ARG, "x and out must be non-NULL");
    if (!aligned(x, 16) || !aligned(out, 16)) return fail(JM_ERR_ARG, "x and out must be 16-byte aligned");
    const size_t need = jm::ws_bytes(s, B);
    if (need > (size_t)JM_NOALLOC_SCRATCH_BYTES)
        return fail(JM_ERR_SHAPE, "B=%d needs %zu bytes of workspace; the fixed no-allocation workspace holds %zu "
                    "(use jm_layer_ffn_batch, or fewer tokens per call)", B, need, (size_t)JM_NOALLOC_SCRATCH_BYTES);
    void* base = (s->device >= 0 && s->device < MAX_DEVICES) ? scratch_ptr[s->device] : nullptr;
    if (!base) return fail(JM_ERR_ARG, "the no-allocation workspace of device %d is not resolved", s->device);
    JM_HIP(hipSetDevice(s->device), "hipSetDevice");
    jm::Ws w;
    jm::ws_layout(s, B, (char*)base, &w);
    hipStream_t st = (hipStream_t)stream;
    if (int rc = jm::ffn_enqueue(s, layer, x, B, out, jm::FfnIo{}, false, st, &w)) return rc;
    const int k = s->topk;
    if (topk_idx) JM_HIP(hipMemcpyAsync(topk_idx, w.top, (size_t)B * k * 4, hipMemcpyDeviceToDevice, st), "copy top-k");
    if (topk_w) JM_HIP(hipMemcpyAsync(topk_w, w.tw, (size_t)B * k * 4, hipMemcpyDeviceToDevice, st), "copy top-k weights");
    return 0;
}

int jm_store_profile(jm_store* s, int enable) {
    if (int rc = check_store(s)) return rc;
    JM_HIP(hipSetDevice(s->device), "hipSetDevice");
    if (enable && !s->prof) {
        // no system-scope fence: the marks then cost the stream little more
        // than the kernels' own boundaries
        for (int i = 0; i <= JM_STAGES; i++)
            JM_HIP(hipEventCreateWithFlags(&s->ev[i], hipEventDisableSystemFence), "hipEventCreate");
        s->prof = 1;
    } else if (!enable && s->prof) {
        JM_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
        for (int i = 0; i <= JM_STAGES; i++) (void)hipEventDestroy(s->ev[i]);
        s->prof = 0;
    }
    return 0;
}

int jm_store_stage_ms(jm_store* s, float* ms, int n) {
    if (int rc = check_store(s)) return rc;
    if (!s->prof) return fail(JM_ERR_ARG, "profiling is off (jm_store_profile)");
    if (!ms || n < JM_STAGES) return fail(JM_ERR_ARG, "need room for %d stage times", JM_STAGES);
    JM_HIP(hipEventSynchronize(s->ev[JM_STAGES]), "hipEventSynchronize");
    for (int i = 0; i < JM_STAGES; i++)
        JM_HIP(hipEventElapsedTime(&ms[i], s->ev[i], s->ev[i + 1]), "hipEventElapsedTime");
    return 0;
}

int jm_store_copy_workspace(const jm_store* s, int field, void* dst, uint64_t bytes, void* stream) {
    if (int rc = check_moe_store(s, "jm_store_copy_workspace")) return rc;
    if (!dst) return fail(JM_ERR_ARG, "destination is NULL");
    const size_t nslot = (size_t)s->last_B * s->topk;
    const void* src = nullptr;
    size_t cap = 0;
    switch (field) {
        case JM_WS_LOGITS: src = s->w.logits; cap = (size_t)s->last_B * s->E * 4; break;
        case JM_WS_SEG_OFF: src = s->w.seg_off; cap = (size_t)(s->E + 1) * 4; break;
        case JM_WS_SEG_SLOT: src = s->w.seg_slot; cap = nslot * 4; break;
        case JM_WS_ACTIVE: src = s->w.active; cap = (size_t)s->E * 4; break;
        case JM_WS_N_ACTIVE: src = s->w.n_active; cap = 4; break;
        case JM_WS_FIRST_SLOT: src = s->w.first_slot; cap = (size_t)s->E * 4; break;
        case JM_WS_ACT: src = s->w.act; cap = nslot * s->m * 4; break;
        case JM_WS_Y: src = s->w.y; cap = nslot * s->d * 4; break;
        case JM_WS_N_DENSE_TILES: src = s->w.n_tiles; cap = 4; break;
        default: return fail(JM_ERR_ARG, "unknown workspace field %d", field);
    }
    if (!src || s->last_B == 0) return fail(JM_ERR_ARG, "no call has run on this store yet");
    if (s->dec_last && field != JM_WS_LOGITS && field != JM_WS_ACT)
        return fail(JM_ERR_ARG, "field %d is written only by the dispatch path (B * topk > %d)", field, JM_DEC_SLOTS);
    if (bytes > cap) return fail(JM_ERR_ARG, "%llu bytes requested, field holds %zu", (unsigned long long)bytes, cap);
    JM_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream), "workspace copy");
    return 0;
}

int jm_router(const void* gate_w, int dtype, const float* x, int B, int E, int d, int topk,
              int renorm, float* logits, int32_t* top, float* tw, void* stream) {
    if (!gate_w || !x || !logits || !top || !tw) return fail(JM_ERR_ARG, "NULL argument to jm_router");
    if (B < 0 || E <= 0 || E > JM_MAX_E || d <= 0 || d % 8 || topk <= 0 || topk > E || topk > JM_MAX_TOPK)
        return fail(JM_ERR_SHAPE, "bad router shape (B=%d E=%d d=%d topk=%d)", B, E, d, topk);
    if (B == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    JM_HIP(jm::launch_router(gate_w, dtype == JM_DTYPE_BF16, x, logits, B, E, d, st), "router launch");
    JM_HIP(jm::launch_topk(logits, B, E, topk, renorm ? 1 : 0, top, tw, st), "top-k launch");
    return 0;
}

int jm_dispatch(const int32_t* top, int nslot, int E, int topk, int32_t* seg_off, int32_t* seg_slot,
                int32_t* active, int32_t* n_active, int32_t* first_slot, int32_t* comb, void* stream) {
    if (!top || !seg_off || !seg_slot || !active || !n_active || !first_slot || !comb)
        return fail(JM_ERR_ARG, "NULL argument to jm_dispatch");
    if (nslot < 0 || nslot > JM_MAX_SLOTS || E <= 0 || E > JM_MAX_E || topk <= 0 || topk > JM_MAX_TOPK ||
        nslot % topk)
        return fail(JM_ERR_SHAPE, "need 0 <= nslot <= %d (a multiple of topk <= %d) and 0 < E <= %d",
                    JM_MAX_SLOTS, JM_MAX_TOPK, JM_MAX_E);
    int dev = 0, lds_max = 0;
    JM_HIP(hipGetDevice(&dev), "hipGetDevice");
    JM_HIP(hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev), "hipDeviceGetAttribute");
    if ((size_t)jm::dispatch_lds_ints(nslot, E) * 4 > (size_t)lds_max)
        return fail(JM_ERR_SHAPE, "%d slots over %d experts exceed the dispatch's LDS", nslot, E);
    JM_HIP(jm::launch_dispatch(top, nslot, E, topk, seg_off, seg_slot, active, n_active, first_slot, comb,
                               (hipStream_t)stream), "dispatch launch");
    return 0;
}

int jm_q4_dequant(float* out, const uint8_t* packed, const uint16_t* scales, int64_t numel, int group,
                  void* stream) {
    if (!out || !packed || !scales) return fail(JM_ERR_ARG, "NULL argument to jm_q4_dequant");
    if (group != 32 && group != 64) return fail(JM_ERR_SHAPE, "group must be 32 or 64");
    if (numel < 0) return fail(JM_ERR_SHAPE, "numel must be >= 0");
    JM_HIP(jm::launch_dequant(packed, scales, numel, group, out, (hipStream_t)stream), "dequant launch");
    return 0;
}

int jm_q4_gemm_f32(float* out, const float* X, int T, const uint8_t* packed, const uint16_t* scales,
                   int m, int d, int group, void* stream) {
    if (!out || !X || !packed || !scales) return fail(JM_ERR_ARG, "NULL argument to jm_q4_gemm_f32");
    if (group != 32 && group != 64) return fail(JM_ERR_SHAPE, "group must be 32 or 64");
    if (T < 0 || m < 0 || d <= 0 || d % group) return fail(JM_ERR_SHAPE, "bad q4_gemm shape (T=%d m=%d d=%d)", T, m, d);
    if (d / group > 64) return fail(JM_ERR_SHAPE, "d / group must be <= 64");
    if ((d / 2) % 16) return fail(JM_ERR_SHAPE, "d must be a multiple of 32 (16-byte packed rows)");
    if (!aligned(packed, 16) || !aligned(X, 16)) return fail(JM_ERR_ARG, "packed and X must be 16-byte aligned");
    if (T == 0 || m == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    // from jm_set_q4_gemm_min_tokens tokens on the matrix cores (int8 digit
    // pairs of X)
    const bool mfma = T >= g_q4_gemm_min_t.load(std::memory_order_relaxed) && jm::q4_gemm_mfma_ok(m, d, group) &&
                      aligned(scales, 16);
    const size_t ng = (size_t)d / group;
    const size_t dig_bytes = align256((size_t)T * ng * JM_NDIG * (group / 8) * 4);
    const size_t sc_bytes = align256((size_t)T * ng * 4);
    const size_t need = mfma ? jm::q4_gemm_mfma_ws(T, m, d, group) : dig_bytes + sc_bytes;
    PluginWs ws;
    if (int rc = plugin_ws(st, need, &ws)) return rc;
    hipError_t e;
    if (mfma) {
        e = jm::launch_q4_gemm_mfma(packed, scales, X, T, m, d, group, ws.p, out, st);
    } else {
        uint32_t* dig = (uint32_t*)ws.p;
        float* dsc = (float*)((char*)ws.p + dig_bytes);
        e = jm::launch_prep_digits(X, d, T, d, group, dig, dsc, st);
        if (e == hipSuccess) e = jm::launch_q4_rows(packed, scales, m, d, group, dig, dsc, T, out, m, st);
    }
    const hipError_t f = ws.async ? hipFreeAsync(ws.p, st) : hipSuccess;
    if (e != hipSuccess) return hip_fail(e, "q4_gemm launch");
    if (f != hipSuccess) return hip_fail(f, "hipFreeAsync");
    return 0;
}

int jm_set_q4_gemm_min_tokens(int tokens) {
    if (tokens < 0) return fail(JM_ERR_ARG, "tokens must be >= 0 (0 = default)");
    g_q4_gemm_min_t.store(tokens == 0 ? JM_Q4_GEMM_MIN_T : tokens, std::memory_order_relaxed);
    return 0;
}

int jm_get_q4_gemm_min_tokens(void) { return g_q4_gemm_min_t.load(std::memory_order_relaxed); }

// ------------------------------------------------- block stages one by one

int jm_expert_gateup(jm_store* s, int layer, const float* x, const int32_t* top, int B, float* act, void* stream) {
    jm::RouteArgs r{};
    jm::ExpertArgs a{};
    if (int rc = stage_setup(s, layer, top, B, "jm_expert_gateup", (hipStream_t)stream, &r, &a)) return rc;
    if (B == 0) return 0;
    if (!x || !act || !aligned(x, 16) || !aligned(act, 16))
        return fail(JM_ERR_ARG, "jm_expert_gateup: x and act must be non-NULL and 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    const jm::Ws& w = s->w;
    // the tokens' digits as the router writes them, then gate/up + SwiGLU
    // of every slot into act (fp32) and the act digits
    JM_HIP(jm::launch_prep_digits(x, s->d, B, s->d, s->group, w.xdig, w.xscale, st, s->ndig), "digits launch");
    a.act = act;
    JM_HIP(jm::launch_gateup(a, a.umax, st), "gate/up launch");
    return 0;
}

int jm_expert_down(jm_store* s, int layer, const float* act, const int32_t* top, const float* tw, int B, float* y,
                   void* stream) {
    jm::RouteArgs r{};
    jm::ExpertArgs a{};
    if (int rc = stage_setup(s, layer, top, B, "jm_expert_down", (hipStream_t)stream, &r, &a)) return rc;
    if (B == 0) return 0;
    if (!act || !tw || !y || !aligned(act, 16) || !aligned(y, 16))
        return fail(JM_ERR_ARG, "jm_expert_down: act, tw and y must be non-NULL, act and y 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    const jm::Ws& w = s->w;
    // act's digits in 32-value groups, as the gate/up epilogue writes them,
    // then y[slot] = tw[slot] * (down rows . act[slot])
    JM_HIP(jm::launch_prep_digits(act, s->m, B * s->topk, s->m, 32, w.adig, w.ascale, st, s->ndig), "digits launch");
    a.tw = tw;
    a.y = y;
    JM_HIP(jm::launch_down(a, a.umax, st), "down launch");
    return 0;
}

int jm_combine(jm_store* s, const float* y, const int32_t* top, int B, float* out, void* stream) {
    jm::RouteArgs r{};
    jm::ExpertArgs a{};
    if (int rc = stage_setup(s, 0, top, B, "jm_combine", (hipStream_t)stream, &r, &a)) return rc;
    if (B == 0) return 0;
    if (!y || !out || !aligned(y, 16) || !aligned(out, 16))
        return fail(JM_ERR_ARG, "jm_combine: y and out must be non-NULL and 16-byte aligned");
    JM_HIP(jm::launch_combine(y, s->w.comb, B, s->topk, s->d, nullptr, out, (hipStream_t)stream), "combine launch");
    return 0;
}

int jm_expert_job(const jm_expert_job_t* j, void* stream) {
    if (!j) return fail(JM_ERR_ARG, "job is NULL");
    if (!j->pk_g || !j->sc_g || !j->pk_u || !j->sc_u || !j->pk_d || !j->sc_d || !j->x || !j->scratch)
        return fail(JM_ERR_ARG, "jm_expert_job: NULL pointer in the job");
    const int m = j->m_gg, d = j->d_in, G = j->group;
    if (G != 32 && G != 64) return fail(JM_ERR_SHAPE, "group must be 32 or 64");
    if (m <= 0 || d <= 0 || j->m_d != d || j->d_m != m)
        return fail(JM_ERR_SHAPE, "jm_expert_job: need m_gg, d_in > 0, m_d == d_in and d_m == m_gg (got %d %d %d %d)",
                    m, d, j->m_d, j->d_m);
    if (d % G || m % G || d / G > 64 || m / G > 64 || (d / 2) % 16 || (m / 2) % 16)
        return fail(JM_ERR_SHAPE, "jm_expert_job: d_in and m_gg must be multiples of 32 and of group, at most 64 groups");
    if (!aligned(j->pk_g, 16) || !aligned(j->pk_u, 16) || !aligned(j->pk_d, 16) || !aligned(j->x, 16))
        return fail(JM_ERR_ARG, "jm_expert_job: packed records and x must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    const size_t dx = align256((size_t)(d / G) * JM_NDIG * (G / 8) * 4), sx = align256((size_t)(d / G) * 4);
    const size_t gu = align256((size_t)2 * m * 4);
    const size_t da = align256((size_t)(m / G) * JM_NDIG * (G / 8) * 4), sa = align256((size_t)(m / G) * 4);
    PluginWs ws;
    if (int rc = plugin_ws(st, dx + sx + gu + da + sa, &ws)) return rc;
    char* p = (char*)ws.p;
    uint32_t* dig_x = (uint32_t*)p;
    float* sc_x = (float*)(p + dx);
    float* gbuf = (float*)(p + dx + sx);
    uint32_t* dig_a = (uint32_t*)(p + dx + sx + gu);
    float* sc_a = (float*)(p + dx + sx + gu + da);
    float* act = j->scratch;
    float* wout = j->scratch + m;
    // g and u rows against x, act = SiLU(g) * u (expert_ffn.c:165-172),
    // then prob * (down rows . act) (:173-190)
    hipError_t e = jm::launch_prep_digits(j->x, d, 1, d, G, dig_x, sc_x, st);
    if (e == hipSuccess) e = jm::launch_q4_rows(j->pk_g, j->sc_g, m, d, G, dig_x, sc_x, 1, gbuf, m, st);
    if (e == hipSuccess) e = jm::launch_q4_rows(j->pk_u, j->sc_u, m, d, G, dig_x, sc_x, 1, gbuf + m, m, st);
    if (e == hipSuccess) e = jm::launch_swiglu_vec(gbuf, m, act, st);
    if (e == hipSuccess) e = jm::launch_prep_digits(act, m, 1, m, G, dig_a, sc_a, st);
    if (e == hipSuccess) e = jm::launch_q4_rows(j->pk_d, j->sc_d, d, m, G, dig_a, sc_a, 1, wout, d, st);
    if (e == hipSuccess) e = jm::launch_scale_vec(wout, d, j->prob, st);
    const hipError_t f = ws.async ? hipFreeAsync(ws.p, st) : hipSuccess;
    if (e != hipSuccess) return hip_fail(e, "expert_job launch");
    if (f != hipSuccess) return hip_fail(f, "hipFreeAsync");
    return 0;
}

int jm_q4_gemv_f32(float* out, const float* x, const uint8_t* packed, const uint16_t* scales,
                   int m, int d, int group, void* stream) {
    return jm_q4_gemm_f32(out, x, 1, packed, scales, m, d, group, stream);
}

}  // extern "C"
