// Dense branch of the grouped Q4 expert product (gfx950 int8 MFMA), taken by
// the experts whose segment holds at least `dense_min` tokens (prefill-sized
// batches, skewed routing).  The same contraction as the wave-item kernels
// in jm_experts.hip (decode_kernel.c:1365-1383), as tiled products:
//
//   k_gateup_mfma  per (expert, 32-token tile, 128 intermediate rows):
//                  G = X . Wg^T and U = X . Wu^T over d, then
//                  act = (G / (1 + expf_fast(-G))) * U, written as int8
//                  digit pairs for the down product (and as float)
//   k_down_mfma    per (expert, 32-token tile, 512 hidden rows in two passes):
//                  y[slot] = w_slot * (act . Wd^T) over the intermediate
//
// Operands:
//   weights  the signed nibbles q - 8 as int8, unpacked in registers from
//            the packed record (each wave streams its own rows);
//   tokens   two int8 digits per value with one float scale per token and
//            Q4 group (jm_device.h: encode_i8_group_wave): the router kernel
//            writes them for x, the gate/up epilogue for act.
// v_mfma_i32_32x32x32_i8 tiles, tokens on the A side (i), weight rows on the
// B side (n), in the lane layout of jm_mx.h; the lo plane's accumulator
// starts at -8 times the tokens' group sums (wdigits takes q, not q - 8).
// So a lane holds one weight row and 16 tokens: the row's group scale is one
// value per lane, the tokens' scales 16.
//
// Per Q4 group of a lane's row and its 16 tokens the two digit products are
// exact int32 sums (hi and lo), combined as 256 hi + lo (exact, below 2^24 in
// magnitude), converted to float and accumulated as
//   acc += (float(256 hi + lo) * s_token) * s_row.
//
// The whole contraction of a tile's 32 tokens (both digit planes) stays in
// LDS for the block's lifetime, so the main loop has no barriers: each wave
// streams its weight rows through a ring of register stages and reads its
// token operands from LDS.
#include <atomic>
#include <type_traits>

#include "jm_device.h"
#include "jm_items.h"
#include "jm_kernels.h"
#include "jm_mx.h"

namespace jm {

constexpr int MT = JM_DENSE_TILE;   // tokens per tile (32)
static_assert(MT == 32, "the tile's tokens are the 32 A rows of one MFMA");
constexpr int MTHREADS = 512;       // 8 waves per block
constexpr int NWAVE = MTHREADS / 64;
constexpr int GU_ROWS = 128;        // intermediate rows of a gate/up block (both matrices)
constexpr int DN_ROWS = 256;        // hidden rows of one pass of a down block (8 waves x 32)
constexpr int DN_BLOCK_ROWS = 512;  // hidden rows of a down block: two passes over its staged act digits
constexpr int KMAX = 2048;          // longest contraction the kernels take
constexpr int KPAD = 16;            // bytes of padding per LDS token row (bank spread)
constexpr int KPH_MAX = 1024;       // columns of a token phase (the tokens' LDS holds one phase)
constexpr int SSC = 256;            // columns of a weight super-stage: 128 bytes (one cache line) per row
constexpr int WRS = 144;            // LDS bytes per row of a wave's weight buffer (128 + bank spread)
constexpr int WBUF = 32 * WRS;      // one super-stage of a wave's 32 rows

struct TileInfo {
    int slot0;      // first position of the tile in seg_slot
    int nt;         // tokens in the tile (1..MT)
    int e;          // expert id
};

__device__ __forceinline__ TileInfo tile_at(const ExpertArgs& a, int t) {
    const int2 tl = a.tiles[t];
    const ExpertWork wk = a.work[tl.x];
    TileInfo ti;
    ti.slot0 = wk.s0 + tl.y * MT;
    ti.nt = min(MT, wk.n - tl.y * MT);
    ti.e = wk.e;
    return ti;
}

// LDS layout of a block with contraction length K:
//   q    the tile's token digits of one phase (kph columns): token i's plane
//        p (0 hi, 1 lo) at q + (p * MT + i) * (kph + KPAD), in int8 operand
//        order; kph + KPAD = 16 mod 256 bytes puts the 16 token rows of a
//        ds_read_b128 half-wave in distinct banks
//   s    the tokens' scales over all of K: group g, token i at s[g * MT + i]
//   c    -8 times the tokens' group sums of 256 h + l, laid out as s
//   tok  the tile's token (gate/up) or slot (down) rows, then its slot ids
//        (gate/up) or routing weights (down)
//   w    per wave, two super-stage buffers of its 32 weight rows (WRS bytes
//        per row)
struct Lay {
    int kph;
    size_t s, c, tok, w, total;
    __host__ __device__ constexpr Lay(int K, int G)
        : kph(K < KPH_MAX ? K : KPH_MAX),
          s((size_t)2 * MT * ((K < KPH_MAX ? K : KPH_MAX) + KPAD)),
          c(s + (size_t)(K / G) * MT * 4),
          tok(c + (size_t)(K / G) * MT * 4),
          w(tok + 2 * MT * 4),
          total(tok + 2 * MT * 4 + (size_t)NWAVE * 2 * WBUF) {}
};

// Stage the tile's digit planes, columns [c0, c0 + kph), into q: token i's
// rows are row src[i] of hi/lo [.][K].  All threads; no branches, so each
// thread's loads of a batch are all in flight together (indices past the
// end repeat the last piece, stored again to the same place).
__device__ __forceinline__ void stage_phase(const int8_t* __restrict__ hi, const int8_t* __restrict__ lo,
                                            const int* src, int K, int c0, int kph, int8_t* q) {
    constexpr int BATCH = 8;
    // an opaque thread index: the addresses below are recomputed at each
    // staging instead of being kept live across the caller's main loop
    int tid = threadIdx.x;
    __asm__ volatile("" : "+v"(tid));
    const int KP = kph + KPAD;
    const int pieces = kph / 16;                  // 16-byte pieces per token row
    const int total = 2 * MT * pieces;
    // u / pieces as a multiply-high: exact for u * pieces < 2^32
    const unsigned magic = 0xFFFFFFFFu / (unsigned)pieces + 1u;
    for (int base = 0; base < total; base += MTHREADS * BATCH) {
        uint4 v[BATCH];
        int dst[BATCH];
#pragma unroll
        for (int j = 0; j < BATCH; j++) {
            const unsigned u = (unsigned)min(base + j * MTHREADS + tid, total - 1);
            const int r = (int)__umulhi(u, magic);                // plane * MT + token
            const int pc = (int)u - r * pieces;
            v[j] = *(const uint4*)((r >= MT ? lo : hi) + (size_t)src[r & (MT - 1)] * K + c0 + pc * 16);
            dst[j] = r * KP + pc * 16;
        }
#pragma unroll
        for (int j = 0; j < BATCH; j++) *(uint4*)(q + dst[j]) = v[j];
    }
}

// The tile's token scales and group-sum corrections of ng groups (padding
// tokens, i >= nt: 0); token row r's groups start at r * stride.
__device__ __forceinline__ void stage_scales(const float* __restrict__ sc, const int* __restrict__ qc, const int* src,
                                             int nt, int ng, int stride, float* s, int* c) {
    for (int u = threadIdx.x; u < ng * MT; u += MTHREADS) {
        const int g = u / MT, i = u % MT;
        const size_t o = (size_t)src[i] * stride + g;
        s[u] = i < nt ? sc[o] : 0.0f;
        c[u] = i < nt ? -8 * qc[o] : 0;
    }
}

// A wave's weight stream.  A super-stage is SSC columns of the wave's 32
// rows: one 128-byte line per row, read as 4 coalesced loads per lane (load
// k: lane L takes row 8 k + L / 8, bytes 16 (L % 8) of the line), then
// written to the wave's own LDS buffer and read back per stage in the MFMA
// layout (lane n % 32 its row).  Two super-stages are in flight.  With the
// lines come this lane's row's scales of the super-stage's groups (4 stages
// x 64 / G groups).
template <int G>
struct WStream {
    static constexpr int NSC = 4 * 64 / G;        // scales per super-stage
    typedef typename std::conditional<NSC == 4, uint2, uint4>::type ScT;
    uint4 wb[2][4];                               // [0]: the next super-stage, [1]: the one after
    ScT sc[2];
    const uint8_t* wbase;                         // the wave's first row
    const uint8_t* srow;                          // this lane's row's scales
    size_t rowb;                                  // bytes per row
    int nss;                                      // super-stages over K
    __device__ __forceinline__ void load(int slot, int S) {
        S = S < nss ? S : nss - 1;
        const int L = threadIdx.x & 63;
#pragma unroll
        for (int k = 0; k < 4; k++)
            wb[slot][k] = *(const uint4*)(wbase + (size_t)(8 * k + L / 8) * rowb + (size_t)S * (SSC / 2) + 16 * (L % 8));
        sc[slot] = *(const ScT*)(srow + (size_t)S * NSC * 2);
    }
    // write the next super-stage's lines to LDS buffer wl and return its
    // scales; the one after moves up and super-stage S is requested behind it
    __device__ __forceinline__ ScT advance(uint8_t* wl, int S) {
        const int L = threadIdx.x & 63;
#pragma unroll
        for (int k = 0; k < 4; k++) *(uint4*)(wl + (8 * k + L / 8) * WRS + 16 * (L % 8)) = wb[0][k];
        const ScT r = sc[0];
#pragma unroll
        for (int k = 0; k < 4; k++) wb[0][k] = wb[1][k];
        sc[0] = sc[1];
        load(1, S);
        return r;
    }
};

// scale u (0..NSC-1) of a super-stage's packed fp16 scales, as float
template <int G>
__device__ __forceinline__ float sc_at(const typename WStream<G>::ScT& v, int u) {
    uint32_t w;
    if (G == 64) w = u < 2 ? ((const uint2&)v).x : ((const uint2&)v).y;
    else w = u < 2 ? ((const uint4&)v).x : u < 4 ? ((const uint4&)v).y : u < 6 ? ((const uint4&)v).z : ((const uint4&)v).w;
    return fp16_hw((uint16_t)(w >> (16 * (u & 1))));
}

// A wave's token operands of one stage: both sub-steps, both digit planes.
// Stage columns (relative to the token phase) start at c; lane half h.
//   G = 64: one group; sub-step u takes values 32 h + 16 u + 0..15.
//   G = 32: two groups; sub-step u (= group u) takes values 32 u + 16 h + 0..15.
struct AOps {
    int4v ah0, ah1, al0, al1;
};

template <int G>
__device__ __forceinline__ AOps load_aops(const int8_t* qh, const int8_t* ql, int c, int h) {
    const int o0 = G == 64 ? c + 32 * h : c + 16 * h;
    const int o1 = G == 64 ? o0 + 16 : o0 + 32;
    return AOps{*(const int4v*)(qh + o0), *(const int4v*)(qh + o1), *(const int4v*)(ql + o0),
                *(const int4v*)(ql + o1)};
}

// The weight operands of one stage from the wave's LDS buffer (row n, lane
// half h), as int8 (q - 8): sub-step 0 and 1 (see AOps).
template <int G>
__device__ __forceinline__ void load_bops(const uint8_t* wl, int n, int h, int cs, int4v& b0, int4v& b1) {
    const uint8_t* r = wl + n * WRS + 32 * cs;
    if (G == 64) {
        const uint4 w = *(const uint4*)(r + 16 * h);
        b0 = wdigits(w.x, w.y);
        b1 = wdigits(w.z, w.w);
    } else {
        const uint2 w0 = *(const uint2*)(r + 8 * h), w1 = *(const uint2*)(r + 16 + 8 * h);
        b0 = wdigits(w0.x, w0.y);
        b1 = wdigits(w1.x, w1.y);
    }
}

// The 16 tokens' scales of one group (this lane's half h)
struct SxOps {
    float4 s[4];
};

__device__ __forceinline__ SxOps load_sx(const float* s, int g, int h) {
    const float* sg = s + (size_t)g * MT + 4 * h;
    return SxOps{{*(const float4*)(sg), *(const float4*)(sg + 8), *(const float4*)(sg + 16),
                  *(const float4*)(sg + 24)}};
}

// The 16 tokens' corrections of one group (this lane's half h), in the
// accumulator layout: register v holds token 8 (v / 4) + 4 h + v % 4.
__device__ __forceinline__ int16v load_corr(const int* c, int g, int h) {
    const int* cg = c + (size_t)g * MT + 4 * h;
    const int8v a = __builtin_shufflevector(*(const int4v*)cg, *(const int4v*)(cg + 8), 0, 1, 2, 3, 4, 5, 6, 7);
    const int8v b = __builtin_shufflevector(*(const int4v*)(cg + 16), *(const int4v*)(cg + 24), 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
}

// The integer products of one stage: per group of the stage, hi and lo
// digit planes.  The lo products accumulate onto o.il, which the caller sets
// to the group's corrections: with unsigned nibbles q, 256 ih + il is then
// the exact sum of (256 h + l) (q - 8).
template <int G>
struct IOps {
    int16v ih[64 / G], il[64 / G];
};

template <int G>
__device__ __forceinline__ void stage_mfma(IOps<G>& o, const AOps& a, const int4v& b0, const int4v& b1) {
    if (G == 64) {
        o.ih[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a.ah0, b0, int16v{}, 0, 0, 0);
        o.il[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a.al0, b0, o.il[0], 0, 0, 0);
        o.ih[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a.ah1, b1, o.ih[0], 0, 0, 0);
        o.il[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a.al1, b1, o.il[0], 0, 0, 0);
    } else {
        o.ih[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a.ah0, b0, int16v{}, 0, 0, 0);
        o.il[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a.al0, b0, o.il[0], 0, 0, 0);
        o.ih[G == 64 ? 0 : 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a.ah1, b1, int16v{}, 0, 0, 0);
        o.il[G == 64 ? 0 : 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a.al1, b1, o.il[G == 64 ? 0 : 1], 0, 0, 0);
    }
}

// acc += 256 * ih + il of one group, times each token's scale, times the
// row's scale
__device__ __forceinline__ void group_acc(floatx16& acc, const int16v& ih, const int16v& il, const SxOps& sx,
                                          float ws) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float sv[4] = {sx.s[k].x, sx.s[k].y, sx.s[k].z, sx.s[k].w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int v = 4 * k + j;
            const int iv = ih[v] * 256 + il[v];
            acc[v] = __builtin_fmaf(__fmul_rn((float)iv, sv[j]), ws, acc[v]);
        }
    }
}

// Where a block's token digits come from, for the phase restaging.
struct TokSrc {
    const int8_t* hi;
    const int8_t* lo;
    const int* rows;
    int K;
};

// The contraction of one wave: its 32 weight rows (lane n = l % 32 holds
// row n) against the tile's 32 tokens over K columns, into acc.  The token
// digits of the first phase and all the scales are in LDS, and the weight
// stream's first two super-stages are in flight.  Stage c's token operands
// are read one stage ahead; for G = 64 stage c's MFMAs are issued before
// stage c - 1's scale epilogue (products alternate by stage parity), so
// each wave has independent MFMA and VALU work at every point.  At each
// token phase boundary the block restages the tokens (two barriers).
template <int G, bool AHEAD = true>
__device__ __forceinline__ void wave_product(floatx16& acc, WStream<G>& ws, uint8_t* wl, int8_t* q,
                                             const float* s, const int* cc, const TokSrc& ts, const Lay& ly) {
    constexpr int NG = 64 / G;                    // groups per stage
    constexpr bool PIPE = G == 64;
    const int lane = threadIdx.x & 63;
    const int n = lane & 31, h = lane >> 5;
    const int KP = ly.kph + KPAD;
    const int8_t* qh = q + (size_t)n * KP;
    const int8_t* ql = q + (size_t)(MT + n) * KP;
    const int sspp = ly.kph / SSC;                // super-stages per token phase
    const int nss = ws.nss;
    AOps ab[2];
    IOps<G> pr[PIPE ? 2 : 1];
    float wsp[PIPE ? 2 : 1][NG];
    // AHEAD (G = 64): the next stage's weight operands (within a
    // super-stage) and this stage's token scales (for the epilogue of the
    // stage before) are requested one stage ahead, so that the stage's
    // MFMAs and epilogue wait on no LDS read of their own stage
    int4v bn0, bn1;
    SxOps sxn;
    const int nph = (nss + sspp - 1) / sspp;
#pragma unroll 1
    for (int ph = 0; ph < nph; ph++) {
      if (ph > 0) {
        __syncthreads();                          // every wave is done with the previous phase
        stage_phase(ts.hi, ts.lo, ts.rows, ts.K, ph * ly.kph, ly.kph, q);
        __syncthreads();
      }
      const int s_end = min(nss, (ph + 1) * sspp);
#pragma unroll 1
      for (int S = ph * sspp; S < s_end; S++) {
        const bool pstart = S % sspp == 0, pend = S + 1 == s_end;
        uint8_t* wbuf = wl + (S & 1) * WBUF;
        const typename WStream<G>::ScT scs = ws.advance(wbuf, S + 2);
        const int cp = (S % sspp) * SSC;          // the super-stage's first column within the phase
        if (PIPE && pstart) ab[0] = load_aops<G>(qh, ql, cp, h);
        if (PIPE && AHEAD) load_bops<G>(wbuf, n, h, 0, bn0, bn1);
#pragma unroll
        for (int cs = 0; cs < 4; cs++) {
            __builtin_amdgcn_sched_barrier(0);
            const int c = 4 * S + cs;             // stage index over K
            const int cur = cs & 1, prv = cur ^ 1;
            const int pc = PIPE ? cur : 0, pp = PIPE ? prv : 0;
            if (PIPE && !AHEAD) {
                if (!(cs == 3 && pend)) ab[prv] = load_aops<G>(qh, ql, cp + 64 * (cs + 1), h);
                SxOps sxp;
                if (c > 0) sxp = load_sx(s, c - 1, h);
                int4v b0, b1;
                load_bops<G>(wbuf, n, h, cs, b0, b1);
                pr[pc].il[0] = load_corr(cc, c, h);
                stage_mfma<G>(pr[pc], ab[cur], b0, b1);
                wsp[pc][0] = sc_at<G>(scs, cs);
                if (c > 0) group_acc(acc, pr[pp].ih[0], pr[pp].il[0], sxp, wsp[pp][0]);
            } else if (PIPE) {
                const int4v b0 = bn0, b1 = bn1;
                pr[pc].il[0] = load_corr(cc, c, h);
                const SxOps sxp = sxn;
                // requests for the next stage
                if (!(cs == 3 && pend)) ab[prv] = load_aops<G>(qh, ql, cp + 64 * (cs + 1), h);
                if (cs < 3) load_bops<G>(wbuf, n, h, cs + 1, bn0, bn1);
                sxn = load_sx(s, c, h);
                stage_mfma<G>(pr[pc], ab[cur], b0, b1);
                wsp[pc][0] = sc_at<G>(scs, cs);
                if (c > 0) group_acc(acc, pr[pp].ih[0], pr[pp].il[0], sxp, wsp[pp][0]);
            } else {
                ab[cur] = load_aops<G>(qh, ql, cp + 64 * cs, h);
                int4v b0, b1;
                load_bops<G>(wbuf, n, h, cs, b0, b1);
#pragma unroll
                for (int u = 0; u < NG; u++) pr[0].il[u] = load_corr(cc, NG * c + u, h);
                stage_mfma<G>(pr[0], ab[cur], b0, b1);
#pragma unroll
                for (int u = 0; u < NG; u++) wsp[0][u] = sc_at<G>(scs, NG * cs + u);
#pragma unroll
                for (int u = 0; u < NG; u++)
                    group_acc(acc, pr[0].ih[u], pr[0].il[u], load_sx(s, NG * c + u, h), wsp[0][u]);
            }
        }
      }
    }
    if (PIPE) {
        // the last stage's epilogue (stage 4 nss - 1 is odd: its products sit in buffer 1)
        group_acc(acc, pr[PIPE ? 1 : 0].ih[0], pr[PIPE ? 1 : 0].il[0], AHEAD ? sxn : load_sx(s, 4 * nss - 1, h),
                  wsp[PIPE ? 1 : 0][0]);
    }
}

// ------------------------------------------------------------------ gate/up

template <int G>
__device__ __forceinline__ void gateup_tile(const ExpertArgs& a, const TileInfo& ti, int rblk, unsigned char* sm) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int d = a.d, m = a.m, ng = d / G;
    const Lay ly(d, G);
    const int mat = w & 1, rq = w >> 1;           // this wave: gate (0) or up (1), rows 32 rq .. 32 rq + 31
    const int r0 = rblk * GU_ROWS;                // the block's first intermediate row
    int8_t* q = (int8_t*)sm;
    float* s = (float*)(sm + ly.s);
    int* cc = (int*)(sm + ly.c);
    int* tok = (int*)(sm + ly.tok);
    uint8_t* wl = sm + ly.w + (size_t)w * 2 * WBUF;
    int* slots = tok + MT;
    if (tid < MT) {
        const int sl = a.seg_slot[ti.slot0 + (tid < ti.nt ? tid : 0)];   // padding: the first slot
        slots[tid] = sl;
        tok[tid] = sl / a.topk;
    }
    unsigned long long so, po;
    a.rec.get(mat, a.key0 + ti.e, so, po);
    const int n = lane & 31;
    const int wrow0 = r0 + 32 * rq;               // the wave's first row
    WStream<G> ws;
    ws.wbase = a.blob + po + (size_t)wrow0 * (d / 2);
    ws.srow = a.blob + so + (size_t)(wrow0 + n) * ng * 2;
    ws.rowb = d / 2;
    ws.nss = d / SSC;
    ws.load(0, 0);
    ws.load(1, 1);
    __syncthreads();
    stage_phase(a.xqh, a.xql, tok, d, 0, ly.kph, q);
    stage_scales(a.xqs, a.xqc, tok, ti.nt, ng, ng, s, cc);
    __syncthreads();
    floatx16 acc = {};
    wave_product<G>(acc, ws, wl, q, s, cc, TokSrc{a.xqh, a.xql, tok, d}, ly);

    // SwiGLU: both matrices' sums to LDS (over the token digits), then one
    // wave per (token, 64-row piece) forms act, its digits and scale
    __syncthreads();
    const int h = lane >> 5;
    constexpr int RP = GU_ROWS + 4;               // padded LDS row of one token's sums
    float* gu = (float*)sm;                       // [2][MT][RP]
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int i = 8 * (v / 4) + 4 * h + (v % 4);
        gu[((size_t)mat * MT + i) * RP + 32 * rq + n] = acc[v];
    }
    __syncthreads();
    const int mg = m / G;
    for (int it = w; it < MT * (GU_ROWS / 64); it += NWAVE) {
        const int i = it / (GU_ROWS / 64), piece = it % (GU_ROWS / 64);
        if (i >= ti.nt) continue;                 // wave-uniform
        const int slot = slots[i];
        const int rr = 64 * piece + lane;         // row within the block
        // SiLU(g) * u, dividing as the reference does (decode_kernel.c:1375)
        const float g = gu[(size_t)i * RP + rr], u = gu[((size_t)MT + i) * RP + rr];
        const float av = swiglu(g, u);
        const int row = r0 + rr;
        a.act[(size_t)slot * m + row] = av;
        const int g0 = row / G;                   // this lane's group (a G-lane segment)
        encode_i8_group_wave<G>(av, true, a.aqh + (size_t)slot * m + (size_t)g0 * G,
                                a.aql + (size_t)slot * m + (size_t)g0 * G, a.aqs + (size_t)slot * mg + g0,
                                a.aqc + (size_t)slot * mg + g0);
    }
}

// The experts under dense_min (n_tiles[1] entries of the small list) as
// wave items, run by the blocks past the tiles (first = the first such
// block, nblk = how many): virtual block v of 8 waves takes the 8
// consecutive items 8 (v % vpe) + w of small entry v / vpe.  The blocks are
// dispatched after the tiles' and fill the grid's last round.  The grid
// always has at least (row blocks) x (small experts) of them: an expert
// under dense_min frees a whole tile of max_tiles = slots / 32 + E.
template <int G, int LPR, int NDIG>
__device__ __forceinline__ void small_gateup(const ExpertArgs& a, int first, int nblk, unsigned char* sm) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int vpe = a.m / wi::GU_ROWS / NWAVE;
    const int nv = a.n_tiles[1] * vpe;
    // per group of 4 waves, the act-scale slots of wi::gateup_item
    float (*gm)[2][4] = (float (*)[2][4])sm;
    int (*gb)[2][4] = (int (*)[2][4])(sm + 2 * sizeof(float[2][4]));
#pragma unroll 1
    for (int v = first; v < nv; v += nblk) {
        wi::gateup_item<G, NDIG, LPR, 1, false>(a, a.top, a.small[v / vpe], (v % vpe) * NWAVE + w, gm[w >> 2],
                                                   gb[w >> 2]);
        __syncthreads();                          // the slots serve the next item
    }
}

// 1-D grid: block f < n_tiles x (m / GU_ROWS) is tile f % n_tiles, row
// block f / n_tiles; the rest run the small experts' items.
template <int G, int LPR, int NDIG>
__global__ void __launch_bounds__(MTHREADS, 1)
k_gateup_mfma(ExpertArgs a) {
    extern __shared__ __align__(16) unsigned char sm[];
    const int nt = a.n_tiles[0], ntb = nt * (a.m / GU_ROWS);
    const int f = blockIdx.x;
    if (f < ntb) {
        gateup_tile<G>(a, tile_at(a, f % nt), f / nt, sm);
        return;
    }
    small_gateup<G, LPR, NDIG>(a, f - ntb, (int)gridDim.x - ntb, sm);
}

// --------------------------------------------------------------------- down

template <int G>
__device__ __forceinline__ void down_tile(const ExpertArgs& a, const TileInfo& ti, int rblk, unsigned char* sm) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int d = a.d, m = a.m, ng = m / G;
    const Lay ly(m, G);
    int8_t* q = (int8_t*)sm;
    float* s = (float*)(sm + ly.s);
    int* cc = (int*)(sm + ly.c);
    int* tok = (int*)(sm + ly.tok);
    float* tws = (float*)(tok + MT);
    uint8_t* wl = sm + ly.w + (size_t)w * 2 * WBUF;
    if (tid < MT) {
        const int sl = a.seg_slot[ti.slot0 + (tid < ti.nt ? tid : 0)];   // padding: the first slot
        tok[tid] = sl;
        tws[tid] = a.tw[sl];
    }
    unsigned long long so, po;
    a.rec.get(2, a.key0 + ti.e, so, po);
    const int n = lane & 31, h = lane >> 5;
    WStream<G> ws;
    ws.rowb = m / 2;
    ws.nss = m / SSC;
    auto start = [&](int pass) __attribute__((always_inline)) {
        const int wrow0 = rblk * DN_BLOCK_ROWS + pass * DN_ROWS + 32 * w;
        ws.wbase = a.blob + po + (size_t)wrow0 * (m / 2);
        ws.srow = a.blob + so + (size_t)(wrow0 + n) * ng * 2;
        ws.load(0, 0);
        ws.load(1, 1);
        return wrow0 + n;
    };
    int row = start(0);
    __syncthreads();
    stage_phase(a.aqh, a.aql, tok, m, 0, ly.kph, q);
    stage_scales(a.aqs, a.aqc, tok, ti.nt, ng, ng, s, cc);
    __syncthreads();
    // the staged act digits serve DN_BLOCK_ROWS / DN_ROWS passes over the rows
#pragma unroll 1
    for (int pass = 0; pass < DN_BLOCK_ROWS / DN_ROWS; pass++) {
        floatx16 acc = {};
        wave_product<G>(acc, ws, wl, q, s, cc, TokSrc{a.aqh, a.aql, tok, m}, ly);
        const int r = row;
        if (pass + 1 < DN_BLOCK_ROWS / DN_ROWS) row = start(pass + 1);
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int i = 8 * (v / 4) + 4 * h + (v % 4);
            if (i < ti.nt) a.y[(size_t)tok[i] * d + r] = __fmul_rn(tws[i], acc[v]);
        }
    }
}

// The small experts' down items (wi::down_item, no barriers) on the blocks
// past the tiles, 8 consecutive items of one entry per virtual block.
template <int G, int LPR, int NDIG>
__device__ __forceinline__ void small_down(const ExpertArgs& a, int first, int nblk) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int vpe = a.d / wi::DN_ROWS / NWAVE;
    const int nv = a.n_tiles[1] * vpe;
#pragma unroll 1
    for (int v = first; v < nv; v += nblk)
        wi::down_item<G, NDIG, LPR, 1>(a, a.small[v / vpe], (v % vpe) * NWAVE + w);
}

// 1-D grid as k_gateup_mfma's, with row blocks of DN_BLOCK_ROWS hidden rows.
template <int G, int LPR, int NDIG>
__global__ void __launch_bounds__(MTHREADS, 1)
k_down_mfma(ExpertArgs a) {
    extern __shared__ __align__(16) unsigned char sm[];
    const int nt = a.n_tiles[0], ntb = nt * (a.d / DN_BLOCK_ROWS);
    const int f = blockIdx.x;
    if (f < ntb) {
        down_tile<G>(a, tile_at(a, f % nt), f / nt, sm);
        return;
    }
    small_down<G, LPR, NDIG>(a, f - ntb, (int)gridDim.x - ntb);
}

// ------------------------------------------------------ plain Q4 product

// out[t][row] = X[t] . dequant(W[row]) for one Q4 matrix (the plugin
// product q4_gemm_f32, expert_ffn.c:200-215, at prefill-sized T): block
// (32-token tile, npass x 256 rows, K split z), 8 waves x 32 rows per pass
// over the tile's staged digits, as the down kernel without routing.  The
// digits of X come from k_prep_i8.  With gridDim.z > 1 split z covers the
// columns [z kl, z kl + kl) (whole Q4 groups and super-stages) and writes
// its partial sums to out + z T m, which k_sum_splits adds in split order.
template <int G>
__global__ void __launch_bounds__(MTHREADS, 1)
k_q4_gemm_mfma(const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales,
               const int8_t* __restrict__ xqh, const int8_t* __restrict__ xql, const float* __restrict__ xqs,
               const int* __restrict__ xqc, int T, int m, int d, int kl, int npass, float* __restrict__ out) {
    extern __shared__ __align__(16) unsigned char sm[];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int ng = d / G;                         // groups per row (the scales' row stride)
    const int k0 = (int)blockIdx.z * kl;          // the split's first column
    const Lay ly(kl, G);
    const int t0 = blockIdx.x * MT;
    const int nt = min(MT, T - t0);
    float* const o = out + (size_t)blockIdx.z * T * m;
    int8_t* q = (int8_t*)sm;
    float* s = (float*)(sm + ly.s);
    int* cc = (int*)(sm + ly.c);
    int* tok = (int*)(sm + ly.tok);
    uint8_t* wl = sm + ly.w + (size_t)w * 2 * WBUF;
    if (tid < MT) tok[tid] = t0 + (tid < nt ? tid : 0);   // padding: the tile's first token
    const int n = lane & 31, h = lane >> 5;
    WStream<G> ws;
    ws.rowb = d / 2;
    ws.nss = kl / SSC;
    auto start = [&](int pass) __attribute__((always_inline)) {
        const int wrow0 = (blockIdx.y * npass + pass) * DN_ROWS + 32 * w;
        ws.wbase = packed + (size_t)wrow0 * (d / 2) + k0 / 2;
        ws.srow = (const uint8_t*)scales + ((size_t)(wrow0 + n) * ng + k0 / G) * 2;
        ws.load(0, 0);
        ws.load(1, 1);
        return wrow0 + n;
    };
    int row = start(0);
    __syncthreads();
    stage_phase(xqh + k0, xql + k0, tok, d, 0, ly.kph, q);
    stage_scales(xqs + k0 / G, xqc + k0 / G, tok, nt, kl / G, ng, s, cc);
    __syncthreads();
#pragma unroll 1
    for (int pass = 0; pass < npass; pass++) {
        floatx16 acc = {};
        // (operands one stage ahead would spill this kernel's registers)
        wave_product<G, false>(acc, ws, wl, q, s, cc, TokSrc{xqh + k0, xql + k0, tok, d}, ly);
        const int r = row;
        if (pass + 1 < npass) row = start(pass + 1);
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int i = 8 * (v / 4) + 4 * h + (v % 4);
            if (i < nt) o[(size_t)(t0 + i) * m + r] = acc[v];
        }
    }
}

// out[i] = the sum of the ns partial products part[z][i], z = 0, 1, ... in
// order (n4 float4 elements each).
__global__ void __launch_bounds__(256)
k_sum_splits(const float4* __restrict__ part, long long n4, int ns, float4* __restrict__ out) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    float4 v[8];
#pragma unroll
    for (int z = 0; z < 8; z++)
        if (z < ns) v[z] = part[(size_t)z * n4 + i];
    float4 r = v[0];
#pragma unroll
    for (int z = 1; z < 8; z++)
        if (z < ns) {
            r.x = __fadd_rn(r.x, v[z].x);
            r.y = __fadd_rn(r.y, v[z].y);
            r.z = __fadd_rn(r.z, v[z].z);
            r.w = __fadd_rn(r.w, v[z].w);
        }
    out[i] = r;
}

// Int8 digit pairs and scales of T rows of d floats, one G-lane segment per
// Q4 group (the encoding of the block's router kernels).
template <int G>
__global__ void __launch_bounds__(256)
k_prep_i8(const float* __restrict__ X, int T, int d, int8_t* __restrict__ hi, int8_t* __restrict__ lo,
          float* __restrict__ sc, int* __restrict__ qc) {
    const long long seg = ((long long)blockIdx.x * blockDim.x + threadIdx.x) / G;
    const int ng = d / G;
    const bool ok = seg < (long long)T * ng;
    const long long sg = ok ? seg : 0;
    const int t = (int)(sg / ng), g = (int)(sg % ng);
    const size_t o = (size_t)t * d + (size_t)g * G;
    const float v = ok ? X[o + (threadIdx.x & (G - 1))] : 0.0f;
    encode_i8_group_wave<G>(v, ok, hi + o, lo + o, sc + (size_t)t * ng + g, qc + (size_t)t * ng + g);
}

// Contractions the kernels take: multiples of the weight super-stage, and
// one token phase or whole phases; row counts of whole blocks.
static bool mfma_k_ok(int K) { return K % SSC == 0 && K <= KMAX && (K <= KPH_MAX || K % KPH_MAX == 0); }

bool mfma_shape_ok(int d, int m) {
    return d % DN_BLOCK_ROWS == 0 && m % GU_ROWS == 0 && mfma_k_ok(d) && mfma_k_ok(m);
}

namespace {

template <int G>
constexpr size_t gateup_lds(int d) {
    return Lay(d, G).total > (size_t)2 * MT * (GU_ROWS + 4) * 4 ? Lay(d, G).total
                                                                 : (size_t)2 * MT * (GU_ROWS + 4) * 4;
}

// Dynamic LDS above 64 KiB must be allowed per kernel: once per device,
// for the largest contraction the kernels take.
constexpr int MAX_DEV = 64;
std::atomic<unsigned> g_lds_set[MAX_DEV];

hipError_t allow_lds() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= MAX_DEV) return hipErrorInvalidDevice;
    if (g_lds_set[dev].load(std::memory_order_acquire)) return hipSuccess;
#define JM_MF(N) \
        {(const void*)k_gateup_mfma<64, 32, N>, gateup_lds<64>(KMAX)}, {(const void*)k_gateup_mfma<64, 64, N>, gateup_lds<64>(KMAX)}, \
        {(const void*)k_gateup_mfma<32, 32, N>, gateup_lds<32>(KMAX)}, {(const void*)k_gateup_mfma<32, 64, N>, gateup_lds<32>(KMAX)}, \
        {(const void*)k_down_mfma<64, 32, N>, Lay(KMAX, 64).total}, {(const void*)k_down_mfma<64, 64, N>, Lay(KMAX, 64).total}, \
        {(const void*)k_down_mfma<32, 32, N>, Lay(KMAX, 32).total}, {(const void*)k_down_mfma<32, 64, N>, Lay(KMAX, 32).total}
    const struct { const void* f; size_t b; } k[18] = {
        JM_MF(4), JM_MF(5),
        {(const void*)k_q4_gemm_mfma<64>, Lay(KMAX, 64).total}, {(const void*)k_q4_gemm_mfma<32>, Lay(KMAX, 32).total}};
#undef JM_MF
    for (const auto& x : k) {
        e = hipFuncSetAttribute(x.f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)x.b);
        if (e != hipSuccess) return e;
    }
    g_lds_set[dev].store(1u, std::memory_order_release);
    return hipSuccess;
}

}  // namespace

// Lanes per row segment of the small experts' wave items: rows of C columns
// (C / 32 chunks of 16 bytes; C <= KMAX, so one chunk per lane).
static int item_lanes(int C) { return C / 32 <= 32 ? 32 : 64; }

// Grids of max_tiles x (row blocks) blocks, one row of blocks more: the
// blocks past the device's tile count run the small experts' wave items.
hipError_t launch_gateup_mfma(const ExpertArgs& a, int max_tiles, hipStream_t st) {
    if (max_tiles == 0) return hipSuccess;
    if (!mfma_shape_ok(a.d, a.m) || (a.group != 64 && a.group != 32)) return hipErrorInvalidValue;
    if (!a.small || (a.m / wi::GU_ROWS) % NWAVE) return hipErrorInvalidValue;
    hipError_t e = allow_lds();
    if (e != hipSuccess) return e;
    const int rb = a.m / GU_ROWS;
    const dim3 grid((unsigned)((max_tiles + 1) * rb));
    const bool l64 = item_lanes(a.d) == 64;
    if (a.ndig != 4 && a.ndig != 5) return hipErrorInvalidValue;
#define JM_GM(GG, L) do { if (a.ndig == 5) hipLaunchKernelGGL((k_gateup_mfma<GG, L, 5>), grid, dim3(MTHREADS), gateup_lds<GG>(a.d), st, a); \
                          else hipLaunchKernelGGL((k_gateup_mfma<GG, L, 4>), grid, dim3(MTHREADS), gateup_lds<GG>(a.d), st, a); } while (0)
    if (a.group == 64) {
        if (l64) JM_GM(64, 64);
        else JM_GM(64, 32);
    } else {
        if (l64) JM_GM(32, 64);
        else JM_GM(32, 32);
    }
#undef JM_GM
    return hipGetLastError();
}

hipError_t launch_down_mfma(const ExpertArgs& a, int max_tiles, hipStream_t st) {
    if (max_tiles == 0) return hipSuccess;
    if (!mfma_shape_ok(a.d, a.m) || (a.group != 64 && a.group != 32)) return hipErrorInvalidValue;
    if (!a.small || (a.d / wi::DN_ROWS) % NWAVE) return hipErrorInvalidValue;
    hipError_t e = allow_lds();
    if (e != hipSuccess) return e;
    const int rb = a.d / DN_BLOCK_ROWS;
    const dim3 grid((unsigned)((max_tiles + 1) * rb));
    const bool l64 = item_lanes(a.m) == 64;
    if (a.ndig != 4 && a.ndig != 5) return hipErrorInvalidValue;
#define JM_DM(GG, L) do { if (a.ndig == 5) hipLaunchKernelGGL((k_down_mfma<GG, L, 5>), grid, dim3(MTHREADS), Lay(a.m, GG).total, st, a); \
                          else hipLaunchKernelGGL((k_down_mfma<GG, L, 4>), grid, dim3(MTHREADS), Lay(a.m, GG).total, st, a); } while (0)
    if (a.group == 64) {
        if (l64) JM_DM(64, 64);
        else JM_DM(64, 32);
    } else {
        if (l64) JM_DM(32, 64);
        else JM_DM(32, 32);
    }
#undef JM_DM
    return hipGetLastError();
}

static size_t pad256(size_t n) { return (n + 255) & ~(size_t)255; }

bool q4_gemm_mfma_ok(int m, int d, int group) {
    // whole 256-row passes; each row's scales of a super-stage in one
    // aligned 8-byte (G = 64) or 16-byte (G = 32) load
    return m % DN_ROWS == 0 && mfma_k_ok(d) && (group == 64 || group == 32) &&
           ((d / group) * 2) % (group == 64 ? 8 : 16) == 0;
}

// K splits of the plain product: when the grid of token tiles x row blocks
// would leave most of the 256 CUs idle, ns blocks share each one's
// contraction (ns a divisor of the super-stages over d, at most 8): the
// smallest ns that fills one round of 256 blocks, else the largest.
int q4_gemm_splits(int T, int m, int d) {
    const long long blocks = (long long)((T + MT - 1) / MT) * (m / DN_ROWS);
    const int nss = d / SSC;
    int ns = 1;
    for (int c = 2; c <= 8 && blocks * ns < 256; c++)
        if (nss % c == 0 && mfma_k_ok(d / c)) ns = c;
    return ns;
}

size_t q4_gemm_mfma_ws(int T, int m, int d, int group) {
    const int ns = q4_gemm_splits(T, m, d);
    return pad256((size_t)T * d) * 2 + pad256((size_t)T * (d / group) * 4) * 2 +
           (ns > 1 ? pad256((size_t)ns * T * m * 4) : 0);
}

hipError_t launch_q4_gemm_mfma(const uint8_t* packed, const uint16_t* scales, const float* X, int T, int m, int d,
                               int group, void* ws, float* out, hipStream_t st) {
    if (T == 0 || m == 0) return hipSuccess;
    if (!q4_gemm_mfma_ok(m, d, group)) return hipErrorInvalidValue;
    hipError_t e = allow_lds();
    if (e != hipSuccess) return e;
    int8_t* hi = (int8_t*)ws;
    int8_t* lo = hi + pad256((size_t)T * d);
    float* sc = (float*)(lo + pad256((size_t)T * d));
    int* qc = (int*)((char*)sc + pad256((size_t)T * (d / group) * 4));
    float* part = (float*)((char*)qc + pad256((size_t)T * (d / group) * 4));
    const long long lanes = (long long)T * d;
    const unsigned pblocks = (unsigned)((lanes + 255) / 256);
    const int ns = q4_gemm_splits(T, m, d);
    const int kl = d / ns;
    float* dst = ns > 1 ? part : out;
    // two passes per block when the rows allow and the grid still fills the chip
    const int tiles = (T + MT - 1) / MT;
    const int npass = (m % (2 * DN_ROWS) == 0 && (long long)tiles * (m / (2 * DN_ROWS)) >= 256) ? 2 : 1;
    const dim3 grid((unsigned)tiles, (unsigned)(m / (DN_ROWS * npass)), (unsigned)ns);
    if (group == 64) {
        hipLaunchKernelGGL(k_prep_i8<64>, dim3(pblocks), dim3(256), 0, st, X, T, d, hi, lo, sc, qc);
        hipLaunchKernelGGL(k_q4_gemm_mfma<64>, grid, dim3(MTHREADS), Lay(kl, 64).total, st, packed, scales, hi, lo, sc,
                           qc, T, m, d, kl, npass, dst);
    } else {
        hipLaunchKernelGGL(k_prep_i8<32>, dim3(pblocks), dim3(256), 0, st, X, T, d, hi, lo, sc, qc);
        hipLaunchKernelGGL(k_q4_gemm_mfma<32>, grid, dim3(MTHREADS), Lay(kl, 32).total, st, packed, scales, hi, lo, sc,
                           qc, T, m, d, kl, npass, dst);
    }
    if (ns > 1) {
        const long long n4 = (long long)T * m / 4;
        hipLaunchKernelGGL(k_sum_splits, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, (const float4*)part, n4,
                           ns, (float4*)out);
    }
    return hipGetLastError();
}

}  // namespace jm
