// Dense branch of the grouped Q4 expert product (gfx950 MFMA), taken by the
// experts whose segment holds at least `dense_min` tokens (prefill-sized
// batches, skewed routing).  The same contraction as the wave-item kernels
// in jm_experts.hip (decode_kernel.c:1365-1383), as tiled products:
//
//   k_gateup_mfma  per (expert, 64-token tile, 128 intermediate rows):
//                  G = X . Wg^T and U = X . Wu^T over d, then
//                  act = (G / (1 + expf_fast(-G))) * U
//   k_down_mfma    per (expert, 64-token tile, 128 hidden rows; 256 for a
//                  tile of up to 32 tokens):
//                  y[slot] = w_slot * (act . Wd^T) over the intermediate
//
// Operands, per 64-column (narrow down tiles: 32-column) stage of the
// contraction, staged in LDS:
//   weights  the signed nibbles q - 8 as fp16 (exact), one fp32 scale per
//            row and Q4 group applied to the fp32 accumulator of that group;
//   tokens   each fp32 value split into hi = fp16(v) and lo = fp16(v - hi)
//            (by the router kernel for x, by the gate/up epilogue for act),
//            two products per tile, so the activations keep 22 significant
//            bits.  A row whose largest magnitude reaches 2^15 (x: a token;
//            act: a slot's 128-row block) is split as v * 2^-p instead, and
//            its products are scaled back by 2^p (exact): the gate/up
//            epilogue for x, the down kernel's group scales for act, so the
//            fp16 range never clips an activation.
// Both operands keep each 8-column group in the order 0 4 1 5 2 6 3 7 that
// the nibble dequantisation produces; the contraction does not care.
// v_mfma_f32_32x32x16_f16 tiles with the tokens on the A side: lane l holds
// one weight row (n = l % 32) and 16 tokens, so a group's scale is one value
// per lane.  Lane layout (checked on the device): A[i][k] at lane i % 32,
// k = 8 * (l / 32) + j; B[k][n] at lane n % 32, k = 8 * (l / 32) + j;
// D register v of lane l = (i = 8 (v / 4) + 4 (l / 32) + v % 4, n = l % 32).
//
// Two stages stream into registers while the stage in LDS is multiplied;
// the next stage goes to the other LDS buffer after the MFMAs (double
// buffering).
#include "jm_device.h"
#include "jm_kernels.h"

namespace jm {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int MT = JM_DENSE_TILE;   // tokens per tile of the tile list

__device__ __forceinline__ void split_hi_lo(float v, _Float16& h, _Float16& l) {
    h = (_Float16)v;
    l = (_Float16)(v - (float)h);
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// 32 nibbles (one 16-byte piece; word c holds values 8c..8c+7, value i in
// bits 4i..4i+3) as q - 8 in fp16, to 4 x 16 bytes of LDS in the MFMA
// column order (0 4 1 5 2 6 3 7 per 8 values): the fp16 bits 0x6400 | q
// are 1024 + q exactly, and one packed subtraction of 1032 leaves q - 8.
__device__ __forceinline__ void nibbles_to_lds(uint4 p, _Float16* dst) {
    const uint32_t w[4] = {p.x, p.y, p.z, p.w};
    const half2_t bias = {(_Float16)1032.0f, (_Float16)1032.0f};
#pragma unroll
    for (int c = 0; c < 4; c++) {
        uint32_t t[4];
#pragma unroll
        for (int i = 0; i < 4; i++) t[i] = ((w[c] >> (4 * i)) & 0x000F000Fu) | 0x64006400u;   // values (i, i + 4)
        half8 h;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const half2_t v = __builtin_bit_cast(half2_t, t[i]) - bias;
            h[2 * i] = v[0];
            h[2 * i + 1] = v[1];
        }
        *(half8*)(dst + 8 * c) = h;
    }
}

struct TileInfo {
    int slot0;      // first position of the tile in seg_slot
    int nt;         // tokens in the tile (1..MT)
    int e;          // expert id
};

__device__ __forceinline__ bool tile_info(const ExpertArgs& a, int t, TileInfo* ti) {
    if (t >= *a.n_tiles) return false;
    const int2 tl = a.tiles[t];
    const ExpertWork wk = a.work[tl.x];
    ti->slot0 = wk.s0 + tl.y * MT;
    ti->nt = min(MT, wk.n - tl.y * MT);
    ti->e = wk.e;
    return true;
}

constexpr int MTHREADS = 512;       // 8 waves per block
constexpr int MROWS = 128;          // weight rows of one block column (blockIdx.y)

// Tile shapes.  A wide tile (33..64 tokens, and every gate/up tile) is
// multiplied by one block per 128 weight rows: 8 waves of 32 tokens x 32
// rows (2 token halves x 4 row quarters), 64-column stages.  A narrow down
// tile (up to 32 tokens: most experts of a skewed prefill batch) is
// multiplied by one block per 256 rows, the even block of each pair of
// block columns (the odd one exits): 8 waves of the same 32 tokens x 32
// rows each, 32-column stages.  Both shapes issue the same MFMAs per wave
// and stream the same bytes per block; the narrow one halves the blocks of
// a narrow tile and multiplies no padding half.
template <bool NARROW>
struct Shape {
    static constexpr int TOK = NARROW ? 32 : 64;      // tokens per tile
    static constexpr int ROWS = NARROW ? 256 : 128;   // weight rows per block
    static constexpr int KS = NARROW ? 32 : 64;       // contraction columns per stage
    static constexpr int KP = KS + 8;                 // padded LDS row in halves (80 / 144 bytes: 16-byte aligned, bank-spread)
    static constexpr int XPC = KS / 8;                // 8-value token pieces per token and stage
    static constexpr int XTHR = TOK * XPC;            // threads staging tokens (128 / 512)
    static constexpr int WPR = KS / 32;               // 16-byte weight pieces per row and stage
};

// Scale groups of a stage: NGS scale values per row, each over KSG MFMA
// k-steps; a 64-value group spans SPG = 2 narrow stages, and its two halves'
// partial sums are summed before the scale is applied.
template <int G, int KS_>
struct Groups {
    static constexpr int NGS = KS_ >= G ? KS_ / G : 1;
    static constexpr int KSG = (KS_ >= G ? G : KS_) / 16;
    static constexpr int SPG = KS_ >= G ? 1 : G / KS_;
    static_assert(SPG == 1 || SPG == 2, "a scale group spans one or two stages");
};

// narrow tiles need whole 256-row blocks
__device__ __forceinline__ bool narrow_rows_ok(int rows) { return rows % (2 * MROWS) == 0; }

// ------------------------------------------------------------------ gate/up

template <int G, bool NARROW>
struct GuLds {
    using S = Shape<NARROW>;
    _Float16 xh[2][S::TOK * S::KP], xl[2][S::TOK * S::KP];
    _Float16 wl[2][2][S::ROWS * S::KP];
    float scl[2][2][S::ROWS][Groups<G, S::KS>::NGS];
    int tok[S::TOK];
    float xf[S::TOK];              // 2^p of each token's split
    float amx[4][S::TOK];          // max |act| of each token over each row quarter's 32 rows
};

// Stage registers of one thread: 8 token values (hi and lo), one 16-byte
// piece of one row of one matrix, that row's scales for the stage.
template <int NGS>
struct StageRegs {
    uint4 h, l;
    uint4 w;
    uint16_t sc[NGS];
};

template <int G, bool NARROW>
__device__ __forceinline__ void gateup_tile(const ExpertArgs& a, const TileInfo& ti, unsigned char* sm) {
    using S = Shape<NARROW>;
    using Q = Groups<G, S::KS>;
    GuLds<G, NARROW>& L = *reinterpret_cast<GuLds<G, NARROW>*>(sm);
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = tid >> 6;
    const int row0 = blockIdx.y * MROWS;          // first intermediate row of the block
    const int d = a.d, ng = d / G, nstage = d / S::KS;
    if (tid < S::TOK) {
        const int b = tid < ti.nt ? a.seg_slot[ti.slot0 + tid] / a.topk : -1;
        L.tok[tid] = b;
        L.xf[tid] = b >= 0 ? a.xexp[b] : 1.0f;
    }
    unsigned long long so[2], po[2];
    a.rec.get(0, a.key0 + ti.e, so[0], po[0]);
    a.rec.get(1, a.key0 + ti.e, so[1], po[1]);
    __syncthreads();

    // staging assignment: tokens (threads < XTHR, 8 values each of one
    // token), weights (every thread one 16-byte piece of one row of one
    // matrix)
    const bool xthr = S::XTHR == MTHREADS || tid < S::XTHR;   // wave-uniform
    const int xt = (tid / S::XPC) % S::TOK, xpart = tid % S::XPC;
    const int wm = tid >> 8, widx = tid & 255;
    const int wrow = widx / S::WPR, wpiece = widx % S::WPR;
    const int xb = L.tok[xt];
    const size_t xo = (size_t)(xb >= 0 ? xb : 0) * d + xpart * 8;
    const uint8_t* wpk = a.blob + po[wm] + (size_t)(row0 + wrow) * (d / 2) + wpiece * 16;
    const uint16_t* wsc = (const uint16_t*)(a.blob + so[wm]) + (size_t)(row0 + wrow) * ng;

    // every load is unconditional (past the last stage: the last stage again)
    auto load_stage = [&](StageRegs<Q::NGS>& r, int s) __attribute__((always_inline)) {
        s = s < nstage ? s : nstage - 1;
        if (xthr) {
            r.h = *(const uint4*)(a.xsh + xo + s * S::KS);
            r.l = *(const uint4*)(a.xsl + xo + s * S::KS);
        }
        r.w = *(const uint4*)(wpk + s * (S::KS / 2));
#pragma unroll
        for (int j = 0; j < Q::NGS; j++) r.sc[j] = wsc[(s * S::KS) / G + j];
    };
    auto store_stage = [&](const StageRegs<Q::NGS>& r, int buf) __attribute__((always_inline)) {
        if (xthr) {
            const unsigned keep = xb >= 0 ? 0xFFFFFFFFu : 0u;     // padding tokens stage zeros
            *(uint4*)&L.xh[buf][xt * S::KP + xpart * 8] = make_uint4(r.h.x & keep, r.h.y & keep, r.h.z & keep, r.h.w & keep);
            *(uint4*)&L.xl[buf][xt * S::KP + xpart * 8] = make_uint4(r.l.x & keep, r.l.y & keep, r.l.z & keep, r.l.w & keep);
        }
        nibbles_to_lds(r.w, &L.wl[buf][wm][wrow * S::KP + wpiece * 32]);
        if (wpiece == 0) {
#pragma unroll
            for (int j = 0; j < Q::NGS; j++) L.scl[buf][wm][wrow][j] = fp16_hw(r.sc[j]);
        }
    };

    // this wave's token half and 32-row slice
    const int th = NARROW ? 0 : (w & 1), rq = NARROW ? w : (w >> 1);
    const int ai = th * 32 + (lane & 31), bn = rq * 32 + (lane & 31), kq = 8 * (lane >> 5);
    floatx16 tg = {}, tu = {};
    floatx16 cg = {}, cu = {};                    // partial sums carried into a group's second stage
    // fresh: the stage starts a scale group; apply: it ends one
    auto mfma_stage = [&](int buf, bool fresh, bool apply) __attribute__((always_inline)) {
#pragma unroll
        for (int gs = 0; gs < Q::NGS; gs++) {
            floatx16 ag = fresh ? floatx16{} : cg, au = fresh ? floatx16{} : cu;
#pragma unroll
            for (int k2 = 0; k2 < Q::KSG; k2++) {
                const int k0 = (gs * Q::KSG + k2) * 16 + kq;
                const half8 a_h = *(const half8*)&L.xh[buf][ai * S::KP + k0];
                const half8 a_l = *(const half8*)&L.xl[buf][ai * S::KP + k0];
                const half8 b_g = *(const half8*)&L.wl[buf][0][bn * S::KP + k0];
                const half8 b_u = *(const half8*)&L.wl[buf][1][bn * S::KP + k0];
                ag = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_h, b_g, ag, 0, 0, 0);
                ag = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_l, b_g, ag, 0, 0, 0);
                au = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_h, b_u, au, 0, 0, 0);
                au = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_l, b_u, au, 0, 0, 0);
            }
            if (apply) {
                const float sg = L.scl[buf][0][bn][gs], su = L.scl[buf][1][bn][gs];
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    tg[v] = __builtin_fmaf(sg, ag[v], tg[v]);
                    tu[v] = __builtin_fmaf(su, au[v], tu[v]);
                }
            } else {
                cg = ag;
                cu = au;
            }
        }
    };
    // stages s + 1 and s + 2 stream into registers while stage s (in LDS) is
    // multiplied; nstage is even, so buffer 0 always holds an even stage
    StageRegs<Q::NGS> r0, r1;
    load_stage(r0, 0);
    load_stage(r1, 1);
    store_stage(r0, 0);
    load_stage(r0, 2);
    __syncthreads();
    for (int s = 0; s < nstage; s += 2) {
        mfma_stage(0, true, Q::SPG == 1);         // stage s; r1 = s + 1, r0 = s + 2 in flight
        store_stage(r1, 1);
        load_stage(r1, s + 3);
        __syncthreads();
        mfma_stage(1, Q::SPG == 1, true);         // stage s + 1; r0 = s + 2, r1 = s + 3
        store_stage(r0, 0);
        load_stage(r0, s + 4);
        __syncthreads();
    }
    // act = SiLU(g) * u for this lane's row and 16 tokens (the token's
    // split prescale undone first)
    const int r = row0 + bn;
    float av[16];
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int i = th * 32 + 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
        const float f = L.xf[i];
        av[v] = swiglu(__fmul_rn(tg[v], f), __fmul_rn(tu[v], f));
        // the token's max |act| over this half-wave's 32 rows
        const float mx = seg_max<32>(i < ti.nt ? fabsf(av[v]) : 0.0f);
        if ((lane & 31) == 0) L.amx[rq][i] = mx;
    }
    __syncthreads();
    const int nb = a.m / MROWS;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int i = th * 32 + 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
        if (i < ti.nt) {
            const int slot = a.seg_slot[ti.slot0 + i];
            // one prescale per (slot, this block's 128 rows)
            const int pe = split_exp(fmaxf(fmaxf(L.amx[0][i], L.amx[1][i]), fmaxf(L.amx[2][i], L.amx[3][i])));
            if (rq == 0 && (lane & 31) == 0) a.aexp[(size_t)slot * nb + blockIdx.y] = exp2i(pe);
            _Float16 hh, ll;
            split_hi_lo(__fmul_rn(av[v], exp2i(-pe)), hh, ll);
            a.act[(size_t)slot * a.m + r] = av[v];
            const size_t o = (size_t)slot * a.m + (r & ~7) + mfma_slot(r & 7);
            a.act_h[o] = hh;
            a.act_l[o] = ll;
        }
    }
}

// Gate/up takes every tile in the wide shape: with narrow tiles in 256-row
// blocks the 512-token Zipf-routed block's gate/up took 167 us instead of
// 160 (twice the stages of half the MFMA work each, and the per-stage
// latency is what bounds it), while the down product, with a third of the
// contraction, gains from the halved block count.
template <int G>
__global__ void __launch_bounds__(MTHREADS, 1)
k_gateup_mfma(ExpertArgs a) {
    TileInfo ti;
    if (!tile_info(a, blockIdx.x, &ti)) return;
    __shared__ __align__(16) unsigned char sm[sizeof(GuLds<G, false>)];
    gateup_tile<G, false>(a, ti, sm);
}

// --------------------------------------------------------------------- down

template <int G, bool NARROW>
struct DnLds {
    using S = Shape<NARROW>;
    _Float16 xh[2][S::TOK * S::KP], xl[2][S::TOK * S::KP];
    _Float16 wl[2][S::ROWS * S::KP];
    float scl[2][S::ROWS][Groups<G, S::KS>::NGS];
    int tok[S::TOK];
};

template <int G, bool NARROW>
__device__ __forceinline__ void down_tile(const ExpertArgs& a, const TileInfo& ti, unsigned char* sm) {
    using S = Shape<NARROW>;
    using Q = Groups<G, S::KS>;
    DnLds<G, NARROW>& L = *reinterpret_cast<DnLds<G, NARROW>*>(sm);
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = tid >> 6;
    const int row0 = blockIdx.y * MROWS;          // first hidden row of the block
    const int m = a.m, ng = m / G, nstage = m / S::KS;
    if (tid < S::TOK) L.tok[tid] = tid < ti.nt ? a.seg_slot[ti.slot0 + tid] : -1;
    unsigned long long so, po;
    a.rec.get(2, a.key0 + ti.e, so, po);
    __syncthreads();
    // act blocks split with a prescale (a magnitude past 2^15): the tile then
    // scales each token's group products back by 2^p of its 128-column block
    const int nb = m / MROWS;
    int any = 0;
    for (int q = tid; q < S::TOK * nb; q += MTHREADS) {
        const int sl = L.tok[q / nb];
        if (sl >= 0 && a.aexp[(size_t)sl * nb + q % nb] != 1.0f) any = 1;
    }
    const bool scaled = __syncthreads_or(any) != 0;

    // staging: act (threads < XTHR, 8 columns of one token each), weights
    // (threads 0..255, one 16-byte piece of one row each)
    const bool xthr = S::XTHR == MTHREADS || tid < S::XTHR;   // wave-uniform
    const bool wthr = tid < 256;                               // wave-uniform
    const int xt = (tid / S::XPC) % S::TOK, xpart = tid % S::XPC;
    const int widx = tid & 255;
    const int wrow = widx / S::WPR, wpiece = widx % S::WPR;
    const int xs = L.tok[xt];
    const size_t xo = (size_t)(xs >= 0 ? xs : 0) * m + xpart * 8;
    const uint8_t* wpk = a.blob + po + (size_t)(row0 + wrow) * (m / 2) + wpiece * 16;
    const uint16_t* wsc = (const uint16_t*)(a.blob + so) + (size_t)(row0 + wrow) * ng;

    auto load_stage = [&](StageRegs<Q::NGS>& r, int s) __attribute__((always_inline)) {
        s = s < nstage ? s : nstage - 1;
        if (xthr) {
            r.h = *(const uint4*)(a.act_h + xo + s * S::KS);
            r.l = *(const uint4*)(a.act_l + xo + s * S::KS);
        }
        if (wthr) {
            r.w = *(const uint4*)(wpk + s * (S::KS / 2));
#pragma unroll
            for (int j = 0; j < Q::NGS; j++) r.sc[j] = wsc[(s * S::KS) / G + j];
        }
    };
    auto store_stage = [&](const StageRegs<Q::NGS>& r, int buf) __attribute__((always_inline)) {
        if (xthr) {
            const unsigned keep = xs >= 0 ? 0xFFFFFFFFu : 0u;     // padding tokens stage zeros
            *(uint4*)&L.xh[buf][xt * S::KP + xpart * 8] = make_uint4(r.h.x & keep, r.h.y & keep, r.h.z & keep, r.h.w & keep);
            *(uint4*)&L.xl[buf][xt * S::KP + xpart * 8] = make_uint4(r.l.x & keep, r.l.y & keep, r.l.z & keep, r.l.w & keep);
        }
        if (wthr) {
            nibbles_to_lds(r.w, &L.wl[buf][wrow * S::KP + wpiece * 32]);
            if (wpiece == 0) {
#pragma unroll
                for (int j = 0; j < Q::NGS; j++) L.scl[buf][wrow][j] = fp16_hw(r.sc[j]);
            }
        }
    };

    const int th = NARROW ? 0 : (w & 1), rq = NARROW ? w : (w >> 1);
    const int ai = th * 32 + (lane & 31), bn = rq * 32 + (lane & 31), kq = 8 * (lane >> 5);
    floatx16 tot = {};
    floatx16 carry = {};                          // partial sum carried into a group's second stage
    auto mfma_stage = [&](int buf, int st, bool fresh, bool apply) __attribute__((always_inline)) {
#pragma unroll
        for (int gs = 0; gs < Q::NGS; gs++) {
            floatx16 acc = fresh ? floatx16{} : carry;
#pragma unroll
            for (int k2 = 0; k2 < Q::KSG; k2++) {
                const int k0 = (gs * Q::KSG + k2) * 16 + kq;
                const half8 a_h = *(const half8*)&L.xh[buf][ai * S::KP + k0];
                const half8 a_l = *(const half8*)&L.xl[buf][ai * S::KP + k0];
                const half8 b = *(const half8*)&L.wl[buf][bn * S::KP + k0];
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_h, b, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_l, b, acc, 0, 0, 0);
            }
            if (apply) {
                const float sc = L.scl[buf][bn][gs];
                if (scaled) {
                    // stages never straddle a 128-column block
                    const int g128 = st * S::KS / MROWS;
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        const int sl = L.tok[th * 32 + 8 * (v / 4) + 4 * (lane >> 5) + (v % 4)];
                        const float f = sl >= 0 ? a.aexp[(size_t)sl * nb + g128] : 1.0f;
                        tot[v] = __builtin_fmaf(__fmul_rn(sc, f), acc[v], tot[v]);
                    }
                } else {
#pragma unroll
                    for (int v = 0; v < 16; v++) tot[v] = __builtin_fmaf(sc, acc[v], tot[v]);
                }
            } else {
                carry = acc;
            }
        }
    };
    StageRegs<Q::NGS> r0, r1;
    load_stage(r0, 0);
    load_stage(r1, 1);
    store_stage(r0, 0);
    load_stage(r0, 2);
    __syncthreads();
    for (int s = 0; s < nstage; s += 2) {
        mfma_stage(0, s, true, Q::SPG == 1);
        store_stage(r1, 1);
        load_stage(r1, s + 3);
        __syncthreads();
        mfma_stage(1, s + 1, Q::SPG == 1, true);
        store_stage(r0, 0);
        load_stage(r0, s + 4);
        __syncthreads();
    }
    const int r = row0 + bn;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int i = th * 32 + 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
        if (i < ti.nt) {
            const int slot = L.tok[i];
            a.y[(size_t)slot * a.d + r] = __fmul_rn(a.tw[slot], tot[v]);
        }
    }
}

template <int G>
__global__ void __launch_bounds__(MTHREADS, 1)
k_down_mfma(ExpertArgs a) {
    TileInfo ti;
    if (!tile_info(a, blockIdx.x, &ti)) return;
    constexpr size_t W = sizeof(DnLds<G, false>), N = sizeof(DnLds<G, true>);
    __shared__ __align__(16) unsigned char sm[W > N ? W : N];
    if (ti.nt <= 32 && narrow_rows_ok(a.d)) {
        if (blockIdx.y & 1) return;               // the even block of the pair takes all 256 rows
        down_tile<G, true>(a, ti, sm);
    } else {
        down_tile<G, false>(a, ti, sm);
    }
}

// the MFMA branch needs whole 128-row tiles and an even number of 64-column
// stages on both products (narrow tiles also take 256-row blocks where the
// rows allow)
bool mfma_shape_ok(int d, int m) { return d % MROWS == 0 && m % MROWS == 0 && (d / 64) % 2 == 0 && (m / 64) % 2 == 0; }

hipError_t launch_gateup_mfma(const ExpertArgs& a, int max_tiles, hipStream_t st) {
    if (max_tiles == 0) return hipSuccess;
    if (!mfma_shape_ok(a.d, a.m)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)max_tiles, (unsigned)(a.m / MROWS));
    if (a.group == 64) hipLaunchKernelGGL(k_gateup_mfma<64>, grid, dim3(MTHREADS), 0, st, a);
    else hipLaunchKernelGGL(k_gateup_mfma<32>, grid, dim3(MTHREADS), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_down_mfma(const ExpertArgs& a, int max_tiles, hipStream_t st) {
    if (max_tiles == 0) return hipSuccess;
    if (!mfma_shape_ok(a.d, a.m)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)max_tiles, (unsigned)(a.d / MROWS));
    if (a.group == 64) hipLaunchKernelGGL(k_down_mfma<64>, grid, dim3(MTHREADS), 0, st, a);
    else hipLaunchKernelGGL(k_down_mfma<32>, grid, dim3(MTHREADS), 0, st, a);
    return hipGetLastError();
}

}  // namespace jm
