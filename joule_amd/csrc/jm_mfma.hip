// Dense branch of the grouped Q4 expert product (gfx950 MFMA), taken by the
// experts whose segment holds at least `dense_min` tokens (prefill-sized
// batches, skewed routing).  The same contraction as the wave-item kernels
// in jm_experts.hip (decode_kernel.c:1365-1383), as tiled products:
//
//   k_gateup_mfma  per (expert, 64-token tile, 128 intermediate rows):
//                  G = X . Wg^T and U = X . Wu^T over d, then
//                  act = (G / (1 + expf_fast(-G))) * U
//   k_down_mfma    per (expert, 64-token tile, 128 hidden rows):
//                  y[slot] = w_slot * (act . Wd^T) over the intermediate
//
// Operands, per 64-column stage of the contraction, staged in LDS:
//   weights  the signed nibbles q - 8 as fp16 (exact), one fp32 scale per
//            row and Q4 group applied to the fp32 accumulator of that group;
//   tokens   each fp32 value split into hi = fp16(v) and lo = fp16(v - hi)
//            (by the router kernel for x, by the gate/up epilogue for act),
//            two products per tile, so the activations keep 22 significant
//            bits (|v| < 65504).
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

constexpr int MT = JM_DENSE_TILE;   // tokens per tile
constexpr int KS = 64;              // contraction columns per stage
constexpr int KP = KS + 8;          // padded LDS row, in halves (144 bytes: 16-byte aligned, bank-spread)

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

constexpr int MTHREADS = 512;       // 8 waves: 2 token halves x 4 row quarters of the 128-row tile
constexpr int MROWS = 128;          // weight rows per block

// ------------------------------------------------------------------ gate/up

// Stage registers of one thread: 8 token values, one 16-byte piece of one
// row of one matrix, that row's scales for the stage.
// Stage registers of one thread: 8 token values (hi and lo), one 16-byte
// piece of one row of one matrix, that row's scales for the stage.
template <int NGS>
struct GuStage {
    uint4 h, l;
    uint4 w;
    uint16_t sc[NGS];
};

template <int G>
__global__ void __launch_bounds__(MTHREADS, 1)
k_gateup_mfma(ExpertArgs a) {
    TileInfo ti;
    if (!tile_info(a, blockIdx.x, &ti)) return;
    constexpr int NGS = KS / G;                   // scale groups per stage
    constexpr int KSG = G / 16;                   // MFMA k-steps per scale group
    __shared__ __align__(16) _Float16 xh[2][MT * KP], xl[2][MT * KP], wl[2][2][MROWS * KP];
    __shared__ float scl[2][2][MROWS][NGS];
    __shared__ int tok_b[MT];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = tid >> 6;
    const int rt = blockIdx.y;                    // 128-row tile of the intermediate
    const int d = a.d, ng = d / G, nstage = d / KS;
    if (tid < MT) tok_b[tid] = tid < ti.nt ? a.seg_slot[ti.slot0 + tid] / a.topk : -1;
    unsigned long long so[2], po[2];
    a.rec.get(0, a.key0 + ti.e, so[0], po[0]);
    a.rec.get(1, a.key0 + ti.e, so[1], po[1]);
    __syncthreads();

    // staging assignment: tokens (8 threads x 8 values each), weights (one
    // 16-byte piece of one row of one matrix)
    const int xt = tid >> 3, xpart = tid & 7;
    const int wm = tid >> 8, wrow = (tid & 255) >> 1, wpiece = tid & 1;
    const int xb = tok_b[xt];
    const size_t xo = (size_t)(xb >= 0 ? xb : 0) * d + xpart * 8;
    const uint8_t* wpk = a.blob + po[wm] + (size_t)(rt * MROWS + wrow) * (d / 2) + wpiece * 16;
    const uint16_t* wsc = (const uint16_t*)(a.blob + so[wm]) + (size_t)(rt * MROWS + wrow) * ng;

    // every load is unconditional (past the last stage: the last stage again),
    // so that each wait counts exactly the loads it needs
    auto load_stage = [&](GuStage<NGS>& r, int s) __attribute__((always_inline)) {
        s = s < nstage ? s : nstage - 1;
        r.h = *(const uint4*)(a.xsh + xo + s * KS);
        r.l = *(const uint4*)(a.xsl + xo + s * KS);
        r.w = *(const uint4*)(wpk + s * (KS / 2));
#pragma unroll
        for (int j = 0; j < NGS; j++) r.sc[j] = wsc[s * NGS + j];
    };
    auto store_stage = [&](const GuStage<NGS>& r, int buf) __attribute__((always_inline)) {
        const unsigned keep = xb >= 0 ? 0xFFFFFFFFu : 0u;     // padding tokens stage zeros
        *(uint4*)&xh[buf][xt * KP + xpart * 8] = make_uint4(r.h.x & keep, r.h.y & keep, r.h.z & keep, r.h.w & keep);
        *(uint4*)&xl[buf][xt * KP + xpart * 8] = make_uint4(r.l.x & keep, r.l.y & keep, r.l.z & keep, r.l.w & keep);
        nibbles_to_lds(r.w, &wl[buf][wm][wrow * KP + wpiece * 32]);
        if (wpiece == 0) {
#pragma unroll
            for (int j = 0; j < NGS; j++) scl[buf][wm][wrow][j] = fp16_hw(r.sc[j]);
        }
    };

    const int th = w & 1, rq = w >> 1;            // this wave's token half and row quarter
    const int ai = th * 32 + (lane & 31), bn = rq * 32 + (lane & 31), kq = 8 * (lane >> 5);
    floatx16 tg = {}, tu = {};
    auto mfma_stage = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int gs = 0; gs < NGS; gs++) {
            floatx16 ag = {}, au = {};
#pragma unroll
            for (int k2 = 0; k2 < KSG; k2++) {
                const int k0 = (gs * KSG + k2) * 16 + kq;
                const half8 a_h = *(const half8*)&xh[buf][ai * KP + k0];
                const half8 a_l = *(const half8*)&xl[buf][ai * KP + k0];
                const half8 b_g = *(const half8*)&wl[buf][0][bn * KP + k0];
                const half8 b_u = *(const half8*)&wl[buf][1][bn * KP + k0];
                ag = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_h, b_g, ag, 0, 0, 0);
                ag = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_l, b_g, ag, 0, 0, 0);
                au = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_h, b_u, au, 0, 0, 0);
                au = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_l, b_u, au, 0, 0, 0);
            }
            const float sg = scl[buf][0][bn][gs], su = scl[buf][1][bn][gs];
#pragma unroll
            for (int v = 0; v < 16; v++) {
                tg[v] = __builtin_fmaf(sg, ag[v], tg[v]);
                tu[v] = __builtin_fmaf(su, au[v], tu[v]);
            }
        }
    };
    // stages s + 1 and s + 2 stream into registers while stage s (in LDS) is
    // multiplied; nstage is even
    GuStage<NGS> r0, r1;
    load_stage(r0, 0);
    load_stage(r1, 1);
    store_stage(r0, 0);
    load_stage(r0, 2);
    __syncthreads();
    for (int s = 0; s < nstage; s += 2) {
        mfma_stage(0);                            // stage s; r1 = s + 1, r0 = s + 2 in flight
        store_stage(r1, 1);
        load_stage(r1, s + 3);
        __syncthreads();
        mfma_stage(1);                            // stage s + 1; r0 = s + 2, r1 = s + 3
        store_stage(r0, 0);
        load_stage(r0, s + 4);
        __syncthreads();
    }
    // act = SiLU(g) * u for this lane's row and 16 tokens
    const int r = rt * MROWS + bn;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int i = th * 32 + 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
        if (i < ti.nt) {
            const int slot = a.seg_slot[ti.slot0 + i];
            const float av = swiglu(tg[v], tu[v]);
            _Float16 hh, ll;
            split_hi_lo(av, hh, ll);
            a.act[(size_t)slot * a.m + r] = av;
            const size_t o = (size_t)slot * a.m + (r & ~7) + mfma_slot(r & 7);
            a.act_h[o] = hh;
            a.act_l[o] = ll;
        }
    }
}

// --------------------------------------------------------------------- down

template <int NGS>
struct DnStage {
    uint4 h, l;
    uint4 w;
    uint16_t sc[NGS];
};

template <int G>
__global__ void __launch_bounds__(MTHREADS, 1)
k_down_mfma(ExpertArgs a) {
    TileInfo ti;
    if (!tile_info(a, blockIdx.x, &ti)) return;
    constexpr int NGS = KS / G;
    constexpr int KSG = G / 16;
    __shared__ __align__(16) _Float16 xh[2][MT * KP], xl[2][MT * KP], wl[2][MROWS * KP];
    __shared__ float scl[2][MROWS][NGS];
    __shared__ int tok_s[MT];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = tid >> 6;
    const int rt = blockIdx.y;                    // 128-row tile of the hidden dimension
    const int m = a.m, ng = m / G, nstage = m / KS;
    if (tid < MT) tok_s[tid] = tid < ti.nt ? a.seg_slot[ti.slot0 + tid] : -1;
    unsigned long long so, po;
    a.rec.get(2, a.key0 + ti.e, so, po);
    __syncthreads();

    const int xt = tid >> 3, xpart = tid & 7;     // act: 8 threads x 8 columns per token
    const int wrow = (tid & 255) >> 1, wpiece = tid & 1;   // threads 0..255 stage the weights
    const bool wthr = tid < 2 * MROWS;
    const int xs = tok_s[xt];
    const size_t xo = (size_t)(xs >= 0 ? xs : 0) * m + xpart * 8;
    const uint8_t* wpk = a.blob + po + (size_t)(rt * MROWS + wrow) * (m / 2) + wpiece * 16;
    const uint16_t* wsc = (const uint16_t*)(a.blob + so) + (size_t)(rt * MROWS + wrow) * ng;

    auto load_stage = [&](DnStage<NGS>& r, int s) __attribute__((always_inline)) {
        s = s < nstage ? s : nstage - 1;
        r.h = *(const uint4*)(a.act_h + xo + s * KS);
        r.l = *(const uint4*)(a.act_l + xo + s * KS);
        r.w = *(const uint4*)(wpk + s * (KS / 2));
#pragma unroll
        for (int j = 0; j < NGS; j++) r.sc[j] = wsc[s * NGS + j];
    };
    auto store_stage = [&](const DnStage<NGS>& r, int buf) __attribute__((always_inline)) {
        const unsigned keep = xs >= 0 ? 0xFFFFFFFFu : 0u;     // padding tokens stage zeros
        *(uint4*)&xh[buf][xt * KP + xpart * 8] = make_uint4(r.h.x & keep, r.h.y & keep, r.h.z & keep, r.h.w & keep);
        *(uint4*)&xl[buf][xt * KP + xpart * 8] = make_uint4(r.l.x & keep, r.l.y & keep, r.l.z & keep, r.l.w & keep);
        if (wthr) {
            nibbles_to_lds(r.w, &wl[buf][wrow * KP + wpiece * 32]);
            if (wpiece == 0) {
#pragma unroll
                for (int j = 0; j < NGS; j++) scl[buf][wrow][j] = fp16_hw(r.sc[j]);
            }
        }
    };

    const int th = w & 1, rq = w >> 1;
    const int ai = th * 32 + (lane & 31), bn = rq * 32 + (lane & 31), kq = 8 * (lane >> 5);
    floatx16 tot = {};
    auto mfma_stage = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int gs = 0; gs < NGS; gs++) {
            floatx16 acc = {};
#pragma unroll
            for (int k2 = 0; k2 < KSG; k2++) {
                const int k0 = (gs * KSG + k2) * 16 + kq;
                const half8 a_h = *(const half8*)&xh[buf][ai * KP + k0];
                const half8 a_l = *(const half8*)&xl[buf][ai * KP + k0];
                const half8 b = *(const half8*)&wl[buf][bn * KP + k0];
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_h, b, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_l, b, acc, 0, 0, 0);
            }
            const float sc = scl[buf][bn][gs];
#pragma unroll
            for (int v = 0; v < 16; v++) tot[v] = __builtin_fmaf(sc, acc[v], tot[v]);
        }
    };
    DnStage<NGS> r0, r1;
    load_stage(r0, 0);
    load_stage(r1, 1);
    store_stage(r0, 0);
    load_stage(r0, 2);
    __syncthreads();
    for (int s = 0; s < nstage; s += 2) {
        mfma_stage(0);
        store_stage(r1, 1);
        load_stage(r1, s + 3);
        __syncthreads();
        mfma_stage(1);
        store_stage(r0, 0);
        load_stage(r0, s + 4);
        __syncthreads();
    }
    const int r = rt * MROWS + bn;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int i = th * 32 + 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
        if (i < ti.nt) {
            const int slot = tok_s[i];
            a.y[(size_t)slot * a.d + r] = __fmul_rn(a.tw[slot], tot[v]);
        }
    }
}

// the MFMA branch needs whole 128-row tiles and an even number of 64-column
// stages on both products
bool mfma_shape_ok(int d, int m) { return d % MROWS == 0 && m % MROWS == 0 && (d / KS) % 2 == 0 && (m / KS) % 2 == 0; }

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
