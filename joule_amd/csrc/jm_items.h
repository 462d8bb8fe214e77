// Wave items of the grouped Q4 expert product (gfx950), shared by the
// wave-item kernels (jm_experts.hip) and the MFMA kernels (jm_mfma.hip),
// whose surplus blocks run the small experts' items in their last round.
// The arithmetic is described at the top of jm_experts.hip.
#pragma once

#include <type_traits>

#include "jm_device.h"
#include "jm_kernels.h"
#include "jm_q4dot.h"

namespace jm {
namespace wi {

__device__ __forceinline__ uint4 flip_nibbles(uint4 v) {
    return make_uint4(v.x ^ 0x88888888u, v.y ^ 0x88888888u, v.z ^ 0x88888888u, v.w ^ 0x88888888u);
}

// sum over the 8 nibble pairs of the four words of a chunk (weights already
// XOR 0x8) for one digit, added to acc shifted by one digit (Horner over the
// digits)
__device__ __forceinline__ int chunk_digit(const uint4& w, const uint4& d, int acc) {
    acc = dot8(w.x, d.x, acc << 4);
    acc = dot8(w.y, d.y, acc);
    acc = dot8(w.z, d.z, acc);
    return dot8(w.w, d.w, acc);
}

// Digits of one token for one 16-byte chunk: NDIG words-quads and a scale.
template <int NDIG>
struct ChunkDigits {
    uint4 d[NDIG];
    float s;
};

// Exact sum over a 32-value chunk of (q - 8) * a for weights f (signed
// nibbles) and one token's digits of the chunk (Horner over the digit
// planes: v_dot8 accumulates in place, so one chain needs one zero).
template <int NDIG>
__device__ __forceinline__ int chunk_dot(const uint4& f, const ChunkDigits<NDIG>& cd) {
    int iv = 0;
#pragma unroll
    for (int k = NDIG - 1; k >= 0; k--) iv = chunk_digit(f, cd.d[k], iv);
    return iv;
}

constexpr int GU_ROWS = 8;     // gate/up rows per wave item (a block's 4 items share an act scale)
constexpr int DN_ROWS = 16;    // down rows per wave item

// ------------------------------------------------------------------ gate/up

// One wave item of the gate/up product: entry u (BALLOT: a slot of the
// top-k table; otherwise an entry of the dispatch path's work table),
// intermediate rows [GU_ROWS c, GU_ROWS (c + 1)).  gmax / gbad are the LDS
// slots where the 4 waves holding rows 32 (c / 4) .. 32 (c / 4) + 31 of a
// slot meet for their act scale, behind a block-wide barrier per token: the
// caller gives every wave of a block the same u (so the same token count)
// and items c of one group of 4 in one group of 4 waves.
template <int G, int NDIG, int LPR, int QC, bool BALLOT>
__device__ __forceinline__ void gateup_item(const ExpertArgs& a, const int* top, int u, int c,
                                            float (&gmax)[2][4], int (&gbad)[2][4]) {
    constexpr int RPI = JM_WAVE / LPR;
    constexpr int S = GU_ROWS / RPI;
    const int lane = threadIdx.x & 63;
    // the expert, its record offsets and its slots
    unsigned long long so_g, po_g, so_u, po_u;
    int n;
    BallotSlots bs;
    TableSlots ts;
    if constexpr (BALLOT) {
        if (u >= a.nslot) return;
        int e;
        if (!bs.init(top, a.nslot, a.E, u, &e)) return;
        n = bs.n;
        a.rec.get(0, a.key0 + e, so_g, po_g);
        a.rec.get(1, a.key0 + e, so_u, po_u);
    } else {
        if (u >= a.umax) return;
        const ExpertWork wk = a.work[u];
        if (wk.n == 0 || wk.n >= a.dense_min) return;     // none, or the MFMA branch's
        n = wk.n;
        ts.init(a.seg_slot, wk.s0, wk.n);
        so_g = wk.sc[0]; po_g = wk.pk[0];
        so_u = wk.sc[1]; po_u = wk.pk[1];
    }
    auto next_slot = [&]() { if constexpr (BALLOT) return bs.next(); else return ts.next(); };
    const int col = lane & (LPR - 1), rsub = lane / LPR;
    const int cpr = a.d / 32, ngroups = a.d / G;
    const int row0 = c * GU_ROWS + rsub;
    const uint8_t* pk_g = a.blob + po_g;
    const uint16_t* sc_g = (const uint16_t*)(a.blob + so_g);
    const uint8_t* pk_u = a.blob + po_u;
    const uint16_t* sc_u = (const uint16_t*)(a.blob + so_u);

    // chunks past the row (lanes beyond C/32) read chunk 0 and count zero:
    // every load is unconditional, so the loads of all steps are in flight
    // together
    bool live[QC];
    int chk[QC], grp[QC], half[QC];
#pragma unroll
    for (int q = 0; q < QC; q++) {
        const int ch = col + LPR * q;
        live[q] = ch < cpr;
        chk[q] = live[q] ? ch : 0;
        grp[q] = chk[q] * 32 / G;
        half[q] = (chk[q] * 32 % G) / 32;
    }
    auto load_tok = [&](ChunkDigits<NDIG> (&td)[QC], int slot) {
        const size_t b = (size_t)(slot / a.topk);
#pragma unroll
        for (int q = 0; q < QC; q++) {
            const size_t gi = b * ngroups + grp[q];
            const uint4* p = (const uint4*)(a.xdig + gi * (NDIG * (G / 8))) + half[q];
#pragma unroll
            for (int k = 0; k < NDIG; k++) td[q].d[k] = p[k * (G / 32)];
            td[q].s = a.xscale[gi];
        }
    };

    // requests in the order of use: the first token's digits, then the
    // weight rows step by step.  The memory counter retires loads in order,
    // so the first token's arithmetic on step s waits only for the loads up
    // to step s while the later steps' rows are still arriving.
    ChunkDigits<NDIG> cur[QC], nxt[QC];
    int slot = next_slot();
    load_tok(cur, slot);
    __builtin_amdgcn_sched_barrier(0);
    uint4 wg[S][QC], wu[S][QC];
    uint16_t hg[S][QC], hu[S][QC];
#pragma unroll
    for (int s = 0; s < S; s++) {
        const int row = row0 + s * RPI;
#pragma unroll
        for (int q = 0; q < QC; q++) {
            const size_t o = (size_t)row * (a.d / 2) + (size_t)chk[q] * 16;
            wg[s][q] = *(const uint4*)(pk_g + o);
            wu[s][q] = *(const uint4*)(pk_u + o);
            hg[s][q] = sc_g[(size_t)row * ngroups + grp[q]];
            hu[s][q] = sc_u[(size_t)row * ngroups + grp[q]];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // after transpose_sum, row i = s * RPI + r of the item is in lanes
    // LPR * r + 8 * s (gate) and + 4 (up)
    const int i8 = lane & 7;
    const int src = LPR * (i8 % RPI) + 8 * (i8 / RPI);
    // the item's gate and up partial sums (value 2s + m: step s, m = 0 gate,
    // 1 up) for one token.  The first token takes the steps in order with a
    // scheduling barrier after each, turning each step's rows into signed
    // nibbles (q - 8) in place, so that its arithmetic on step s waits only
    // for the loads up to step s; the later tokens reuse the signed rows.
    auto parts = [&](const ChunkDigits<NDIG> (&cd)[QC], float (&part)[2 * S], auto first) {
#pragma unroll
        for (int s = 0; s < S; s++) {
            float pg = 0.0f, pu = 0.0f;
#pragma unroll
            for (int q = 0; q < QC; q++) {
                if constexpr (decltype(first)::value) {
                    wg[s][q] = flip_nibbles(wg[s][q]);
                    wu[s][q] = flip_nibbles(wu[s][q]);
                }
                int ig = 0, iu = 0;
#pragma unroll
                for (int k = NDIG - 1; k >= 0; k--) {
                    ig = chunk_digit(wg[s][q], cd[q].d[k], ig);
                    iu = chunk_digit(wu[s][q], cd[q].d[k], iu);
                }
                const float xs = live[q] ? cd[q].s : 0.0f;
                pg = __fadd_rn(pg, __fmul_rn((float)ig, __fmul_rn(xs, fp16_hw(hg[s][q]))));
                pu = __fadd_rn(pu, __fmul_rn((float)iu, __fmul_rn(xs, fp16_hw(hu[s][q]))));
            }
            part[2 * s] = pg;
            part[2 * s + 1] = pu;
            if constexpr (decltype(first)::value) __builtin_amdgcn_sched_barrier(0);
        }
    };
    // SwiGLU of the item's 8 rows for the token of slot sl: the 8 act values
    // to lanes 0..7, then fp32 act and their digits.  The 4 waves of the
    // block hold rows 32 cb .. 32 cb + 31 of the same slot (items 4 cb ..
    // 4 cb + 3) and share one digit scale: the maxima meet in LDS (a
    // block-uniform barrier: the waves have the same slot and token count).
    const int wib = c & 3, cb = c >> 2;
    auto finish = [&](float (&part)[2 * S], int sl, int t) {
        static_assert(2 * S == LPR / 4, "one transposed value per 4 lanes");
        const float tot = transpose_sum<LPR>(part);
        const float up = dpp_f<DPP_ROL4>(tot);          // lanes with bit 2 clear: gate here, up 4 lanes on
        const float av = swiglu(tot, up);
        const float mine = __shfl(av, src, JM_WAVE);
        if (lane < 8) a.act[(size_t)sl * a.m + c * GU_ROWS + lane] = mine;
        const float am = lane < 8 ? fabsf(mine) : 0.0f;
        const int bad = seg_or<8>(!(am <= 3.4028235e38f) ? 1 : 0);
        const float mx8 = seg_max<8>(am);
        if (lane == 0) {
            gmax[t & 1][wib] = mx8;
            gbad[t & 1][wib] = bad;
        }
        __syncthreads();
        const float mx = fmaxf(fmaxf(gmax[t & 1][0], gmax[t & 1][1]), fmaxf(gmax[t & 1][2], gmax[t & 1][3]));
        const bool nf = (gbad[t & 1][0] | gbad[t & 1][1] | gbad[t & 1][2] | gbad[t & 1][3]) != 0;
        const size_t gi = (size_t)sl * (a.m / 32) + cb;
        encode_digits_shared<NDIG>(mine, mx, nf, lane < 8, a.adig + gi * (NDIG * 4) + wib);
        if (wib == 0 && lane == 0) a.ascale[gi] = digit_scale<NDIG>(mx, nf);
    };
    int nslot = 0;
    if (n > 1) {
        nslot = next_slot();
        load_tok(nxt, nslot);
    }
    {
        float part[2 * S];
        parts(cur, part, std::true_type{});
        finish(part, slot, 0);
    }
    for (int t = 1; t < n; t++) {
        slot = nslot;
#pragma unroll
        for (int q = 0; q < QC; q++) cur[q] = nxt[q];
        if (t + 1 < n) {
            nslot = next_slot();
            load_tok(nxt, nslot);
        }
        float part[2 * S];
        parts(cur, part, std::false_type{});
        finish(part, slot, t);
    }
}


// One wave item of the down product: work-table entry u, hidden rows
// [DN_ROWS c, DN_ROWS (c + 1)), into y (no barriers).
template <int G, int NDIG, int LPR, int QC>
__device__ __forceinline__ void down_item(const ExpertArgs& a, int u, int c) {
    constexpr int RPI = JM_WAVE / LPR;
    constexpr int S = DN_ROWS / RPI;
    const int lane = threadIdx.x & 63;
    if (u >= a.umax) return;
    const ExpertWork wk = a.work[u];
    if (wk.n == 0 || wk.n >= a.dense_min) return;         // none, or the MFMA branch's
    TableSlots ts;
    ts.init(a.seg_slot, wk.s0, wk.n);
    const int col = lane & (LPR - 1), rsub = lane / LPR;
    const int cpr = a.m / 32, ngroups = a.m / G;
    const int row0 = c * DN_ROWS + rsub;
    const uint8_t* pk_d = a.blob + wk.pk[2];
    const uint16_t* sc_d = (const uint16_t*)(a.blob + wk.sc[2]);

    // chunks past the row read chunk 0 and count zero (unconditional loads)
    bool live[QC];
    int chk[QC], grp[QC];
#pragma unroll
    for (int q = 0; q < QC; q++) {
        const int ch = col + LPR * q;
        live[q] = ch < cpr;
        chk[q] = live[q] ? ch : 0;
        grp[q] = chk[q] * 32 / G;
    }
    uint4 wd[S][QC];
    uint16_t hd[S][QC];
#pragma unroll
    for (int s = 0; s < S; s++) {
        const int row = row0 + s * RPI;
#pragma unroll
        for (int q = 0; q < QC; q++) {
            wd[s][q] = *(const uint4*)(pk_d + (size_t)row * (a.m / 2) + (size_t)chk[q] * 16);
            hd[s][q] = sc_d[(size_t)row * ngroups + grp[q]];
        }
    }

    // act digits of a chunk (32 values, one scale)
    auto load_act = [&](ChunkDigits<NDIG> (&ad)[QC], int slot) {
#pragma unroll
        for (int q = 0; q < QC; q++) {
            const size_t gi = (size_t)slot * (a.m / 32) + chk[q];
            const uint4* p = (const uint4*)(a.adig + gi * (NDIG * 4));
#pragma unroll
            for (int k = 0; k < NDIG; k++) ad[q].d[k] = p[k];
            ad[q].s = a.ascale[gi];
        }
    };

    __builtin_amdgcn_sched_barrier(0);
    ChunkDigits<NDIG> cd[QC], nd[QC];
    int slot = ts.next();
    float wt = a.tw[slot];
    load_act(cd, slot);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < S; s++)
#pragma unroll
        for (int q = 0; q < QC; q++) wd[s][q] = flip_nibbles(wd[s][q]);

    for (int t = 0; t < wk.n; t++) {
        int nslot = 0;
        float nwt = 0.0f;
        if (t + 1 < wk.n) {
            nslot = ts.next();
            nwt = a.tw[nslot];
            load_act(nd, nslot);
        }
        float part[S];
#pragma unroll
        for (int s = 0; s < S; s++) {
            float ps = 0.0f;
#pragma unroll
            for (int q = 0; q < QC; q++) {
                const int iv = chunk_dot(wd[s][q], cd[q]);
                ps = __builtin_fmaf((float)iv, live[q] ? __fmul_rn(cd[q].s, fp16_hw(hd[s][q])) : 0.0f, ps);
            }
            part[s] = ps;
        }
        static_assert(S == LPR / 4, "one transposed value per 4 lanes");
        // row s * RPI + r of the item ends in lanes LPR * r + 4 * s
        const float v = transpose_sum<LPR>(part);
        if ((lane & 3) == 0)
            a.y[(size_t)slot * a.d + c * DN_ROWS + ((lane & (LPR - 1)) >> 2) * RPI + rsub] = __fmul_rn(wt, v);
        if (t + 1 < wk.n) {
            slot = nslot;
            wt = nwt;
#pragma unroll
            for (int q = 0; q < QC; q++) cd[q] = nd[q];
        }
    }
}


}  // namespace wi
}  // namespace jm
