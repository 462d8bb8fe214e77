// Grouped Q4 expert product of the MoE block (gfx950), three launches:
//
//   k_gateup   per (active expert, 8 intermediate rows), one wave:
//              g = gate_row . x, u = up_row . x for every token routed to the
//              expert, act = (g / (1 + expf_fast(-g))) * u
//              (decode_kernel.c:1365-1375), and the 8 act values re-encoded
//              as digits with one scale for the down pass
//   k_down     per (active expert, 16 hidden rows), one wave:
//              y[slot][r] = w_slot * (down_row . act_slot) (:1376-1383)
//   k_combine  out[b] = the token's k expert rows summed in the reference's
//              union order (:1502-1507)
//
// Lane layout: a row of C columns is read as C/32 chunks of 16 bytes (32
// packed weights); lane col of an LPR-lane row segment holds chunks col,
// col + LPR, ... so that each load instruction of a wave covers whole rows
// of contiguous memory (one 1 KiB row per instruction for C = 2048).  A wave
// item issues every weight load of its rows before any arithmetic; the
// registers then serve each token of the expert's segment in turn while the
// next token's digits load.  Waves are independent: no barriers, no LDS.
// The work table (written by the dispatch, longest segments first) gives a
// wave its expert, segment and record offsets in one scalar load.
//
// The chunk dot runs on v_dot8_i32_i4: the packed nibbles XOR 0x8 are the
// signed values q - 8, and each activation value is given as NDIG signed
// base-16 digits of an exact integer a = rint(x / s), so sum (q - 8) * a is
// exact; it is scaled by s * (fp16 weight scale) in fp32.  Token digits come
// in groups of G values (one scale per weight group); act digits in groups
// of 8 (one scale per gate/up wave item).
#include "jm_device.h"
#include "jm_kernels.h"
#include "jm_q4dot.h"

namespace jm {

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

constexpr int GU_ROWS = 8;     // gate/up rows per wave item = act values per act scale
constexpr int DN_ROWS = 16;    // down rows per wave item

// ------------------------------------------------------------------ gate/up

template <int G, int NDIG, int LPR, int QC>
__global__ void __launch_bounds__(256)
k_gateup(ExpertArgs a) {
    constexpr int RPI = JM_WAVE / LPR;
    constexpr int S = GU_ROWS / RPI;
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nchunk = a.m / GU_ROWS;
    const int u = item / nchunk, c = item % nchunk;
    if (u >= a.umax) return;
    const ExpertWork wk = a.work[u];
    if (wk.n == 0) return;
    const int slotv = lane < wk.n ? a.seg_slot[wk.s0 + lane] : 0;   // slots of the first 64 tokens
    const int col = lane & (LPR - 1), rsub = lane / LPR;
    const int cpr = a.d / 32, ngroups = a.d / G;
    const int row0 = c * GU_ROWS + rsub;
    const uint8_t* pk_g = a.blob + wk.pk[0];
    const uint16_t* sc_g = (const uint16_t*)(a.blob + wk.sc[0]);
    const uint8_t* pk_u = a.blob + wk.pk[1];
    const uint16_t* sc_u = (const uint16_t*)(a.blob + wk.sc[1]);

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

    // keep every weight load ahead of the first token's digits and of all
    // arithmetic: waiting for the digits then also waits for the weights
    // (the memory counter retires loads in order), but nothing is issued late
    __builtin_amdgcn_sched_barrier(0);
    ChunkDigits<NDIG> cur[QC], nxt[QC];
    int slot = __builtin_amdgcn_readlane(slotv, 0);
    load_tok(cur, slot);
    __builtin_amdgcn_sched_barrier(0);
    // signed nibbles once, for every token
#pragma unroll
    for (int s = 0; s < S; s++)
#pragma unroll
        for (int q = 0; q < QC; q++) { wg[s][q] = flip_nibbles(wg[s][q]); wu[s][q] = flip_nibbles(wu[s][q]); }

    // after transpose_sum, row i = s * RPI + r of the item is in lanes
    // LPR * r + 8 * s (gate) and + 4 (up)
    const int i8 = lane & 7;
    const int src = LPR * (i8 % RPI) + 8 * (i8 / RPI);
    for (int t = 0; t < wk.n; t++) {
        int nslot = 0;
        if (t + 1 < wk.n) {
            nslot = t + 1 < 64 ? __builtin_amdgcn_readlane(slotv, t + 1) : a.seg_slot[wk.s0 + t + 1];
            load_tok(nxt, nslot);
        }
        float part[2 * S];                   // value 2s + m: step s, m = 0 gate, 1 up
#pragma unroll
        for (int s = 0; s < S; s++) {
            float pg = 0.0f, pu = 0.0f;
#pragma unroll
            for (int q = 0; q < QC; q++) {
                int ig = 0, iu = 0;
#pragma unroll
                for (int k = NDIG - 1; k >= 0; k--) {
                    ig = chunk_digit(wg[s][q], cur[q].d[k], ig);
                    iu = chunk_digit(wu[s][q], cur[q].d[k], iu);
                }
                const float xs = live[q] ? cur[q].s : 0.0f;
                pg = __fadd_rn(pg, __fmul_rn((float)ig, __fmul_rn(xs, fp16_hw(hg[s][q]))));
                pu = __fadd_rn(pu, __fmul_rn((float)iu, __fmul_rn(xs, fp16_hw(hu[s][q]))));
            }
            part[2 * s] = pg;
            part[2 * s + 1] = pu;
        }
        static_assert(2 * S == LPR / 4, "one transposed value per 4 lanes");
        const float tot = transpose_sum<LPR>(part);
        const float up = dpp_f<DPP_ROL4>(tot);          // lanes with bit 2 clear: gate here, up 4 lanes on
        const float av = swiglu(tot, up);
        // the item's 8 act values to lanes 0..7, then fp32 act and one
        // 8-value digit group
        const float mine = __shfl(av, src, JM_WAVE);
        if (lane < 8) a.act[(size_t)slot * a.m + c * GU_ROWS + lane] = mine;
        const size_t ai = (size_t)slot * (a.m / 8) + c;
        encode_group_wave<8, NDIG>(mine, lane < 8, a.adig + ai * NDIG, a.ascale + ai);
        if (t + 1 < wk.n) {
            slot = nslot;
#pragma unroll
            for (int q = 0; q < QC; q++) cur[q] = nxt[q];
        }
    }
}

// -------------------------------------------------------------------- down

template <int G, int NDIG, int LPR, int QC>
__global__ void __launch_bounds__(256)
k_down(ExpertArgs a) {
    constexpr int RPI = JM_WAVE / LPR;
    constexpr int S = DN_ROWS / RPI;
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nchunk = a.d / DN_ROWS;
    const int u = item / nchunk, c = item % nchunk;
    if (u >= a.umax) return;
    const ExpertWork wk = a.work[u];
    if (wk.n == 0) return;
    const int slotv = lane < wk.n ? a.seg_slot[wk.s0 + lane] : 0;
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

    // act digits of a chunk: 4 groups of 8 values, NDIG words each, 4 scales
    auto load_act = [&](uint32_t (&dg)[QC][4][NDIG], float4 (&sc)[QC], int slot) {
#pragma unroll
        for (int q = 0; q < QC; q++) {
            const size_t ai = (size_t)slot * (a.m / 8) + (size_t)chk[q] * 4;
            const uint4* p = (const uint4*)(a.adig + ai * NDIG);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                static_assert(NDIG == 4, "act digit loads assume 4 digits (one uint4 per 8 values)");
                const uint4 v = p[j];
                dg[q][j][0] = v.x; dg[q][j][1] = v.y; dg[q][j][2] = v.z; dg[q][j][3] = v.w;
            }
            sc[q] = *(const float4*)(a.ascale + ai);
        }
    };

    __builtin_amdgcn_sched_barrier(0);
    uint32_t cd[QC][4][NDIG], nd[QC][4][NDIG];
    float4 cs[QC], ns[QC];
    int slot = __builtin_amdgcn_readlane(slotv, 0);
    float wt = a.tw[slot];
    load_act(cd, cs, slot);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < S; s++)
#pragma unroll
        for (int q = 0; q < QC; q++) wd[s][q] = flip_nibbles(wd[s][q]);

    for (int t = 0; t < wk.n; t++) {
        int nslot = 0;
        float nwt = 0.0f;
        if (t + 1 < wk.n) {
            nslot = t + 1 < 64 ? __builtin_amdgcn_readlane(slotv, t + 1) : a.seg_slot[wk.s0 + t + 1];
            nwt = a.tw[nslot];
            load_act(nd, ns, nslot);
        }
        float part[S];
#pragma unroll
        for (int s = 0; s < S; s++) {
            float ps = 0.0f;
#pragma unroll
            for (int q = 0; q < QC; q++) {
                const uint32_t fw[4] = {wd[s][q].x, wd[s][q].y, wd[s][q].z, wd[s][q].w};
                const float sj[4] = {cs[q].x, cs[q].y, cs[q].z, cs[q].w};
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    int iv = 0;
#pragma unroll
                    for (int k = NDIG - 1; k >= 0; k--) iv = dot8(fw[j], cd[q][j][k], iv << 4);
                    acc = __fadd_rn(acc, __fmul_rn((float)iv, sj[j]));
                }
                ps = __fadd_rn(ps, live[q] ? __fmul_rn(acc, fp16_hw(hd[s][q])) : 0.0f);
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
            for (int q = 0; q < QC; q++) {
                cs[q] = ns[q];
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int k = 0; k < NDIG; k++) cd[q][j][k] = nd[q][j][k];
            }
        }
    }
}

// ----------------------------------------------------------------- combine

__global__ void __launch_bounds__(256)
k_combine(const float* __restrict__ y, const int* __restrict__ comb, int B, int k, int d,
          float* __restrict__ out) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    const int d4 = d / 4;
    if (idx >= B * d4) return;
    const int b = idx / d4, r = 4 * (idx % d4);
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // no early exit: the loads of all k slots can be in flight together
#pragma unroll 8
    for (int i = 0; i < k; i++) {
        const int s = comb[b * k + i];
        const float4 v = s >= 0 ? *(const float4*)(y + (size_t)s * d + r) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (s >= 0) {
            acc.x = __fadd_rn(acc.x, v.x); acc.y = __fadd_rn(acc.y, v.y);
            acc.z = __fadd_rn(acc.z, v.z); acc.w = __fadd_rn(acc.w, v.w);
        }
    }
    *(float4*)(out + (size_t)b * d + r) = acc;
}

// lanes per row segment and 16-byte chunks per lane for rows of C columns
static inline void row_lanes(int C, int* lpr, int* qc) {
    const int cpr = C / 32;
    *qc = (cpr + 63) / 64;
    const int raw = (cpr + *qc - 1) / *qc;
    *lpr = raw <= 16 ? 16 : raw <= 32 ? 32 : 64;
}

hipError_t launch_gateup(const ExpertArgs& a, int umax, hipStream_t st) {
    const long long waves = (long long)umax * (a.m / GU_ROWS);
    if (waves == 0) return hipSuccess;
    const dim3 grid((unsigned)((waves + 3) / 4));
    int lpr, qc;
    row_lanes(a.d, &lpr, &qc);
#define JM_GU(GG, L, Q) hipLaunchKernelGGL((k_gateup<GG, JM_NDIG, L, Q>), grid, dim3(256), 0, st, a)
#define JM_GUG(GG) if (qc == 2) JM_GU(GG, 64, 2); else if (lpr == 64) JM_GU(GG, 64, 1); \
                   else if (lpr == 32) JM_GU(GG, 32, 1); else JM_GU(GG, 16, 1);
    if (qc > 2) return hipErrorInvalidValue;
    if (a.group == 64) { JM_GUG(64) } else { JM_GUG(32) }
#undef JM_GUG
#undef JM_GU
    return hipGetLastError();
}

hipError_t launch_down(const ExpertArgs& a, int umax, hipStream_t st) {
    const long long waves = (long long)umax * (a.d / DN_ROWS);
    if (waves == 0) return hipSuccess;
    const dim3 grid((unsigned)((waves + 3) / 4));
    int lpr, qc;
    row_lanes(a.m, &lpr, &qc);
#define JM_DN(GG, L, Q) hipLaunchKernelGGL((k_down<GG, JM_NDIG, L, Q>), grid, dim3(256), 0, st, a)
#define JM_DNG(GG) if (qc == 2) JM_DN(GG, 64, 2); else if (lpr == 64) JM_DN(GG, 64, 1); \
                   else if (lpr == 32) JM_DN(GG, 32, 1); else JM_DN(GG, 16, 1);
    if (qc > 2) return hipErrorInvalidValue;
    if (a.group == 64) { JM_DNG(64) } else { JM_DNG(32) }
#undef JM_DNG
#undef JM_DN
    return hipGetLastError();
}

hipError_t launch_combine(const float* y, const int* comb, int B, int k, int d, float* out, hipStream_t st) {
    const long long n = (long long)B * (d / 4);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, y, comb, B, k, d, out);
    return hipGetLastError();
}

}  // namespace jm
