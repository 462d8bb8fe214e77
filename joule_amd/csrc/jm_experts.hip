// Grouped Q4 expert product of the MoE block (gfx950).
//
// Decode path (B * topk <= 256 slots), two launches after the routing:
//   k_gateup<BALLOT>  per (slot, 8 intermediate rows), one wave (for batches
//                     of up to JM_GU_TOPK_MAX_B tokens each block of 4 waves
//                     first computes the top-k of every token); the wave of
//                     an expert's first slot finds all its slots by a ballot
//                     over the top-k table (others exit) and computes
//                     g = gate_row . x, u = up_row . x for each of them,
//                     act = (g / (1 + expf_fast(-g))) * u
//                     (decode_kernel.c:1365-1375), and the 8 act values
//                     re-encoded as digits with one scale for the down pass
//   k_down_comb       per chunk of 8 hidden rows, one block: every routed
//                     expert's rows against the act of each of its slots,
//                     y = w_slot * (down_row . act) (:1376-1383) into LDS,
//                     then out[b][rows] = the token's k values summed in the
//                     reference's union order (:1502-1507)
// Dispatch path (more slots): the same gate/up over the work table the
// dispatch kernel writes, k_down per (expert, 16 hidden rows) into y, and
// k_combine; experts with dense_min or more slots are left to the MFMA
// kernels (jm_mfma.hip).
//
// Lane layout: a row of C columns is read as C/32 chunks of 16 bytes (32
// packed weights); lane col of an LPR-lane row segment holds chunks col,
// col + LPR, ... so that each load instruction of a wave covers whole rows
// of contiguous memory (one 1 KiB row per instruction for C = 2048).  A wave
// item issues every weight load of its rows before any arithmetic; the
// registers then serve each token of the expert in turn while the next
// token's digits load.
//
// The chunk dot runs on v_dot8_i32_i4: the packed nibbles XOR 0x8 are the
// signed values q - 8, and each activation value is given as NDIG signed
// base-16 digits of an exact integer a = rint(x / s), so sum (q - 8) * a is
// exact; it is scaled by s * (fp16 weight scale) in fp32.  Token digits come
// in groups of G values (one scale per weight group); act digits in groups
// of 32 (one scale per chunk of a down row: the 4 gate/up wave items of a
// block, which hold 32 consecutive rows of one slot, share it).
#include "jm_items.h"

namespace jm {

using namespace wi;

// ------------------------------------------------------------------ gate/up

// EPL > 0 (decode path, small batches): the block first computes the top-k
// of every token from the router scores itself (softmax, top-k and renorm as
// k_topk: decode_kernel.c:1425-1448, topk_wave), its 4 waves taking tokens
// w, w + 4, ...; block 0 also writes the table for the down kernel and the
// caller.  This replaces the top-k launch.
template <int G, int NDIG, int LPR, int QC, bool BALLOT, int EPL>
__global__ void __launch_bounds__(256)
k_gateup(ExpertArgs a) {
    __shared__ float gmax[2][4];       // per token parity: each wave's max |act|
    __shared__ int gbad[2][4];         // and whether it saw a non-finite value
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int item = blockIdx.x * 4 + wave;
    const int nchunk = a.m / GU_ROWS;
    const int* top = a.top;
    if constexpr (BALLOT && EPL > 0) {
        constexpr int EP = EPL > 0 ? EPL : 1;
        __shared__ int top_s[JM_DEC_SLOTS];
        __shared__ float tw_s[JM_DEC_SLOTS];
        __shared__ float p_s[4][64 * EP];
        for (int b = wave; b < a.B; b += 4)
            topk_wave<EP>(a.logits + (size_t)b * a.E, a.E, a.topk, a.renorm, p_s[wave],
                          top_s + b * a.topk, tw_s + b * a.topk);
        __syncthreads();
        if (blockIdx.x == 0)
            for (int i = threadIdx.x; i < a.nslot; i += 256) {
                a.top_w[i] = top_s[i];
                a.tw_w[i] = tw_s[i];
            }
        top = top_s;
    }
    gateup_item<G, NDIG, LPR, QC, BALLOT>(a, top, item / nchunk, item % nchunk, gmax, gbad);
}

// -------------------------------------------------------------------- down

template <int G, int NDIG, int LPR, int QC>
__global__ void __launch_bounds__(256)
k_down(ExpertArgs a) {
    const int item = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nchunk = a.d / DN_ROWS;
    down_item<G, NDIG, LPR, QC>(a, item / nchunk, item % nchunk);
}

// ---------------------------------------------------------- down + combine

constexpr int DC_ROWS = 8;             // hidden rows per block

// Threads per block and experts in flight per wave of the down/combine
// kernel: one expert in flight, with 16 waves for rows of at most 32 chunks
// (m <= 1024; 13.4 us on the Qwen3 block at B = 8 against 14.4 for 12
// waves with two experts, 17.4 for 16-row blocks, 20 to 22 for 4-row
// blocks) and 12 waves for wider rows, whose registers do not fit 16.
template <int LPR>
struct DcShape {
    static constexpr int THREADS = LPR <= 32 ? 1024 : 768;
    static constexpr int NR = 1;
};

// Decode path: block c owns hidden rows [c * DC_ROWS, (c + 1) * DC_ROWS) of
// every token.  It lists the routed experts in the reference's union order
// (first appearance over the slots); wave w of NW takes experts w, w + NW,
// ..., keeping NR of them in flight (each expert's rows, and the act digits of
// its first slot, requested in that order), writes w_slot * (rows . act_slot)
// for each slot into LDS, and finally sums each token's values in union
// order.  Every block streams the same bytes: the rows of all routed
// experts.
template <int G, int NDIG, int LPR, int QC>
__global__ void __launch_bounds__(DcShape<LPR>::THREADS)
k_down_comb(ExpertArgs a) {
    constexpr int DC_THREADS = DcShape<LPR>::THREADS;
    constexpr int DC_WAVES = DC_THREADS / 64;
    constexpr int R = DC_ROWS;
    constexpr int RPI = JM_WAVE / LPR;          // rows per load instruction
    constexpr int S = R / RPI;                  // load steps per expert
    static_assert(S >= 1 && S * RPI == R, "whole rows per step");
    constexpr int NR = DcShape<LPR>::NR;        // experts in flight per wave
    static_assert(JM_DEC_SLOTS <= DC_THREADS, "a slot per thread");
    __shared__ int top_l[JM_DEC_SLOTS], ulist[JM_DEC_SLOTS], comb_l[JM_DEC_SLOTS];
    __shared__ int first_l[JM_MAX_E];
    __shared__ float tw_l[JM_DEC_SLOTS];
    __shared__ float ypart[JM_DEC_SLOTS * R];
    __shared__ int wcnt[JM_DEC_SLOTS / 64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = blockIdx.x;
    const int nslot = a.nslot, E = a.E, k = a.topk;

    if (tid < nslot) tw_l[tid] = a.tw[tid];
    int e_me;
    const int U = decode_union<JM_DEC_SLOTS>(a.top, nslot, E, top_l, first_l, ulist, wcnt, &e_me);
    // each token's slots ranked by the first slot of their expert (distinct
    // experts -> distinct keys); slots without an expert last, as -1
    if (tid < nslot) {
        const int b = tid / k, i = tid % k;
        const int key = e_me >= 0 ? first_l[e_me] : 0x7FFFFFFF;
        int rnk = 0;
        for (int j = 0; j < k; j++) {
            const int ej = top_l[b * k + j];
            const int kj = (ej >= 0 && ej < E) ? first_l[ej] : 0x7FFFFFFF;
            rnk += (kj < key) || (kj == key && j < i);
        }
        comb_l[b * k + rnk] = e_me >= 0 ? tid : -1;
    }
    __syncthreads();

    const int col = lane & (LPR - 1), rsub = lane / LPR;
    const int cpr = a.m / 32, ngroups = a.m / G;
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
    // act digits of a chunk (32 values, one scale)
    struct Act {
        ChunkDigits<NDIG> c[QC];
    };
    auto load_act = [&](Act& ad, int slot) {
#pragma unroll
        for (int q = 0; q < QC; q++) {
            const size_t gi = (size_t)slot * (a.m / 32) + chk[q];
            const uint4* p = (const uint4*)(a.adig + gi * (NDIG * 4));
#pragma unroll
            for (int k = 0; k < NDIG; k++) ad.c[q].d[k] = p[k];
            ad.c[q].s = a.ascale[gi];
        }
    };
    struct Rows {
        uint4 wd[S][QC];
        uint16_t hd[S][QC];
    };
    // expert u: the act digits of its first slot, then its rows
    auto issue = [&](Rows& rw, Act& ad, int u) {
        const int s0 = ulist[u];
        const int e = top_l[s0];
        load_act(ad, s0);
        unsigned long long so, po;
        a.rec.get(2, a.key0 + e, so, po);
        const uint8_t* pk = a.blob + po;
        const uint16_t* scl = (const uint16_t*)(a.blob + so);
#pragma unroll
        for (int s = 0; s < S; s++) {
            const int row = c * R + rsub + s * RPI;
#pragma unroll
            for (int q = 0; q < QC; q++) {
                rw.wd[s][q] = *(const uint4*)(pk + (size_t)row * (a.m / 2) + (size_t)chk[q] * 16);
                rw.hd[s][q] = scl[(size_t)row * ngroups + grp[q]];
            }
        }
    };
    auto slot_dot = [&](const Rows& rw, const Act& ad, int slot) {
        float part[S];
#pragma unroll
        for (int s = 0; s < S; s++) {
            float ps = 0.0f;
#pragma unroll
            for (int q = 0; q < QC; q++) {
                const int iv = chunk_dot(flip_nibbles(rw.wd[s][q]), ad.c[q]);
                ps = __builtin_fmaf((float)iv, live[q] ? __fmul_rn(ad.c[q].s, fp16_hw(rw.hd[s][q])) : 0.0f, ps);
            }
            part[s] = ps;
        }
        // row s * RPI + rsub of the block's rows ends in the lanes with
        // (lane % LPR) / (LPR / S) == s
        const float v = transpose_reduce<LPR, S>(part);
        if ((lane & (LPR / S - 1)) == 0) {
            const int s_idx = (lane & (LPR - 1)) / (LPR / S);
            ypart[slot * R + s_idx * RPI + rsub] = __fmul_rn(tw_l[slot], v);
        }
    };
    // all slots of expert u; the later slots' digits are requested on demand
    auto expert = [&](const Rows& rw, const Act& ad, int u) {
        const int s0 = ulist[u];
        BallotSlots bs;
        bs.init_lds(top_l, nslot, top_l[s0]);
        (void)bs.next();                      // s0
        slot_dot(rw, ad, s0);
        for (int t = 1; t < bs.n; t++) {
            const int slot = bs.next();
            Act more;
            load_act(more, slot);
            slot_dot(rw, more, slot);
        }
    };
    const int nj = U > w ? (U - w + DC_WAVES - 1) / DC_WAVES : 0;   // this wave's experts
    Rows rw[NR];
    Act ad[NR];
#pragma unroll
    for (int q = 0; q < NR; q++)
        if (q < nj) issue(rw[q], ad[q], w + q * DC_WAVES);
    for (int j0 = 0; j0 < nj; j0 += NR) {
#pragma unroll
        for (int q = 0; q < NR; q++) {
            const int j = j0 + q;
            if (j < nj) {
                expert(rw[q], ad[q], w + j * DC_WAVES);
                if (j + NR < nj) issue(rw[q], ad[q], w + (j + NR) * DC_WAVES);
            }
        }
    }
    __syncthreads();
    for (int o = tid; o < a.B * R; o += DC_THREADS) {
        const int b = o / R, rr = o % R;
        float acc = 0.0f;
        for (int j = 0; j < k; j++) {
            const int sl = comb_l[b * k + j];
            if (sl >= 0) acc = __fadd_rn(acc, ypart[sl * R + rr]);
        }
        const size_t oi = (size_t)b * a.d + (size_t)c * R + rr;
        // the residual add h + block of the decoder layer (resid may be out)
        a.out[oi] = a.resid ? __fadd_rn(a.resid[oi], acc) : acc;
    }
}

// ----------------------------------------------------------------- combine

__global__ void __launch_bounds__(256)
k_combine(const float* __restrict__ y, const int* __restrict__ comb, int B, int k, int d,
          const float* resid, float* out) {
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
    if (resid) {   // the residual add h + block of the decoder layer
        const float4 h = *(const float4*)(resid + (size_t)b * d + r);
        acc = make_float4(__fadd_rn(h.x, acc.x), __fadd_rn(h.y, acc.y), __fadd_rn(h.z, acc.z), __fadd_rn(h.w, acc.w));
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

template <bool BALLOT, int EPL>
static hipError_t gateup_launch(const ExpertArgs& a, long long items, hipStream_t st) {
    const long long waves = items * (a.m / GU_ROWS);
    if (waves == 0) return hipSuccess;
    const dim3 grid((unsigned)((waves + 3) / 4));
    int lpr, qc;
    row_lanes(a.d, &lpr, &qc);
    if (a.ndig != 4 && a.ndig != 5) return hipErrorInvalidValue;
#define JM_GU(GG, L, Q) do { if (a.ndig == 5) hipLaunchKernelGGL((k_gateup<GG, 5, L, Q, BALLOT, EPL>), grid, dim3(256), 0, st, a); \
                             else hipLaunchKernelGGL((k_gateup<GG, 4, L, Q, BALLOT, EPL>), grid, dim3(256), 0, st, a); } while (0)
#define JM_GUG(GG) if (qc == 2) JM_GU(GG, 64, 2); else if (lpr == 64) JM_GU(GG, 64, 1); \
                   else if (lpr == 32) JM_GU(GG, 32, 1); else JM_GU(GG, 16, 1);
    if (qc > 2) return hipErrorInvalidValue;
    if (a.group == 64) { JM_GUG(64) } else { JM_GUG(32) }
#undef JM_GUG
#undef JM_GU
    return hipGetLastError();
}

hipError_t launch_gateup(const ExpertArgs& a, int umax, hipStream_t st) {
    return gateup_launch<false, 0>(a, umax, st);
}

bool gateup_topk(int B, int E) { return B <= JM_GU_TOPK_MAX_B && E <= JM_MAX_E; }

hipError_t launch_gateup_dec(const ExpertArgs& a, hipStream_t st) {
    if (a.nslot > JM_DEC_SLOTS) return hipErrorInvalidValue;
    if (!gateup_topk(a.B, a.E)) return gateup_launch<true, 0>(a, a.nslot, st);
    if (!a.logits || !a.top_w || !a.tw_w) return hipErrorInvalidValue;
    return a.E <= 128 ? gateup_launch<true, 2>(a, a.nslot, st) : gateup_launch<true, 8>(a, a.nslot, st);
}

hipError_t launch_down_comb(const ExpertArgs& a, hipStream_t st) {
    if (a.nslot > JM_DEC_SLOTS || a.E > JM_MAX_E || a.d % DC_ROWS) return hipErrorInvalidValue;
    if (a.nslot == 0) return hipSuccess;
    const dim3 grid((unsigned)(a.d / DC_ROWS));
    int lpr, qc;
    row_lanes(a.m, &lpr, &qc);
    if (a.ndig != 4 && a.ndig != 5) return hipErrorInvalidValue;
#define JM_DC(GG, L, Q) do { if (a.ndig == 5) hipLaunchKernelGGL((k_down_comb<GG, 5, L, Q>), grid, dim3(DcShape<L>::THREADS), 0, st, a); \
                             else hipLaunchKernelGGL((k_down_comb<GG, 4, L, Q>), grid, dim3(DcShape<L>::THREADS), 0, st, a); } while (0)
#define JM_DCG(GG) if (qc == 2) JM_DC(GG, 64, 2); else if (lpr == 64) JM_DC(GG, 64, 1); \
                   else if (lpr == 32) JM_DC(GG, 32, 1); else JM_DC(GG, 16, 1);
    if (qc > 2) return hipErrorInvalidValue;
    if (a.group == 64) { JM_DCG(64) } else { JM_DCG(32) }
#undef JM_DCG
#undef JM_DC
    return hipGetLastError();
}

hipError_t launch_down(const ExpertArgs& a, int umax, hipStream_t st) {
    const long long waves = (long long)umax * (a.d / DN_ROWS);
    if (waves == 0) return hipSuccess;
    const dim3 grid((unsigned)((waves + 3) / 4));
    int lpr, qc;
    row_lanes(a.m, &lpr, &qc);
    if (a.ndig != 4 && a.ndig != 5) return hipErrorInvalidValue;
#define JM_DN(GG, L, Q) do { if (a.ndig == 5) hipLaunchKernelGGL((k_down<GG, 5, L, Q>), grid, dim3(256), 0, st, a); \
                             else hipLaunchKernelGGL((k_down<GG, 4, L, Q>), grid, dim3(256), 0, st, a); } while (0)
#define JM_DNG(GG) if (qc == 2) JM_DN(GG, 64, 2); else if (lpr == 64) JM_DN(GG, 64, 1); \
                   else if (lpr == 32) JM_DN(GG, 32, 1); else JM_DN(GG, 16, 1);
    if (qc > 2) return hipErrorInvalidValue;
    if (a.group == 64) { JM_DNG(64) } else { JM_DNG(32) }
#undef JM_DNG
#undef JM_DN
    return hipGetLastError();
}

hipError_t launch_combine(const float* y, const int* comb, int B, int k, int d, const float* resid,
                          float* out, hipStream_t st) {
    const long long n = (long long)B * (d / 4);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, y, comb, B, k, d,
                       resid, out);
    return hipGetLastError();
}

}  // namespace jm
