// Small-batch decode path of the MoE block (gfx950): B * topk <= 64 slots,
// two launches.
//
//   k_front     one persistent block of 8 waves per CU.
//     router      (router inside the launch) wave 0 of block g < ceil(E/8) B
//                 computes the scores of expert group g mod ceil(E/8) for
//                 token g / ceil(E/8) with the chains of k_router_grp
//                 (jm_chain.h: the same bits, decode_kernel.c:234-256,
//                 693-718) and publishes each score as a 64-bit word
//                 (score bits | tag << 32) with an agent-scope store.  The
//                 readers poll those words until every one carries this
//                 call's tag: one word holds both the value and its
//                 freshness, so no fence orders anything (a release fence
//                 writes back a whole L2 and costs more than a launch).
//     digits      every block writes the B tokens' digits into its own LDS:
//                 encoded from x (router inside) or copied from the router
//                 kernel's.
//     top-k       every block selects every token's experts from the scores
//                 (topk_vals: k_topk's arithmetic, decode_kernel.c:1425-1448)
//                 and lists the routed experts in union order (:1449-1485).
//     gate/up     wave items (expert, 8 intermediate rows), items i, i + NW,
//                 ... per wave, two in flight: the next item's 16 KiB of rows
//                 stream while the current one is multiplied against each
//                 of its slots' tokens (decode_kernel.c:1365-1375).  Rows
//                 are read with buffer loads: an item past the end requests
//                 nothing (its offsets lie outside a zero-length range), so
//                 every wave issues the same loads in the same order and the
//                 memory counter waits stay exact.  The 8 act values of a
//                 slot get a digit scale of their own (no cross-wave max),
//                 and the outputs wait in LDS until the wave's last item:
//                 stores count on the same counter as loads, and a store
//                 between two items' loads would make every wait cover it.
//   k_down_lds  one block of 16 waves per 8 hidden rows: every routed
//               expert's 8 down rows are requested at once (up to 4 experts
//               per wave), the act digits of all slots are copied into LDS
//               beside them (direct-to-LDS loads), then each slot's
//               w_slot * (rows . act) (:1376-1383) goes to LDS and each
//               token's k values are summed in the reference's union order
//               (:1502-1507).
#include <atomic>

#include "jm_bufld.h"
#include "jm_chain.h"
#include "jm_items.h"

namespace jm {

using namespace wi;

namespace {

constexpr int FR_THREADS = 512;
constexpr int FR_WAVES = FR_THREADS / 64;
constexpr int FR_MAX_E = 256;
constexpr int FR_OUT = JM_FRONT_SLOTS;    // staged outputs per wave: its items have distinct experts
constexpr int FR_SPIN = 1 << 16;          // polls of one token's scores before giving up (~0.1 s)

__host__ __device__ constexpr size_t align_up(size_t n, size_t a) { return (n + a - 1) / a * a; }

// one staged gate/up output: a slot's 8 act values of one item
struct FrontOut {
    int slot, c;
    uint32_t scale;           // bf16 bits of the 8 values' digit scale
    uint32_t pad;
    float act[8];
    uint32_t dig[4];          // one word per digit plane
};
static_assert(sizeof(FrontOut) == 64, "64-byte staged outputs");

// Digits of 8 consecutive values of one token (one word per digit plane,
// nibble i = value i), the G-value group's scale from the G/8 lanes that
// hold its words (aligned lane groups).  The same digits as
// encode_group_both: a = rint(v * (R / max)) written as 4 balanced base-16
// digits.  Biased by 0x8888 each nibble of a + 0x8888 is its digit + 8, so
// the planes are a nibble transpose of the 8 biased integers, XOR 8 per
// nibble.  The 0x1.8p23 addition rounds to the nearest integer (ties to
// even) and leaves it in the low bits.
template <int G>
__device__ __forceinline__ void encode_word8(const float (&v)[8], bool ok, uint32_t (&P)[4], float* s_out) {
    constexpr int LG = G / 8;
    float am = 0.0f;
    int bad = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float x = fabsf(v[i]);
        am = fmaxf(am, x);
        bad |= !(x <= 3.4028235e38f);
    }
    if (!ok) { am = 0.0f; bad = 0; }
    bad = seg_or<LG>(bad);
    const float mx = seg_max<LG>(am);
    *s_out = digit_scale<4>(mx, bad != 0);
    const float inv = (mx > 0.0f && !bad) ? __fdiv_rn((float)Digits<4>::R, mx) : 0.0f;
    uint32_t u[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        u[i] = bad ? 0x8888u : __float_as_uint(__fadd_rn(__fmul_rn(v[i], inv), 12582912.0f)) + 0x8888u;
    // A_m = u_{2m} | u_{2m+1} << 16 (low halves)
    const uint32_t A0 = __builtin_amdgcn_perm(u[1], u[0], 0x05040100u);
    const uint32_t A1 = __builtin_amdgcn_perm(u[3], u[2], 0x05040100u);
    const uint32_t A2 = __builtin_amdgcn_perm(u[5], u[4], 0x05040100u);
    const uint32_t A3 = __builtin_amdgcn_perm(u[7], u[6], 0x05040100u);
    // bytes b of A0..A3 gathered: L (b = 0, 2) and H (b = 1, 3) of the even
    // and odd values
    const uint32_t T01 = __builtin_amdgcn_perm(A1, A0, 0x05010400u);
    const uint32_t T23 = __builtin_amdgcn_perm(A3, A2, 0x05010400u);
    const uint32_t T01o = __builtin_amdgcn_perm(A1, A0, 0x07030602u);
    const uint32_t T23o = __builtin_amdgcn_perm(A3, A2, 0x07030602u);
    const uint32_t Le = __builtin_amdgcn_perm(T23, T01, 0x05040100u);
    const uint32_t He = __builtin_amdgcn_perm(T23, T01, 0x07060302u);
    const uint32_t Lo = __builtin_amdgcn_perm(T23o, T01o, 0x05040100u);
    const uint32_t Ho = __builtin_amdgcn_perm(T23o, T01o, 0x07060302u);
    constexpr uint32_t M = 0x0F0F0F0Fu;
    P[0] = ((Le & M) | ((Lo << 4) & ~M)) ^ 0x88888888u;
    P[1] = (((Le >> 4) & M) | (Lo & ~M)) ^ 0x88888888u;
    P[2] = ((He & M) | ((Ho << 4) & ~M)) ^ 0x88888888u;
    P[3] = (((He >> 4) & M) | (Ho & ~M)) ^ 0x88888888u;
}

// The digit scale of 8 act values as bf16 bits, rounded up so that every
// |v| / scale stays within R (NaN when a value is not finite).
__device__ __forceinline__ uint32_t act_scale_bf16(float mx, bool bad) {
    if (bad) return 0x7FC0u;
    const uint32_t u = __float_as_uint(__fdiv_rn(mx, (float)Digits<4>::R));
    return ((u + 0xFFFFu) & 0xFFFF0000u) >> 16;
}

// G: token group; LPR = d / 32 lanes per row (one 16-byte chunk each); EPL:
// scores per lane in the top-k; ROUTER: the router runs inside the launch.
template <int G, int LPR, int EPL, bool ROUTER, bool WBF16>
__global__ void __launch_bounds__(FR_THREADS)
k_front(FrontArgs a) {
    constexpr int d = LPR * 32;
    constexpr int DV = d / 512;
    constexpr int RPI = JM_WAVE / LPR;           // rows per load instruction
    constexpr int S = GU_ROWS / RPI;             // load steps per matrix per item
    constexpr int NG = d / G;                    // token groups
    constexpr int W8 = d / 8;                    // digit words per plane per token
    constexpr int TP = d / 8 + 4;
    static_assert(2 * S == LPR / 4, "one transposed value per 4 lanes");
    extern __shared__ __align__(16) unsigned char dsm[];
    __shared__ float xT[ROUTER ? 8 * TP : 4];
    __shared__ int top_s[JM_FRONT_SLOTS], top_l[JM_FRONT_SLOTS], ulist[JM_FRONT_SLOTS], ue[JM_FRONT_SLOTS];
    __shared__ float tw_s[JM_FRONT_SLOTS];
    __shared__ int first_l[FR_MAX_E];
    __shared__ int wcnt[1];
    __shared__ float p_s[FR_WAVES][64 * EPL];
    __shared__ unsigned long long rec_l[JM_FRONT_SLOTS][4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int B = a.B, E = a.E, k = a.topk, m = a.m, nslot = B * k;
    uint32_t* xd = (uint32_t*)dsm;                                    // [B][4][W8]
    float* xs = (float*)(dsm + align_up((size_t)B * d * 2, 16));     // [B][NG]
    // this wave's staged outputs, then its scale scratch
    FrontOut* outs = (FrontOut*)(dsm + align_up((size_t)B * d * 2, 16) + align_up((size_t)B * NG * 4, 16) +
                                 (size_t)w * (FR_OUT * sizeof(FrontOut) + 16 * NG * 2));

    unsigned tag = 0;
    if constexpr (ROUTER) {
        tag = a.sync[0] + 1u;
        // router wave: scores of one expert group for one token
        const int ngrp = (E + 7) / 8;
        if (w == 0 && (int)blockIdx.x < ngrp * B) {
            using C = Chain<DV, WBF16>;
            constexpr int XV = d / 256;
            constexpr int NB = C::NC < 16 ? C::NC : 16;
            const int eg = blockIdx.x % ngrp, b = blockIdx.x / ngrp;
            const uint4* wt = (const uint4*)a.wt;
            float4 xv[XV];
            const float4* xb = (const float4*)(a.x + (size_t)b * d);
#pragma unroll
            for (int i = 0; i < XV; i++) xv[i] = xb[lane + 64 * i];
            uint4 buf[NB][C::CP];
#pragma unroll
            for (int c = 0; c < NB; c++) C::load(buf[c], wt, eg, c, lane);
            stage_chain_order<XV, TP>(xv, xT);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const float acc = router_chains<DV, WBF16, NB>(buf, wt, eg, xT);
            const int e = 8 * eg + (lane >> 3);
            if ((lane & 7) == 0 && e < E) {
                a.logits[(size_t)b * E + e] = acc;
                __hip_atomic_store(a.ll + (size_t)b * E + e,
                                   ((unsigned long long)tag << 32) | __float_as_uint(acc), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        // the B tokens' digits into this block's LDS: word i = 8 values,
        // G/8 consecutive threads per group; the tokens' loads of 4 words
        // per thread are requested together
        constexpr int EW = 4;
        for (int i0 = 0; i0 < B * W8; i0 += EW * FR_THREADS) {
            float4 xl[EW][2];
#pragma unroll
            for (int r = 0; r < EW; r++) {
                const int i = i0 + r * FR_THREADS + tid;
                const int wi = i < B * W8 ? i : 0;
                const float4* xp = (const float4*)(a.x + (size_t)(wi / W8) * d + 8 * (wi % W8));
                xl[r][0] = xp[0];
                xl[r][1] = xp[1];
            }
#pragma unroll
            for (int r = 0; r < EW; r++) {
                const int i = i0 + r * FR_THREADS + tid;
                const bool ok = i < B * W8;
                const int wi = ok ? i : 0;
                const int b = wi / W8, j = wi % W8;
                const float v[8] = {xl[r][0].x, xl[r][0].y, xl[r][0].z, xl[r][0].w,
                                    xl[r][1].x, xl[r][1].y, xl[r][1].z, xl[r][1].w};
                uint32_t P[4];
                float sc;
                encode_word8<G>(v, ok, P, &sc);
                if (ok) {
#pragma unroll
                    for (int kk = 0; kk < 4; kk++) xd[(b * 4 + kk) * W8 + j] = P[kk];
                    if (j % (G / 8) == 0) xs[b * NG + j / (G / 8)] = sc;
                }
            }
        }
    } else {
        // the router kernel's digits [b][group][plane][G/8] -> [b][plane][word]
        // with direct-to-LDS loads, all in flight together: one wave load per
        // (token, plane), lane L the words 4L .. 4L + 3 (W8 / 4 lanes), then
        // the scales [b][group] as they lie, 1 KiB per wave load
        for (int p = w; p < B * 4; p += FR_WAVES) {
            const int b = p / 4, kk = p % 4;
            if (lane < W8 / 4) {
                const int j = 4 * lane;
                const uint32_t* src = a.xdig + ((size_t)(b * NG + j / (G / 8)) * 4 + kk) * (G / 8) + j % (G / 8);
                __builtin_amdgcn_global_load_lds((const void*)src,
                                                 (__attribute__((address_space(3))) void*)(xd + (size_t)p * W8), 16, 0, 0);
            }
        }
        const int sbytes = B * NG * 4;
        for (int p = w; p * 1024 < sbytes; p += FR_WAVES) {
            if (p * 1024 + lane * 16 < sbytes)
                __builtin_amdgcn_global_load_lds((const void*)((const char*)a.xscale + p * 1024 + lane * 16),
                                                 (__attribute__((address_space(3))) void*)((char*)xs + p * 1024), 16, 0, 0);
        }
    }

    // top-k of every token: wave w takes tokens w, w + 8, ...
    for (int b = w; b < B; b += FR_WAVES) {
        float v[EPL];
        if constexpr (ROUTER) {
            const unsigned long long* src = a.ll + (size_t)b * E;
            for (int spin = 0;; spin++) {
                bool fresh = true;
#pragma unroll
                for (int j = 0; j < EPL; j++) {
                    const int e = lane + 64 * j;
                    if (e < E) {
                        const unsigned long long q = __hip_atomic_load(src + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        fresh = fresh && (unsigned)(q >> 32) == tag;
                        v[j] = __uint_as_float((unsigned)q);
                    } else {
                        v[j] = 0.0f;
                    }
                }
                if (__all(fresh)) break;
                if (spin >= FR_SPIN) {
                    if (lane == 0) atomicAdd(a.sync + 1, 1u);
                    break;
                }
                __builtin_amdgcn_s_sleep(8);
            }
        } else {
#pragma unroll
            for (int j = 0; j < EPL; j++) {
                const int e = lane + 64 * j;
                v[j] = e < E ? a.logits_in[(size_t)b * E + e] : 0.0f;
            }
        }
        topk_vals<EPL>(v, E, k, a.renorm, p_s[w], top_s + b * k, tw_s + b * k);
    }
    // this wave's direct-to-LDS copies complete before any wave reads them
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __syncthreads();
    const int U = decode_union<JM_FRONT_SLOTS>(top_s, nslot, E, top_l, first_l, ulist, wcnt);
    if (tid < U) {
        const int e = top_s[ulist[tid]];
        ue[tid] = e;
        unsigned long long so, po;
        a.rec.get(0, a.key0 + e, so, po);
        rec_l[tid][0] = (unsigned long long)(a.blob + so);
        rec_l[tid][1] = (unsigned long long)(a.blob + po);
        a.rec.get(1, a.key0 + e, so, po);
        rec_l[tid][2] = (unsigned long long)(a.blob + so);
        rec_l[tid][3] = (unsigned long long)(a.blob + po);
    }
    if (blockIdx.x == 0 && tid < nslot) {
        a.top[tid] = top_s[tid];
        a.tw[tid] = tw_s[tid];
    }
    __syncthreads();

    // gate/up items
    const int nch = m / GU_ROWS;
    const int NBK = gridDim.x, NW = NBK * FR_WAVES;
    const int gw = w * NBK + blockIdx.x;
    const int NI = U * nch;
    const int nmax = (NI + NW - 1) / NW;         // the same for every wave: waves past NI issue nothing
    const int col = lane & (LPR - 1), rsub = lane / LPR;
    const int grp = col * 32 / G;
    const int rec_pk = m * d / 2, rec_sc = m * NG * 2;
    const int tslot = lane < nslot ? top_s[lane] : -1;
    const int i8 = lane & 7;
    const int src = LPR * (i8 % RPI) + 8 * (i8 / RPI);

    // per item: the 8 gate and 8 up rows (one 16-byte chunk per lane and
    // row) and their fp16 scales, 8 * NG contiguous per matrix, as one
    // 16-byte piece per lane of NG lanes each (two loads instead of one
    // per lane and row: every load instruction holds a slot of the memory
    // pipeline whatever its size)
    static_assert(NG <= 64, "one load per matrix for the scales");
    uint4 wg[2][S], wu[2][S], sg[2], su[2];
    uint16_t* scr = (uint16_t*)(outs + FR_OUT);                      // this wave's 16 * NG scales
    auto issue = [&](int bi, int it) {
        const bool ok = it < NI;
        const int iu = ok ? it : 0;
        const int u = iu / nch, c = iu % nch;
        const __amdgpu_buffer_rsrc_t rgs = rsrc(uniform64(rec_l[u][0]), ok ? rec_sc : 0);
        const __amdgpu_buffer_rsrc_t rgp = rsrc(uniform64(rec_l[u][1]), ok ? rec_pk : 0);
        const __amdgpu_buffer_rsrc_t rus = rsrc(uniform64(rec_l[u][2]), ok ? rec_sc : 0);
        const __amdgpu_buffer_rsrc_t rup = rsrc(uniform64(rec_l[u][3]), ok ? rec_pk : 0);
#pragma unroll
        for (int s = 0; s < S; s++) {
            const int row = c * GU_ROWS + rsub + s * RPI;
            const unsigned o = (unsigned)row * (d / 2) + (unsigned)col * 16;
            wg[bi][s] = bload16(rgp, o);
            wu[bi][s] = bload16(rup, o);
        }
        // lanes past NG read past the range: zero, no access
        const unsigned so = lane < NG ? (unsigned)c * GU_ROWS * NG * 2 + (unsigned)lane * 16 : 0xFFFFFFF0u;
        sg[bi] = bload16(rgs, so);
        su[bi] = bload16(rus, so);
    };
    int nout = 0;
    auto compute = [&](int bi, int it) {
        const bool ok = it < NI;
        const int iu = ok ? it : 0;
        const int u = iu / nch, c = iu % nch;
        const int e = ok ? ue[u] : -2;
        // the weights as signed nibbles q - 8 (this waits for the item's
        // loads), kept in registers for all the item's slots (the empty asm:
        // the compiler would otherwise redo the XOR for every slot)
#pragma unroll
        for (int s = 0; s < S; s++) {
            wg[bi][s] = flip_nibbles(wg[bi][s]);
            wu[bi][s] = flip_nibbles(wu[bi][s]);
            asm volatile("" : "+v"(wg[bi][s].x), "+v"(wg[bi][s].y), "+v"(wg[bi][s].z), "+v"(wg[bi][s].w));
            asm volatile("" : "+v"(wu[bi][s].x), "+v"(wu[bi][s].y), "+v"(wu[bi][s].z), "+v"(wu[bi][s].w));
        }
        // the scales through this wave's LDS: row r's group g at [r][g]
        // (gate), [8 + r][g] (up); each lane's 2 S of them as floats
        if (lane < NG) {
            *(uint4*)(scr + 8 * lane) = sg[bi];
            *(uint4*)(scr + 8 * NG * 1 + 8 * lane) = su[bi];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float hgf[S], huf[S];
#pragma unroll
        for (int s = 0; s < S; s++) {
            const int r = rsub + s * RPI;
            hgf[s] = fp16_hw(scr[r * NG + grp]);
            huf[s] = fp16_hw(scr[(GU_ROWS + r) * NG + grp]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        unsigned long long msk = __ballot(tslot == e);
        while (msk) {
            const int sl = __builtin_ctzll(msk);
            msk &= msk - 1;
            const int b = sl / k;
            ChunkDigits<4> cd;
            const uint32_t* xb = xd + (size_t)b * 4 * W8 + 4 * col;
#pragma unroll
            for (int kk = 0; kk < 4; kk++) cd.d[kk] = *(const uint4*)(xb + kk * W8);
            cd.s = xs[b * NG + grp];
            float part[2 * S];
#pragma unroll
            for (int s = 0; s < S; s++) {
                // sum over the digit planes 16^k (w . d_k): one short chain per
                // plane, then Horner over the four exact partial sums
                int pg[4], pu[4];
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    pg[kk] = chunk_digit(wg[bi][s], cd.d[kk], 0);
                    pu[kk] = chunk_digit(wu[bi][s], cd.d[kk], 0);
                }
                const int ig = ((((pg[3] << 4) + pg[2]) << 4) + pg[1]) * 16 + pg[0];
                const int iu2 = ((((pu[3] << 4) + pu[2]) << 4) + pu[1]) * 16 + pu[0];
                part[2 * s] = __fmul_rn((float)ig, __fmul_rn(cd.s, hgf[s]));
                part[2 * s + 1] = __fmul_rn((float)iu2, __fmul_rn(cd.s, huf[s]));
            }
            // row i of the item: gate total in lanes LPR (i % RPI) + 8 (i / RPI),
            // up 4 lanes on
            const float tot = transpose_sum<LPR>(part);
            const float upv = dpp_f<DPP_ROL4>(tot);
            const float av = swiglu(tot, upv);
            const float mine = __shfl(av, src, JM_WAVE);
            // the 8 act values' digits with their own scale
            const float am = lane < 8 ? fabsf(mine) : 0.0f;
            const bool bad = seg_or<8>(lane < 8 && !(am <= 3.4028235e38f) ? 1 : 0) != 0;
            const float mx = seg_max<8>(am);
            const uint32_t sb = act_scale_bf16(mx, bad);
            const float sv = __uint_as_float(sb << 16);
            const float inv = (mx > 0.0f && !bad) ? __fdiv_rn(1.0f, sv) : 0.0f;
            int dg[4];
            split_digits<4>((int)rintf(__fmul_rn(mine, inv)), dg);
            uint32_t word[4];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) word[kk] = (uint32_t)seg_or<8>((dg[kk] & 15) << (4 * i8));
            // (front_ok keeps a wave's outputs within FR_OUT: its items have
            // distinct experts, so at most one output per slot)
            FrontOut& o = outs[nout < FR_OUT ? nout : FR_OUT - 1];
            if (lane < 8) o.act[lane] = mine;
            if (lane < 4) o.dig[lane] = lane == 0 ? word[0] : lane == 1 ? word[1] : lane == 2 ? word[2] : word[3];
            if (lane == 0) {
                o.slot = sl;
                o.c = c;
                o.scale = sb;
            }
            nout = nout < FR_OUT ? nout + 1 : FR_OUT;
        }
    };
#pragma unroll
    for (int bi = 0; bi < 2; bi++)
#pragma unroll
        for (int s = 0; s < S; s++) {
            wg[bi][s] = make_uint4(0, 0, 0, 0);
            wu[bi][s] = make_uint4(0, 0, 0, 0);
            sg[bi] = make_uint4(0, 0, 0, 0);
            su[bi] = make_uint4(0, 0, 0, 0);
        }
    // iteration j0 = -2 only issues the first two items; every later one
    // computes items j0, j0 + 1 and issues j0 + 2, j0 + 3
    for (int j0 = -2; j0 < nmax; j0 += 2) {
        if (j0 >= 0) compute(0, gw + j0 * NW);
        __builtin_amdgcn_sched_barrier(0);
        issue(0, gw + (j0 + 2) * NW);
        __builtin_amdgcn_sched_barrier(0);
        if (j0 >= 0) compute(1, gw + (j0 + 1) * NW);
        __builtin_amdgcn_sched_barrier(0);
        issue(1, gw + (j0 + 3) * NW);
        __builtin_amdgcn_sched_barrier(0);
    }
    // the staged outputs
    const int ncol = m / 32;
    for (int i = 0; i < nout; i++) {
        const FrontOut& o = outs[i];
        const int sl = __builtin_amdgcn_readfirstlane(o.slot), c = __builtin_amdgcn_readfirstlane(o.c);
        const int j = c & 3, cc = c >> 2;
        if (lane < 8) a.act[(size_t)sl * m + c * GU_ROWS + lane] = o.act[lane];
        if (lane < 4) a.adig[(((size_t)sl * 4 + j) * ncol + cc) * 4 + lane] = o.dig[lane];
        if (lane == 0) a.ascale[((size_t)sl * ncol + cc) * 4 + j] = (uint16_t)o.scale;
    }
}

// ------------------------------------------------------------------ down

constexpr int DL_ROWS = 8;
constexpr int DL_THREADS = 1024;
constexpr int DL_WAVES = DL_THREADS / 64;
constexpr int DL_NR = JM_FRONT_SLOTS / DL_WAVES;     // experts per wave (U <= 64)
// 16-byte pieces per thread of the act copy: 64 slots of m <= 1024 values,
// 2 bytes of digits and 1/4 byte of scale per value
constexpr int DL_PIECES = (JM_FRONT_SLOTS * (2 * 1024 + 1024 / 4) / 16 + DL_THREADS - 1) / DL_THREADS;
// of which requested before the rows (all of them for intermediate sizes up
// to 768 at 64 slots), the rest after: registers for the rows
constexpr int DL_EARLY = (JM_FRONT_SLOTS * (2 * 768 + 768 / 4) / 16 + DL_THREADS - 1) / DL_THREADS;

// LPR lanes per down row (m / 32 chunks, the ones past the row dead).
template <int G, int LPR>
__global__ void __launch_bounds__(DL_THREADS)
k_down_lds(DownArgs a) {
    constexpr int R = DL_ROWS;
    constexpr int RPI = JM_WAVE / LPR;
    constexpr int S = R / RPI;
    static_assert(S >= 1 && S * RPI == R, "whole rows per step");
    extern __shared__ __align__(16) unsigned char dsm[];
    __shared__ int top_l[JM_FRONT_SLOTS], ulist[JM_FRONT_SLOTS], comb_l[JM_FRONT_SLOTS];
    __shared__ int first_l[FR_MAX_E];
    __shared__ float tw_l[JM_FRONT_SLOTS];
    __shared__ float ypart[JM_FRONT_SLOTS * R];
    __shared__ int wcnt[1];
    __shared__ unsigned long long drec[JM_FRONT_SLOTS][2];   // down scales, packed rows of each routed expert
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = blockIdx.x;
    const int k = a.topk, E = a.E, m = a.m, nslot = a.B * k;
    const int ncol = m / 32, cpr = m / 32, ngroups = m / G;
    const size_t dbytes = (size_t)nslot * 2 * m, sbytes = (size_t)nslot * m / 4;
    unsigned char* adl = dsm;                                     // [nslot][4][ncol][4] u32
    unsigned char* asl = dsm + align_up(dbytes, 1024);           // [nslot][ncol][4] bf16

    if (blockIdx.x == 0 && tid == 0 && a.sync) a.sync[0] = a.sync[0] + 1u;
    // the top-k table first (the union order, then the rows, depend on it),
    // then every slot's act digits and scales in 16-byte pieces (clamped
    // into their region), held in registers while the rows are requested and
    // written to LDS afterwards, so that their round trip overlaps the rows'.
    // (Direct-to-LDS loads would make the compiler wait for every load
    // before each later LDS access, serialising the row requests.)
    const int ts = tid < nslot ? tid : 0;
    const int t_me = a.top[ts];
    const float w_me = a.tw[ts];
    __builtin_amdgcn_sched_barrier(0);          // the table's loads ahead of the copies'
    const int nd16 = (int)(dbytes / 16), ns16 = (int)(sbytes / 16);
    auto piece = [&](int p) {
        return p < nd16 ? (const uint4*)a.adig + p
                        : (const uint4*)a.ascale + (p - nd16 < ns16 ? p - nd16 : ns16 - 1);
    };
    uint4 cp[DL_EARLY];
#pragma unroll
    for (int i = 0; i < DL_EARLY; i++) cp[i] = *piece(tid + i * DL_THREADS);
    if (tid < nslot) {
        top_l[tid] = t_me;
        tw_l[tid] = w_me;
    }
    int e_me;
    const int U = decode_union<JM_FRONT_SLOTS>(top_l, nslot, E, top_l, first_l, ulist, wcnt, &e_me);
    // each token's slots ranked by the first slot of their expert
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
    // the routed experts' record addresses, before any row is requested (a
    // lookup between two experts' requests would wait for all of them)
    if (tid < U) {
        unsigned long long so, po;
        a.rec.get(2, a.key0 + top_l[ulist[tid]], so, po);
        drec[tid][0] = (unsigned long long)(a.blob + so);
        drec[tid][1] = (unsigned long long)(a.blob + po);
    }
    __syncthreads();
    // this wave's experts u = w + 16 q: every row requested now
    const int colr = lane & (LPR - 1), rsub = lane / LPR;
    const bool live = colr < cpr;
    const int chk = live ? colr : 0;
    const int rec_pk = a.d * m / 2, rec_sc = a.d * ngroups * 2;
    uint4 wd[DL_NR][S];
    uint32_t hd[DL_NR][S];
#pragma unroll
    for (int q = 0; q < DL_NR; q++) {
        const int u = w + DL_WAVES * q;
        const bool ok = u < U;
        const int uu = ok ? u : 0;
        const __amdgpu_buffer_rsrc_t rp = rsrc(uniform64(drec[uu][1]), ok ? rec_pk : 0);
        const __amdgpu_buffer_rsrc_t rs = rsrc(uniform64(drec[uu][0]), ok ? rec_sc : 0);
#pragma unroll
        for (int s = 0; s < S; s++) {
            const int row = c * R + rsub + s * RPI;
            wd[q][s] = bload16(rp, (unsigned)row * (m / 2) + (unsigned)chk * 16);
            hd[q][s] = bload2(rs, ((unsigned)row * ngroups + (unsigned)(chk * 32 / G)) * 2);
        }
    }
    // the act copies to LDS (they arrived before the rows: requested
    // earlier); the rows may still be in flight (each expert's dot waits for
    // its own rows only).  The empty asm keeps the copies' loads where they
    // are: the compiler would otherwise move each into its store's branch.
#pragma unroll
    for (int i = 0; i < DL_EARLY; i++)
        asm volatile("" : "+v"(cp[i].x), "+v"(cp[i].y), "+v"(cp[i].z), "+v"(cp[i].w));
    auto put = [&](int p, const uint4& v) {
        if (p < nd16) ((uint4*)adl)[p] = v;
        else if (p < nd16 + ns16) ((uint4*)asl)[p - nd16] = v;
    };
#pragma unroll
    for (int i = 0; i < DL_EARLY; i++) put(tid + i * DL_THREADS, cp[i]);
    // pieces past DL_EARLY per thread (intermediate sizes above 768 at 64
    // slots) are requested only now: waiting for them waits for the rows too
    if ((nd16 + ns16) > DL_EARLY * DL_THREADS) {
        uint4 late[DL_PIECES - DL_EARLY];
#pragma unroll
        for (int i = 0; i < DL_PIECES - DL_EARLY; i++) late[i] = *piece(tid + (DL_EARLY + i) * DL_THREADS);
#pragma unroll
        for (int i = 0; i < DL_PIECES - DL_EARLY; i++) put(tid + (DL_EARLY + i) * DL_THREADS, late[i]);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < DL_NR; q++) {
        const int u = w + DL_WAVES * q;
        if (u < U) {
            const int e = top_l[ulist[u]];
#pragma unroll
            for (int s = 0; s < S; s++) {
                wd[q][s] = flip_nibbles(wd[q][s]);
                asm volatile("" : "+v"(wd[q][s].x), "+v"(wd[q][s].y), "+v"(wd[q][s].z), "+v"(wd[q][s].w));
            }
            const int t = lane < nslot ? top_l[lane] : -1;
            unsigned long long msk = __ballot(t == e);
            while (msk) {
                const int sl = __builtin_ctzll(msk);
                msk &= msk - 1;
                uint4 ad[4];
#pragma unroll
                for (int j = 0; j < 4; j++)
                    ad[j] = *(const uint4*)(adl + (((size_t)sl * 4 + j) * ncol + chk) * 16);
                const uint2 sv = *(const uint2*)(asl + ((size_t)sl * ncol + chk) * 8);
                const float as[4] = {__uint_as_float(sv.x << 16), __uint_as_float(sv.x & 0xFFFF0000u),
                                     __uint_as_float(sv.y << 16), __uint_as_float(sv.y & 0xFFFF0000u)};
                float part[S];
#pragma unroll
                for (int s = 0; s < S; s++) {
                    const uint32_t wj[4] = {wd[q][s].x, wd[q][s].y, wd[q][s].z, wd[q][s].w};
                    float t2 = 0.0f;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        int iv = dot8(wj[j], ad[j].w, 0);
                        iv = dot8(wj[j], ad[j].z, iv << 4);
                        iv = dot8(wj[j], ad[j].y, iv << 4);
                        iv = dot8(wj[j], ad[j].x, iv << 4);
                        t2 = __builtin_fmaf((float)iv, as[j], t2);
                    }
                    part[s] = __fmul_rn(t2, live ? fp16_hw((uint16_t)hd[q][s]) : 0.0f);
                }
                const float v = transpose_reduce<LPR, S>(part);
                if ((lane & (LPR / S - 1)) == 0) {
                    const int s_idx = (lane & (LPR - 1)) / (LPR / S);
                    ypart[sl * R + s_idx * RPI + rsub] = __fmul_rn(tw_l[sl], v);
                }
            }
        }
    }
    __syncthreads();
    for (int o = tid; o < a.B * R; o += DL_THREADS) {
        const int b = o / R, rr = o % R;
        float acc = 0.0f;
        for (int j = 0; j < k; j++) {
            const int sl = comb_l[b * k + j];
            if (sl >= 0) acc = __fadd_rn(acc, ypart[sl * R + rr]);
        }
        const size_t oi = (size_t)b * a.d + (size_t)c * R + rr;
        a.out[oi] = a.resid ? __fadd_rn(a.resid[oi], acc) : acc;
    }
}

// token digits, their scales, then per wave the staged outputs followed by
// the scale scratch of one item (16 rows of d / G fp16 scales)
size_t front_lds(int B, int d, int G) {
    return align_up((size_t)B * d * 2, 16) + align_up((size_t)B * (d / G) * 4, 16) +
           (size_t)FR_WAVES * (FR_OUT * sizeof(FrontOut) + (size_t)16 * (d / G) * 2);
}

size_t down_lds(int nslot, int m) {
    return align_up((size_t)nslot * 2 * m, 1024) + align_up((size_t)nslot * m / 4, 1024);
}

constexpr int MAX_DEV = 64;
std::atomic<unsigned> g_front_lds[MAX_DEV];

// dynamic LDS up to the device's per-block limit less the kernel's static LDS
hipError_t allow(const void* f, int lmax) {
    hipFuncAttributes at;
    hipError_t e = hipFuncGetAttributes(&at, f);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lmax - (int)at.sharedSizeBytes);
}

// every instance may take up to 160 KiB of dynamic LDS (checked per call
// against the device's limit by front_ok)
#define JM_FRONT_INSTANCES(X)                                                                          \
    X(64, 64, 1) X(64, 64, 2) X(64, 64, 4) X(64, 32, 1) X(64, 32, 2) X(64, 32, 4)                      \
    X(32, 64, 1) X(32, 64, 2) X(32, 64, 4) X(32, 32, 1) X(32, 32, 2) X(32, 32, 4)

hipError_t allow_front_lds() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= MAX_DEV) return hipErrorInvalidDevice;
    if (g_front_lds[dev].load(std::memory_order_acquire)) return hipSuccess;
    int lmax = 0;
    e = hipDeviceGetAttribute(&lmax, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    if (e != hipSuccess) return e;
#define JM_ALLOW(GG, LL, EE)                                                                  \
    if (e == hipSuccess) e = allow((const void*)k_front<GG, LL, EE, false, false>, lmax);       \
    if (e == hipSuccess) e = allow((const void*)k_front<GG, LL, EE, true, false>, lmax);        \
    if (e == hipSuccess) e = allow((const void*)k_front<GG, LL, EE, true, true>, lmax);
    JM_FRONT_INSTANCES(JM_ALLOW)
#undef JM_ALLOW
    const void* dk[] = {(const void*)k_down_lds<64, 16>, (const void*)k_down_lds<64, 32>,
                        (const void*)k_down_lds<32, 16>, (const void*)k_down_lds<32, 32>};
    for (const void* f : dk)
        if (e == hipSuccess) e = allow(f, lmax);
    if (e != hipSuccess) return e;
    g_front_lds[dev].store(1u, std::memory_order_release);
    return hipSuccess;
}

// static LDS of the kernels (the largest instance), beside the dynamic part
constexpr size_t FRONT_STATIC = 8 * (2048 / 8 + 4) * 4 + 5 * JM_FRONT_SLOTS * 4 + FR_MAX_E * 4 + 16 +
                                FR_WAVES * 64 * 4 * 4 + JM_FRONT_SLOTS * 32;
constexpr size_t DOWN_STATIC = 4 * JM_FRONT_SLOTS * 4 + FR_MAX_E * 4 + JM_FRONT_SLOTS * DL_ROWS * 4 + 16;

}  // namespace

bool front_ok(int B, int E, int d, int m, int topk, int group, int n_cu, int lds_max) {
    const int nslot = B * topk;
    if (B <= 0 || nslot > JM_FRONT_SLOTS || E <= 0 || E > FR_MAX_E) return false;
    if (d != 1024 && d != 2048) return false;
    if (group != 32 && group != 64) return false;
    if (m % 32 || m > 1024 || m <= 0) return false;
    if ((long long)nslot * m % 64) return false;   // the act copy moves whole 16-byte pieces
    // a wave's items belong to distinct experts (the staged outputs fit)
    if ((long long)n_cu * FR_WAVES < m / GU_ROWS || n_cu <= 0) return false;
    if (front_lds(B, d, group) + FRONT_STATIC > (size_t)lds_max) return false;
    if (down_lds(nslot, m) + DOWN_STATIC > (size_t)lds_max) return false;
    return true;
}

bool front_router_ok(int B, int E, int n_cu) { return (long long)((E + 7) / 8) * B <= n_cu; }

hipError_t launch_front(const FrontArgs& a, int n_cu, int lds_max, hipStream_t st) {
    if (!front_ok(a.B, a.E, a.d, a.m, a.topk, a.group, n_cu, lds_max)) return hipErrorInvalidValue;
    const bool router = a.wt != nullptr;
    if (router && !front_router_ok(a.B, a.E, n_cu)) return hipErrorInvalidValue;
    hipError_t e = allow_front_lds();
    if (e != hipSuccess) return e;
    const size_t lds = front_lds(a.B, a.d, a.group);
    const dim3 grid((unsigned)n_cu), blk(FR_THREADS);
    const int lpr = a.d / 32;
    const int epl = a.E <= 64 ? 1 : a.E <= 128 ? 2 : 4;
#define JM_FR(GG, LL, EE)                                                                              \
    if (a.group == GG && lpr == LL && epl == EE) {                                                     \
        if (!router) hipLaunchKernelGGL((k_front<GG, LL, EE, false, false>), grid, blk, lds, st, a);    \
        else if (a.wt_bf16) hipLaunchKernelGGL((k_front<GG, LL, EE, true, true>), grid, blk, lds, st, a); \
        else hipLaunchKernelGGL((k_front<GG, LL, EE, true, false>), grid, blk, lds, st, a);             \
        return hipGetLastError();                                                                      \
    }
    JM_FRONT_INSTANCES(JM_FR)
#undef JM_FR
    return hipErrorInvalidValue;
}

hipError_t launch_down_lds(const DownArgs& a, int n_cu, int lds_max, hipStream_t st) {
    const int nslot = a.B * a.topk;
    if (!front_ok(a.B, a.E, a.d, a.m, a.topk, a.group, n_cu, lds_max) || a.d % DL_ROWS) return hipErrorInvalidValue;
    hipError_t e = allow_front_lds();
    if (e != hipSuccess) return e;
    const size_t lds = down_lds(nslot, a.m);
    const dim3 grid((unsigned)(a.d / DL_ROWS)), blk(DL_THREADS);
    const int cpr = a.m / 32;
    const int lpr = cpr <= 16 ? 16 : 32;
#define JM_DL(GG, LL) \
    if (a.group == GG && lpr == LL) { hipLaunchKernelGGL((k_down_lds<GG, LL>), grid, blk, lds, st, a); return hipGetLastError(); }
    JM_DL(64, 16) JM_DL(64, 32) JM_DL(32, 16) JM_DL(32, 32)
#undef JM_DL
    return hipErrorInvalidValue;
}

}  // namespace jm
