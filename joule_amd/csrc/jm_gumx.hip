// Small-batch gate/up of the MoE block on the matrix cores (gfx950): B <= 8
// tokens, B * topk <= 64 slots; one persistent block of 8 waves per compute
// unit (at most one block per item).
//
//   top-k   every block selects every token's experts from the router
//           kernel's scores (topk_vals: k_topk's arithmetic,
//           decode_kernel.c:1425-1448) and lists the routed experts in union
//           order (:1449-1485); block 0 writes the table for the down kernel
//           and the caller.
//   items   (routed expert, 32 intermediate rows): items b, b + grid, ... of
//           block b.  The block's 8 waves split the item's hidden columns
//           (d / 8 each) and multiply its 32 gate and 32 up rows against all
//           B tokens on v_mfma_i32_32x32x32_i8 (jm_mx.h): the tokens on the
//           A side as int8 digit pairs (row t: token t's hi digits, row
//           8 + t: its lo digits, rows 16..31 zero), the rows on the B side
//           as unsigned nibbles q (lane n % 32: row n).  Per Q4 group the two
//           digit products are exact int32 sums, and 256 hi + lo - 8 (the
//           group's digit sum) is the exact sum of a (q - 8); it is scaled by
//           the token's and the row's scale and accumulated in fp32
//           (decode_kernel.c:1365-1375).  Only the tokens routed to the
//           item's expert are scaled: the others' products cost the matrix
//           cores nothing that they would not spend anyway.  The waves'
//           partial sums meet in LDS; one wave per item (in turn) adds them
//           in wave order, applies SwiGLU and stages act (fp32) and its
//           digits for the down kernel in LDS, one scale per 32 values (the
//           item's rows, the decode path's act format); each wave writes its
//           staged outputs after its last item, since a store between two
//           items' loads would make every later wait on the memory counter
//           cover it.
//   Each wave keeps two items' rows in flight: an item's loads are issued
//   before the one before it is multiplied.  The barrier between the waves'
//   partial sums and their reduction orders LDS only, so that the loads in
//   flight are not waited for.
#include <algorithm>

#include "jm_bufld.h"
#include "jm_device.h"
#include "jm_kernels.h"
#include "jm_mx.h"

namespace jm {

namespace {

constexpr int GX_THREADS = 512;
constexpr int GX_WAVES = GX_THREADS / 64;
constexpr int GX_ROWS = 32;            // intermediate rows per item: the products' 32 columns
constexpr int GX_MAX_B = 8;            // tokens: A rows t (hi digits) and 8 + t (lo digits)
constexpr int GX_SLOTS = 64;
constexpr int GX_MAX_E = 256;
constexpr int GX_NE = 64;              // staged act outputs (slot, item) per block; a full list is written out early

// NB bytes (4, 8 or 16) of a row's scales
template <int NB>
__device__ __forceinline__ uint4 bload_sc(__amdgpu_buffer_rsrc_t r, unsigned off) {
    if constexpr (NB == 16) {
        return bload16(r, off);
    } else if constexpr (NB == 8) {
        const uint2 v = bload8(r, off);
        return make_uint4(v.x, v.y, 0u, 0u);
    } else {
        return make_uint4(bload4(r, off), 0u, 0u, 0u);
    }
}

// fp16 scale j of a row's scale piece, as float
__device__ __forceinline__ float sc_half(const uint4& v, int j) {
    const uint32_t w = j < 2 ? v.x : j < 4 ? v.y : j < 6 ? v.z : v.w;
    return fp16_hw((uint16_t)(w >> (16 * (j & 1))));
}

// One wave's share of an item in registers: per 64-column stage of its
// columns, 16 bytes per lane of each matrix's row (G = 64: bytes 16 h ..
// 16 h + 15 of the stage's group; G = 32: bytes 8 h .. 8 h + 7 of each of
// the stage's two groups), and the row's fp16 scales of the wave's groups.
template <int NST>
struct GxBuf {
    uint4 g[NST], u[NST];
    uint4 sg, su;
};

template <int G, int D, int EPL>
__global__ void __launch_bounds__(GX_THREADS)
k_gu_mx(GuMxArgs a) {
    constexpr int NG = D / G;                   // groups per row
    constexpr int NST = D / 64 / GX_WAVES;      // 64-column stages per wave
    constexpr int NGW = NST * (64 / G);         // groups per wave
    constexpr int SCB = 2 * NGW;                // scale bytes per row and wave
    static_assert(NST >= 1 && SCB >= 4 && SCB <= 16, "a wave's scales in one load");
    __shared__ int top_s[GX_SLOTS], top_l[GX_SLOTS], ulist[GX_SLOTS];
    __shared__ float tw_s[GX_SLOTS];
    __shared__ int first_l[GX_MAX_E];
    __shared__ int wcnt[1];
    __shared__ float p_s[GX_WAVES][64 * EPL];
    __shared__ unsigned long long rec_l[GX_SLOTS][4];
    __shared__ unsigned long long smask_l[GX_SLOTS];   // slots of each union entry
    __shared__ int tmask_l[GX_SLOTS];                  // tokens of each union entry
    __shared__ int uidx[GX_MAX_E];                     // union entry of each routed expert
    __shared__ __align__(16) float tsq[NG * GX_MAX_B];     // token scales [group][token]
    __shared__ __align__(16) int tcq[NG * GX_MAX_B];       // -8 times the tokens' group sums
    __shared__ float ost[GX_NE][GX_ROWS];              // staged act values of (slot, item) pairs
    __shared__ int ometa[GX_NE];                       // their slot * 1024 + item chunk
    __shared__ float red[2][GX_WAVES][2][GX_MAX_B][GX_ROWS];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int B = a.B, E = a.E, k = a.topk, m = a.m, nslot = B * k;
    const int n = lane & 31, hh = lane >> 5;

    // this wave's token operands (they do not depend on the routing): A row
    // n < 8 token n's hi digits, 8 <= n < 16 token n - 8's lo digits, in the
    // columns of the wave's stages (sub-step 0 and 1 of each, jm_mx.h order)
    const bool arow = n < 16 && (n & 7) < B;
    const int8_t* ap = (n < 8 ? a.xqh : a.xql) + (size_t)(arow ? (n & 7) : 0) * D;
    int4v A[NST][2];
#pragma unroll
    for (int s = 0; s < NST; s++) {
        const int c0 = 64 * (w * NST + s);
        const int o0 = G == 64 ? c0 + 32 * hh : c0 + 16 * hh;
        const int o1 = G == 64 ? o0 + 16 : o0 + 32;
        A[s][0] = *(const int4v*)(ap + o0);
        A[s][1] = *(const int4v*)(ap + o1);
    }
    for (int i = tid; i < NG * GX_MAX_B; i += GX_THREADS) {
        const int g = i / GX_MAX_B, b = i % GX_MAX_B;
        tsq[i] = b < B ? a.xqs[b * NG + g] : 0.0f;
        tcq[i] = b < B ? -8 * a.xqc[b * NG + g] : 0;
    }
    // top-k of every token: wave w takes tokens w, w + 8, ...
    for (int b = w; b < B; b += GX_WAVES) {
        float v[EPL];
#pragma unroll
        for (int j = 0; j < EPL; j++) {
            const int e = lane + 64 * j;
            v[j] = e < E ? a.logits[(size_t)b * E + e] : 0.0f;
        }
        topk_vals<EPL>(v, E, k, a.renorm, p_s[w], top_s + b * k, tw_s + b * k);
    }
    __syncthreads();
    const int U = decode_union<GX_SLOTS>(top_s, nslot, E, top_l, first_l, ulist, wcnt);
    if (tid < U) {
        const int e = top_s[ulist[tid]];
        uidx[e] = tid;
        smask_l[tid] = 0ull;
        tmask_l[tid] = 0;
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
    // each union entry's slots and tokens
    if (tid < nslot) {
        const int e = top_s[tid];
        if (e >= 0 && e < E) {
            const int u = uidx[e];
            atomicOr(&smask_l[u], 1ull << tid);
            atomicOr(&tmask_l[u], 1 << (tid / k));
        }
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < NST; s++) {
        if (!arow) {
            A[s][0] = int4v{0, 0, 0, 0};
            A[s][1] = int4v{0, 0, 0, 0};
        }
    }

    const int nch = m / GX_ROWS;
    const int NI = U * nch;
    const int NB = gridDim.x;
    const int nj = (int)blockIdx.x < NI ? (NI - 1 - (int)blockIdx.x) / NB + 1 : 0;   // block-uniform
    const int rec_pk = m * (D / 2), rec_sc = m * NG * 2;

    GxBuf<NST> buf[2];
    // the loads of item j of this block (j >= nj: zero-length ranges, no access)
    auto issue = [&](GxBuf<NST>& bf, int j) {
        const bool ok = j < nj;
        const int it = ok ? (int)blockIdx.x + j * NB : 0;
        const int u = it / nch, c = it % nch;
        const __amdgpu_buffer_rsrc_t rgs = rsrc(uniform64(rec_l[u][0]), ok ? rec_sc : 0);
        const __amdgpu_buffer_rsrc_t rgp = rsrc(uniform64(rec_l[u][1]), ok ? rec_pk : 0);
        const __amdgpu_buffer_rsrc_t rus = rsrc(uniform64(rec_l[u][2]), ok ? rec_sc : 0);
        const __amdgpu_buffer_rsrc_t rup = rsrc(uniform64(rec_l[u][3]), ok ? rec_pk : 0);
        const unsigned row = (unsigned)(c * GX_ROWS + n);
#pragma unroll
        for (int s = 0; s < NST; s++) {
            const unsigned cb = row * (unsigned)(D / 2) + 32u * (unsigned)(w * NST + s);
            if constexpr (G == 64) {
                bf.g[s] = bload16(rgp, cb + 16u * hh);
                bf.u[s] = bload16(rup, cb + 16u * hh);
            } else {
                const uint2 g0 = bload8(rgp, cb + 8u * hh), g1 = bload8(rgp, cb + 16u + 8u * hh);
                const uint2 u0 = bload8(rup, cb + 8u * hh), u1 = bload8(rup, cb + 16u + 8u * hh);
                bf.g[s] = make_uint4(g0.x, g0.y, g1.x, g1.y);
                bf.u[s] = make_uint4(u0.x, u0.y, u1.x, u1.y);
            }
        }
        const unsigned so = row * (unsigned)(NG * 2) + (unsigned)(SCB * w);
        bf.sg = bload_sc<SCB>(rgs, so);
        bf.su = bload_sc<SCB>(rus, so);
    };
    // the staged outputs to global memory: act, its digits (one half-wave
    // per (slot, item): the scale is the max over its 32 values) and the
    // scale.  Written after the last item, so that no store sits between
    // two items' loads in the memory counter's order (only a full list is
    // written earlier).
    int ne = 0;                                  // staged entries (block-uniform)
    auto flush = [&]() {
        lds_barrier();
        for (int e0 = 0; e0 < ne; e0 += 2 * GX_WAVES) {
            const int e = e0 + 2 * w + hh;
            if (e < ne) {
                const float av = ost[e][n];
                const int meta = ometa[e];
                const int sl = meta >> 10, c = meta & 1023;
                a.act[(size_t)sl * m + c * GX_ROWS + n] = av;
                const float am = fabsf(av);
                const bool nf = seg_or<32>(!(am <= 3.4028235e38f) ? 1 : 0) != 0;
                const float mx = seg_max<32>(am);
                const float inv = (mx > 0.0f && !nf) ? __fdiv_rn((float)Digits<JM_NDIG>::R, mx) : 0.0f;
                int dgt[JM_NDIG];
                split_digits<JM_NDIG>((int)rintf(__fmul_rn(av, inv)), dgt);
                const size_t gi = (size_t)sl * (m / 32) + c;
#pragma unroll
                for (int kk = 0; kk < JM_NDIG; kk++) {
                    const int word = seg_or<8>((dgt[kk] & 15) << (4 * (n & 7)));
                    if ((n & 7) == 0) a.adig[gi * (JM_NDIG * 4) + kk * 4 + (n >> 3)] = (uint32_t)word;
                }
                if (n == 0) a.ascale[gi] = digit_scale<JM_NDIG>(mx, nf);
            }
        }
        lds_barrier();
        ne = 0;
    };
    // item j: the waves' partial sums, their sums over the waves (the act
    // values, staged)
    auto compute = [&](GxBuf<NST>& bf, int j) {
        const int it = (int)blockIdx.x + j * NB;
        const int u = it / nch, c = it % nch;
        const unsigned long long sm = smask_l[u];
        const int tb = tmask_l[u];
        const int nsl = __popcll(sm);
        float fg[4] = {0.0f, 0.0f, 0.0f, 0.0f}, fu[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        // acc += (256 hi + lo - 8 sum) * s_token * s_row (lane half hh holds
        // tokens 4 hh + q: hi in register q, lo in 4 + q; all four are
        // scaled, the routed ones are kept)
        auto epi = [&](const int16v& dg, const int16v& du, int gi) {
            const int gg = w * NGW + gi;
            const float hg = sc_half(bf.sg, gi), hu = sc_half(bf.su, gi);
            const float4 ts4 = *(const float4*)(tsq + gg * GX_MAX_B + 4 * hh);
            const int4 tc4 = *(const int4*)(tcq + gg * GX_MAX_B + 4 * hh);
            const float ts[4] = {ts4.x, ts4.y, ts4.z, ts4.w};
            const int tc[4] = {tc4.x, tc4.y, tc4.z, tc4.w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int ig = dg[q] * 256 + dg[4 + q] + tc[q];
                const int iu = du[q] * 256 + du[4 + q] + tc[q];
                fg[q] = __builtin_fmaf(__fmul_rn((float)ig, ts[q]), hg, fg[q]);
                fu[q] = __builtin_fmaf(__fmul_rn((float)iu, ts[q]), hu, fu[q]);
            }
        };
#pragma unroll
        for (int s = 0; s < NST; s++) {
            const int4v bg0 = wdigits(bf.g[s].x, bf.g[s].y), bg1 = wdigits(bf.g[s].z, bf.g[s].w);
            const int4v bu0 = wdigits(bf.u[s].x, bf.u[s].y), bu1 = wdigits(bf.u[s].z, bf.u[s].w);
            if constexpr (G == 64) {
                int16v dg = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[s][0], bg0, int16v{}, 0, 0, 0);
                int16v du = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[s][0], bu0, int16v{}, 0, 0, 0);
                dg = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[s][1], bg1, dg, 0, 0, 0);
                du = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[s][1], bu1, du, 0, 0, 0);
                epi(dg, du, s);
            } else {
                // one group's two products live at a time (registers)
                const int16v dg0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[s][0], bg0, int16v{}, 0, 0, 0);
                const int16v du0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[s][0], bu0, int16v{}, 0, 0, 0);
                epi(dg0, du0, 2 * s);
                __builtin_amdgcn_sched_barrier(0);
                const int16v dg1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[s][1], bg1, int16v{}, 0, 0, 0);
                const int16v du1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[s][1], bu1, int16v{}, 0, 0, 0);
                epi(dg1, du1, 2 * s + 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (ne + nsl > GX_NE) flush();           // block-uniform
        const int rb = j & 1;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (tb & (1 << (4 * hh + q))) {
                red[rb][w][0][4 * hh + q][n] = fg[q];
                red[rb][w][1][4 * hh + q][n] = fu[q];
            }
        }
        lds_barrier();
        // thread t < 32 nsl (counted from wave j mod 8, so that the waves
        // take turns): row t % 32 of the item's (t / 32)-th slot
        const int t = (tid + 64 * (j % GX_WAVES)) % GX_THREADS;
        if (t < 32 * nsl) {
            unsigned long long ms = sm;
            for (int z = 0; z < (t >> 5); z++) ms &= ms - 1;
            const int sl = __builtin_ctzll(ms);
            const int b = sl / k, r = t & 31;
            float g = 0.0f, up = 0.0f;
#pragma unroll
            for (int ww = 0; ww < GX_WAVES; ww++) {
                g = __fadd_rn(g, red[rb][ww][0][b][r]);
                up = __fadd_rn(up, red[rb][ww][1][b][r]);
            }
            ost[ne + (t >> 5)][r] = swiglu(g, up);
            if (r == 0) ometa[ne + (t >> 5)] = sl * 1024 + c;
        }
        ne += nsl;
    };

    issue(buf[0], 0);
    __builtin_amdgcn_sched_barrier(0);
    issue(buf[1], 1);
    __builtin_amdgcn_sched_barrier(0);
    for (int j = 0; j < nj; j += 2) {
        compute(buf[0], j);
        __builtin_amdgcn_sched_barrier(0);
        issue(buf[0], j + 2);
        __builtin_amdgcn_sched_barrier(0);
        if (j + 1 < nj) compute(buf[1], j + 1);
        __builtin_amdgcn_sched_barrier(0);
        issue(buf[1], j + 3);
        __builtin_amdgcn_sched_barrier(0);
    }
    flush();
}

#define JM_GX_INSTANCES(X) \
    X(64, 2048, 1) X(64, 2048, 2) X(64, 2048, 4) X(64, 1024, 1) X(64, 1024, 2) X(64, 1024, 4) \
    X(32, 2048, 1) X(32, 2048, 2) X(32, 2048, 4) X(32, 1024, 1) X(32, 1024, 2) X(32, 1024, 4)

}  // namespace

bool gu_mx_ok(int B, int E, int d, int m, int topk, int group) {
    if (B < 1 || B > GX_MAX_B || topk < 1 || (long long)B * topk > GX_SLOTS) return false;
    if (E < topk || E > GX_MAX_E) return false;
    if (d != 1024 && d != 2048) return false;
    if (group != 32 && group != 64) return false;
    return m > 0 && m % GX_ROWS == 0;
}

hipError_t launch_gu_mx(const GuMxArgs& a, int n_cu, hipStream_t st) {
    if (!gu_mx_ok(a.B, a.E, a.d, a.m, a.topk, a.group) || n_cu <= 0) return hipErrorInvalidValue;
    if (!a.logits || !a.xqh || !a.xql || !a.xqs || !a.xqc || !a.top || !a.tw || !a.act || !a.adig || !a.ascale)
        return hipErrorInvalidValue;
    // at most one block per item: min(E, B * topk) routed experts
    const long long items = (long long)std::min(a.E, a.B * a.topk) * (a.m / GX_ROWS);
    const dim3 grid((unsigned)std::min<long long>(n_cu, items)), blk(GX_THREADS);
    const int epl = a.E <= 64 ? 1 : a.E <= 128 ? 2 : 4;
#define JM_GX(GG, DD, EE)                                                                  \
    if (a.group == GG && a.d == DD && epl == EE) {                                         \
        hipLaunchKernelGGL((k_gu_mx<GG, DD, EE>), grid, blk, 0, st, a);                    \
        return hipGetLastError();                                                          \
    }
    JM_GX_INSTANCES(JM_GX)
#undef JM_GX
    return hipErrorInvalidValue;
}

}  // namespace jm
