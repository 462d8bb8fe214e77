// Routing front of the MoE block (gfx950):
//
//   k_router_grp     one wave per (expert group of 8, token): router scores
//                    in the reference's 8-chain order (decode_kernel.c:
//                    234-256, 693-718) and a share of the token's x digits
//                    for the expert dots
//   k_router_quad    the same from 144 tokens, 4 tokens per block from one
//                    read of the table
//   k_topk           (jm_kernels.hip) one wave per token: softmax + top-k +
//                    renormalisation (:1425-1448)
//   k_dispatch_work  dispatch path only (more than 256 slots): block 0 the
//                    counting sort of all slots (:1449-1485), the expert
//                    work table and the token tiles of the experts that take
//                    the MFMA branch; from 144 tokens the other blocks encode
//                    the tokens' digits (the router then skips its encode)
//
// No block waits for or reads data written by another block of the same
// launch: on MI355X each XCD has its own L2, and a device-scope handoff
// inside a kernel (release fence + atomic ticket) costs more than a kernel
// boundary.
//
// Router chains: lane L = 8 * e_local + r of a wave runs the FMA chain r of
// expert 8 * eg + e_local, the 8 lanes of an expert holding the 8 partial
// sums the reference keeps in the 8 lanes of an AVX2 register.  The router
// table is read from a copy in which the 64 chains of an expert group are
// interleaved in 16-byte pieces: piece i of lane L's chain (values 8t + r
// for t in the piece) sits at [eg][i][L], so each load instruction of a wave
// reads 1 KiB of contiguous memory.  The token is staged in LDS in the
// chains' order.
#include <algorithm>

#include "jm_chain.h"
#include "jm_device.h"
#include "jm_kernels.h"

namespace jm {


// Interleaved copy of the router tables (L layers of E experts; E padded
// to Ep = a multiple of 8 per layer, the padding left as the caller cleared
// it).  Value j of expert e is value t = j / 8 of chain r = j % 8; with P
// values per 16-byte piece (8 bf16 or 4 float32) it goes to piece t / P of
// lane 8 * (e % 8) + r in expert group e / 8:
//   out[l][e/8][t/P][8*(e%8) + r][t%P] = in[l][e][j]
// as float32 or, when every value is exactly a bf16 (the reference's own
// table type), as bf16 bits.
template <bool IN_BF16, bool OUT_BF16>
__global__ void __launch_bounds__(256)
k_router_transpose(const void* __restrict__ in, void* __restrict__ out, long long rows, int E, int Ep,
                   int d) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * d) return;
    const long long row = i / d;
    const int j = (int)(i % d);
    const long long l = row / E;
    const int e = (int)(row % E);
    const float v = IN_BF16 ? bf16_bits_to_f32(((const uint16_t*)in)[i]) : ((const float*)in)[i];
    constexpr int P = OUT_BF16 ? 8 : 4;
    const int t = j >> 3, lane = ((e & 7) << 3) | (j & 7);
    const long long o = l * Ep * d + ((((long long)(e >> 3) * (d / 8 / P) + t / P) * 64 + lane) * P + t % P);
    if (OUT_BF16) ((uint16_t*)out)[o] = (uint16_t)(__float_as_uint(v) >> 16);
    else ((float*)out)[o] = v;
}

// ORs the low 16 bits of every float32 value into *flag (0: all bf16-exact)
__global__ void __launch_bounds__(256)
k_bf16_exact(const float* __restrict__ in, long long n, unsigned* __restrict__ flag) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    unsigned low = i < n ? (__float_as_uint(in[i]) & 0xFFFFu) : 0u;
    low = (unsigned)seg_or<64>((int)(low != 0));
    if ((threadIdx.x & 63) == 0 && low) atomicOr(flag, 1u);
}

hipError_t launch_router_transpose(const void* in, int in_bf16, void* out, int out_bf16, long long rows,
                                   int E, int d, hipStream_t st) {
    const long long n = rows * d;
    const int Ep = router_experts_padded(E);
    const dim3 grid((unsigned)((n + 255) / 256));
#define JM_TR(A, B) hipLaunchKernelGGL((k_router_transpose<A, B>), grid, dim3(256), 0, st, in, out, rows, E, Ep, d)
    if (in_bf16 && out_bf16) JM_TR(true, true);
    else if (in_bf16) JM_TR(true, false);
    else if (out_bf16) JM_TR(false, true);
    else JM_TR(false, false);
#undef JM_TR
    return hipGetLastError();
}

hipError_t launch_bf16_exact(const float* in, long long n, unsigned* flag, hipStream_t st) {
    hipLaunchKernelGGL(k_bf16_exact, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, in, n, flag);
    return hipGetLastError();
}


// Where the encodes of NT groups go: entry t receives group p of token b
// (its x digits and their scale; for the MFMA branch also its digit pairs,
// their scale and integer sum).
template <int G, int NDIG, int NT>
struct EncDst {
    uint32_t* dig[NT];
    float* sc[NT];
    int8_t* hi[NT];
    int8_t* lo[NT];
    float* qs[NT];
    int* qc[NT];
    __device__ __forceinline__ void set(int t, const RouteArgs& a, size_t b, int p, bool i8) {
        const size_t ng = (size_t)(a.d / G), g = b * ng + p, o = b * a.d + (size_t)p * G;
        dig[t] = a.xdig + g * (NDIG * (G / 8));
        sc[t] = a.xscale + g;
        hi[t] = a.xqh + (i8 ? o : 0);
        lo[t] = a.xql + (i8 ? o : 0);
        qs[t] = a.xqs + g;
        qc[t] = a.xqc + g;
    }
};

// x digits of token b staged in xT (chain order), wave eg's share of the
// token's groups over ngrp waves: one G-value group per G-lane segment (and,
// for the MFMA branch, the same group as int8 digit pairs), two groups at a
// time so that their reduction chains interleave.  Run before the router
// chains: it needs only the staged token, so it runs while the table's
// chunks arrive.
template <int G, int NDIG, int d>
__device__ __forceinline__ void encode_token_share(const RouteArgs& a, int b, int eg, int ngrp, const float* xT) {
    constexpr int TP = d / 8 + 4;
    constexpr int ng = d / G;
    constexpr int PPW = JM_WAVE / G;
    const int lane = threadIdx.x & 63;
    const int sub = lane / G;
    const bool i8 = a.xqh != nullptr;
    for (int base = eg * PPW; base < ng; base += 2 * ngrp * PPW) {
        float v[2];
        bool ok[2];
        EncDst<G, NDIG, 2> dst;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int p = base + u * ngrp * PPW + sub;
            ok[u] = p < ng;
            const int pp = ok[u] ? p : 0;
            const int j = pp * G + (lane & (G - 1));
            v[u] = ok[u] ? xT[(size_t)(j & 7) * TP + (j >> 3)] : 0.0f;
            dst.set(u, a, (size_t)b, pp, i8);
        }
        encode_groups_n<G, NDIG, 2>(v, ok, dst.dig, dst.sc, i8, dst.hi, dst.lo, dst.qs, dst.qc);
    }
}

// Router scores of one expert group (8 experts) for one token: block
// (eg, b) is one wave; lane 8 * el + r runs chain r of expert 8 * eg + el
// with up to 16 chunks of its chain in flight.  The block also encodes its
// share of the token's x digits (groups eg, eg + groups, ...) from the
// staged token.  The top-k then runs per token in k_topk once every score
// is written: a per-token block would have to pull the whole table through
// one CU.
// LAYER: the decoder-layer variant, which first adds the o_proj slices to x
// and applies the RMSNorm (a separate instance, so that the plain block's
// router keeps its register budget).
template <int G, int NDIG, int DV, bool WBF16, bool LAYER>
__global__ void __launch_bounds__(64)
k_router_grp(RouteArgs a) {
    using C = Chain<DV, WBF16>;
    constexpr int d = DV * 512;
    constexpr int T = d / 8;
    constexpr int TP = T + 4;                // padded LDS row: the 8 residues fall in different banks
    __shared__ float xT[8 * TP];             // the token, x[8t + r] at [r][t]
    const int eg = blockIdx.x, b = blockIdx.y;
    const int lane = threadIdx.x;
    const int r = lane & 7, el = lane >> 3;
    const int ngrp = gridDim.x;
    const uint4* wt = (const uint4*)a.wt;

    // the token's loads first, so that staging it waits only for them
    constexpr int XV = d / 4 / 64;           // float4 of the token per lane
    float4 xv[XV];
    const float4* xb = (const float4*)(a.x + (size_t)b * d);
#pragma unroll
    for (int i = 0; i < XV; i++) xv[i] = xb[lane + 64 * i];
    // The decoder layer's inputs (the o_proj slices, up to RG_PS of them,
    // and the norm weight) are requested next, before the table: all of
    // them return in the first memory round trip instead of one round trip
    // per slice.  The table's chunks in flight are fewer in this variant so
    // that the slices fit in registers; the rest are requested as the chain
    // consumes the first ones.
    constexpr int RG_PS = LAYER ? 4 : 1;
    float4 sv[RG_PS][XV];
    uint2 nwv[LAYER ? XV : 1];
    const size_t sstride = (size_t)a.B * d / 4;
    const float4* xp = (const float4*)(a.xpart + (size_t)b * d);
    if (LAYER && a.xpart) {
#pragma unroll
        for (int s = 0; s < RG_PS; s++) {
            const int sc = s < a.nxpart ? s : a.nxpart - 1;     // clamped: every load in bounds
#pragma unroll
            for (int i = 0; i < XV; i++) sv[s][i] = xp[sc * sstride + lane + 64 * i];
        }
    }
    if (LAYER && a.norm_w) {
        const uint2* nw = (const uint2*)a.norm_w;
#pragma unroll
        for (int i = 0; i < (LAYER ? XV : 1); i++) nwv[i] = nw[lane + 64 * i];
    }
    constexpr int NBM = LAYER ? 6 : 16;
    constexpr int NB = C::NC < NBM ? C::NC : NBM;
    uint4 buf[NB][C::CP];
#pragma unroll
    for (int c = 0; c < NB; c++) C::load(buf[c], wt, eg, c, lane);
    if (LAYER && a.xpart) {
        // the decoder layer's residual add before the MoE block
        // (decode_kernel.c:1546-1547): x + the attention output, which comes
        // as the o_proj's column slices, summed in slice order
        float4 ps[XV];
#pragma unroll
        for (int i = 0; i < XV; i++) ps[i] = sv[0][i];
#pragma unroll
        for (int s = 1; s < RG_PS; s++) {
            if (s < a.nxpart) {
#pragma unroll
                for (int i = 0; i < XV; i++) {
                    const float4 u = sv[s][i];
                    ps[i] = make_float4(__fadd_rn(ps[i].x, u.x), __fadd_rn(ps[i].y, u.y), __fadd_rn(ps[i].z, u.z),
                                        __fadd_rn(ps[i].w, u.w));
                }
            }
        }
        for (int sl = RG_PS; sl < a.nxpart; sl++) {
#pragma unroll
            for (int i = 0; i < XV; i++) {
                const float4 u = xp[sl * sstride + lane + 64 * i];
                ps[i] = make_float4(__fadd_rn(ps[i].x, u.x), __fadd_rn(ps[i].y, u.y), __fadd_rn(ps[i].z, u.z),
                                    __fadd_rn(ps[i].w, u.w));
            }
        }
#pragma unroll
        for (int i = 0; i < XV; i++)
            xv[i] = make_float4(__fadd_rn(xv[i].x, ps[i].x), __fadd_rn(xv[i].y, ps[i].y), __fadd_rn(xv[i].z, ps[i].z),
                                __fadd_rn(xv[i].w, ps[i].w));
        if (eg == 0 && a.xmid) {
            float4* xm = (float4*)(a.xmid + (size_t)b * d);
#pragma unroll
            for (int i = 0; i < XV; i++) xm[lane + 64 * i] = xv[i];
        }
    }
    if (LAYER && a.norm_w) {
        // the decoder layer's RMSNorm of the token first (decode_kernel.c:224-230,
        // applied at :1549): x * (1 / sqrtf_fast(sum x^2 / d + eps)) * w
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < XV; i++) {
            ss = __builtin_fmaf(xv[i].x, xv[i].x, ss);
            ss = __builtin_fmaf(xv[i].y, xv[i].y, ss);
            ss = __builtin_fmaf(xv[i].z, xv[i].z, ss);
            ss = __builtin_fmaf(xv[i].w, xv[i].w, ss);
        }
        const float inv = rms_inv(seg_sum<64>(ss), d, a.eps);
#pragma unroll
        for (int i = 0; i < (LAYER ? XV : 1); i++) {
            const uint2 w = nwv[i];
            xv[i].x = __fmul_rn(__fmul_rn(xv[i].x, inv), bf16_bits_to_f32(w.x & 0xFFFFu));
            xv[i].y = __fmul_rn(__fmul_rn(xv[i].y, inv), bf16_bits_to_f32(w.x >> 16));
            xv[i].z = __fmul_rn(__fmul_rn(xv[i].z, inv), bf16_bits_to_f32(w.y & 0xFFFFu));
            xv[i].w = __fmul_rn(__fmul_rn(xv[i].w, inv), bf16_bits_to_f32(w.y >> 16));
        }
    }
    stage_chain_order<XV, TP>(xv, xT);
    __syncthreads();
    encode_token_share<G, NDIG, d>(a, b, eg, ngrp, xT);
    const float acc = router_chains<DV, WBF16, NB>(buf, wt, eg, xT);
    const int e = 8 * eg + el;
    if (r == 0 && e < a.E) a.logits[(size_t)b * a.E + e] = acc;
}

// The same for batches of many tokens: block (4 expert groups, 4 tokens),
// one wave per group.  Wave w first stages token 4 * blockIdx.y + w in LDS
// (with the decoder layer's slice sum and RMSNorm, LAYER); then each wave
// runs its group's chains for the 4 tokens from one read of its table
// chunks, each token's chain in the same order as k_router_grp's, so the
// scores are the same bits.  The table is read once per 4 tokens instead of
// once per token.  The x digits and the MFMA-branch digit pairs of the 4 tokens
// are shared out over the grid's waves as k_router_grp shares them.
constexpr int RQ_T = 4;             // tokens per block
template <int G, int NDIG, int DV, bool WBF16, bool LAYER>
__global__ void __launch_bounds__(256)
k_router_quad(RouteArgs a) {
    using C = Chain<DV, WBF16>;
    constexpr int d = DV * 512;
    constexpr int T = d / 8;
    constexpr int TP = T + 4;
    __shared__ float xT[RQ_T][8 * TP];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int eg = blockIdx.x * 4 + w;           // this wave's expert group
    const int ngrp = (a.E + 7) / 8, nvg = gridDim.x * 4;
    const int b0 = blockIdx.y * RQ_T;
    const int r = lane & 7, el = lane >> 3;
    const uint4* wt = (const uint4*)a.wt;
    const bool chains = eg < ngrp;

    constexpr int XV = d / 4 / 64;
    constexpr int NB = C::NC < 16 ? C::NC : 16;
    // wave w stages token b0 + w: its loads first, so that staging waits
    // for them only, then the table's
    const int bw = b0 + w;
    float4 xv[XV];
    {
        const float4* xb = (const float4*)(a.x + (size_t)(bw < a.B ? bw : b0) * d);
#pragma unroll
        for (int i = 0; i < XV; i++) xv[i] = xb[lane + 64 * i];
    }
    __builtin_amdgcn_sched_barrier(0);      // the token's loads ahead of the table's
    // The table's first chunks, unconditionally (group 0 stands in for a
    // wave past the last group): behind a branch, the staging below would
    // wait for every table load as well as the token's.
    uint4 buf[NB][C::CP];
    {
        const int egl = chains ? eg : 0;
#pragma unroll
        for (int c = 0; c < NB; c++) C::load(buf[c], wt, egl, c, lane);
    }
    {
        const int b = bw;
        if (b < a.B) {
            if (LAYER && a.xpart) {
                const float4* xp = (const float4*)(a.xpart + (size_t)b * d);
                const size_t sstride = (size_t)a.B * d / 4;
                float4 ps[XV];
#pragma unroll
                for (int i = 0; i < XV; i++) ps[i] = xp[lane + 64 * i];
                for (int sl = 1; sl < a.nxpart; sl++) {
#pragma unroll
                    for (int i = 0; i < XV; i++) {
                        const float4 u = xp[sl * sstride + lane + 64 * i];
                        ps[i] = make_float4(__fadd_rn(ps[i].x, u.x), __fadd_rn(ps[i].y, u.y), __fadd_rn(ps[i].z, u.z),
                                            __fadd_rn(ps[i].w, u.w));
                    }
                }
#pragma unroll
                for (int i = 0; i < XV; i++)
                    xv[i] = make_float4(__fadd_rn(xv[i].x, ps[i].x), __fadd_rn(xv[i].y, ps[i].y),
                                        __fadd_rn(xv[i].z, ps[i].z), __fadd_rn(xv[i].w, ps[i].w));
                if (blockIdx.x == 0 && a.xmid) {
                    float4* xm = (float4*)(a.xmid + (size_t)b * d);
#pragma unroll
                    for (int i = 0; i < XV; i++) xm[lane + 64 * i] = xv[i];
                }
            }
            if (LAYER && a.norm_w) {
                float ss = 0.0f;
#pragma unroll
                for (int i = 0; i < XV; i++) {
                    ss = __builtin_fmaf(xv[i].x, xv[i].x, ss);
                    ss = __builtin_fmaf(xv[i].y, xv[i].y, ss);
                    ss = __builtin_fmaf(xv[i].z, xv[i].z, ss);
                    ss = __builtin_fmaf(xv[i].w, xv[i].w, ss);
                }
                const float inv = rms_inv(seg_sum<64>(ss), d, a.eps);
                const uint2* nw = (const uint2*)a.norm_w;
#pragma unroll
                for (int i = 0; i < XV; i++) {
                    const uint2 wv = nw[lane + 64 * i];
                    xv[i].x = __fmul_rn(__fmul_rn(xv[i].x, inv), bf16_bits_to_f32(wv.x & 0xFFFFu));
                    xv[i].y = __fmul_rn(__fmul_rn(xv[i].y, inv), bf16_bits_to_f32(wv.x >> 16));
                    xv[i].z = __fmul_rn(__fmul_rn(xv[i].z, inv), bf16_bits_to_f32(wv.y & 0xFFFFu));
                    xv[i].w = __fmul_rn(__fmul_rn(xv[i].w, inv), bf16_bits_to_f32(wv.y >> 16));
                }
            }
            if (LAYER && blockIdx.x == 0 && a.xn) {
                float4* xo = (float4*)(a.xn + (size_t)b * d);
#pragma unroll
                for (int i = 0; i < XV; i++) xo[lane + 64 * i] = xv[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < XV; i++) xv[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        float* xw = xT[w];
#pragma unroll
        for (int i = 0; i < XV; i++) {
            const int j = 4 * (lane + 64 * i);
            xw[((j + 0) & 7) * TP + ((j + 0) >> 3)] = xv[i].x;
            xw[((j + 1) & 7) * TP + ((j + 1) >> 3)] = xv[i].y;
            xw[((j + 2) & 7) * TP + ((j + 2) >> 3)] = xv[i].z;
            xw[((j + 3) & 7) * TP + ((j + 3) >> 3)] = xv[i].w;
        }
    }
    __syncthreads();
    const int nt = min(RQ_T, a.B - b0);           // tokens of this block (>= 1)
    // x digits (one G-value group per G-lane segment) and the MFMA digit
    // pairs of the block's tokens, this wave's share over the grid's nvg
    // waves, before the chains: they need only the staged tokens, so they
    // run while the table's chunks are still arriving.  The tokens of a
    // group are encoded together (unconditionally, the stores guarded), so
    // that their reduction chains interleave.  With enc_late the dispatch
    // launch encodes them instead, on the CUs its one dispatch block leaves
    // idle.
    constexpr int ng = d / G;
    constexpr int PPW = JM_WAVE / G;
    const int sub = lane / G;
    const bool i8 = a.xqh != nullptr;
    for (int base = a.enc_late ? ng : eg * PPW; base < ng; base += nvg * PPW) {
        const int p = base + sub;
        const bool ok = p < ng;
        const int pp = ok ? p : 0;
        const int j = pp * G + (lane & (G - 1));
        float v[RQ_T];
        bool st[RQ_T];
        EncDst<G, NDIG, RQ_T> dst;
#pragma unroll
        for (int t = 0; t < RQ_T; t++) {
            st[t] = ok && t < nt;
            v[t] = st[t] ? xT[t][(size_t)(j & 7) * TP + (j >> 3)] : 0.0f;
            dst.set(t, a, (size_t)b0 + (t < nt ? t : 0), pp, i8);
        }
        encode_groups_n<G, NDIG, RQ_T>(v, st, dst.dig, dst.sc, i8, dst.hi, dst.lo, dst.qs, dst.qc);
    }
    if (chains) {
        float acc[RQ_T];
#pragma unroll
        for (int t = 0; t < RQ_T; t++) acc[t] = 0.0f;
        // each token's chain in k_router_grp's order: chunk c's fused
        // multiply-adds for the 4 tokens interleaved (4 independent chains
        // in flight), pinned before the loads of chunk c + NB
#pragma unroll
        for (int c = 0; c < C::NC; c++) {
            const float* const xr[RQ_T] = {xT[0] + (size_t)r * TP, xT[1] + (size_t)r * TP, xT[2] + (size_t)r * TP,
                                            xT[3] + (size_t)r * TP};
            C::template fma_chunk_n<RQ_T>(buf[c % NB], xr, c, acc);
            static_assert(RQ_T == 4, "one pin per chunk for the 4 tokens");
            __asm__ volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]) : : "memory");
            if (c + NB < C::NC) C::load(buf[c % NB], wt, eg, c + NB, lane);
        }
        const int e = 8 * eg + el;
#pragma unroll
        for (int t = 0; t < RQ_T; t++) {
            float v = acc[t];
            v = __fadd_rn(v, __shfl_xor(v, 4, JM_WAVE));
            v = __fadd_rn(v, __shfl_xor(v, 2, JM_WAVE));
            v = __fadd_rn(v, __shfl_xor(v, 1, JM_WAVE));
            if (r == 0 && e < a.E && t < nt) a.logits[(size_t)(b0 + t) * a.E + e] = v;
        }
    }
}

// The dispatch launch's token encode (enc_late): the x digits and, for the
// MFMA branch, the digit pairs of every token, from a.xenc (the tokens as the
// router scored them).  Item (ENC_T tokens, group position) per wave, one
// G-value group per G-lane segment, the tokens' loads issued together; the
// same values as the router's encode.  Two tokens per item measured best:
// at 512 tokens the block took 1.2 us less than with 4 (0.9 us at 64); with
// 1 token per item it took as long at 512 and 0.4 us more at 64 tokens (when
// the encode moved here from 64 tokens on).
// (The 4 encodes of a 4-token item through
// encode_groups_n made the 512-token block about 0.5 us slower.)
constexpr int ENC_T = 2;
template <int G, int NDIG>
__device__ __forceinline__ void encode_late(const RouteArgs& a, int gw, int nw) {
    constexpr int PPW = JM_WAVE / G;
    const int lane = threadIdx.x & 63, sub = lane / G;
    const int d = a.d, ng = d / G, ngw = ng / PPW;
    const int nq = (a.B + ENC_T - 1) / ENC_T;
    const bool i8 = a.xqh != nullptr;
    for (int it = gw; it < nq * ngw; it += nw) {
        const int q = it / ngw;
        const int p = (it - q * ngw) * PPW + sub;
        const int b0 = q * ENC_T;
        const int nt = min(ENC_T, a.B - b0);
        float v[ENC_T];
#pragma unroll
        for (int t = 0; t < ENC_T; t++) {
            const size_t b = (size_t)b0 + (t < nt ? t : 0);
            v[t] = a.xenc[b * d + (size_t)p * G + (lane & (G - 1))];
        }
        EncDst<G, NDIG, ENC_T> dst;
#pragma unroll
        for (int t = 0; t < ENC_T; t++) {
            const bool st = t < nt;
            dst.set(t, a, (size_t)b0 + (st ? t : 0), p, i8);
            encode_group_both<G, NDIG>(st ? v[t] : 0.0f, st, dst.dig[t], dst.sc[t], i8, dst.hi[t], dst.lo[t],
                                       dst.qs[t], dst.qc[t]);
        }
    }
}

// Dispatch and work table of all slots from the top-k table (dispatch
// path), on block 0; with enc_late, the blocks past it encode the tokens.
template <int G, int NDIG>
__global__ void __launch_bounds__(1024)
k_dispatch_work(RouteArgs a) {
    extern __shared__ int lds_i[];
    if (blockIdx.x > 0) {
        encode_late<G, NDIG>(a, (blockIdx.x - 1) * (blockDim.x / JM_WAVE) + (threadIdx.x >> 6),
                             (gridDim.x - 1) * (blockDim.x / JM_WAVE));
        return;
    }
    ExpertRec rec;
    if ((int)threadIdx.x < a.E) rec = load_expert_rec(a.rec, a.key0, threadIdx.x);
    // the work entries' slot counts come back in LDS (over the expert
    // counts, dead by then); the scan below uses the dispatch's scan scratch
    int* const wn = lds_i;
    unsigned* const wsum = (unsigned*)(lds_i + 3 * a.E + 1);
    dispatch_block<false>(a.top, a.B * a.topk, a.E, a.topk, lds_i, a.seg_off, a.seg_slot, a.active,
                   a.n_active, a.first_slot, a.comb, a.work, a.umax, &rec, wn);
    // the dense experts' token tiles, in work-table order, and the list of
    // the experts under dense_min (their wave items run on the MFMA grids)
    lds_barrier();
    const int u = threadIdx.x;
    int ct = 0, sm = 0;
    if (u < a.umax) {
        const int n = wn[u];
        ct = n >= a.dense_min ? (n + JM_DENSE_TILE - 1) / JM_DENSE_TILE : 0;
        sm = n > 0 && n < a.dense_min;
    }
    uint2 tot;
    const uint2 ex = block_exclusive_scan2(make_uint2((unsigned)ct, (unsigned)sm), wsum, &tot);
    for (int j = 0; j < ct; j++) a.tiles[ex.x + j] = make_int2(u, j);
    if (sm) a.small[ex.y] = u;
    if (threadIdx.x == 0) {
        a.n_tiles[0] = (int)tot.x;
        a.n_tiles[1] = (int)tot.y;
    }
}

hipError_t launch_route_tok(const RouteArgs& a, hipStream_t st) {
    if (a.B == 0) return hipSuccess;
    const int ngrp = (a.E + 7) / 8;
    const bool quad = a.B >= JM_ROUTER_QUAD_MIN_B;
    const dim3 grid((unsigned)ngrp, (unsigned)a.B);
    const dim3 gridq((unsigned)((ngrp + 3) / 4), (unsigned)((a.B + RQ_T - 1) / RQ_T));
    if (a.ndig != 4 && a.ndig != 5) return hipErrorInvalidValue;
#define JM_RTN(GG, N, DVV, BF, LY)                                                                  \
    if (quad) hipLaunchKernelGGL((k_router_quad<GG, N, DVV, BF, LY>), gridq, dim3(256), 0, st, a); \
    else hipLaunchKernelGGL((k_router_grp<GG, N, DVV, BF, LY>), grid, dim3(64), 0, st, a)
#define JM_RT1(GG, DVV, BF, LY) if (a.ndig == 5) { JM_RTN(GG, 5, DVV, BF, LY); } else { JM_RTN(GG, 4, DVV, BF, LY); }
#define JM_RT(GG, DVV, BF) if (a.xpart || a.norm_w) { JM_RT1(GG, DVV, BF, true); } else { JM_RT1(GG, DVV, BF, false); }
#define JM_RTB(GG, DVV) if (a.wt_bf16) { JM_RT(GG, DVV, true); } else { JM_RT(GG, DVV, false); }
#define JM_RTD(GG) switch (a.d / 512) { case 1: JM_RTB(GG, 1); break; case 2: JM_RTB(GG, 2); break; \
        case 3: JM_RTB(GG, 3); break; case 4: JM_RTB(GG, 4); break; case 6: JM_RTB(GG, 6); break; \
        case 8: JM_RTB(GG, 8); break; default: return hipErrorInvalidValue; }
    if (a.group == 64) { JM_RTD(64) } else { JM_RTD(32) }
#undef JM_RTD
#undef JM_RTB
#undef JM_RT
#undef JM_RT1
#undef JM_RTN
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.skip_topk) return e;
    return launch_topk(a.logits, a.B, a.E, a.topk, a.renorm, a.top, a.tw, st);
}

// Blocks of 16 encode waves past the dispatch block: one item per wave up
// to 1024 blocks, more per wave past that.
constexpr int ENC_LATE_MAX_BLOCKS = 1024;

hipError_t launch_dispatch_work(const RouteArgs& a, hipStream_t st) {
    int nenc = 0;
    if (a.enc_late) {
        if (a.group != 32 && a.group != 64) return hipErrorInvalidValue;
        if (a.ndig != 4 && a.ndig != 5) return hipErrorInvalidValue;
        const long long items = (long long)((a.B + ENC_T - 1) / ENC_T) * (a.d / 64);
        nenc = (int)std::min<long long>(ENC_LATE_MAX_BLOCKS, (items + 15) / 16);
    }
    const dim3 grid((unsigned)(1 + nenc));
    const size_t lds = (size_t)dispatch_lds_ints(a.B * a.topk, a.E) * 4;
    if (a.group == 64) {
        if (a.ndig == 5) hipLaunchKernelGGL((k_dispatch_work<64, 5>), grid, dim3(1024), lds, st, a);
        else hipLaunchKernelGGL((k_dispatch_work<64, 4>), grid, dim3(1024), lds, st, a);
    } else {
        if (a.ndig == 5) hipLaunchKernelGGL((k_dispatch_work<32, 5>), grid, dim3(1024), lds, st, a);
        else hipLaunchKernelGGL((k_dispatch_work<32, 4>), grid, dim3(1024), lds, st, a);
    }
    return hipGetLastError();
}

}  // namespace jm
