// The router's FMA chains (gfx950), shared by the router kernels
// (jm_route.hip) and the front kernel's router waves (jm_front.hip), so that
// every path computes the same bits.
//
// Lane L = 8 * e_local + r of a wave runs the FMA chain r of expert
// 8 * eg + e_local over the values j = r (mod 8) in increasing order (the 8
// lanes of an AVX2 register of the reference, decode_kernel.c:234-256,
// 693-718).  The router table is read from the interleaved copy in which
// piece i of lane L's chain (16 bytes) sits at [eg][i][L], so each load
// instruction of a wave reads 1 KiB of contiguous memory.  The token is
// staged in LDS in the chains' order: x[8t + r] at [r][t] of a row of
// T + 4 floats.
#pragma once

#include "jm_device.h"

namespace jm {

// Chain loads in chunks of CP pieces (16 chain values of a bf16 table, 8
// of a float32 one); a ring of chunks is kept in flight, the loads of chunk
// c + ring issued as soon as chunk c's registers are consumed.
template <int DV, bool WBF16>
struct Chain {
    static constexpr int T = DV * 64;                 // chain length (d / 8)
    static constexpr int P = WBF16 ? 8 : 4;           // chain values per 16-byte piece
    static constexpr int NP = T / P;                  // pieces per chain
    static constexpr int CP = 2;                      // pieces per chunk
    static constexpr int NC = NP / CP;                // chunks

    static __device__ __forceinline__ void load(uint4 (&buf)[CP], const uint4* __restrict__ wt, int eg,
                                                int c, int lane) {
        const uint4* p = wt + ((size_t)eg * NP + (size_t)c * CP) * 64 + lane;
#pragma unroll
        for (int i = 0; i < CP; i++) buf[i] = p[(size_t)i * 64];
    }

    // The same for NT tokens at once (staged rows xr[t]): every token's x
    // values of the chunk are read first, then each weight value is applied
    // to the NT chains in turn, so that NT independent chains are in flight
    // (each chain's values still in order).
    template <int NT>
    static __device__ __forceinline__ void fma_chunk_n(const uint4 (&buf)[CP], const float* const (&xr)[NT], int c,
                                                       float (&acc)[NT]) {
        constexpr int NV = CP * P;                    // values per chunk
        float4 xq[NT][NV / 4];
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int i = 0; i < NV / 4; i++) xq[t][i] = ((const float4*)xr[t] + (size_t)c * NV / 4)[i];
#pragma unroll
        for (int v = 0; v < NV; v++) {
            const unsigned wd = ((const unsigned*)&buf[v / P])[WBF16 ? (v % P) / 2 : v % P];
            const float wv = WBF16 ? __uint_as_float((v & 1) ? (wd & 0xFFFF0000u) : (wd << 16)) : __uint_as_float(wd);
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float4 q = xq[t][v / 4];
                const float xv = (v & 3) == 0 ? q.x : (v & 3) == 1 ? q.y : (v & 3) == 2 ? q.z : q.w;
                acc[t] = __builtin_fmaf(wv, xv, acc[t]);
            }
        }
    }

    // acc += chunk c of the chain (values in order), x from the staged row
    static __device__ __forceinline__ float fma_chunk(const uint4 (&buf)[CP], const float* xr, int c,
                                                      float acc) {
        const float4* xq = (const float4*)xr + (size_t)c * CP * P / 4;
#pragma unroll
        for (int i = 0; i < CP; i++) {
            if (WBF16) {
                const float4 x0 = xq[2 * i], x1 = xq[2 * i + 1];
                const unsigned w[4] = {buf[i].x, buf[i].y, buf[i].z, buf[i].w};
                acc = __builtin_fmaf(__uint_as_float(w[0] << 16), x0.x, acc);
                acc = __builtin_fmaf(__uint_as_float(w[0] & 0xFFFF0000u), x0.y, acc);
                acc = __builtin_fmaf(__uint_as_float(w[1] << 16), x0.z, acc);
                acc = __builtin_fmaf(__uint_as_float(w[1] & 0xFFFF0000u), x0.w, acc);
                acc = __builtin_fmaf(__uint_as_float(w[2] << 16), x1.x, acc);
                acc = __builtin_fmaf(__uint_as_float(w[2] & 0xFFFF0000u), x1.y, acc);
                acc = __builtin_fmaf(__uint_as_float(w[3] << 16), x1.z, acc);
                acc = __builtin_fmaf(__uint_as_float(w[3] & 0xFFFF0000u), x1.w, acc);
            } else {
                const float4 xv = xq[i];
                acc = __builtin_fmaf(__uint_as_float(buf[i].x), xv.x, acc);
                acc = __builtin_fmaf(__uint_as_float(buf[i].y), xv.y, acc);
                acc = __builtin_fmaf(__uint_as_float(buf[i].z), xv.z, acc);
                acc = __builtin_fmaf(__uint_as_float(buf[i].w), xv.w, acc);
            }
        }
        return acc;
    }
};

// Staged token row x[8t + r] -> xT[r * TP + t] (TP = d / 8 + 4), from the
// float4s xv[i] = x[4 (lane + 64 i) .. + 3] of one wave.
template <int XV, int TP>
__device__ __forceinline__ void stage_chain_order(const float4 (&xv)[XV], float* xT) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < XV; i++) {
        const int j = 4 * (lane + 64 * i);
        xT[((j + 0) & 7) * TP + ((j + 0) >> 3)] = xv[i].x;
        xT[((j + 1) & 7) * TP + ((j + 1) >> 3)] = xv[i].y;
        xT[((j + 2) & 7) * TP + ((j + 2) >> 3)] = xv[i].z;
        xT[((j + 3) & 7) * TP + ((j + 3) >> 3)] = xv[i].w;
    }
}

// Router score of expert 8 eg + (lane >> 3) for the token staged in xT, in
// every lane of its 8 (chain sums added in the AVX2 order: (r, r^4), then
// ^2, then ^1).  buf holds the first NB chunks already requested; chunk
// c + NB is requested as soon as chunk c's registers are consumed.
template <int DV, bool WBF16, int NB>
__device__ __forceinline__ float router_chains(uint4 (&buf)[NB][2], const uint4* wt, int eg, const float* xT) {
    using C = Chain<DV, WBF16>;
    static_assert(C::CP == 2, "two pieces per chunk");
    constexpr int TP = DV * 64 + 4;
    const int lane = threadIdx.x & 63;
    const float* xr = xT + (size_t)(lane & 7) * TP;
    float acc = 0.0f;
    // Pinned order: chunk c's token reads and fused multiply-adds, then the
    // loads of chunk c + NB into the registers chunk c used.  The empty asm
    // takes the running sum and fences memory operations, so the compiler
    // neither sinks the arithmetic to the end of the chain nor hoists later
    // chunks' reads.
#pragma unroll
    for (int c = 0; c < C::NC; c++) {
        acc = C::fma_chunk(buf[c % NB], xr, c, acc);
        __asm__ volatile("" : "+v"(acc) : : "memory");
        if (c + NB < C::NC) C::load(buf[c % NB], wt, eg, c + NB, lane);
    }
    acc = __fadd_rn(acc, __shfl_xor(acc, 4, JM_WAVE));
    acc = __fadd_rn(acc, __shfl_xor(acc, 2, JM_WAVE));
    acc = __fadd_rn(acc, __shfl_xor(acc, 1, JM_WAVE));
    return acc;
}

}  // namespace jm
