// Routing front of the MoE block (gfx950):
//
//   k_router   router scores in the reference's 8-chain order
//              (decode_kernel.c:234-256, 693-718) and the x digits for the
//              expert dots
//   k_select   top-k of every token (decode_kernel.c:1425-1448), then the
//              dispatch of all slots (:1449-1485) and the expert work table,
//              in one block (B <= 64); larger batches run the multi-block
//              top-k and the single-block dispatch as two launches
//
// Blocks never wait for or read data written by other blocks of the same
// launch: on MI355X each XCD has its own L2, and a device-scope handoff
// inside a kernel costs an L2 write-back and invalidate, while the kernel
// boundary does that once.
//
// k_router: grid (ceil(E/8), ceil(B/4)), 256 threads.  Wave w of block
// (eg, g) owns token b = 4g + w; lane L = 8 * e_local + r runs the FMA
// chain r of expert 8*eg + e_local: the 8 lanes of an expert hold the 8
// partial sums that the reference keeps in the 8 lanes of an AVX2 register.
// The router table is read from a copy in which the 64 chains of an expert
// group are interleaved in 16-byte pieces: piece i of lane L's chain
// (values 8t + r for t in the piece) sits at [eg][i][L], so each load
// instruction of a wave reads 1 KiB of contiguous memory.  The token is
// staged in LDS in the chains' order.
#include <algorithm>

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

constexpr int ROUTE_TOK = 4;         // tokens per block (one per wave)
constexpr int ROUTE_EXP = 8;         // experts per block
constexpr int CH = 16;               // float4 per chain chunk (64 values)

// DV = d / 512.  A lane's chain is T = d/8 values: with a bf16 table it is
// T/8 uint4 (32 for d = 2048), all loaded at once; with a float32 table it
// is T/4 float4, loaded in chunks of 64 values, two chunks in flight.  The
// token's loads are issued first and every loop is unrolled, so each wait
// covers exactly the loads it needs (the memory counter retires loads in
// issue order).
template <int DV, bool WBF16>
__device__ __forceinline__ float router_chain(const void* wt_base, int e, int r, const float* xr, bool live,
                                              float4 (&xv4)[DV * 2], float* dst, bool tok, int lane) {
    constexpr int T = DV * 64;
    constexpr int TP = T + 4;
    float acc = 0.0f;
    if (WBF16) {
        constexpr int NW = T / 8;                      // uint4 per chain
        const uint4* wp = (const uint4*)wt_base + (size_t)(e >> 3) * NW * 64 + (((e & 7) << 3) | r);
        uint4 W[NW];
        if (live) {
#pragma unroll
            for (int i = 0; i < NW; i++) W[i] = wp[(size_t)i * 64];
        }
        if (tok) {
#pragma unroll
            for (int i = 0; i < DV * 2; i++) {
                const int j = 4 * (lane + 64 * i);
                dst[((j + 0) & 7) * TP + ((j + 0) >> 3)] = xv4[i].x;
                dst[((j + 1) & 7) * TP + ((j + 1) >> 3)] = xv4[i].y;
                dst[((j + 2) & 7) * TP + ((j + 2) >> 3)] = xv4[i].z;
                dst[((j + 3) & 7) * TP + ((j + 3) >> 3)] = xv4[i].w;
            }
        }
        __syncthreads();
        if (live) {
            const float4* xq = (const float4*)xr;
#pragma unroll
            for (int i = 0; i < NW; i++) {
                const float4 x0 = xq[2 * i], x1 = xq[2 * i + 1];
                const unsigned w[4] = {W[i].x, W[i].y, W[i].z, W[i].w};
                acc = __builtin_fmaf(__uint_as_float(w[0] << 16), x0.x, acc);
                acc = __builtin_fmaf(__uint_as_float(w[0] & 0xFFFF0000u), x0.y, acc);
                acc = __builtin_fmaf(__uint_as_float(w[1] << 16), x0.z, acc);
                acc = __builtin_fmaf(__uint_as_float(w[1] & 0xFFFF0000u), x0.w, acc);
                acc = __builtin_fmaf(__uint_as_float(w[2] << 16), x1.x, acc);
                acc = __builtin_fmaf(__uint_as_float(w[2] & 0xFFFF0000u), x1.y, acc);
                acc = __builtin_fmaf(__uint_as_float(w[3] << 16), x1.z, acc);
                acc = __builtin_fmaf(__uint_as_float(w[3] & 0xFFFF0000u), x1.w, acc);
            }
        }
    } else {
        const float4* wp = (const float4*)wt_base + (size_t)(e >> 3) * (T / 4) * 64 + (((e & 7) << 3) | r);
        float4 A[CH], Bv[CH];
        if (live) {
#pragma unroll
            for (int i = 0; i < CH; i++) A[i] = wp[(size_t)i * 64];
            if (DV > 1) {
#pragma unroll
                for (int i = 0; i < CH; i++) Bv[i] = wp[(size_t)(CH + i) * 64];
            }
        }
        if (tok) {
#pragma unroll
            for (int i = 0; i < DV * 2; i++) {
                const int j = 4 * (lane + 64 * i);
                dst[((j + 0) & 7) * TP + ((j + 0) >> 3)] = xv4[i].x;
                dst[((j + 1) & 7) * TP + ((j + 1) >> 3)] = xv4[i].y;
                dst[((j + 2) & 7) * TP + ((j + 2) >> 3)] = xv4[i].z;
                dst[((j + 3) & 7) * TP + ((j + 3) >> 3)] = xv4[i].w;
            }
        }
        __syncthreads();
        if (live) {
            const float4* xq = (const float4*)xr;
#pragma unroll
            for (int c = 0; c < DV; c += 2) {
#pragma unroll
                for (int i = 0; i < CH; i++) {
                    const float4 xv = xq[c * CH + i];
                    acc = __builtin_fmaf(A[i].x, xv.x, acc);
                    acc = __builtin_fmaf(A[i].y, xv.y, acc);
                    acc = __builtin_fmaf(A[i].z, xv.z, acc);
                    acc = __builtin_fmaf(A[i].w, xv.w, acc);
                }
                if (c + 2 < DV) {
#pragma unroll
                    for (int i = 0; i < CH; i++) A[i] = wp[(size_t)((c + 2) * CH + i) * 64];
                }
                if (c + 1 < DV) {
#pragma unroll
                    for (int i = 0; i < CH; i++) {
                        const float4 xv = xq[(c + 1) * CH + i];
                        acc = __builtin_fmaf(Bv[i].x, xv.x, acc);
                        acc = __builtin_fmaf(Bv[i].y, xv.y, acc);
                        acc = __builtin_fmaf(Bv[i].z, xv.z, acc);
                        acc = __builtin_fmaf(Bv[i].w, xv.w, acc);
                    }
                    if (c + 3 < DV) {
#pragma unroll
                        for (int i = 0; i < CH; i++) Bv[i] = wp[(size_t)((c + 3) * CH + i) * 64];
                    }
                }
            }
        }
    }
    return acc;
}

template <int G, int NDIG, int DV, bool WBF16>
__global__ void __launch_bounds__(256)
k_router(RouteArgs a) {
    extern __shared__ float lds[];
    constexpr int d = DV * 512;
    constexpr int T = d / 8;                 // chain length
    constexpr int TP = T + 4;                // padded LDS row: the 8 residues fall in different banks
    float* xT = lds;
    const int eg = blockIdx.x, g = blockIdx.y;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane & 7, el = lane >> 3;
    const int e = eg * ROUTE_EXP + el;
    const int b = g * ROUTE_TOK + w;
    const bool tok = b < a.B;
    const bool live = tok && e < a.E;

    float4 xv4[DV * 2];
    if (tok) {
        const float4* xb = (const float4*)(a.x + (size_t)b * d);
#pragma unroll
        for (int i = 0; i < DV * 2; i++) xv4[i] = xb[lane + 64 * i];
    }
    float* dst = xT + (size_t)w * 8 * TP;
    const float* xr = xT + (size_t)w * 8 * TP + (size_t)r * TP;
    float acc = router_chain<DV, WBF16>(a.wt, live ? e : 0, r, xr, live, xv4, dst, tok, lane);
    // horizontal sum in the AVX2 order: (r, r^4), then ^2, then ^1
    acc = __fadd_rn(acc, __shfl_xor(acc, 4, JM_WAVE));
    acc = __fadd_rn(acc, __shfl_xor(acc, 2, JM_WAVE));
    acc = __fadd_rn(acc, __shfl_xor(acc, 1, JM_WAVE));
    if (live && r == 0) a.logits[(size_t)b * a.E + e] = acc;

    // x digits of this block's share of the token group's (token, group)
    // pairs, read from the staged copy: x[bt][j] = xT[bt%4][j%8][j/8]
    constexpr int ng = d / G;
    const int ntok = min(ROUTE_TOK, a.B - g * ROUTE_TOK);
    const int npairs = ntok * ng;
    const int nblk = gridDim.x;
    constexpr int PPW = JM_WAVE / G;
    const int sub = lane / G;
    for (int base = (eg + nblk * w) * PPW; base < npairs; base += nblk * 4 * PPW) {
        const int p = base + sub;
        const bool ok = p < npairs;
        const int tl = ok ? p / ng : 0;
        const int gg = ok ? p % ng : 0;
        const int j = gg * G + (lane & (G - 1));
        const float v = ok ? xT[(size_t)tl * 8 * TP + (size_t)(j & 7) * TP + (j >> 3)] : 0.0f;
        const int bt = g * ROUTE_TOK + tl;
        encode_group_wave<G, NDIG>(v, ok, a.xdig + ((size_t)bt * ng + gg) * (NDIG * (G / 8)),
                                   a.xscale + (size_t)bt * ng + gg);
    }
}

// Top-k of every token (wave w takes tokens w, w + 16, ...) into LDS, then
// the dispatch of all slots and the work table; one block of 1024 threads.
// The record offsets of expert tid are requested first so that they arrive
// while the top-k runs.
template <int EPL>
__global__ void __launch_bounds__(1024)
k_select(RouteArgs a) {
    extern __shared__ int lds_i[];
    ExpertRec rec;
    if ((int)threadIdx.x < a.E) rec = load_expert_rec(a.rec_off, a.LE, a.key0, threadIdx.x);
    const int w = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const int nslot = a.B * a.topk;
    int* top_l = lds_i;                                  // [nslot]
    float* tw_l = (float*)(top_l + nslot);               // [nslot]
    int* rank_l = (int*)(tw_l + nslot);                  // [nslot]
    int* rest = lds_i + (3 * nslot + 3) / 4 * 4;          // 16-byte aligned
    float* p_lds = (float*)rest + (size_t)w * 64 * EPL;
    for (int b = w; b < a.B; b += nw)
        topk_wave<EPL>(a.logits + (size_t)b * a.E, a.E, a.topk, a.renorm, p_lds,
                       top_l + b * a.topk, tw_l + b * a.topk);
    __syncthreads();
    for (int i = threadIdx.x; i < nslot; i += blockDim.x) {
        a.top[i] = top_l[i];
        a.tw[i] = tw_l[i];
    }
    dispatch_block(top_l, nslot, a.E, a.topk, rest, a.seg_off, a.seg_slot, a.active, a.n_active,
                   a.first_slot, a.comb, rank_l, a.work, a.umax, &rec);
}

// Dispatch and work table alone, after the multi-block top-k (large B).
__global__ void __launch_bounds__(1024)
k_dispatch_work(RouteArgs a) {
    extern __shared__ int lds_i[];
    ExpertRec rec;
    if ((int)threadIdx.x < a.E) rec = load_expert_rec(a.rec_off, a.LE, a.key0, threadIdx.x);
    dispatch_block(a.top, a.B * a.topk, a.E, a.topk, lds_i, a.seg_off, a.seg_slot, a.active,
                   a.n_active, a.first_slot, a.comb, a.rank_scratch, a.work, a.umax, &rec);
}

static size_t dispatch_lds_bytes(int E) { return (size_t)dispatch_lds_ints(E) * 4; }

hipError_t launch_route(const RouteArgs& a, hipStream_t st) {
    const dim3 grid((unsigned)((a.E + ROUTE_EXP - 1) / ROUTE_EXP), (unsigned)((a.B + ROUTE_TOK - 1) / ROUTE_TOK));
    const size_t xl = (size_t)ROUTE_TOK * 8 * (a.d / 8 + 4) * 4;
#define JM_RT(GG, DVV) do { if (a.wt_bf16) hipLaunchKernelGGL((k_router<GG, JM_NDIG, DVV, true>), grid, dim3(256), xl, st, a); \
                           else hipLaunchKernelGGL((k_router<GG, JM_NDIG, DVV, false>), grid, dim3(256), xl, st, a); } while (0)
#define JM_RTD(GG) switch (a.d / 512) { case 1: JM_RT(GG, 1); break; case 2: JM_RT(GG, 2); break; \
        case 3: JM_RT(GG, 3); break; case 4: JM_RT(GG, 4); break; case 6: JM_RT(GG, 6); break; \
        case 8: JM_RT(GG, 8); break; default: return hipErrorInvalidValue; }
    if (a.group == 64) { JM_RTD(64) } else { JM_RTD(32) }
#undef JM_RTD
#undef JM_RT
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int epl = a.E <= 64 ? 1 : a.E <= 128 ? 2 : a.E <= 256 ? 4 : 8;
    if (a.B <= 64) {
        const size_t lds = (size_t)(3 * a.B * a.topk + 3) / 4 * 16 + std::max((size_t)16 * 64 * epl * 4, dispatch_lds_bytes(a.E));
#define JM_SEL(EPL) hipLaunchKernelGGL(k_select<EPL>, dim3(1), dim3(1024), lds, st, a)
        if (epl == 1) JM_SEL(1); else if (epl == 2) JM_SEL(2); else if (epl == 4) JM_SEL(4); else JM_SEL(8);
#undef JM_SEL
    } else {
        e = launch_topk(a.logits, a.B, a.E, a.topk, a.renorm, a.top, a.tw, st);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k_dispatch_work, dim3(1), dim3(1024), dispatch_lds_bytes(a.E), st, a);
    }
    return hipGetLastError();
}

}  // namespace jm
