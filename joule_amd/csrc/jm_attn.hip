// Decoder-layer kernels around the MoE block: the bf16 projections (with the
// RMSNorm before them and the residual add after them fused in), decode
// attention over a bf16 KV cache, and the final RMSNorm.  They follow the
// reference's layer_attn_batch / decode_layers_batch
// (decode_kernel.c:1120-1234, 1518-1556) step for step, regrouped into few
// launches:
//
//   k_gemv_part   Wq/Wk/Wv . (h * norm1 weight), per 512-column slice
//                                                             (:224-230, :1126-1145)
//   k_qk_ss       whole-vector QK-norm only: each token's sums of squares
//                 of q and k                                   (:1155-1167)
//   k_attn_part   the slices summed, RMSNorm row scale, bias, per-head or
//                 whole-vector QK-norm and RoPE of the block's heads (:1146-1199; the k
//                 and v rows appended to the cache by the split that holds
//                 the token's position), then scores, softmax and P.V over
//                 one 128-position split of the cache           (:1200-1222)
//   k_attn_comb   the splits merged per head                   (flash-decoding merge)
//   k_gemv_part   Wo . att per slice; the MoE router sums the slices into
//                 the residual                                  (:1225-1232, :1546-1547)
//   k_rms_rows    the final RMSNorm                            (:1556)
//
// The projections are HBM-bound GEMVs split over 512-column slices: every
// 16-byte weight load of a lane serves all the batch's tokens, whose slice
// (16 KiB at 8 tokens) sits in LDS, and the consumer adds the slices.
// Attention streams the cache once: one block per (position split, KV head,
// token) reads 128 positions of K and V (256 bytes each per head) and serves
// every query head of that KV head.
#include "jm_device.h"
#include "jm_kernels.h"

namespace jm {

// ------------------------------------------------------------------ GEMV

// Partial products of column slices: part[s][b][row] = sum over the
// columns k of slice s of W[row][k] * x[b][k] (* norm_w[k]), rows of the
// stacked matrices w[0..2], on the matrix cores.  Block (row group, slice,
// group of 8 tokens): WV waves of 16 rows.  v_mfma_f32_16x16x32_bf16 with
// the weight rows as the A operand straight from memory (lane l: row
// row0 + l % 16, columns 32 ks + 8 (l / 16) .. + 7, one 16-byte load per
// k-step, all requested first) and the tokens as B columns: column n < 8
// holds bf16(x) of token n, column n + 8 the rest bf16(x - bf16(x)); the
// block stages them in LDS in operand order.  Columns n and n ^ 8 of the
// product (one DPP move) add up to the token's dot product at float32-level
// accuracy.  The consumer sums the slices (and applies the RMSNorm row
// scale), so that a projection spreads over hundreds of waves.
template <int SW, int WV>
__global__ void __launch_bounds__(WV * 64)
k_gemv_part(GemvArgs a) {
    constexpr int NK = SW / 32;                    // k-steps
    __shared__ __align__(16) uint4 xb[NK][64];     // B operands, [k-step][lane]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    const int slice = blockIdx.y, tb0 = blockIdx.z * 8;
    const int row0 = (blockIdx.x * WV + w) * 16;
    const int k0 = slice * SW;
    const bool live = row0 < a.N;                  // wave-uniform
    // this wave's rows (a 16-row tile lies in one matrix: rows[i] % 16 == 0)
    const int row = live ? row0 + n : 0;
    const uint16_t* wr;
    if (row < a.rows[0]) wr = a.w[0] + (size_t)row * a.K;
    else if (row < a.rows[0] + a.rows[1]) wr = a.w[1] + (size_t)(row - a.rows[0]) * a.K;
    else wr = a.w[2] + (size_t)(row - a.rows[0] - a.rows[1]) * a.K;
    const uint16_t* wp = wr + k0 + 8 * g;
    // requests first: the tokens' slice (needed first; thread tid serves
    // token tb0 + tid % 8 throughout), then the weight rows
    constexpr int NI = NK * 32;                    // staging items (8 columns of one token)
    constexpr int XI = (NI + WV * 64 - 1) / (WV * 64);     // per thread, the last one partial
    static_assert((WV * 64) % 8 == 0, "token fixed per thread");
    const int tx = tid & 7;
    const bool tin = tb0 + tx < a.B;
    float4 xv[XI][2];
    uint4 nwv[XI];
#pragma unroll
    for (int it = 0; it < XI; it++) {
        const int i = (tid + it * WV * 64) % NI;   // items past NI repeat one (same token), not stored
        const int c = k0 + 32 * (i >> 5) + 8 * ((i >> 3) & 3);
        const float4* xp = (const float4*)(a.x + (size_t)(tin ? tb0 + tx : tb0) * a.K + c);
        xv[it][0] = xp[0];
        xv[it][1] = xp[1];
        if (a.norm_w) nwv[it] = *(const uint4*)(a.norm_w + c);
    }
    uint4 wa[NK];
#pragma unroll
    for (int ks = 0; ks < NK; ks++) wa[ks] = *(const uint4*)(wp + 32 * ks);
    __builtin_amdgcn_sched_barrier(0);             // keep every request ahead of the staging
    // the tokens' slice (times the norm weight), split into hi and lo
    // columns; with a.rss the first row group's blocks also sum the squares
    // of the slice (before the norm weight) per token
    __shared__ float ssw[WV][8];
    const bool want_ss = a.rss && blockIdx.x == 0;    // block-uniform
    float ss = 0.0f;
#pragma unroll
    for (int it = 0; it < XI; it++) {
        const int i = tid + it * WV * 64;
        if (NI % (WV * 64) != 0 && i >= NI) break;         // the partial last item of the thread
        const int ks = i >> 5, gg = (i >> 3) & 3;
        float v[8] = {xv[it][0].x, xv[it][0].y, xv[it][0].z, xv[it][0].w,
                      xv[it][1].x, xv[it][1].y, xv[it][1].z, xv[it][1].w};
        if (tin) {
#pragma unroll
            for (int e = 0; e < 8; e++) ss = __builtin_fmaf(v[e], v[e], ss);
            if (a.norm_w) {
                const uint32_t nn[4] = {nwv[it].x, nwv[it].y, nwv[it].z, nwv[it].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    v[2 * e] = __fmul_rn(v[2 * e], bf16_bits_to_f32(nn[e] & 0xFFFFu));
                    v[2 * e + 1] = __fmul_rn(v[2 * e + 1], bf16_bits_to_f32(nn[e] >> 16));
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = 0.0f;
        }
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int e = 0; e < 4; e++) split_bf16x2(v[2 * e], v[2 * e + 1], hi[e], lo[e]);
        xb[ks][16 * gg + tx] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        xb[ks][16 * gg + 8 + tx] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    }
    if (want_ss) {
        // lanes with equal lane % 8 serve one token
        ss = __fadd_rn(ss, __shfl_xor(ss, 8, JM_WAVE));
        ss = __fadd_rn(ss, __shfl_xor(ss, 16, JM_WAVE));
        ss = __fadd_rn(ss, __shfl_xor(ss, 32, JM_WAVE));
        if (lane < 8) ssw[w][lane] = ss;
    }
    __syncthreads();
    if (want_ss && tid < 8 && tb0 + tid < a.B) {
        float t = ssw[0][tid];
#pragma unroll
        for (int u = 1; u < WV; u++) t = __fadd_rn(t, ssw[u][tid]);
        a.rss[(size_t)slice * a.B + tb0 + tid] = t;
    }
    if (!live) return;

    // two accumulators break the dependence chain of the k-steps
    floatx4 acc[2] = {floatx4{0.0f, 0.0f, 0.0f, 0.0f}, floatx4{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
    for (int ks = 0; ks < NK; ks++)
        acc[ks & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wa[ks]),
                                                              __builtin_bit_cast(bf16x8, xb[ks][lane]),
                                                              acc[ks & 1], 0, 0, 0);
    // lane (g, n): rows row0 + 4 g + i of column n; token n = hi + lo columns
    float tot[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float c = __fadd_rn(acc[0][i], acc[1][i]);
        tot[i] = __fadd_rn(c, dpp_f<DPP_ROR8>(c));
    }
    if (n < 8 && tb0 + n < a.B)
        *(float4*)(a.part + ((size_t)slice * a.B + tb0 + n) * a.N + row0 + 4 * g) =
            make_float4(tot[0], tot[1], tot[2], tot[3]);
}

// ------------------------------------------------------------------ GEMM
//
// The same product for many tokens at once (a prefill chunk): part[0][b][row]
// = sum over all K columns of W[row][k] * x[b][k] (* norm_w[k]), one output
// slice.  Block (128-row tile, 64-token tile), 8 waves: 2 token halves x 4
// row quarters of 32, each wave a 32 x 32 tile by v_mfma_f32_32x32x16_bf16
// with the tokens on the A side (split into bf16 hi and lo, two products
// per k-step, as the GEMV splits them) and the weight rows on the B side.
// Operands go through LDS in 64-column stages, two stages streaming into
// registers while the stage in LDS is multiplied.  Lane layout as the dense
// expert branch's: A[i][k] at lane i % 32, k = 8 (l / 32) + j; B[k][n] at
// lane n % 32, k = 8 (l / 32) + j; D register v of lane l = (i = 8 (v / 4)
// + 4 (l / 32) + v % 4, n = l % 32).  Each weight byte crosses HBM once per
// token tile instead of once per 8 tokens.
constexpr int GM_T = 64;            // tokens per block
constexpr int GM_R = 128;           // weight rows per block
constexpr int GM_KS = 64;           // columns per stage
constexpr int GM_KP = GM_KS + 8;    // padded LDS row, in bf16 (144 bytes: 16-byte aligned, bank-spread)

struct GmStage {
    float4 x0, x1;                  // 8 columns of one token
    uint4 nw;                       // their norm weights (bf16)
    uint4 w[2];                     // 2 x 8 columns of weight rows
    int s;                          // the stage (before clamping to the last one)
};

__global__ void __launch_bounds__(512, 1)
k_gemm_bf16(GemvArgs a) {
    typedef float floatx16 __attribute__((ext_vector_type(16)));
    __shared__ __align__(16) uint16_t xh[2][GM_T * GM_KP], xl[2][GM_T * GM_KP], wl[2][GM_R * GM_KP];
    __shared__ float ss_l[GM_T][8];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    // the first row tile also sums each token's squares (the RMSNorm of the
    // layer input, for the consumer) from the values it stages
    const bool want_ss = a.rss && blockIdx.x == 0;
    float ss = 0.0f;
    const int row0 = blockIdx.x * GM_R, tb0 = blockIdx.y * GM_T;
    // block z takes the z-th of gridDim.z equal column ranges and writes
    // slice z of part (and of rss)
    const int K = a.K, nstage = K / GM_KS / (int)gridDim.z, kz = blockIdx.z;
    const int kcol0 = kz * nstage * GM_KS;
    // the 128-row tile lies in one matrix (row counts are multiples of 128)
    const uint16_t* wm;
    int wr0;
    if (row0 < a.rows[0]) { wm = a.w[0]; wr0 = row0; }
    else if (row0 < a.rows[0] + a.rows[1]) { wm = a.w[1]; wr0 = row0 - a.rows[0]; }
    else { wm = a.w[2]; wr0 = row0 - a.rows[0] - a.rows[1]; }
    // staging: token xt, columns 8 xp .. 8 xp + 7; weight rows wrw and
    // wrw + 64, columns 8 wp .. 8 wp + 7
    const int xt = tid >> 3, xp = tid & 7;
    const int wrw = tid >> 3, wp = tid & 7;
    const bool xlive = tb0 + xt < a.B;
    const float* xrow = a.x + (size_t)(xlive ? tb0 + xt : 0) * K + kcol0 + 8 * xp;
    const uint16_t* wp0 = wm + (size_t)(wr0 + wrw) * K + kcol0 + 8 * wp;
    const uint16_t* wp1 = wp0 + (size_t)64 * K;

    // every load is unconditional (past the last stage: the last stage again)
    auto load_stage = [&](GmStage& r, int s) __attribute__((always_inline)) {
        r.s = s;
        s = s < nstage ? s : nstage - 1;
        const float4* xs = (const float4*)(xrow + s * GM_KS);
        r.x0 = xs[0];
        r.x1 = xs[1];
        if (a.norm_w) r.nw = *(const uint4*)(a.norm_w + kcol0 + s * GM_KS + 8 * xp);
        r.w[0] = *(const uint4*)(wp0 + s * GM_KS);
        r.w[1] = *(const uint4*)(wp1 + s * GM_KS);
    };
    auto store_stage = [&](const GmStage& r, int buf) __attribute__((always_inline)) {
        float v[8] = {r.x0.x, r.x0.y, r.x0.z, r.x0.w, r.x1.x, r.x1.y, r.x1.z, r.x1.w};
        if (want_ss && r.s < nstage) {
#pragma unroll
            for (int e = 0; e < 8; e++) ss = __builtin_fmaf(v[e], v[e], ss);
        }
        if (a.norm_w) {
            const uint32_t nn[4] = {r.nw.x, r.nw.y, r.nw.z, r.nw.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                v[2 * e] = __fmul_rn(v[2 * e], bf16_bits_to_f32(nn[e] & 0xFFFFu));
                v[2 * e + 1] = __fmul_rn(v[2 * e + 1], bf16_bits_to_f32(nn[e] >> 16));
            }
        }
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int e = 0; e < 4; e++) split_bf16x2(v[2 * e], v[2 * e + 1], hi[e], lo[e]);
        const unsigned keep = xlive ? 0xFFFFFFFFu : 0u;     // tokens past B stage zeros
        *(uint4*)&xh[buf][xt * GM_KP + 8 * xp] = make_uint4(hi[0] & keep, hi[1] & keep, hi[2] & keep, hi[3] & keep);
        *(uint4*)&xl[buf][xt * GM_KP + 8 * xp] = make_uint4(lo[0] & keep, lo[1] & keep, lo[2] & keep, lo[3] & keep);
        *(uint4*)&wl[buf][wrw * GM_KP + 8 * wp] = r.w[0];
        *(uint4*)&wl[buf][(wrw + 64) * GM_KP + 8 * wp] = r.w[1];
    };

    const int th = w & 1, rq = w >> 1;            // this wave's token half and row quarter
    const int ai = th * 32 + (lane & 31), bn = rq * 32 + (lane & 31), kq = 8 * (lane >> 5);
    floatx16 acc = {};
    auto mfma_stage = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int k2 = 0; k2 < GM_KS / 16; k2++) {
            const int k0 = k2 * 16 + kq;
            const bf16x8 a_h = *(const bf16x8*)&xh[buf][ai * GM_KP + k0];
            const bf16x8 a_l = *(const bf16x8*)&xl[buf][ai * GM_KP + k0];
            const bf16x8 b = *(const bf16x8*)&wl[buf][bn * GM_KP + k0];
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_h, b, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_l, b, acc, 0, 0, 0);
        }
    };
    // stages s + 1 and s + 2 stream into registers while stage s (in LDS) is
    // multiplied; nstage is even
    GmStage r0, r1;
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
    const int n = row0 + bn;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int t = tb0 + th * 32 + 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
        if (t < a.B) a.part[((size_t)kz * a.B + t) * a.N + n] = acc[v];
    }
    if (want_ss) {
        ss_l[xt][xp] = ss;
        __syncthreads();
        if (tid < GM_T && tb0 + tid < a.B) {
            float t = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) t = __fadd_rn(t, ss_l[tid][i]);
            a.rss[(size_t)kz * a.B + tb0 + tid] = t;
        }
    }
}

bool gemm_shape_ok(const GemvArgs& a) {
    return a.K % (2 * GM_KS) == 0 && a.rows[0] % GM_R == 0 && a.rows[1] % GM_R == 0 && a.rows[2] % GM_R == 0;
}

static int device_cus() {
    static int ncu = 0;
    if (ncu == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
            ncu = 256;
    }
    return ncu;
}

// Column ranges (K slices) of the GEMM, 1, 2 or 4: one block per CU runs at
// a time, so a grid of (N / 128) x (B / 64) tiles that leaves CUs idle in
// its last round is split along K into more, shorter blocks.  Time is
// modelled as rounds x (1 / slices + 0.15), the constant a block's fixed
// part (prologue, output stores); ties keep fewer slices (fewer partial
// outputs to write and sum).
int gemm_slices(const GemvArgs& a) {
    const int ncu = device_cus();
    const long long tiles = (long long)(a.N / GM_R) * ((a.B + GM_T - 1) / GM_T);
    const int nstage = a.K / GM_KS;
    int best = 1;
    double best_t = 1e30;
    for (int kz : {1, 2, 4}) {
        if (nstage % (2 * kz) != 0) continue;
        const long long rounds = (tiles * kz + ncu - 1) / ncu;
        const double t = (double)rounds * (1.0 / kz + 0.15);
        if (t < best_t - 1e-9) {
            best_t = t;
            best = kz;
        }
    }
    return best;
}

hipError_t launch_gemm_bf16(const GemvArgs& a, hipStream_t st) {
    if (a.B == 0 || a.N == 0) return hipSuccess;
    if (!gemm_shape_ok(a)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)(a.N / GM_R), (unsigned)((a.B + GM_T - 1) / GM_T), (unsigned)gemm_slices(a));
    hipLaunchKernelGGL(k_gemm_bf16, grid, dim3(512), 0, st, a);
    return hipGetLastError();
}

bool gemv_shape_ok(int K) { return K > 0 && K % 1024 == 0 && K <= 8192; }

int gemv_slice_cols(int K) { return K >= 4096 && K % 1024 == 0 ? 1024 : 512; }

// Waves per block (16 rows each) of a projection: the one of 5, 4 and 2
// whose grid fills its last round of the CUs best (one block per CU and
// round), the larger on ties.  A grid of 1.25 rounds (320 blocks on 256
// CUs) leaves the CUs with two blocks to set the time.
static int gemv_waves(int N, int slices, int zgroups) {
    const int ncu = device_cus();
    int best = 4;
    double best_eff = -1.0;
    for (int wv : {5, 4, 2}) {
        const long long nb = (long long)((N + 16 * wv - 1) / (16 * wv)) * slices * zgroups;
        const long long rounds = (nb + ncu - 1) / ncu;
        const double eff = (double)nb / (double)(rounds * ncu);
        if (eff > best_eff + 1e-9) {
            best_eff = eff;
            best = wv;
        }
    }
    return best;
}

hipError_t launch_gemv_part(const GemvArgs& a, hipStream_t st) {
    if (a.B == 0 || a.N == 0) return hipSuccess;
    if (a.rows[0] % 16 || a.rows[1] % 16 || a.rows[2] % 16) return hipErrorInvalidValue;
    const int sw = gemv_slice_cols(a.K);
    const int zg = (a.B + 7) / 8;
    const int wv = gemv_waves(a.N, a.K / sw, zg);
    const dim3 grid((unsigned)((a.N + 16 * wv - 1) / (16 * wv)), (unsigned)(a.K / sw), (unsigned)zg);
#define JM_GV(SWV, WVV) hipLaunchKernelGGL((k_gemv_part<SWV, WVV>), grid, dim3(WVV * 64), 0, st, a)
    if (sw == 1024) {
        if (wv == 5) JM_GV(1024, 5);
        else if (wv == 2) JM_GV(1024, 2);
        else JM_GV(1024, 4);
    } else {
        if (wv == 5) JM_GV(512, 5);
        else if (wv == 2) JM_GV(512, 2);
        else JM_GV(512, 4);
    }
#undef JM_GV
    return hipGetLastError();
}

// ------------------------------------------------------------- attention

// Partial sums over 16 lanes of QPK per-head dot products; head h's total
// ends in the lanes j (= lane % 16) with j / (16 / QPK) == h.
template <int QPK>
__device__ __forceinline__ float head_reduce16(float (&v)[QPK]) {
    if constexpr (QPK == 8) {
        transpose_level<8, 8>(v);
        transpose_level<4, 4>(v);
        const bool hi = (threadIdx.x & 2) != 0;
        const float keep = hi ? v[1] : v[0], send = hi ? v[0] : v[1];
        float t = __fadd_rn(keep, dpp_f<DPP_XOR2>(send));
        return __fadd_rn(t, dpp_f<DPP_XOR1>(t));
    } else {
        return transpose_reduce<16, QPK>(v);
    }
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_round(float f) { return __uint_as_float(f32_to_bf16_rne(f) << 16); }

// Four consecutive projection values of one token (rows row .. row + 3 of
// the stacked q, k, v outputs, dimensions 4 j .. 4 j + 3 of one head) with
// everything their finish reads, requested together: the first
// min(nslice, 4) column slices, the slices' sums of squares of h, the bias,
// the per-head norm weight and the RoPE factors at pos.
struct Fin4 {
    float4 sl[4];
    float rs[4];
    float4 bias;
    uint2 nw;
    float4 c, sn;
};

__device__ __forceinline__ void fin4_load(Fin4& f, const AttnArgs& a, int b, int row, const float* bias, int brow,
                                          const uint16_t* nw, bool rope, int pos, int j) {
    constexpr int HD = 128;
    const int ns = a.nslice < 4 ? a.nslice : 4;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int sl = u < ns ? u : 0;          // clamped: the select in fin4_value drops it
        f.sl[u] = *(const float4*)(a.qkv + ((size_t)sl * a.B + b) * a.nqkv + row);
        f.rs[u] = a.rss[(size_t)sl * a.B + b];
    }
    f.bias = bias ? *(const float4*)(bias + brow) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    f.nw = nw ? *(const uint2*)(nw + 4 * j) : make_uint2(0u, 0u);
    if (rope) {
        const size_t ci = (size_t)pos * HD + 4 * (j & 15);
        f.c = *(const float4*)(a.cos + ci);
        f.sn = *(const float4*)(a.sin + ci);
    }
}

// The norm weight of q head (isq) or k head `head` of the layer: per head,
// the one [128] vector; over the whole vector, the head's 128 entries.
__device__ __forceinline__ const uint16_t* qk_weight(const AttnArgs& a, bool isq, int head) {
    const uint16_t* w = isq ? a.qn : a.kn;
    if (!w) return nullptr;
    return a.qk_norm == 2 ? w + (size_t)head * 128 : w;
}

// The four values finished (decode_kernel.c:1126-1199): the column slices
// summed in slice order, times the RMSNorm row scale of h (the projections
// were taken of h * norm weight), plus the bias; then, for a q or k head,
// the QK-norm with weight nw (norm 1: the head's RMSNorm, :1174-1189;
// norm 2: the whole vector's, with its sum of squares from k_qk_ss,
// :1155-1167) and RoPE rotate-half at
// pos (:1190-1194, :259-266) over the aligned 32-lane segment that holds
// the head (lane j: dimensions 4 j .. 4 j + 3; dim i pairs with i + 64,
// i.e. lane j with j ^ 16; first half a cos - b sin, second a sin + b cos).
__device__ __forceinline__ void fin4_value(float (&v)[4], const Fin4& f, const AttnArgs& a, int b, int row,
                                           int norm, bool rope, int j) {
    constexpr int HD = 128;
    const int ns = a.nslice < 4 ? a.nslice : 4;
    float4 acc = f.sl[0];
    float ss = f.rs[0];
#pragma unroll
    for (int u = 1; u < 4; u++) {
        const bool in = u < ns;
        acc.x = in ? __fadd_rn(acc.x, f.sl[u].x) : acc.x;
        acc.y = in ? __fadd_rn(acc.y, f.sl[u].y) : acc.y;
        acc.z = in ? __fadd_rn(acc.z, f.sl[u].z) : acc.z;
        acc.w = in ? __fadd_rn(acc.w, f.sl[u].w) : acc.w;
        ss = in ? __fadd_rn(ss, f.rs[u]) : ss;
    }
    for (int sl = 4; sl < a.nslice; sl++) {     // wider inputs (d = 3072, 8192): the rest of the slices
        const float4 t = *(const float4*)(a.qkv + ((size_t)sl * a.B + b) * a.nqkv + row);
        acc.x = __fadd_rn(acc.x, t.x);
        acc.y = __fadd_rn(acc.y, t.y);
        acc.z = __fadd_rn(acc.z, t.z);
        acc.w = __fadd_rn(acc.w, t.w);
        ss = __fadd_rn(ss, a.rss[(size_t)sl * a.B + b]);
    }
    const float inv = rms_inv(ss, a.d, a.eps);
    v[0] = __fadd_rn(__fmul_rn(acc.x, inv), f.bias.x);
    v[1] = __fadd_rn(__fmul_rn(acc.y, inv), f.bias.y);
    v[2] = __fadd_rn(__fmul_rn(acc.z, inv), f.bias.z);
    v[3] = __fadd_rn(__fmul_rn(acc.w, inv), f.bias.w);
    if (norm) {
        float hinv;
        if (norm == 1) {
            float sq = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++) sq = __builtin_fmaf(v[e], v[e], sq);
            // the reference sums the head's squares in dimension order; the
            // tree here changes the sum by rounding only
            hinv = rms_inv(seg_sum<32>(sq), HD, a.eps);
        } else {
            const bool isq = row < a.H * HD;
            hinv = rms_inv(a.qkss[(size_t)b * 2 + (isq ? 0 : 1)], (isq ? a.H : a.KH) * HD, a.eps);
        }
        const uint32_t nn[4] = {f.nw.x & 0xFFFFu, f.nw.x >> 16, f.nw.y & 0xFFFFu, f.nw.y >> 16};
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = __fmul_rn(__fmul_rn(v[e], hinv), bf16_bits_to_f32(nn[e]));
    }
    if (rope) {
        const bool lo = j < 16;
        const float c[4] = {f.c.x, f.c.y, f.c.z, f.c.w}, sn[4] = {f.sn.x, f.sn.y, f.sn.z, f.sn.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float other = __shfl_xor(v[e], 16, JM_WAVE);
            v[e] = lo ? __builtin_fmaf(v[e], c[e], -__fmul_rn(other, sn[e]))
                      : __builtin_fmaf(other, sn[e], __fmul_rn(v[e], c[e]));
        }
    }
}

// The k and v rows of one KV head of one token, for one wave: lanes 0..31
// the k head (norm, RoPE), lanes 32..63 the v head.
struct KvFin {
    Fin4 f;
    int row;
    bool isk;
};

__device__ __forceinline__ void kv_load(KvFin& k, const AttnArgs& a, int b, int kh, int pos, int lane) {
    constexpr int HD = 128;
    k.isk = lane < 32;
    const int j = lane & 31;
    k.row = (k.isk ? a.H + kh : a.H + a.KH + kh) * HD + 4 * j;
    fin4_load(k.f, a, b, k.row, k.isk ? a.bk : a.bv, kh * HD + 4 * j, k.isk ? qk_weight(a, false, kh) : nullptr,
              k.isk, pos, j);
}

// Finished and appended to the token's caches kc, vc at pos (:1195-1199);
// with kvn, also kept there (kvn[0]: k, kvn[1]: v, bf16).
__device__ __forceinline__ void kv_store(const KvFin& k, const AttnArgs& a, int b, int kh, int pos, int lane,
                                         gptr<uint16_t> kc, gptr<uint16_t> vc, uint16_t (*kvn)[128]) {
    constexpr int HD = 128;
    const int j = lane & 31;
    float v[4];
    fin4_value(v, k.f, a, b, k.row, k.isk && a.kn ? a.qk_norm : 0, k.isk, j);
    uint16_t hb4[4];
#pragma unroll
    for (int e = 0; e < 4; e++) hb4[e] = (uint16_t)f32_to_bf16_rne(v[e]);
    if (kvn) {
#pragma unroll
        for (int e = 0; e < 4; e++) kvn[k.isk ? 0 : 1][4 * j + e] = hb4[e];
    }
    const gptr<uint16_t> dst = (k.isk ? kc : vc) + ((size_t)pos * a.KH + kh) * HD + 4 * j;
    *(uint2*)dst = make_uint2(hb4[0] | ((uint32_t)hb4[1] << 16), hb4[2] | ((uint32_t)hb4[3] << 16));
}

// The whole-vector QK-norm (decode_kernel.c:1155-1167) needs each token's
// sum of squares over all of q (H * 128 values) and all of k (KH * 128)
// before the attention blocks, which finish one KV head each, can scale
// their heads.  One block per token finishes every q and k value as
// fin4_value does (slices, row scale, bias: the same bits) and sums the
// squares; qkss[b] = (q sum, k sum).
__global__ void __launch_bounds__(256)
k_qk_ss(AttnArgs a) {
    constexpr int HD = 128;
    __shared__ float red[2][4];
    const int b = blockIdx.x, tid = threadIdx.x;
    const int nq = a.H * HD / 4, nqk = (a.H + a.KH) * HD / 4;   // float4 groups of q, of q and k
    float sq = 0.0f, sk = 0.0f;
    for (int u = tid; u < nqk; u += 256) {
        const bool isq = u < nq;
        const int row = 4 * u;                    // q rows, then the k rows, as stacked in qkv
        Fin4 f;
        fin4_load(f, a, b, row, isq ? a.bq : a.bk, isq ? row : row - a.H * HD, nullptr, false, 0, 0);
        float v[4];
        fin4_value(v, f, a, b, row, 0, false, 0);
        float t = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) t = __builtin_fmaf(v[e], v[e], t);
        if (isq) sq = __fadd_rn(sq, t);
        else sk = __fadd_rn(sk, t);
    }
    sq = seg_sum<64>(sq);
    sk = seg_sum<64>(sk);
    if ((tid & 63) == 0) {
        red[0][tid >> 6] = sq;
        red[1][tid >> 6] = sk;
    }
    __syncthreads();
    if (tid < 2) a.qkss[(size_t)b * 2 + tid] = __fadd_rn(__fadd_rn(red[tid][0], red[tid][1]),
                                                         __fadd_rn(red[tid][2], red[tid][3]));
}

// The same for float32 caches (the reference's KVCache type): the finished
// values are appended as they are; with kvf, also kept there (kvf[0]: k,
// kvf[1]: v).
__device__ __forceinline__ void kv_store_f32(const KvFin& k, const AttnArgs& a, int b, int kh, int pos, int lane,
                                             gptr<float> kc, gptr<float> vc, float (*kvf)[128]) {
    constexpr int HD = 128;
    const int j = lane & 31;
    float v[4];
    fin4_value(v, k.f, a, b, k.row, k.isk && a.kn ? a.qk_norm : 0, k.isk, j);
    const f32x4_t v4 = f32x4_t{v[0], v[1], v[2], v[3]};
    if (kvf) *(f32x4_t*)&kvf[k.isk ? 0 : 1][4 * j] = v4;
    const gptr<float> dst = (k.isk ? kc : vc) + ((size_t)pos * a.KH + kh) * HD + 4 * j;
    *(gptr<f32x4_t>)dst = v4;
}

// For a batch whose tokens may share a cache (a prefill chunk: the
// positions of one prompt), every token's k and v rows are appended before
// the attention reads the caches: one wave per (KV head, token).
template <bool F32>
__global__ void __launch_bounds__(64)
k_kv_append(AttnArgs a) {
    const int kh = blockIdx.x, b = blockIdx.y;
    const int pos = a.pos[b];
    const unsigned long long* kvp = a.kv + ((size_t)b * a.L + a.layer) * 2;
    KvFin k;
    kv_load(k, a, b, kh, pos, threadIdx.x);
    if (F32) kv_store_f32(k, a, b, kh, pos, threadIdx.x, (gptr<float>)kvp[0], (gptr<float>)kvp[1], nullptr);
    else kv_store(k, a, b, kh, pos, threadIdx.x, (gptr<uint16_t>)kvp[0], (gptr<uint16_t>)kvp[1], nullptr);
}

// The 4 waves' partial outputs of a split block (wave w's at red + w *
// wstride, [QPK][128]) merged with the split's max (the flash-decoding
// merge within the block) into part_o / part_ml:
// thread tid takes head tid / 32, dimensions 4 (tid % 32) .. + 3, so that
// each thread forms the 4 waves' factors of one head once.
template <int QPK>
__device__ __forceinline__ void merge_waves(const AttnArgs& a, int b, int kh, int s, const float* red, int wstride,
                                            const float (*mls)[QPK][2]) {
    constexpr int HD = 128;
    const int tid = threadIdx.x;
    float* po = a.part_o + (((size_t)b * a.KH + kh) * a.S + s) * QPK * HD;
    {
        const int h = tid >> 5, oi = h * HD + 4 * (tid & 31);
        if (h < QPK) {
            const float M = fmaxf(fmaxf(mls[0][h][0], mls[1][h][0]), fmaxf(mls[2][h][0], mls[3][h][0]));
            float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float L = 0.0f;
#pragma unroll
            for (int ww = 0; ww < 4; ww++) {
                const float m = mls[ww][h][0];
                const float f = m == -INFINITY ? 0.0f : expf_fast(__fsub_rn(m, M));
                const float4 r = *(const float4*)&red[(size_t)ww * wstride + oi];
                O.x = __builtin_fmaf(r.x, f, O.x);
                O.y = __builtin_fmaf(r.y, f, O.y);
                O.z = __builtin_fmaf(r.z, f, O.z);
                O.w = __builtin_fmaf(r.w, f, O.w);
                L = __builtin_fmaf(mls[ww][h][1], f, L);
            }
            *(float4*)(po + oi) = O;
            if ((tid & 31) == 0) {
                float* ml = a.part_ml + ((((size_t)b * a.KH + kh) * a.S + s) * QPK + h) * 2;
                ml[0] = M;
                ml[1] = L;
            }
        }
    }
}

// One (position split, KV head, token): QPK query heads over positions
// [128 s, 128 s + 128) of the token's T = pos + 1 cache rows (the row at pos
// finished and appended here), on the matrix cores.  Wave w takes 32 positions
// tw = 128 s + 32 w .. tw + 31 and all 128 head dimensions.
//
// Scores (:1205-1211) by v_mfma_f32_16x16x32_bf16 with the cached K rows
// as the A operand straight from memory (lane l: row tw + 16 mt + l % 16,
// dimensions 32 kk + 8 (l / 16) .. + 7, one 16-byte load) and the query
// heads as B columns: column n < 8 holds bf16(q) of head n, column n + 8 the
// rest bf16(q - bf16(q)) (split in the prologue), so the two columns' sum
// carries 16 significant bits of q against the exact bf16 keys, accumulated
// in fp32.  The sum of
// columns n and n ^ 8 (one DPP move) is the score of head n % 8 at the 4
// positions tw + 16 mt + 4 (l / 16) + i of the lane's accumulator.
//
// Softmax numerators over the wave's 32 positions with the wave's own max
// (:1212-1214), then P . V (:1215-1221) with P as the A operand: row n holds
// head n % 8's weights split the same way (bf16(p) for n < 8, the rest for
// n >= 8), already in the lanes that computed them; the contraction index
// j of lane group g is position 16 (j / 4) + 4 g + j % 4.  V goes through
// LDS (one row per position, 264 bytes, so that the 4 lane groups' reads
// fall in different banks) and is read back per column as the B operand.
// Rows m and m + 8 of the product (lanes l and l ^ 32) are added by one
// transposing step.  The 4 waves' partial outputs are merged with the
// split's max, as the split merge does across splits.
template <int QPK>
__global__ void __launch_bounds__(256)
k_attn_part(AttnArgs a) {
    constexpr int HD = 128, P = 128, PW = 32, VR = 132;
    // Each wave's V rows, then (its own region, once its last P.V read is
    // issued: a wave's LDS operations complete in order) its outputs for the
    // merge.  Until every wave has read them (the barrier after the query
    // columns), the start holds the finished query heads (bf16 hi, lo) and
    // the token's own k and v row (the split that holds it).  34 KB per
    // block: the 544 blocks of an 8-token step at 2049 positions are
    // resident at once (with a separate 16 KB output buffer, two blocks fit
    // a CU and the last 32 ran as a second round).
    __shared__ __align__(16) uint16_t vt[4][PW * VR];
    __shared__ float mls[4][QPK][2];                    // each wave's (max, sum)
    constexpr int RSTRIDE = PW * VR / 2;                // floats between the waves' output regions
    static_assert(QPK * HD <= RSTRIDE, "a wave's outputs fit its V region");
    static_assert(QPK * 2 * HD * 2 + 2 * HD * 2 <= sizeof(vt), "prologue fits the V rows' space");
    float* const red0 = (float*)&vt[0][0];
    uint16_t (*qs)[2][HD] = (uint16_t (*)[2][HD])&vt[0][0];
    uint16_t (*kvn)[HD] = (uint16_t (*)[HD])((char*)&vt[0][0] + QPK * 2 * HD * 2);
    const int kh = blockIdx.x, b = blockIdx.y, s = (int)gridDim.z - 1 - (int)blockIdx.z;
    const int pos = a.pos[b];
    const int T = pos + 1;
    const int t0 = s * P;
    if (t0 >= T) return;                 // past this token's positions (block-uniform)
    // this split holds the token's own row and appends it (block-uniform);
    // without a.append the rows were appended by k_kv_append
    const bool own = a.append && pos < t0 + P;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    const int tw = t0 + PW * w;
    const unsigned long long* kvp = a.kv + ((size_t)b * a.L + a.layer) * 2;
    const gptr<const uint16_t> kc = (gptr<const uint16_t>)kvp[0];
    const gptr<const uint16_t> vc = (gptr<const uint16_t>)kvp[1];
    // requests first, in the order of use: the inputs of the block's
    // query heads and (wave 0 of the split holding the token's row) of its
    // k and v rows, then the K rows, then the V rows (unconditional: row 0
    // past the end; the token's own row, not yet in the cache, is replaced
    // below).  The projections are finished here: every split block
    // finishes its query heads itself; with a.append the split holding the
    // token's row also finishes its k and v, appends them to the cache and
    // uses them in place of the cache row.
    const int qh = tid >> 5, qj = tid & 31;          // query head qh of the block, dimensions 4 qj .. + 3
    const int qrow = (kh * QPK + (qh < QPK ? qh : 0)) * HD + 4 * qj;
    const bool kvw = own && w == 0;                  // wave-uniform
    Fin4 fq;
    fin4_load(fq, a, b, qrow, a.bq, qrow, qk_weight(a, true, kh * QPK + (qh < QPK ? qh : 0)), true, pos, qj);
    KvFin fkv;
    if (kvw) kv_load(fkv, a, b, kh, pos, lane);
    uint4 kr[2][4], vr[8];
#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
        const int t = tw + 16 * mt + n;
        const gptr<const uint16_t> row = kc + ((size_t)(t < T ? t : 0) * a.KH + kh) * HD + 8 * g;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) kr[mt][kk] = load_g16(row + 32 * kk);
    }
    __builtin_amdgcn_sched_barrier(0);      // keep the K requests ahead of the arithmetic
    {
        float v[4];
        fin4_value(v, fq, a, b, qrow, a.qn ? a.qk_norm : 0, true, qj);
        // the V rows once the query's inputs are consumed: the registers
        // they take are the prologue's, so that the kernel stays at 3
        // blocks per CU (the rows arrive while the scores are formed)
#pragma unroll
        for (int jv = 0; jv < 8; jv++) {
            const int t = tw + 4 * jv + g;
            vr[jv] = load_g16(vc + ((size_t)(t < T ? t : 0) * a.KH + kh) * HD + 8 * n);
        }
        if (QPK == 8 || qh < QPK) {                 // whole 32-lane segments
#pragma unroll
            for (int e = 0; e < 4; e++) {
                // split for the matrix cores: hi = bf16(q), lo = bf16(q - hi)
                const uint32_t hi = f32_to_bf16_rne(v[e]);
                qs[qh][0][4 * qj + e] = (uint16_t)hi;
                qs[qh][1][4 * qj + e] = (uint16_t)f32_to_bf16_rne(__fsub_rn(v[e], __uint_as_float(hi << 16)));
            }
        }
        if (kvw) kv_store(fkv, a, b, kh, pos, lane, (gptr<uint16_t>)kc, (gptr<uint16_t>)vc, kvn);
    }
    __syncthreads();
    // the query columns (head n % 8, zero for heads >= QPK; the hi half of
    // the split for n < 8, the lo half above)
    const int hq = n & 7;
    const bool lo_col = n >= 8;
    uint4 qr[4];
#pragma unroll
    for (int kk = 0; kk < 4; kk++)
        qr[kk] = hq < QPK ? *(const uint4*)&qs[hq < QPK ? hq : 0][lo_col ? 1 : 0][8 * g + 32 * kk]
                          : make_uint4(0u, 0u, 0u, 0u);
    if (own) {
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
            if (tw + 16 * mt + n == pos) {
#pragma unroll
                for (int kk = 0; kk < 4; kk++) kr[mt][kk] = *(const uint4*)&kvn[0][8 * g + 32 * kk];
            }
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (tw + 4 * j + g == pos) vr[j] = *(const uint4*)&kvn[1][8 * n];
    }
    __syncthreads();                        // vt is free from here
    bf16x8 qb[4];
#pragma unroll
    for (int kk = 0; kk < 4; kk++) qb[kk] = __builtin_bit_cast(bf16x8, qr[kk]);

    // ---- scores: q . k / sqrtf_fast(hd), as q . k times the divisor's
    // reciprocal (within an ulp of the division)
    floatx4 sacc[2];
#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
        sacc[mt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
            sacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[mt][kk]), qb[kk],
                                                               sacc[mt], 0, 0, 0);
    }
    float sv[8];
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float c = sacc[mt][i];
            const float tot = __fadd_rn(c, dpp_f<DPP_ROR8>(c));
            const int t = tw + 16 * mt + 4 * g + i;
            const float sc = t < T ? __fmul_rn(tot, a.rsdiv) : -INFINITY;
            sv[4 * mt + i] = sc;
            mx = fmaxf(mx, sc);
        }
    // over the lane groups (positions) of the column
    mx = fmaxf(mx, swz_xor16_f(mx));
    mx = fmaxf(mx, __shfl_xor(mx, 32, JM_WAVE));
    const float mref = mx == -INFINITY ? 0.0f : mx;     // a wave wholly past T
    float l = 0.0f;
    uint32_t pp[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float p0 = expf_fast(__fsub_rn(sv[2 * i], mref));
        const float p1 = expf_fast(__fsub_rn(sv[2 * i + 1], mref));
        l = __fadd_rn(__fadd_rn(l, p0), p1);
        uint32_t hi, lo;
        split_bf16x2(p0, p1, hi, lo);
        pp[i] = lo_col ? lo : hi;
    }
    l = __fadd_rn(l, swz_xor16_f(l));
    l = __fadd_rn(l, __shfl_xor(l, 32, JM_WAVE));
    const bf16x8 pa = __builtin_bit_cast(bf16x8, make_uint4(pp[0], pp[1], pp[2], pp[3]));

    // ---- V rows through this wave's LDS rows, read back per column
    uint16_t* vw = vt[w];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        uint2* dst = (uint2*)(vw + (4 * j + g) * VR + 8 * n);
        dst[0] = make_uint2(vr[j].x, vr[j].y);
        dst[1] = make_uint2(vr[j].z, vr[j].w);
    }
    // LDS operations of one wave complete in order; this keeps the compiler
    // from moving the reads above the writes
    __asm__ volatile("" : : : "memory");
    floatx4 oacc[8];
#pragma unroll
    for (int nt = 0; nt < 8; nt++) {
        uint32_t vb[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // two 16-bit reads straight into the low and high halves
            const int j0 = 2 * i, j1 = 2 * i + 1;
            u16x2 e;
            e.x = vw[(16 * (j0 >> 2) + 4 * g + (j0 & 3)) * VR + 16 * nt + n];
            e.y = vw[(16 * (j1 >> 2) + 4 * g + (j1 & 3)) * VR + 16 * nt + n];
            vb[i] = __builtin_bit_cast(uint32_t, e);
        }
        oacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            pa, __builtin_bit_cast(bf16x8, make_uint4(vb[0], vb[1], vb[2], vb[3])),
            floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
    }
    // rows m (hi) and m + 8 (lo) of a head: lanes l and l ^ 32
    float o[32];
#pragma unroll
    for (int nt = 0; nt < 8; nt++)
#pragma unroll
        for (int i = 0; i < 4; i++) o[4 * nt + i] = oacc[nt][i];
    transpose_level<32, 32>(o);
    // now o[4 nt + i] = head 4 (g % 2) + i, dimension 16 (nt + 4 (g / 2)) + n
#pragma unroll
    for (int nt = 0; nt < 4; nt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int hh = 4 * (g & 1) + i;
            if (hh < QPK) red0[(size_t)w * RSTRIDE + hh * HD + 16 * (nt + 4 * (g >> 1)) + n] = o[4 * nt + i];
        }
    if (g == 0 && n < QPK) {
        mls[w][n][0] = mx;
        mls[w][n][1] = l;
    }
    __syncthreads();

    merge_waves<QPK>(a, b, kh, s, red0, RSTRIDE, mls);
}

// The split block over float32 caches, in float32 arithmetic throughout
// (the reference's SDPA, :1200-1222, on its own cache type): the same
// block shape, prologue and partial outputs as k_attn_part, on the vector
// units.  Wave w takes positions tw = 128 s + 32 w .. tw + 31.
//   scores  lane l: position tw + l % 32 and dimensions 64 (l / 32) .. + 63
//           of its K row (16 float4 loads), against the finished query
//           heads in LDS; the two halves' sums added across lanes l, l ^ 32
//   P . V   lane l: dimensions 2 l, 2 l + 1 of the 32 V rows (one float2
//           load per row, a whole row per wave load), the softmax
//           numerators read back from LDS
template <int QPK>
__global__ void __launch_bounds__(256)
k_attn_part_f32(AttnArgs a) {
    constexpr int HD = 128, P = 128, PW = 32;
    __shared__ __align__(16) float qf[QPK][HD];          // the finished query heads
    __shared__ __align__(16) float kvf[2][HD];           // the token's own k and v rows
    __shared__ __align__(16) float pw[4][QPK][PW];       // each wave's softmax numerators
    __shared__ __align__(16) float red[4][QPK * HD];     // each wave's outputs
    __shared__ float mls[4][QPK][2];                     // each wave's (max, sum)
    const int kh = blockIdx.x, b = blockIdx.y, s = (int)gridDim.z - 1 - (int)blockIdx.z;
    const int pos = a.pos[b];
    const int T = pos + 1;
    const int t0 = s * P;
    if (t0 >= T) return;                 // past this token's positions (block-uniform)
    const bool own = a.append && pos < t0 + P;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int pl = lane & 31, hf = lane >> 5;
    const int tw = t0 + PW * w;
    const unsigned long long* kvp = a.kv + ((size_t)b * a.L + a.layer) * 2;
    const gptr<float> kc = (gptr<float>)kvp[0];
    const gptr<float> vc = (gptr<float>)kvp[1];
    // requests first, in the order of use (as k_attn_part): the prologue's
    // inputs, the K rows, the V rows (row 0 past the end)
    const int qh = tid >> 5, qj = tid & 31;
    const int qhc = qh < QPK ? qh : 0;
    const int qrow = (kh * QPK + qhc) * HD + 4 * qj;
    const bool kvw = own && w == 0;                  // wave-uniform
    Fin4 fq;
    fin4_load(fq, a, b, qrow, a.bq, qrow, qk_weight(a, true, kh * QPK + qhc), true, pos, qj);
    KvFin fkv;
    if (kvw) kv_load(fkv, a, b, kh, pos, lane);
    f32x4_t kr[16];
    {
        const int t = tw + pl;
        const gptr<float> row = kc + ((size_t)(t < T ? t : 0) * a.KH + kh) * HD + 64 * hf;
#pragma unroll
        for (int i = 0; i < 16; i++) kr[i] = *(gptr<const f32x4_t>)(row + 4 * i);
    }
    f32x2_t vr[PW];
#pragma unroll
    for (int j = 0; j < PW; j++) {
        const int t = tw + j;
        vr[j] = *(gptr<const f32x2_t>)(vc + ((size_t)(t < T ? t : 0) * a.KH + kh) * HD + 2 * lane);
    }
    __builtin_amdgcn_sched_barrier(0);      // keep every request ahead of the arithmetic
    {
        float v[4];
        fin4_value(v, fq, a, b, qrow, a.qn ? a.qk_norm : 0, true, qj);
        if (qh < QPK) *(float4*)&qf[qh][4 * qj] = make_float4(v[0], v[1], v[2], v[3]);
        if (kvw) kv_store_f32(fkv, a, b, kh, pos, lane, kc, vc, kvf);
    }
    __syncthreads();
    if (own) {
        // the token's own row, not read from the cache (appended above)
        if (tw + pl == pos) {
#pragma unroll
            for (int i = 0; i < 16; i++) kr[i] = *(const f32x4_t*)&kvf[0][64 * hf + 4 * i];
        }
#pragma unroll
        for (int j = 0; j < PW; j++)
            if (tw + j == pos) vr[j] = *(const f32x2_t*)&kvf[1][2 * lane];
    }

    // ---- scores q . k / sqrtf_fast(hd) (as q . k times the divisor's
    // reciprocal), softmax numerators with the wave's own max
    const bool live = tw + pl < T;
    float mx[QPK], lsum[QPK];
#pragma unroll
    for (int h = 0; h < QPK; h++) {
        const float4* q4 = (const float4*)&qf[h][64 * hf];
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float4 q = q4[i];
            acc = __builtin_fmaf(kr[i].x, q.x, acc);
            acc = __builtin_fmaf(kr[i].y, q.y, acc);
            acc = __builtin_fmaf(kr[i].z, q.z, acc);
            acc = __builtin_fmaf(kr[i].w, q.w, acc);
        }
        const float tot = __fadd_rn(acc, __shfl_xor(acc, 32, JM_WAVE));
        const float sc = live ? __fmul_rn(tot, a.rsdiv) : -INFINITY;
        mx[h] = seg_max<32>(sc);
        const float mref = mx[h] == -INFINITY ? 0.0f : mx[h];     // a wave wholly past T
        const float p = expf_fast(__fsub_rn(sc, mref));
        lsum[h] = seg_sum<32>(p);
        if (hf == 0) pw[w][h][pl] = p;
    }
    // LDS operations of one wave complete in order; this keeps the compiler
    // from moving the reads above the writes
    __asm__ volatile("" : : : "memory");

    // ---- P . V over the wave's positions, in position order
    float2 o[QPK];
#pragma unroll
    for (int h = 0; h < QPK; h++) o[h] = make_float2(0.0f, 0.0f);
#pragma unroll
    for (int j4 = 0; j4 < PW / 4; j4++) {
#pragma unroll
        for (int h = 0; h < QPK; h++) {
            const float4 p4 = *(const float4*)&pw[w][h][4 * j4];
            const float pp[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
            for (int u = 0; u < 4; u++) {
                o[h].x = __builtin_fmaf(vr[4 * j4 + u].x, pp[u], o[h].x);
                o[h].y = __builtin_fmaf(vr[4 * j4 + u].y, pp[u], o[h].y);
            }
        }
    }
#pragma unroll
    for (int h = 0; h < QPK; h++) *(float2*)&red[w][h * HD + 2 * lane] = o[h];
    if (lane < QPK) {
        float m = mx[0], l = lsum[0];
#pragma unroll
        for (int h = 1; h < QPK; h++)
            if (lane == h) { m = mx[h]; l = lsum[h]; }
        mls[w][lane][0] = m;
        mls[w][lane][1] = l;
    }
    __syncthreads();
    merge_waves<QPK>(a, b, kh, s, &red[0][0], QPK * HD, mls);
}

// Merge of the splits of one (query head, token): out = sum_s o_s e^(m_s - M)
// / sum_s l_s e^(m_s - M), M the max over the splits.  The splits' weights
// are computed in parallel (128 at a time) and staged in LDS; each thread
// then sums its dimension over them with independent loads.  Up to
// CMB_SR splits (4096 positions), every load is issued first (thread t:
// split t's max and sum, and its dimension of every split), so the merge
// waits for one memory round trip; the sums are the same, in the same order.
constexpr int CMB_SR = 32;

__global__ void __launch_bounds__(128)
k_attn_comb(AttnArgs a, int qpk, float* __restrict__ att) {
    __shared__ float fs[128];
    __shared__ float red[2];
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    const int kh = h / qpk, hq = h % qpk;
    const int ns = (a.pos[b] + 128) / 128;          // splits of T = pos + 1 positions
    const size_t base = ((size_t)b * a.KH + kh) * a.S;
    const float* ml = a.part_ml + (base * qpk + hq) * 2;      // split s at ml[2 qpk s]
    if (ns <= CMB_SR) {
        const float* po = a.part_o + (base * qpk + hq) * 128 + t;
        float pv[CMB_SR];
#pragma unroll
        for (int s = 0; s < CMB_SR; s++) pv[s] = s < ns ? po[(size_t)128 * qpk * s] : 0.0f;
        const float m_t = t < ns ? ml[(size_t)2 * qpk * t] : -INFINITY;
        const float l_t = t < ns ? ml[(size_t)2 * qpk * t + 1] : 0.0f;
        const float mx = seg_max<64>(fmaxf(-INFINITY, m_t));
        if ((t & 63) == 0) red[t >> 6] = mx;
        __syncthreads();
        const float M = fmaxf(red[0], red[1]);
        float f = 0.0f, lsum = 0.0f;
        if (t < ns) {
            f = expf_fast(__fsub_rn(m_t, M));
            lsum = __builtin_fmaf(l_t, f, lsum);
        }
        fs[t] = f;
        __syncthreads();
        float O = 0.0f;
#pragma unroll
        for (int s = 0; s < CMB_SR; s++)
            if (s < ns) O = __builtin_fmaf(pv[s], fs[s], O);
        lsum = seg_sum<64>(lsum);
        if ((t & 63) == 0) red[t >> 6] = lsum;      // every thread read M before the barrier above
        __syncthreads();
        att[((size_t)b * a.H + h) * 128 + t] = __fdiv_rn(O, __fadd_rn(red[0], red[1]));
        return;
    }
    float mx = -INFINITY;
    for (int s = t; s < ns; s += 128) mx = fmaxf(mx, ml[(size_t)2 * qpk * s]);
    mx = seg_max<64>(mx);
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    const float M = fmaxf(red[0], red[1]);
    float lsum = 0.0f, O = 0.0f;
    const float* po = a.part_o + (base * qpk + hq) * 128 + t;  // split s at po[128 qpk s]
    for (int c0 = 0; c0 < ns; c0 += 128) {
        const int s = c0 + t;
        float f = 0.0f;
        if (s < ns) {
            f = expf_fast(__fsub_rn(ml[(size_t)2 * qpk * s], M));
            lsum = __builtin_fmaf(ml[(size_t)2 * qpk * s + 1], f, lsum);
        }
        __syncthreads();
        fs[t] = f;
        __syncthreads();
        const int n = ns - c0 < 128 ? ns - c0 : 128;
#pragma unroll 8
        for (int i = 0; i < n; i++) O = __builtin_fmaf(po[(size_t)128 * qpk * (c0 + i)], fs[i], O);
    }
    lsum = seg_sum<64>(lsum);
    __syncthreads();
    if ((t & 63) == 0) red[t >> 6] = lsum;
    __syncthreads();
    att[((size_t)b * a.H + h) * 128 + t] = __fdiv_rn(O, __fadd_rn(red[0], red[1]));
}

hipError_t launch_attn(const AttnArgs& a, int qpk, float* att, hipStream_t st) {
    if (a.B == 0) return hipSuccess;
    if (a.qk_norm == 2) {
        if (!a.qkss || !a.qn || !a.kn) return hipErrorInvalidValue;
        hipLaunchKernelGGL(k_qk_ss, dim3((unsigned)a.B), dim3(256), 0, st, a);
        hipError_t e0 = hipGetLastError();
        if (e0 != hipSuccess) return e0;
    }
    if (!a.append) {
        if (a.kv_f32) hipLaunchKernelGGL(k_kv_append<true>, dim3((unsigned)a.KH, (unsigned)a.B), dim3(64), 0, st, a);
        else hipLaunchKernelGGL(k_kv_append<false>, dim3((unsigned)a.KH, (unsigned)a.B), dim3(64), 0, st, a);
        hipError_t e0 = hipGetLastError();
        if (e0 != hipSuccess) return e0;
    }
    // Split s of (KV head kh, token b) is block (kh, b, S - 1 - s): the
    // splits are dispatched from the last one, which holds the fewest
    // positions (or none, for a token whose prefix is short).  A block that
    // lands on a CU after others has its first requests served behind
    // theirs; dispatched this way, the blocks that land late are mostly full
    // splits behind light ones rather than full splits behind full ones.
    const dim3 grid((unsigned)a.KH, (unsigned)a.B, (unsigned)a.S);
#define JM_AP(Q) if (a.kv_f32) hipLaunchKernelGGL(k_attn_part_f32<Q>, grid, dim3(256), 0, st, a); \
                 else hipLaunchKernelGGL(k_attn_part<Q>, grid, dim3(256), 0, st, a)
    switch (qpk) {
        case 1: JM_AP(1); break;
        case 2: JM_AP(2); break;
        case 4: JM_AP(4); break;
        case 8: JM_AP(8); break;
        default: return hipErrorInvalidValue;
    }
#undef JM_AP
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_comb, dim3((unsigned)a.H, (unsigned)a.B), dim3(128), 0, st, a, qpk, att);
    return hipGetLastError();
}

// ------------------------------------------------------------ final norm

// out[b] = RMSNorm(x[b]) * w (decode_kernel.c:224-230), one block per token.
__global__ void __launch_bounds__(256)
k_rms_rows(const float* __restrict__ x, const uint16_t* __restrict__ w, int d, float eps,
           float* __restrict__ out) {
    __shared__ float part[4];
    const int b = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + (size_t)b * d;
    float ss = 0.0f;
    for (int i = tid; i < d; i += 256) ss = __builtin_fmaf(xr[i], xr[i], ss);
    ss = seg_sum<64>(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    const float inv = rms_inv(__fadd_rn(__fadd_rn(part[0], part[1]), __fadd_rn(part[2], part[3])), d, eps);
    for (int i = tid; i < d; i += 256)
        out[(size_t)b * d + i] = __fmul_rn(__fmul_rn(xr[i], inv), bf16_bits_to_f32(w[i]));
}

hipError_t launch_rms_rows(const float* x, const uint16_t* w, int B, int d, float eps, float* out,
                           hipStream_t st) {
    if (B == 0) return hipSuccess;
    hipLaunchKernelGGL(k_rms_rows, dim3((unsigned)B), dim3(256), 0, st, x, w, d, eps, out);
    return hipGetLastError();
}

}  // namespace jm
