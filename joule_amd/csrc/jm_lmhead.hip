// The decoder's output end: the lm_head with its argmax, and the embedding
// lookup (decode_kernel.c:964-1062 lm_head_B / lm_head_A, :1597-1600
// embed_lookup).
//
// k_lm_head: logits[b][v] = W[v] . x[b] for 256 rows per block (8 waves x 32
// rows, 4 per iteration, the next iteration's rows requested while the
// current one is multiplied), all of the d columns of up to 8 tokens staged once in
// LDS.  With argmax outputs, each lane keeps the best (value, row) of its
// token over the rows it sees, in increasing row order, and the block writes
// its best per token.  k_argmax_merge merges the blocks' bests.  The argmax
// is lm_head_A's: a row wins only with a strictly larger value than the best
// so far (initial -1e30 at row 0), so ties go to the lowest row and NaN never
// wins; the merges compare (value, row) pairs the same way, which gives the
// same row as one sequential scan.
#include "jm_device.h"
#include "jm_kernels.h"

namespace jm {

// (v, i) better than (bv, bi) in the order of a sequential strict-> scan
__device__ __forceinline__ bool lm_better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

template <int BT, int NP>
__global__ void __launch_bounds__(512)
k_lm_head(LmArgs a) {
    // 32 rows per wave: 4 per iteration (2 at d = 4096, whose double-buffered
    // rows would not fit the registers otherwise)
    constexpr int K = NP * 512, R = NP >= 8 ? 2 : 4, IT = 32 / R, W8 = 8;
    __shared__ __align__(16) float xs[BT * K];
    __shared__ float cv[W8][BT];
    __shared__ int ci[W8][BT];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int tb0 = blockIdx.y * BT;
    const int rowb = blockIdx.x * (W8 * R * IT) + w * (R * IT);
    const uint16_t* W = a.w;

    auto load = [&](uint4 (&buf)[NP][R], int r0) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            int row = r0 + r;
            row = row < a.V ? row : a.V - 1;
            const uint4* p = (const uint4*)(W + (size_t)row * K) + lane;
#pragma unroll
            for (int pg = 0; pg < NP; pg++) buf[pg][r] = p[pg * 64];
        }
    };
    uint4 cur[NP][R], nxt[NP][R];
    load(cur, rowb);
    for (int i = tid; i < BT * K / 4; i += 512) {
        const int b = i / (K / 4), c = 4 * (i % (K / 4));
        const float4 v = tb0 + b < a.B ? *(const float4*)(a.x + (size_t)(tb0 + b) * K + c)
                                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        *(float4*)(xs + b * K + c) = v;
    }
    __syncthreads();

    constexpr int NV = R * BT;
    constexpr int NG = NV < 16 ? NV : 16;
    constexpr int LPV = 64 / NG;              // lanes holding each row total
    float bv = -1e30f;
    int bi = 0;
    for (int it = 0; it < IT; it++) {
        const int r0 = rowb + it * R;
        if (it + 1 < IT) load(nxt, r0 + R);
        float acc[R][BT];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int b = 0; b < BT; b++) acc[r][b] = 0.0f;
#pragma unroll
        for (int pg = 0; pg < NP; pg++) {
            float wf[R][8];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t ww[4] = {cur[pg][r].x, cur[pg][r].y, cur[pg][r].z, cur[pg][r].w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    wf[r][2 * i] = __uint_as_float(ww[i] << 16);
                    wf[r][2 * i + 1] = __uint_as_float(ww[i] & 0xFFFF0000u);
                }
            }
            const int kl = pg * 512 + lane * 8;
#pragma unroll
            for (int b = 0; b < BT; b++) {
                const float4 x0 = *(const float4*)(xs + b * K + kl);
                const float4 x1 = *(const float4*)(xs + b * K + kl + 4);
                const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int r = 0; r < R; r++) {
                    float s = acc[r][b];
#pragma unroll
                    for (int i = 0; i < 8; i++) s = __builtin_fmaf(wf[r][i], xv[i], s);
                    acc[r][b] = s;
                }
                // one token at a time (see k_gemv_part)
#pragma unroll
                for (int r = 0; r < R; r++) __asm__ volatile("" : "+v"(acc[r][b]) : : "memory");
            }
        }
        float* flat = &acc[0][0];
#pragma unroll
        for (int g0 = 0; g0 < NV; g0 += NG) {
            float v[NG];
#pragma unroll
            for (int i = 0; i < NG; i++) v[i] = flat[g0 + i];
            const float tot = transpose_reduce<64, NG>(v);
            if (lane % LPV == 0) {
                const int vi = g0 + lane / LPV;
                const int r = vi / BT, b = vi % BT;          // b is the same for every group
                const int row = r0 + r;
                if (row < a.V && tb0 + b < a.B) {
                    if (a.logits) a.logits[(size_t)(tb0 + b) * a.V + row] = tot;
                    if (tot > bv) { bv = tot; bi = row; }
                }
            }
        }
#pragma unroll
        for (int pg = 0; pg < NP; pg++)
#pragma unroll
            for (int r = 0; r < R; r++) cur[pg][r] = nxt[pg][r];
    }
    if (!a.best_v) return;
    // the lanes holding token b differ in the lane bits above LPV * BT
#pragma unroll
    for (int m = LPV * BT; m < 64; m <<= 1) {
        const float ov = __shfl_xor(bv, m, JM_WAVE);
        const int oi = __shfl_xor(bi, m, JM_WAVE);
        if (lm_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane < LPV * BT && lane % LPV == 0) {
        cv[w][lane / LPV] = bv;
        ci[w][lane / LPV] = bi;
    }
    __syncthreads();
    if (tid < BT && tb0 + tid < a.B) {
        float v = cv[0][tid];
        int i = ci[0][tid];
        for (int ww = 1; ww < W8; ww++)
            if (lm_better(cv[ww][tid], ci[ww][tid], v, i)) { v = cv[ww][tid]; i = ci[ww][tid]; }
        a.best_v[(size_t)blockIdx.x * a.B + tb0 + tid] = v;
        a.best_i[(size_t)blockIdx.x * a.B + tb0 + tid] = i;
    }
}

// out_tok[b] = the best row over the blocks' bests of token b.
__global__ void __launch_bounds__(256)
k_argmax_merge(const float* __restrict__ best_v, const int* __restrict__ best_i, int nblk, int B,
               int* __restrict__ out_tok) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int b = blockIdx.x, t = threadIdx.x;
    float v = -1e30f;
    int i = 0;
    for (int k = t; k < nblk; k += 256) {
        const float kv = best_v[(size_t)k * B + b];
        const int ki = best_i[(size_t)k * B + b];
        if (lm_better(kv, ki, v, i)) { v = kv; i = ki; }
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const float ov = __shfl_xor(v, m, JM_WAVE);
        const int oi = __shfl_xor(i, m, JM_WAVE);
        if (lm_better(ov, oi, v, i)) { v = ov; i = oi; }
    }
    if ((t & 63) == 0) { sv[t >> 6] = v; si[t >> 6] = i; }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < 4; w++)
            if (lm_better(sv[w], si[w], v, i)) { v = sv[w]; i = si[w]; }
        out_tok[b] = i;
    }
}

int lm_blocks(int V) { return (V + 255) / 256; }

bool lm_shape_ok(int d) { return d == 1024 || d == 2048 || d == 4096; }

hipError_t launch_lm_head(const LmArgs& a, int* out_tok, hipStream_t st) {
    if (a.B == 0) return hipSuccess;
    // up to 64 KiB of tokens staged per block (128 KiB at d = 4096)
    const int BT = a.B <= 1 ? 1 : a.B <= 2 ? 2 : a.B <= 4 ? 4 : 8;
    const dim3 grid((unsigned)lm_blocks(a.V), (unsigned)((a.B + BT - 1) / BT));
#define JM_LM(BB, NN) hipLaunchKernelGGL((k_lm_head<BB, NN>), grid, dim3(512), 0, st, a)
#define JM_LMN(BB) switch (a.d) { case 1024: JM_LM(BB, 2); break; case 2048: JM_LM(BB, 4); break; \
        case 4096: JM_LM(BB, 8); break; default: return hipErrorInvalidValue; }
    switch (BT) {
        case 1: JM_LMN(1) break;
        case 2: JM_LMN(2) break;
        case 4: JM_LMN(4) break;
        default: JM_LMN(8) break;
    }
#undef JM_LMN
#undef JM_LM
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !out_tok) return e;
    hipLaunchKernelGGL(k_argmax_merge, dim3((unsigned)a.B), dim3(256), 0, st, a.best_v, a.best_i,
                       lm_blocks(a.V), a.B, out_tok);
    return hipGetLastError();
}

// out[b] = bf16 row tokens[b] of the embedding (decode_kernel.c:1597-1600);
// a token outside [0, V) gives a row of NaN.
__global__ void __launch_bounds__(256)
k_embed(const uint16_t* __restrict__ embed, int V, int d, const int* __restrict__ tokens,
        float* __restrict__ out) {
    const int b = blockIdx.x;
    const int tok = tokens[b];
    const bool ok = tok >= 0 && tok < V;
    const uint16_t* row = embed + (size_t)(ok ? tok : 0) * d;
    for (int i = threadIdx.x; i < d; i += 256)
        out[(size_t)b * d + i] = ok ? bf16_bits_to_f32(row[i]) : __uint_as_float(0x7FC00000u);
}

hipError_t launch_embed(const uint16_t* embed, int V, int d, const int* tokens, int B, float* out,
                        hipStream_t st) {
    if (B == 0) return hipSuccess;
    hipLaunchKernelGGL(k_embed, dim3((unsigned)B), dim3(256), 0, st, embed, V, d, tokens, out);
    return hipGetLastError();
}

// bf16 bits of float32 values that are exactly bf16 (the low half is zero).
__global__ void __launch_bounds__(256)
k_f32_bf16_bits(const float* __restrict__ in, long long n, uint16_t* __restrict__ out) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = (uint16_t)(__float_as_uint(in[i]) >> 16);
}

hipError_t launch_f32_bf16_bits(const float* in, long long n, uint16_t* out, hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_f32_bf16_bits, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, in, n, out);
    return hipGetLastError();
}

}  // namespace jm
