// Decoder-layer kernels around the MoE block: the bf16 projections (with the
// RMSNorm before them and the residual add after them fused in), decode
// attention over a bf16 KV cache, and the final RMSNorm.  They follow the
// reference's layer_attn_batch / decode_layers_batch
// (decode_kernel.c:1120-1234, 1518-1556) step for step, regrouped into few
// launches:
//
//   k_gemv_part   Wq/Wk/Wv . (h * norm1 weight), per 512-column slice
//                                                             (:224-230, :1126-1145)
//   k_qkv_fin     the slices summed, RMSNorm row scale, bias, per-head
//                 QK-norm, RoPE; q out, k and v appended to the cache
//                                                               (:1146-1199)
//   k_attn_part   scores, softmax and P.V over one 128-position split of
//                 the cache                                     (:1200-1222)
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
// stacked matrices w[0..2].  Block (row group, slice, token group): WV waves
// of R rows, each lane holding 8 consecutive columns of its rows per
// 512-column pass (NPS passes per slice); the slice of every token of the
// group staged in LDS.  The consumer sums the slices (and applies the
// RMSNorm row scale), so that each block moves few activation bytes and a
// projection spreads over hundreds of blocks.
template <int BT, int R, int WV, int NPS>
__global__ void __launch_bounds__(WV * 64)
k_gemv_part(GemvArgs a) {
    constexpr int SW = NPS * 512;
    __shared__ __align__(16) float xs[BT * SW];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int slice = blockIdx.y, tb0 = blockIdx.z * BT;
    const int row0 = blockIdx.x * (WV * R) + w * R;
    const int k0 = slice * SW;

    // this wave's rows, 16 bytes per lane per pass, requested first
    uint4 wq[R][NPS];
#pragma unroll
    for (int r = 0; r < R; r++) {
        int row = row0 + r;
        row = row < a.N ? row : a.N - 1;
        const uint16_t* wr;
        if (row < a.rows[0]) wr = a.w[0] + (size_t)row * a.K;
        else if (row < a.rows[0] + a.rows[1]) wr = a.w[1] + (size_t)(row - a.rows[0]) * a.K;
        else wr = a.w[2] + (size_t)(row - a.rows[0] - a.rows[1]) * a.K;
        const uint4* p = (const uint4*)(wr + k0) + lane;
#pragma unroll
        for (int j = 0; j < NPS; j++) wq[r][j] = p[j * 64];
    }
    // the tokens' slice (times the norm weight)
    for (int i = tid; i < BT * SW / 4; i += WV * 64) {
        const int b = i / (SW / 4), c = 4 * (i % (SW / 4));
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (tb0 + b < a.B) {
            v = *(const float4*)(a.x + (size_t)(tb0 + b) * a.K + k0 + c);
            if (a.norm_w) {
                const uint2 nw = *(const uint2*)(a.norm_w + k0 + c);
                v.x = __fmul_rn(v.x, bf16_bits_to_f32(nw.x & 0xFFFFu));
                v.y = __fmul_rn(v.y, bf16_bits_to_f32(nw.x >> 16));
                v.z = __fmul_rn(v.z, bf16_bits_to_f32(nw.y & 0xFFFFu));
                v.w = __fmul_rn(v.w, bf16_bits_to_f32(nw.y >> 16));
            }
        }
        *(float4*)(xs + b * SW + c) = v;
    }
    __syncthreads();

    float acc[R][BT];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < BT; b++) acc[r][b] = 0.0f;
#pragma unroll
    for (int j = 0; j < NPS; j++) {
        float wf[R][8];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t ww[4] = {wq[r][j].x, wq[r][j].y, wq[r][j].z, wq[r][j].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                wf[r][2 * i] = __uint_as_float(ww[i] << 16);
                wf[r][2 * i + 1] = __uint_as_float(ww[i] & 0xFFFF0000u);
            }
        }
#pragma unroll
        for (int b = 0; b < BT; b++) {
            const float4 x0 = *(const float4*)(xs + b * SW + j * 512 + lane * 8);
            const float4 x1 = *(const float4*)(xs + b * SW + j * 512 + lane * 8 + 4);
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int r = 0; r < R; r++) {
                float s = acc[r][b];
#pragma unroll
                for (int i = 0; i < 8; i++) s = __builtin_fmaf(wf[r][i], xv[i], s);
                acc[r][b] = s;
            }
            // one token at a time: the empty asm takes the sums and fences
            // memory, so later tokens' LDS reads are not hoisted into registers
#pragma unroll
            for (int r = 0; r < R; r++) __asm__ volatile("" : "+v"(acc[r][b]) : : "memory");
        }
    }
    // row totals: groups of up to 16 partial sums transposed across the wave
    constexpr int NV = R * BT;
    constexpr int NG = NV < 16 ? NV : 16;
    float* flat = &acc[0][0];
#pragma unroll
    for (int g0 = 0; g0 < NV; g0 += NG) {
        float v[NG];
#pragma unroll
        for (int i = 0; i < NG; i++) v[i] = flat[g0 + i];
        const float tot = transpose_reduce<64, NG>(v);
        constexpr int LPV = 64 / NG;                  // lanes holding each value
        if (lane % LPV == 0) {
            const int vi = g0 + lane / LPV;
            const int r = vi / BT, b = vi % BT;
            const int row = row0 + r;
            if (row < a.N && tb0 + b < a.B) a.part[((size_t)slice * a.B + tb0 + b) * a.N + row] = tot;
        }
    }
}

bool gemv_shape_ok(int K) { return K > 0 && K % 1024 == 0 && K <= 8192; }

int gemv_slice_cols(int K) { return K >= 4096 ? 1024 : 512; }

hipError_t launch_gemv_part(const GemvArgs& a, hipStream_t st) {
    if (a.B == 0 || a.N == 0) return hipSuccess;
    const int BT = a.B <= 1 ? 1 : a.B <= 2 ? 2 : a.B <= 4 ? 4 : 8;
    // shapes from a sweep at 8 tokens: 512-column slices with 8 waves of 4
    // rows for K = 2048 (2.5 TB/s on the qkv projection), 1024-column slices
    // with 16 waves of 2 rows for K = 4096 (o_proj)
    const bool wide = gemv_slice_cols(a.K) == 1024;
    const int R = wide ? 2 : 4, WV = wide ? 16 : 8;
    const dim3 grid((unsigned)((a.N + WV * R - 1) / (WV * R)), (unsigned)(a.K / gemv_slice_cols(a.K)),
                    (unsigned)((a.B + BT - 1) / BT));
#define JM_GP(BB) if (wide) hipLaunchKernelGGL((k_gemv_part<BB, 2, 16, 2>), grid, dim3(1024), 0, st, a); \
                  else hipLaunchKernelGGL((k_gemv_part<BB, 4, 8, 1>), grid, dim3(512), 0, st, a)
    switch (BT) {
        case 1: JM_GP(1); break;
        case 2: JM_GP(2); break;
        case 4: JM_GP(4); break;
        default: JM_GP(8); break;
    }
#undef JM_GP
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

__device__ __forceinline__ float bf16_round(float f) { return __uint_as_float(f32_to_bf16_rne(f) << 16); }

// The projections of one head of one token finished: the column slices
// summed, times the RMSNorm row scale of h, plus the bias (:1126-1145); for
// q and k heads the per-head RMSNorm (:1174-1189) and RoPE rotate-half at
// the token's position (:1190-1194, :259-266).  q heads go to qout; k and v
// heads are appended to the bf16 cache at the position (:1195-1199).
// Block (head in q.., k.., v.., token), one thread per dimension.
__global__ void __launch_bounds__(128)
k_qkv_fin(AttnArgs a) {
    constexpr int HD = 128;
    __shared__ float vals[HD];
    __shared__ float red[2];
    const int hh = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    const int pos = a.pos[b];
    // RMSNorm row scale of the layer input (the projections were taken of
    // h * norm weight)
    const float* hb = a.h + (size_t)b * a.d;
    float ss = 0.0f;
    for (int i = t; i < a.d / 4; i += HD) {
        const float4 v = *(const float4*)(hb + 4 * i);
        ss = __builtin_fmaf(v.x, v.x, ss);
        ss = __builtin_fmaf(v.y, v.y, ss);
        ss = __builtin_fmaf(v.z, v.z, ss);
        ss = __builtin_fmaf(v.w, v.w, ss);
    }
    ss = seg_sum<64>(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    const float inv = rms_inv(__fadd_rn(red[0], red[1]), a.d, a.eps);
    const int row = hh * HD + t;
    float v = a.qkv[(size_t)b * a.nqkv + row];
    for (int sl = 1; sl < a.nslice; sl++) v = __fadd_rn(v, a.qkv[((size_t)sl * a.B + b) * a.nqkv + row]);
    v = __fmul_rn(v, inv);
    const bool isq = hh < a.H, isk = !isq && hh < a.H + a.KH;
    const float* bias = isq ? a.bq : isk ? a.bk : a.bv;
    const int brow = isq ? row : isk ? row - a.H * HD : row - (a.H + a.KH) * HD;
    if (bias) v = __fadd_rn(v, bias[brow]);
    const unsigned long long* kvp = a.kv + ((size_t)b * a.L + a.layer) * 2;
    if (!isq && !isk) {                  // v head: to the cache
        uint16_t* vc = (uint16_t*)kvp[1];
        vc[((size_t)pos * a.KH + (hh - a.H - a.KH)) * HD + t] = (uint16_t)f32_to_bf16_rne(v);
        return;
    }
    const uint16_t* nw = isq ? a.qn : a.kn;
    if (nw) {
        float sq = seg_sum<64>(__fmul_rn(v, v));
        __syncthreads();                 // red[] reused
        if ((t & 63) == 0) red[t >> 6] = sq;
        __syncthreads();
        const float hinv = rms_inv(__fadd_rn(red[0], red[1]), HD, a.eps);
        v = __fmul_rn(__fmul_rn(v, hinv), bf16_bits_to_f32(nw[t]));
    }
    // rotate-half: dim i pairs with i + 64 (first half: a cos - b sin,
    // second half: a sin + b cos, with a = dim i, b = dim i + 64)
    vals[t] = v;
    __syncthreads();
    const float other = vals[t ^ 64];
    const bool lo = t < HD / 2;
    const int ci = lo ? t : t - HD / 2;
    const float c = a.cos[(size_t)pos * HD + ci], sn = a.sin[(size_t)pos * HD + ci];
    const float o = lo ? __builtin_fmaf(v, c, -__fmul_rn(other, sn)) : __builtin_fmaf(other, sn, __fmul_rn(v, c));
    if (isq) {
        a.qout[((size_t)b * a.H + hh) * HD + t] = o;
    } else {
        uint16_t* kc = (uint16_t*)kvp[0];
        kc[((size_t)pos * a.KH + (hh - a.H)) * HD + t] = (uint16_t)f32_to_bf16_rne(o);
    }
}

// One (position split, KV head, token): QPK query heads over positions
// [128 s, 128 s + 128) of the token's T = pos + 1 cache rows (the row at pos
// appended by k_qkv_fin).  256 threads; lane (g, j) of wave w takes
// positions 128 s + 32 w + 4 st + g (st < 8) and head dimensions 8 j ..
// 8 j + 7.
template <int QPK>
__global__ void __launch_bounds__(256)
k_attn_part(AttnArgs a) {
    constexpr int HD = 128, P = 128, SP = P + 4;
    __shared__ __align__(16) float sc[QPK][SP];        // scores, then exp(score - max)
    __shared__ __align__(16) float red[4][QPK * HD];   // per-wave partial outputs
    const int s = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
    const int pos = a.pos[b];
    const int T = pos + 1;
    const int t0 = s * P;
    if (t0 >= T) return;                 // past this token's positions (block-uniform)
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const unsigned long long* kvp = a.kv + ((size_t)b * a.L + a.layer) * 2;
    const uint16_t* kc = (const uint16_t*)kvp[0];
    const uint16_t* vc = (const uint16_t*)kvp[1];
    const int g = lane >> 4, j = lane & 15;
    // the rows: unconditional loads (row 0 past the end)
    uint4 kr[8], vr[8];
#pragma unroll
    for (int st = 0; st < 8; st++) {
        const int t = t0 + 32 * w + 4 * st + g;
        const size_t off = ((size_t)(t < T ? t : 0) * a.KH + kh) * HD + 8 * j;
        kr[st] = *(const uint4*)(kc + off);
        vr[st] = *(const uint4*)(vc + off);
    }
    float q[QPK][8];
#pragma unroll
    for (int h = 0; h < QPK; h++) {
        const float4* qp = (const float4*)(a.qout + ((size_t)b * a.H + kh * QPK + h) * HD + 8 * j);
        const float4 q0 = qp[0], q1 = qp[1];
        q[h][0] = q0.x; q[h][1] = q0.y; q[h][2] = q0.z; q[h][3] = q0.w;
        q[h][4] = q1.x; q[h][5] = q1.y; q[h][6] = q1.z; q[h][7] = q1.w;
    }

    // ---- scores (:1205-1211): q . k / sqrtf_fast(hd)
    constexpr int LPH = 16 / QPK;
#pragma unroll
    for (int st = 0; st < 8; st++) {
        const int t = t0 + 32 * w + 4 * st + g;
        const uint32_t kw[4] = {kr[st].x, kr[st].y, kr[st].z, kr[st].w};
        float kf[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            kf[2 * i] = __uint_as_float(kw[i] << 16);
            kf[2 * i + 1] = __uint_as_float(kw[i] & 0xFFFF0000u);
        }
        float dots[QPK];
#pragma unroll
        for (int h = 0; h < QPK; h++) {
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) d = __builtin_fmaf(q[h][i], kf[i], d);
            dots[h] = d;
        }
        const float tot = head_reduce16<QPK>(dots);
        if (j % LPH == 0) sc[j / LPH][t - t0] = t < T ? __fdiv_rn(tot, a.sdiv) : -INFINITY;
    }
    __syncthreads();

    // ---- softmax numerators over the split (:1212-1214) with the split's
    // own max; the merge rescales by the global one
    if (tid < QPK * 32) {
        const int h = tid >> 5, li = tid & 31;
        float v[4];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[i] = sc[h][li + 32 * i];
            mx = fmaxf(mx, v[i]);
        }
        mx = seg_max<32>(mx);
        float l = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float p = expf_fast(__fsub_rn(v[i], mx));
            sc[h][li + 32 * i] = p;
            l = __fadd_rn(l, p);
        }
        l = seg_sum<32>(l);
        if (li == 0) {
            float* ml = a.part_ml + ((((size_t)b * a.KH + kh) * a.S + s) * QPK + h) * 2;
            ml[0] = mx;
            ml[1] = l;
        }
    }
    __syncthreads();

    // ---- P . V (:1215-1221) over this lane's positions
    float acc[QPK * 8];
#pragma unroll
    for (int i = 0; i < QPK * 8; i++) acc[i] = 0.0f;
#pragma unroll
    for (int st = 0; st < 8; st++) {
        const int t = t0 + 32 * w + 4 * st + g;
        const uint32_t vw[4] = {vr[st].x, vr[st].y, vr[st].z, vr[st].w};
        const bool ok = t < T;
        float vf[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            vf[2 * i] = ok ? __uint_as_float(vw[i] << 16) : 0.0f;
            vf[2 * i + 1] = ok ? __uint_as_float(vw[i] & 0xFFFF0000u) : 0.0f;
        }
#pragma unroll
        for (int h = 0; h < QPK; h++) {
            const float p = sc[h][t - t0];
#pragma unroll
            for (int i = 0; i < 8; i++) acc[h * 8 + i] = __builtin_fmaf(p, vf[i], acc[h * 8 + i]);
        }
    }
    // sum over the 4 lane groups g: two transposing levels leave lane group
    // g with values [g N/4, (g + 1) N/4) of the flat (head, dim) list
    constexpr int N = QPK * 8;
    transpose_level<32, N>(acc);
    transpose_level<16, N / 2>(acc);
#pragma unroll
    for (int i = 0; i < N / 4; i++) {
        const int idx = g * (N / 4) + i;
        red[w][(idx >> 3) * HD + 8 * j + (idx & 7)] = acc[i];
    }
    __syncthreads();
    float* po = a.part_o + (((size_t)b * a.KH + kh) * a.S + s) * QPK * HD;
    for (int o = tid; o < QPK * HD; o += 256)
        po[o] = __fadd_rn(__fadd_rn(red[0][o], red[1][o]), __fadd_rn(red[2][o], red[3][o]));
}

// Merge of the splits of one (query head, token): out = sum_s o_s e^(m_s - M)
// / sum_s l_s e^(m_s - M), M the max over the splits.  The splits' weights
// are computed in parallel (128 at a time) and staged in LDS; each thread
// then sums its dimension over them with independent loads.
__global__ void __launch_bounds__(128)
k_attn_comb(AttnArgs a, int qpk, float* __restrict__ att) {
    __shared__ float fs[128];
    __shared__ float red[2];
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    const int kh = h / qpk, hq = h % qpk;
    const int ns = (a.pos[b] + 128) / 128;          // splits of T = pos + 1 positions
    const size_t base = ((size_t)b * a.KH + kh) * a.S;
    const float* ml = a.part_ml + (base * qpk + hq) * 2;      // split s at ml[2 qpk s]
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
    hipLaunchKernelGGL(k_qkv_fin, dim3((unsigned)(a.H + 2 * a.KH), (unsigned)a.B), dim3(128), 0, st, a);
    hipError_t e0 = hipGetLastError();
    if (e0 != hipSuccess) return e0;
    const dim3 grid((unsigned)a.S, (unsigned)a.KH, (unsigned)a.B);
    switch (qpk) {
        case 1: hipLaunchKernelGGL(k_attn_part<1>, grid, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL(k_attn_part<2>, grid, dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL(k_attn_part<4>, grid, dim3(256), 0, st, a); break;
        case 8: hipLaunchKernelGGL(k_attn_part<8>, grid, dim3(256), 0, st, a); break;
        default: return hipErrorInvalidValue;
    }
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
