// Decoder-layer kernels around the MoE block: the bf16 projections (with the
// RMSNorm before them and the residual add after them fused in), decode
// attention over a bf16 KV cache, and the final RMSNorm.  They follow the
// reference's layer_attn_batch / decode_layers_batch
// (decode_kernel.c:1120-1234, 1518-1556) step for step, regrouped into few
// launches:
//
//   k_gemv_bf16   norm1 + Wq/Wk/Wv (+ bias)  -> qkv        (:224-230, :1126-1145)
//   k_attn_part   per-head QK-norm, RoPE, KV append, scores, softmax and
//                 P.V over one 128-position split of the cache  (:1165-1222)
//   k_attn_comb   the splits merged per head                   (flash-decoding merge)
//   k_gemv_bf16   Wo . att + residual -> h                     (:1225-1232, :1546-1547)
//   k_rms_rows    the final RMSNorm                            (:1556)
//
// The projections are HBM-bound GEMVs: every 16-byte weight load of a lane
// serves all the batch's tokens, whose rows sit in LDS.  Attention streams
// the cache once: one block per (position split, KV head, token) reads 128
// positions of K and V (256 bytes each per head) and serves every query head
// of that KV head.
#include "jm_device.h"
#include "jm_kernels.h"

namespace jm {

// ------------------------------------------------------------------ GEMV

// out[b][row] = (resid[b][row] +) (bias[row] +) W[row] . xn[b], rows of the
// stacked matrices w[0..2]; xn = x, or RMSNorm(x) * norm_w.  Block: 4 waves
// of R rows each; every lane holds 8 consecutive columns of each of its rows
// per 512-column pass, all passes' weights requested up front.  Tokens in
// groups of BT (grid.y); their rows staged in LDS in chunks of KC columns.
template <int BT, int NP, int R>
__global__ void __launch_bounds__(256)
k_gemv_bf16(GemvArgs a) {
    constexpr int K = NP * 512;
    constexpr int KC0 = 16384 / BT;                  // 64 KiB of fp32 rows
    constexpr int KC = K < KC0 ? K : KC0 / 512 * 512;
    constexpr int PPC = KC / 512;                    // passes per chunk
    static_assert(KC >= 512 && K % KC == 0, "chunking");
    __shared__ __align__(16) float xs[BT * KC];
    __shared__ float invl[BT];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int tb0 = blockIdx.y * BT;
    const int row0 = (blockIdx.x * 4 + w) * R;

    // this wave's rows: every pass's 8 columns, requested first
    uint4 wq[NP][R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        int row = row0 + r;
        row = row < a.N ? row : a.N - 1;
        const uint16_t* wr;
        if (row < a.rows[0]) wr = a.w[0] + (size_t)row * K;
        else if (row < a.rows[0] + a.rows[1]) wr = a.w[1] + (size_t)(row - a.rows[0]) * K;
        else wr = a.w[2] + (size_t)(row - a.rows[0] - a.rows[1]) * K;
        const uint4* p = (const uint4*)wr + lane;
#pragma unroll
        for (int pg = 0; pg < NP; pg++) wq[pg][r] = p[pg * 64];
    }
    // RMSNorm scales of the group's tokens (one wave per token)
    if (a.norm_w) {
        for (int b = w; b < BT; b += 4) {
            float ss = 0.0f;
            if (tb0 + b < a.B) {
                const float4* xr = (const float4*)(a.x + (size_t)(tb0 + b) * K);
#pragma unroll
                for (int i = 0; i < K / 256; i++) {
                    const float4 v = xr[lane + 64 * i];
                    ss = __builtin_fmaf(v.x, v.x, ss);
                    ss = __builtin_fmaf(v.y, v.y, ss);
                    ss = __builtin_fmaf(v.z, v.z, ss);
                    ss = __builtin_fmaf(v.w, v.w, ss);
                }
            }
            ss = seg_sum<64>(ss);
            if (lane == 0) invl[b] = rms_inv(ss, K, a.eps);
        }
    }
    float acc[R][BT];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < BT; b++) acc[r][b] = 0.0f;

#pragma unroll
    for (int pg = 0; pg < NP; pg++) {
        if (pg % PPC == 0) {
            // stage columns [kc0, kc0 + KC) of the group's tokens
            const int kc0 = pg * 512;
            __syncthreads();
#pragma unroll 4
            for (int i = tid; i < BT * KC / 4; i += 256) {
                const int b = i / (KC / 4), c = 4 * (i % (KC / 4));
                float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (tb0 + b < a.B) {
                    v = *(const float4*)(a.x + (size_t)(tb0 + b) * K + kc0 + c);
                    if (a.norm_w) {
                        const float inv = invl[b];
                        const uint2 nw = *(const uint2*)(a.norm_w + kc0 + c);
                        v.x = __fmul_rn(__fmul_rn(v.x, inv), bf16_bits_to_f32(nw.x & 0xFFFFu));
                        v.y = __fmul_rn(__fmul_rn(v.y, inv), bf16_bits_to_f32(nw.x >> 16));
                        v.z = __fmul_rn(__fmul_rn(v.z, inv), bf16_bits_to_f32(nw.y & 0xFFFFu));
                        v.w = __fmul_rn(__fmul_rn(v.w, inv), bf16_bits_to_f32(nw.y >> 16));
                    }
                }
                *(float4*)(xs + b * KC + c) = v;
            }
            __syncthreads();
        }
        const int kl = (pg % PPC) * 512 + lane * 8;
        // this pass's weights as floats, once for all tokens; the empty asm
        // keeps the conversion (and the wait for the load) at this pass
        float wf[R][8];
#pragma unroll
        for (int r = 0; r < R; r++) {
            uint32_t ww[4] = {wq[pg][r].x, wq[pg][r].y, wq[pg][r].z, wq[pg][r].w};
            __asm__ volatile("" : "+v"(ww[0]), "+v"(ww[1]), "+v"(ww[2]), "+v"(ww[3]));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                wf[r][2 * i] = __uint_as_float(ww[i] << 16);
                wf[r][2 * i + 1] = __uint_as_float(ww[i] & 0xFFFF0000u);
            }
        }
#pragma unroll
        for (int b = 0; b < BT; b++) {
            const float4 x0 = *(const float4*)(xs + b * KC + kl);
            const float4 x1 = *(const float4*)(xs + b * KC + kl + 4);
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int r = 0; r < R; r++) {
                float s = acc[r][b];
#pragma unroll
                for (int i = 0; i < 8; i++) s = __builtin_fmaf(wf[r][i], xv[i], s);
                acc[r][b] = s;
            }
            // one token's columns at a time: the empty asm takes the running
            // sums and fences memory, so neither are later tokens' LDS reads
            // hoisted nor this token's multiply-adds sunk (either would hold
            // many tokens' columns in registers)
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
            if (row < a.N && tb0 + b < a.B) {
                float y = tot;
                if (row < a.rows[0]) { if (a.bias[0]) y = __fadd_rn(y, a.bias[0][row]); }
                else if (row < a.rows[0] + a.rows[1]) { if (a.bias[1]) y = __fadd_rn(y, a.bias[1][row - a.rows[0]]); }
                else if (a.bias[2]) y = __fadd_rn(y, a.bias[2][row - a.rows[0] - a.rows[1]]);
                const size_t o = (size_t)(tb0 + b) * a.N + row;
                if (a.resid) y = __fadd_rn(a.resid[o], y);
                a.out[o] = y;
            }
        }
    }
}

bool gemv_shape_ok(int K) { return K == 1024 || K == 2048 || K == 4096; }

hipError_t launch_gemv_bf16(const GemvArgs& a, int rows_per_wave, hipStream_t st) {
    if (a.B == 0 || a.N == 0) return hipSuccess;
    const int BT = a.B <= 1 ? 1 : a.B <= 2 ? 2 : a.B <= 4 ? 4 : a.B <= 8 ? 8 : 16;
    const int R = rows_per_wave == 2 ? 2 : 4;
    const dim3 grid((unsigned)((a.N + 4 * R - 1) / (4 * R)), (unsigned)((a.B + BT - 1) / BT));
#define JM_GV(BB, NN, RR) hipLaunchKernelGGL((k_gemv_bf16<BB, NN, RR>), grid, dim3(256), 0, st, a)
#define JM_GVR(BB, NN) if (R == 2) JM_GV(BB, NN, 2); else JM_GV(BB, NN, 4)
#define JM_GVN(BB) switch (a.K) { case 1024: JM_GVR(BB, 2); break; case 2048: JM_GVR(BB, 4); break; \
        case 4096: JM_GVR(BB, 8); break; default: return hipErrorInvalidValue; }
    switch (BT) {
        case 1: JM_GVN(1) break;
        case 2: JM_GVN(2) break;
        case 4: JM_GVN(4) break;
        case 8: JM_GVN(8) break;
        default: JM_GVN(16) break;
    }
#undef JM_GVN
#undef JM_GVR
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

__device__ __forceinline__ float bf16_round(float f) { return __uint_as_float(f32_to_bf16_rne(f) << 16); }

// One (position split, KV head, token): QPK query heads over positions
// [128 s, 128 s + 128) of the token's T = pos + 1.  256 threads; lane
// (g, j) of wave w takes positions 128 s + 32 w + 4 st + g (st < 8) and
// head dimensions 8 j .. 8 j + 7.
template <int QPK>
__global__ void __launch_bounds__(256)
k_attn_part(AttnArgs a) {
    constexpr int HD = 128, P = 128, SP = P + 4;
    __shared__ __align__(16) float qs[QPK][HD];        // the query heads, normalised and rotated
    __shared__ __align__(16) float kvn[2][HD];         // the new k and v, as the bf16 cache holds them
    __shared__ __align__(16) float sc[QPK][SP];        // scores, then exp(score - max)
    __shared__ __align__(16) float red[4][QPK * HD];   // per-wave partial outputs
    const int s = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
    const int pos = a.pos[b];
    const int T = pos + 1;
    const int t0 = s * P;
    if (t0 >= T) return;                 // past this token's positions (block-uniform)
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float* qb = a.qkv + (size_t)b * a.nqkv;
    const unsigned long long* kvp = a.kv + ((size_t)b * a.L + a.layer) * 2;
    uint16_t* kc = (uint16_t*)kvp[0];
    uint16_t* vc = (uint16_t*)kvp[1];

    // ---- the query heads and the new k: per-head RMSNorm (:1174-1189),
    // then RoPE rotate-half at pos (:1190-1194, :259-266); dims i and i + 64
    // are 16 lanes apart in a 32-thread group of 4 dims per thread
    {
        const int grp = tid >> 5, li = tid & 31, dim = 4 * li;
        const bool lo = dim < HD / 2;
        const int ci = lo ? dim : dim - HD / 2;
        const float4 cs = *(const float4*)(a.cos + (size_t)pos * HD + ci);
        const float4 sn = *(const float4*)(a.sin + (size_t)pos * HD + ci);
        for (int it = grp; it <= QPK; it += 8) {
            const bool isk = it == QPK;
            const float* src = qb + (size_t)(isk ? a.H + kh : kh * QPK + it) * HD;
            float v[4];
            {
                const float4 t = *(const float4*)(src + dim);
                v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
            }
            const uint16_t* nw = isk ? a.kn : a.qn;
            if (nw) {
                float ss = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) ss = __builtin_fmaf(v[i], v[i], ss);
                const float inv = rms_inv(seg_sum<32>(ss), HD, a.eps);
                const uint2 wv = *(const uint2*)(nw + dim);
                const uint32_t wb[4] = {wv.x & 0xFFFFu, wv.x >> 16, wv.y & 0xFFFFu, wv.y >> 16};
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = __fmul_rn(__fmul_rn(v[i], inv), bf16_bits_to_f32(wb[i]));
            }
            const float c4[4] = {cs.x, cs.y, cs.z, cs.w}, s4[4] = {sn.x, sn.y, sn.z, sn.w};
            float o[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float other = __shfl_xor(v[i], 16, JM_WAVE);
                // first half: a cos - b sin; second half: a sin + b cos
                // (a = dim i, b = dim i + 64)
                o[i] = lo ? __builtin_fmaf(v[i], c4[i], -__fmul_rn(other, s4[i]))
                          : __builtin_fmaf(other, s4[i], __fmul_rn(v[i], c4[i]));
            }
            if (!isk) {
                *(float4*)(&qs[it][dim]) = make_float4(o[0], o[1], o[2], o[3]);
            } else {
                *(float4*)(&kvn[0][dim]) = make_float4(bf16_round(o[0]), bf16_round(o[1]), bf16_round(o[2]),
                                                       bf16_round(o[3]));
            }
        }
        if (tid < 32) {
            const float4 t = *(const float4*)(qb + (size_t)(a.H + a.KH + kh) * HD + dim);
            *(float4*)(&kvn[1][dim]) = make_float4(bf16_round(t.x), bf16_round(t.y), bf16_round(t.z), bf16_round(t.w));
        }
    }
    __syncthreads();
    // the split holding pos appends the new k and v (:1195-1199)
    if (pos - t0 < P && tid < 64) {
        const int which = tid >> 5, dim = 4 * (tid & 31);
        const float* src = kvn[which];
        const uint2 bits = make_uint2(f32_to_bf16_rne(src[dim]) | (f32_to_bf16_rne(src[dim + 1]) << 16),
                                      f32_to_bf16_rne(src[dim + 2]) | (f32_to_bf16_rne(src[dim + 3]) << 16));
        uint16_t* dst = which ? vc : kc;
        *(uint2*)(dst + ((size_t)pos * a.KH + kh) * HD + dim) = bits;
    }

    // ---- scores (:1205-1211): q . k / sqrtf_fast(hd)
    const int g = lane >> 4, j = lane & 15;
    uint4 kr[8], vr[8];
#pragma unroll
    for (int st = 0; st < 8; st++) {
        const int t = t0 + 32 * w + 4 * st + g;
        const int ta = (t < T && t != pos) ? t : 0;     // unconditional loads; pos and the tail replaced below
        const size_t off = ((size_t)ta * a.KH + kh) * HD + 8 * j;
        kr[st] = *(const uint4*)(kc + off);
        vr[st] = *(const uint4*)(vc + off);
    }
    float q[QPK][8];
#pragma unroll
    for (int h = 0; h < QPK; h++) {
        const float4 q0 = *(const float4*)(&qs[h][8 * j]), q1 = *(const float4*)(&qs[h][8 * j + 4]);
        q[h][0] = q0.x; q[h][1] = q0.y; q[h][2] = q0.z; q[h][3] = q0.w;
        q[h][4] = q1.x; q[h][5] = q1.y; q[h][6] = q1.z; q[h][7] = q1.w;
    }
    constexpr int LPH = 16 / QPK;
#pragma unroll
    for (int st = 0; st < 8; st++) {
        const int t = t0 + 32 * w + 4 * st + g;
        float kf[8];
        if (t == pos) {
#pragma unroll
            for (int i = 0; i < 8; i++) kf[i] = kvn[0][8 * j + i];
        } else {
            const uint32_t kw[4] = {kr[st].x, kr[st].y, kr[st].z, kr[st].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                kf[2 * i] = __uint_as_float(kw[i] << 16);
                kf[2 * i + 1] = __uint_as_float(kw[i] & 0xFFFF0000u);
            }
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
        float vf[8];
        if (t == pos) {
#pragma unroll
            for (int i = 0; i < 8; i++) vf[i] = kvn[1][8 * j + i];
        } else {
            const uint32_t vw[4] = {vr[st].x, vr[st].y, vr[st].z, vr[st].w};
            const bool ok = t < T;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                vf[2 * i] = ok ? __uint_as_float(vw[i] << 16) : 0.0f;
                vf[2 * i + 1] = ok ? __uint_as_float(vw[i] & 0xFFFF0000u) : 0.0f;
            }
        }
#pragma unroll
        for (int h = 0; h < QPK; h++) {
            const float p = sc[h][t - t0];
#pragma unroll
            for (int i = 0; i < 8; i++) acc[h * 8 + i] = __builtin_fmaf(p, vf[i], acc[h * 8 + i]);
        }
    }
    // sum over the 4 lane groups g: two transposing levels leave lane group
    // g with values [g' N/4, (g' + 1) N/4) of the flat (head, dim) list,
    // g' = 2 (g >> 1) + (g & 1) = g
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
// / sum_s l_s e^(m_s - M), M the max over the splits.
__global__ void __launch_bounds__(128)
k_attn_comb(AttnArgs a, int qpk, float* __restrict__ att) {
    const int h = blockIdx.x, b = blockIdx.y, dim = threadIdx.x;
    const int kh = h / qpk, hq = h % qpk;
    const int T = a.pos[b] + 1;
    const int ns = (T + 127) / 128;
    const size_t base = ((size_t)b * a.KH + kh) * a.S;
    float M = -INFINITY;
    for (int s = 0; s < ns; s++) M = fmaxf(M, a.part_ml[((base + s) * qpk + hq) * 2]);
    float L = 0.0f, O = 0.0f;
    for (int s = 0; s < ns; s++) {
        const float* ml = a.part_ml + ((base + s) * qpk + hq) * 2;
        const float f = expf_fast(__fsub_rn(ml[0], M));
        L = __builtin_fmaf(ml[1], f, L);
        O = __builtin_fmaf(a.part_o[((base + s) * qpk + hq) * 128 + dim], f, O);
    }
    att[((size_t)b * a.H + h) * 128 + dim] = __fdiv_rn(O, L);
}

hipError_t launch_attn(const AttnArgs& a, int qpk, float* att, hipStream_t st) {
    if (a.B == 0) return hipSuccess;
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
