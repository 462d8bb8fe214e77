// MoE decode block kernels for gfx950 (CDNA4, wave64).
//
// Stages of one call (the reference's layer_ffn_batch,
// src/jouleai/native/decode_kernel.c:1387-1508):
//
//   k_router_logits  scores[b][e] = gate_w[e] . x[b] in the reference's
//                    8-chain FMA order (decode_kernel.c:234-256, 693-718)
//   k_prep_digits    activation groups -> signed base-16 digits + scale
//   k_topk           softmax with expf_fast, top-k lowest-index ties,
//                    optional renormalisation (decode_kernel.c:1425-1448)
//   k_dispatch       stable counting sort of the B*k slots into per-expert
//                    segments, list of active experts (decode_kernel.c:1449-1485)
//   k_gateup         per (active expert, 64-row block): gate and up Q4 rows
//                    dotted with the segment's tokens, act = SiLU(g)*u, and
//                    the act groups re-encoded as digits for the down pass
//                    (decode_kernel.c:1365-1375)
//   k_down           per (active expert, row block): down Q4 rows dotted with
//                    the act digits, times the routing weight (:1376-1383)
//   k_combine        out[b] = sum of the token's k expert rows in the
//                    reference's union order (:1486-1507)
//
// No atomics touch results, so outputs are deterministic and a token's
// output does not depend on which other tokens share the batch except through
// the summation order of the combine, which follows the reference.
#include "jm_device.h"
#include "jm_kernels.h"

namespace jm {

// ------------------------------------------------------------------ router

// One thread per (token b, expert e, lane r of 8).  Lane r accumulates the
// FMA chain over columns j == r (mod 8) starting from +0; the 8 partials are
// combined as ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)), i.e. xor-butterflies
// 4, 2, 1, which is the reference's horizontal sum.
template <bool BF16>
__global__ void __launch_bounds__(256)
k_router_logits(const void* __restrict__ gate_w, const float* __restrict__ x,
                float* __restrict__ logits, int B, int E, int d) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int r = t & 7;
    const int pair = t >> 3;
    const bool live = pair < B * E;
    const int e = live ? pair % E : 0;
    const int b = live ? pair / E : 0;
    float acc = 0.0f;
    if (live) {
        const float* xb = x + (size_t)b * d;
        if (BF16) {
            const uint16_t* w = (const uint16_t*)gate_w + (size_t)e * d;
#pragma unroll 8
            for (int j = r; j < d; j += 8) acc = __builtin_fmaf(bf16_bits_to_f32(w[j]), xb[j], acc);
        } else {
            const float* w = (const float*)gate_w + (size_t)e * d;
#pragma unroll 8
            for (int j = r; j < d; j += 8) acc = __builtin_fmaf(w[j], xb[j], acc);
        }
    }
    acc = __fadd_rn(acc, __shfl_xor(acc, 4, JM_WAVE));
    acc = __fadd_rn(acc, __shfl_xor(acc, 2, JM_WAVE));
    acc = __fadd_rn(acc, __shfl_xor(acc, 1, JM_WAVE));
    if (live && r == 0) logits[(size_t)b * E + e] = acc;
}

// ------------------------------------------------------ activation digits

// Encode `ngroups` groups of G floats per row of `src` (row stride
// src_stride floats) into digits: dig[row][g][k][w] (NDIG x G/8 words per
// group) and scale[row][g].  One thread per (row, group).
template <int G, int NDIG>
__global__ void __launch_bounds__(256)
k_prep_digits(const float* __restrict__ src, int src_stride, int rows, int ngroups,
              uint32_t* __restrict__ dig, float* __restrict__ scale) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * ngroups) return;
    const int row = t / ngroups, g = t % ngroups;
    const float* v = src + (size_t)row * src_stride + (size_t)g * G;
    float vals[G];
    float mx = 0.0f;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < G; i += 4) {
        const float4 q = *(const float4*)(v + i);
        vals[i] = q.x; vals[i + 1] = q.y; vals[i + 2] = q.z; vals[i + 3] = q.w;
    }
#pragma unroll
    for (int i = 0; i < G; i++) {
        const float a = fabsf(vals[i]);
        bad |= !(a <= 3.4028235e38f);
        mx = fmaxf(mx, a);
    }
    const float s = digit_scale<NDIG>(mx, bad);
    const float inv = (mx > 0.0f && !bad) ? __fdiv_rn((float)Digits<NDIG>::R, mx) : 0.0f;
    uint32_t* out = dig + ((size_t)row * ngroups + g) * (NDIG * (G / 8));
#pragma unroll
    for (int w = 0; w < G / 8; w++) {
        uint32_t word[NDIG];
#pragma unroll
        for (int k = 0; k < NDIG; k++) word[k] = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int a = (int)rintf(__fmul_rn(vals[8 * w + i], inv));
            int dg[NDIG];
            split_digits<NDIG>(a, dg);
#pragma unroll
            for (int k = 0; k < NDIG; k++) word[k] |= ((uint32_t)dg[k] & 15u) << (4 * i);
        }
#pragma unroll
        for (int k = 0; k < NDIG; k++) out[k * (G / 8) + w] = word[k];
    }
    scale[(size_t)row * ngroups + g] = s;
}

// ------------------------------------------------------------------- top-k

// One wave per token.  E <= 64 * EPL.  Writes top[b][i], tw[b][i].
template <int EPL>
__global__ void __launch_bounds__(64)
k_topk(const float* __restrict__ logits, int E, int k, int renorm,
       int* __restrict__ top, float* __restrict__ tw) {
    __shared__ float p_lds[64 * EPL];
    __shared__ float total;
    __shared__ int top_lds[64];
    __shared__ float tw_lds[64];
    const int b = blockIdx.x;
    const int lane = threadIdx.x;
    const float* s = logits + (size_t)b * E;
    float v[EPL];
    float mx = -1e30f;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + 64 * j;
        v[j] = e < E ? s[e] : __int_as_float(0x7FC00000);
        if (v[j] > mx) mx = v[j];          // NaN never wins, as in the reference scan
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float other = __shfl_xor(mx, o, JM_WAVE);
        if (other > mx) mx = other;
    }
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + 64 * j;
        if (e < E) p_lds[e] = expf_fast(__fsub_rn(v[j], mx));
    }
    __syncthreads();
    if (lane == 0) {                       // sequential sum, e = 0..E-1
        float sum = 0.0f;
        for (int e = 0; e < E; e++) sum = __fadd_rn(sum, p_lds[e]);
        total = sum;
    }
    __syncthreads();
    const float sum = total;
    bool used[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + 64 * j;
        v[j] = e < E ? __fdiv_rn(p_lds[e], sum) : __int_as_float(0x7FC00000);
        used[j] = false;
    }
    for (int i = 0; i < k; i++) {
        // lane-local best: strict > over increasing index keeps the lowest
        float bv = -1e30f;
        int bi = -1;
#pragma unroll
        for (int j = 0; j < EPL; j++)
            if (!used[j] && v[j] > bv) { bv = v[j]; bi = lane + 64 * j; }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const float ov = __shfl_xor(bv, o, JM_WAVE);
            const int oi = __shfl_xor(bi, o, JM_WAVE);
            const bool take = (ov > bv) || (ov == bv && oi >= 0 && (bi < 0 || oi < bi));
            if (take) { bv = ov; bi = oi; }
        }
#pragma unroll
        for (int j = 0; j < EPL; j++)
            if (bi == lane + 64 * j) used[j] = true;
        if (lane == 0) { top_lds[i] = bi; tw_lds[i] = bv; }
    }
    __syncthreads();
    if (lane == 0 && renorm) {
        float ss = 0.0f;
        for (int i = 0; i < k; i++) ss = __fadd_rn(ss, tw_lds[i]);
        for (int i = 0; i < k; i++) tw_lds[i] = __fdiv_rn(tw_lds[i], ss);
    }
    __syncthreads();
    if (lane < k) {
        top[(size_t)b * k + lane] = top_lds[lane];
        tw[(size_t)b * k + lane] = tw_lds[lane];
    }
}

// ---------------------------------------------------------------- dispatch

// Single block of 1024 threads.  Stable counting sort of nslot = B*k slots
// by expert id (E <= 512, nslot <= 65536).  The slots are cut into
// DISP_CHUNKS contiguous chunks; per-(chunk, expert) counts live in LDS, a
// slot's position is its expert's segment start + the counts of earlier
// chunks + its rank among equal experts earlier in its own chunk.
// rank_scratch [nslot] is written and read back by the same thread.
constexpr int DISP_CHUNKS = 16;
constexpr int DISP_MAX_E = 512;

__global__ void __launch_bounds__(1024)
k_dispatch(const int* __restrict__ top, int nslot, int E,
           int* __restrict__ seg_off, int* __restrict__ seg_slot, int* __restrict__ active,
           int* __restrict__ n_active, int* __restrict__ first_slot, int* __restrict__ rank_scratch) {
    __shared__ int cnt[DISP_CHUNKS][DISP_MAX_E];
    __shared__ int off_lds[DISP_MAX_E + 1];
    const int tid = threadIdx.x, nth = blockDim.x;
    const int chunk = (nslot + DISP_CHUNKS - 1) / DISP_CHUNKS;
    for (int i = tid; i < DISP_CHUNKS * DISP_MAX_E; i += nth) (&cnt[0][0])[i] = 0;
    __syncthreads();
    for (int s = tid; s < nslot; s += nth) {
        const int e = top[s];
        if (e < 0 || e >= E) { rank_scratch[s] = -1; continue; }
        const int c = s / chunk;
        int rank = 0;
        for (int q = c * chunk; q < s; q++) rank += (top[q] == e);
        rank_scratch[s] = rank;
        atomicAdd(&cnt[c][e], 1);
    }
    __syncthreads();
    for (int e = tid; e < E; e += nth) {       // exclusive prefix over chunks
        int run = 0;
        for (int c = 0; c < DISP_CHUNKS; c++) {
            const int n = cnt[c][e];
            cnt[c][e] = run;
            run += n;
        }
        off_lds[e] = run;                      // per-expert total for now
    }
    __syncthreads();
    if (tid == 0) {
        int acc = 0, U = 0;
        for (int e = 0; e < E; e++) {
            const int n = off_lds[e];
            off_lds[e] = acc;
            if (n > 0) active[U++] = e;
            acc += n;
        }
        off_lds[E] = acc;
        *n_active = U;
    }
    __syncthreads();
    for (int e = tid; e <= E; e += nth) seg_off[e] = off_lds[e];
    for (int s = tid; s < nslot; s += nth) {
        const int rank = rank_scratch[s];
        if (rank < 0) continue;
        const int e = top[s];
        const int pos = off_lds[e] + cnt[s / chunk][e] + rank;
        seg_slot[pos] = s;
        if (pos == off_lds[e]) first_slot[e] = s;
    }
}

// ------------------------------------------------------------ expert rows

// Digits of one token for this lane's group: NDIG x (G/8) words.
template <int G, int NDIG>
struct TokDigits {
    uint32_t w[NDIG][G / 8];
    float s;
};

template <int G, int NDIG>
__device__ __forceinline__ void load_digits(TokDigits<G, NDIG>& td, const uint32_t* __restrict__ dig,
                                            const float* __restrict__ scale, size_t group_index,
                                            bool live) {
    if (!live) {
#pragma unroll
        for (int k = 0; k < NDIG; k++)
#pragma unroll
            for (int w = 0; w < G / 8; w++) td.w[k][w] = 0;
        td.s = 0.0f;
        return;
    }
    const uint4* p = (const uint4*)(dig + group_index * (NDIG * (G / 8)));
#pragma unroll
    for (int k = 0; k < NDIG; k++)
#pragma unroll
        for (int w4 = 0; w4 < G / 32; w4++) {
            const uint4 q = p[k * (G / 32) + w4];
            td.w[k][4 * w4] = q.x; td.w[k][4 * w4 + 1] = q.y;
            td.w[k][4 * w4 + 2] = q.z; td.w[k][4 * w4 + 3] = q.w;
        }
    td.s = scale[group_index];
}

// Integer group dot: sum_j (q_j - 8) * a_j with a_j given by its digits.
// wq holds the G/8 packed words of the weight group already XOR 0x88888888.
template <int G, int NDIG>
__device__ __forceinline__ int group_dot(const uint32_t* wq, const TokDigits<G, NDIG>& td) {
    int acc = 0;
#pragma unroll
    for (int k = NDIG - 1; k >= 0; k--) {
        acc <<= 4;
#pragma unroll
        for (int w = 0; w < G / 8; w++) acc = dot8(wq[w], td.w[k][w], acc);
    }
    return acc;
}

template <int G>
__device__ __forceinline__ void load_group(uint32_t* wq, const uint8_t* __restrict__ p) {
    const uint4* q = (const uint4*)p;
#pragma unroll
    for (int i = 0; i < G / 32; i++) {
        const uint4 v = q[i];
        wq[4 * i] = v.x ^ 0x88888888u; wq[4 * i + 1] = v.y ^ 0x88888888u;
        wq[4 * i + 2] = v.z ^ 0x88888888u; wq[4 * i + 3] = v.w ^ 0x88888888u;
    }
}

// Gate/up pass.  Block = 512 threads (8 waves) per (active expert, block of
// RB = 64 rows).  LPR = d / G lanes per row (one weight group per lane),
// RPW = 64 / LPR rows per wave per step, each wave owns 8 consecutive rows.
template <int G, int NDIG, int NT, int LPR>
__global__ void __launch_bounds__(512)
k_gateup(ExpertArgs a) {
    constexpr int RB = 64;
    constexpr int WAVES = 8;
    constexpr int ROWS_PER_WAVE = RB / WAVES;
    constexpr int RPW = JM_WAVE / LPR;       // LPR == d / G (checked on the host)
    const int nblk = a.m / RB;
    const int u = blockIdx.x / nblk, rb = blockIdx.x % nblk;
    if (u >= *a.n_active) return;
    const int e = a.active[u];
    const int s0 = a.seg_off[e], n = a.seg_off[e + 1] - s0;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane % LPR, rsub = lane / LPR;
    const int ngroups = a.d / G;
    const uint8_t* blob = a.blob;
    const size_t ke = (size_t)a.layer * a.E + e;
    const uint8_t* pk_g = blob + a.off[(0 * a.LE + ke) * 2 + 1];
    const uint16_t* sc_g = (const uint16_t*)(blob + a.off[(0 * a.LE + ke) * 2 + 0]);
    const uint8_t* pk_u = blob + a.off[(1 * a.LE + ke) * 2 + 1];
    const uint16_t* sc_u = (const uint16_t*)(blob + a.off[(1 * a.LE + ke) * 2 + 0]);

    __shared__ float act_lds[NT][RB];
    __shared__ int slot_lds[NT];

    for (int c0 = 0; c0 < n; c0 += NT) {
        const int nt = min(NT, n - c0);
        if (threadIdx.x < NT) slot_lds[threadIdx.x] = threadIdx.x < nt ? a.seg_slot[s0 + c0 + threadIdx.x] : 0;
        __syncthreads();
        TokDigits<G, NDIG> td[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int slot = slot_lds[t];
            const int b = slot / a.topk;
            load_digits<G, NDIG>(td[t], a.xdig, a.xscale, (size_t)b * ngroups + g, t < nt);
        }
        constexpr int steps = ROWS_PER_WAVE / RPW;
#pragma unroll 2
        for (int it = 0; it < steps; it++) {
            const int row_local = wave * ROWS_PER_WAVE + it * RPW + rsub;
            const int row = rb * RB + row_local;
            uint32_t wg[G / 8], wu[G / 8];
            load_group<G>(wg, pk_g + (size_t)row * (a.d / 2) + (size_t)g * (G / 2));
            load_group<G>(wu, pk_u + (size_t)row * (a.d / 2) + (size_t)g * (G / 2));
            const float sg = fp16_hw(sc_g[(size_t)row * ngroups + g]);
            const float su = fp16_hw(sc_u[(size_t)row * ngroups + g]);
#pragma unroll
            for (int t = 0; t < NT; t++) {
                if (t >= nt) break;
                const int ig = group_dot<G, NDIG>(wg, td[t]);
                const int iu = group_dot<G, NDIG>(wu, td[t]);
                float vg = __fmul_rn((float)ig, __fmul_rn(td[t].s, sg));
                float vu = __fmul_rn((float)iu, __fmul_rn(td[t].s, su));
                vg = seg_sum<LPR>(vg);
                vu = seg_sum<LPR>(vu);
                if (g == 0) {
                    const float av = swiglu(vg, vu);
                    act_lds[t][row_local] = av;
                    a.act[(size_t)slot_lds[t] * a.m + row] = av;
                }
            }
        }
        __syncthreads();
        // re-encode the act groups of this row block for the down pass:
        // one thread per (token, group, word)
        constexpr int GPB = RB / G;          // groups per block
        const int nwork = nt * GPB * (G / 8);
        for (int w = threadIdx.x; w < nwork; w += blockDim.x) {
            const int t = w / (GPB * (G / 8));
            const int grp = (w / (G / 8)) % GPB;
            const int word = w % (G / 8);
            const float* gv = &act_lds[t][grp * G];
            float mx = 0.0f;
            bool bad = false;
            for (int i = 0; i < G; i++) {
                const float av = fabsf(gv[i]);
                bad |= !(av <= 3.4028235e38f);
                mx = fmaxf(mx, av);
            }
            const float s = digit_scale<NDIG>(mx, bad);
            const float inv = (mx > 0.0f && !bad) ? __fdiv_rn((float)Digits<NDIG>::R, mx) : 0.0f;
            uint32_t wd[NDIG];
#pragma unroll
            for (int k = 0; k < NDIG; k++) wd[k] = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int q = (int)rintf(__fmul_rn(gv[8 * word + i], inv));
                int dg[NDIG];
                split_digits<NDIG>(q, dg);
#pragma unroll
                for (int k = 0; k < NDIG; k++) wd[k] |= ((uint32_t)dg[k] & 15u) << (4 * i);
            }
            const size_t gi = (size_t)slot_lds[t] * (a.m / G) + (size_t)rb * GPB + grp;
            uint32_t* dst = a.adig + gi * (NDIG * (G / 8));
#pragma unroll
            for (int k = 0; k < NDIG; k++) dst[k * (G / 8) + word] = wd[k];
            if (word == 0) a.ascale[gi] = s;
        }
        __syncthreads();
    }
}

// Down pass.  Block = 512 threads per (active expert, block of RBD rows).
// LPR = lanes per row = next power of two >= m / G; lanes past m / G idle.
template <int G, int NDIG, int NT, int LPR>
__global__ void __launch_bounds__(512)
k_down(ExpertArgs a) {
    constexpr int RBD = 128;
    constexpr int WAVES = 8;
    constexpr int ROWS_PER_WAVE = RBD / WAVES;
    constexpr int RPW = JM_WAVE / LPR;
    const int nblk = a.d / RBD;
    const int u = blockIdx.x / nblk, rb = blockIdx.x % nblk;
    if (u >= *a.n_active) return;
    const int e = a.active[u];
    const int s0 = a.seg_off[e], n = a.seg_off[e + 1] - s0;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane % LPR, rsub = lane / LPR;
    const int ngroups = a.m / G;
    const bool glive = g < ngroups;
    const size_t ke = (size_t)a.layer * a.E + e;
    const uint8_t* pk_d = a.blob + a.off[(2 * a.LE + ke) * 2 + 1];
    const uint16_t* sc_d = (const uint16_t*)(a.blob + a.off[(2 * a.LE + ke) * 2 + 0]);

    for (int c0 = 0; c0 < n; c0 += NT) {
        const int nt = min(NT, n - c0);
        int slot[NT];
        float wt[NT];
        TokDigits<G, NDIG> td[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            slot[t] = t < nt ? a.seg_slot[s0 + c0 + t] : 0;
            wt[t] = t < nt ? a.tw[slot[t]] : 0.0f;
            load_digits<G, NDIG>(td[t], a.adig, a.ascale, (size_t)slot[t] * ngroups + g, t < nt && glive);
        }
        constexpr int steps = ROWS_PER_WAVE / RPW;
#pragma unroll 2
        for (int it = 0; it < steps; it++) {
            const int row = rb * RBD + wave * ROWS_PER_WAVE + it * RPW + rsub;
            uint32_t wd[G / 8];
            float sd = 0.0f;
            if (glive) {
                load_group<G>(wd, pk_d + (size_t)row * (a.m / 2) + (size_t)g * (G / 2));
                sd = fp16_hw(sc_d[(size_t)row * ngroups + g]);
            } else {
#pragma unroll
                for (int w = 0; w < G / 8; w++) wd[w] = 0;
            }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                if (t >= nt) break;
                const int iv = group_dot<G, NDIG>(wd, td[t]);
                float v = glive ? __fmul_rn((float)iv, __fmul_rn(td[t].s, sd)) : 0.0f;
                v = seg_sum<LPR>(v);
                if (g == 0) a.y[(size_t)slot[t] * a.d + row] = __fmul_rn(wt[t], v);
            }
        }
    }
}

// ----------------------------------------------------------------- combine

// out[b][r] = sum over the token's slots, ordered by the first slot at which
// their expert appears in the batch (the reference's union order), from +0.
__global__ void __launch_bounds__(256)
k_combine(const float* __restrict__ y, const int* __restrict__ top,
          const int* __restrict__ first_slot, int k, int d, float* __restrict__ out) {
    const int b = blockIdx.y;
    __shared__ int order[32];
    if (threadIdx.x == 0) {
        int key[32], sl[32], n = 0;
        for (int i = 0; i < k; i++) {
            const int e = top[(size_t)b * k + i];
            if (e < 0) continue;
            const int kk = first_slot[e];
            int p = n++;
            while (p > 0 && key[p - 1] > kk) { key[p] = key[p - 1]; sl[p] = sl[p - 1]; p--; }
            key[p] = kk;
            sl[p] = b * k + i;
        }
        for (int i = 0; i < k; i++) order[i] = i < n ? sl[i] : -1;
    }
    __syncthreads();
    const int r = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (r >= d) return;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int i = 0; i < k; i++) {
        const int s = order[i];
        if (s < 0) break;
        const float4 v = *(const float4*)(y + (size_t)s * d + r);
        acc.x = __fadd_rn(acc.x, v.x); acc.y = __fadd_rn(acc.y, v.y);
        acc.z = __fadd_rn(acc.z, v.z); acc.w = __fadd_rn(acc.w, v.w);
    }
    *(float4*)(out + (size_t)b * d + r) = acc;
}

// ----------------------------------------------------- plain Q4 products

// Exact dequantisation (q - 8) * fp32(scale) of one tensor record.
template <int G>
__global__ void __launch_bounds__(256)
k_dequant(const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales,
          long long numel, float* __restrict__ out) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= numel) return;
    const uint8_t byte = packed[i >> 1];
    const int q = (i & 1) ? (byte >> 4) : (byte & 15);
    out[i] = __fmul_rn((float)(q - 8), fp16_bits_to_f32(scales[i / G]));
}

// Rows of one Q4 matrix against T token digit vectors: out[t][row] (row
// stride ostride).  Block = 256 threads; LPR lanes per row.
template <int G, int NDIG, int NT, int LPR>
__global__ void __launch_bounds__(256)
k_q4_rows(const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales,
          int rows, int cols, const uint32_t* __restrict__ dig, const float* __restrict__ dscale,
          int T, float* __restrict__ out, int ostride) {
    constexpr int RPW = JM_WAVE / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane % LPR, rsub = lane / LPR;
    const int ngroups = cols / G;
    const bool glive = g < ngroups;
    const int row = (blockIdx.x * 4 + wave) * RPW + rsub;
    const bool rlive = row < rows;
    uint32_t wq[G / 8];
    float sw = 0.0f;
    if (glive && rlive) {
        load_group<G>(wq, packed + (size_t)row * (cols / 2) + (size_t)g * (G / 2));
        sw = fp16_hw(scales[(size_t)row * ngroups + g]);
    } else {
#pragma unroll
        for (int w = 0; w < G / 8; w++) wq[w] = 0;
    }
    for (int t0 = 0; t0 < T; t0 += NT) {
#pragma unroll
        for (int tt = 0; tt < NT; tt++) {
            const int t = t0 + tt;
            if (t >= T) break;
            TokDigits<G, NDIG> td;
            load_digits<G, NDIG>(td, dig, dscale, (size_t)t * ngroups + g, glive);
            const int iv = group_dot<G, NDIG>(wq, td);
            float v = (glive && rlive) ? __fmul_rn((float)iv, __fmul_rn(td.s, sw)) : 0.0f;
            v = seg_sum<LPR>(v);
            if (g == 0 && rlive) out[(size_t)t * ostride + row] = v;
        }
    }
}

// ------------------------------------------------------------ host launch

static inline dim3 grid1(long long n, int bs) { return dim3((unsigned)((n + bs - 1) / bs)); }

hipError_t launch_router(const void* gate_w, int bf16, const float* x, float* logits,
                         int B, int E, int d, hipStream_t st) {
    const long long n = (long long)B * E * 8;
    if (bf16)
        hipLaunchKernelGGL(k_router_logits<true>, grid1(n, 256), dim3(256), 0, st, gate_w, x, logits, B, E, d);
    else
        hipLaunchKernelGGL(k_router_logits<false>, grid1(n, 256), dim3(256), 0, st, gate_w, x, logits, B, E, d);
    return hipGetLastError();
}

hipError_t launch_prep_digits(const float* src, int stride, int rows, int cols, int group,
                              uint32_t* dig, float* scale, hipStream_t st) {
    const int ng = cols / group;
    const long long n = (long long)rows * ng;
    if (n == 0) return hipSuccess;
    if (group == 64)
        hipLaunchKernelGGL((k_prep_digits<64, JM_NDIG>), grid1(n, 256), dim3(256), 0, st, src, stride, rows, ng, dig, scale);
    else
        hipLaunchKernelGGL((k_prep_digits<32, JM_NDIG>), grid1(n, 256), dim3(256), 0, st, src, stride, rows, ng, dig, scale);
    return hipGetLastError();
}

hipError_t launch_topk(const float* logits, int B, int E, int k, int renorm, int* top, float* tw,
                       hipStream_t st) {
    if (E <= 64) hipLaunchKernelGGL(k_topk<1>, dim3(B), dim3(64), 0, st, logits, E, k, renorm, top, tw);
    else if (E <= 128) hipLaunchKernelGGL(k_topk<2>, dim3(B), dim3(64), 0, st, logits, E, k, renorm, top, tw);
    else if (E <= 256) hipLaunchKernelGGL(k_topk<4>, dim3(B), dim3(64), 0, st, logits, E, k, renorm, top, tw);
    else hipLaunchKernelGGL(k_topk<8>, dim3(B), dim3(64), 0, st, logits, E, k, renorm, top, tw);
    return hipGetLastError();
}

hipError_t launch_dispatch(const int* top, int nslot, int E, int* seg_off, int* seg_slot,
                           int* active, int* n_active, int* first_slot, int* rank_scratch,
                           hipStream_t st) {
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, st, top, nslot, E, seg_off, seg_slot,
                       active, n_active, first_slot, rank_scratch);
    return hipGetLastError();
}

hipError_t launch_experts(const ExpertArgs& a, int umax, hipStream_t st) {
    const int nblk_gu = a.m / 64;
    const int nblk_dn = a.d / 128;
    const int lpr_gu = a.d / a.group;
    const int lpr_dn = a.m / a.group <= 16 ? 16 : a.m / a.group <= 32 ? 32 : 64;
    const dim3 ggu(umax * nblk_gu);
#define JM_GU(GG, L) hipLaunchKernelGGL((k_gateup<GG, JM_NDIG, JM_NT, L>), ggu, dim3(512), 0, st, a)
    if (a.group == 64) {
        if (lpr_gu == 16) JM_GU(64, 16); else if (lpr_gu == 32) JM_GU(64, 32); else JM_GU(64, 64);
        if (lpr_dn == 16) hipLaunchKernelGGL((k_down<64, JM_NDIG, JM_NT, 16>), dim3(umax * nblk_dn), dim3(512), 0, st, a);
        else if (lpr_dn == 32) hipLaunchKernelGGL((k_down<64, JM_NDIG, JM_NT, 32>), dim3(umax * nblk_dn), dim3(512), 0, st, a);
        else hipLaunchKernelGGL((k_down<64, JM_NDIG, JM_NT, 64>), dim3(umax * nblk_dn), dim3(512), 0, st, a);
    } else {
        if (lpr_gu == 16) JM_GU(32, 16); else if (lpr_gu == 32) JM_GU(32, 32); else JM_GU(32, 64);
        if (lpr_dn == 16) hipLaunchKernelGGL((k_down<32, JM_NDIG, JM_NT, 16>), dim3(umax * nblk_dn), dim3(512), 0, st, a);
        else if (lpr_dn == 32) hipLaunchKernelGGL((k_down<32, JM_NDIG, JM_NT, 32>), dim3(umax * nblk_dn), dim3(512), 0, st, a);
        else hipLaunchKernelGGL((k_down<32, JM_NDIG, JM_NT, 64>), dim3(umax * nblk_dn), dim3(512), 0, st, a);
    }
#undef JM_GU
    return hipGetLastError();
}

hipError_t launch_combine(const float* y, const int* top, const int* first_slot, int B, int k, int d,
                          float* out, hipStream_t st) {
    dim3 grid((unsigned)((d / 4 + 255) / 256), (unsigned)B);
    hipLaunchKernelGGL(k_combine, grid, dim3(256), 0, st, y, top, first_slot, k, d, out);
    return hipGetLastError();
}

hipError_t launch_dequant(const uint8_t* packed, const uint16_t* scales, long long numel, int group,
                          float* out, hipStream_t st) {
    if (numel == 0) return hipSuccess;
    if (group == 64) hipLaunchKernelGGL(k_dequant<64>, grid1(numel, 256), dim3(256), 0, st, packed, scales, numel, out);
    else hipLaunchKernelGGL(k_dequant<32>, grid1(numel, 256), dim3(256), 0, st, packed, scales, numel, out);
    return hipGetLastError();
}

hipError_t launch_q4_rows(const uint8_t* packed, const uint16_t* scales, int rows, int cols, int group,
                          const uint32_t* dig, const float* dscale, int T, float* out, int ostride,
                          hipStream_t st) {
    const int ng = cols / group;
    const int lpr = ng <= 16 ? 16 : ng <= 32 ? 32 : 64;
    const int rows_per_block = 4 * (64 / lpr);
    const dim3 grid((unsigned)((rows + rows_per_block - 1) / rows_per_block));
#define JM_ROWS(GG, L) hipLaunchKernelGGL((k_q4_rows<GG, JM_NDIG, JM_NT, L>), grid, dim3(256), 0, st, \
                                          packed, scales, rows, cols, dig, dscale, T, out, ostride)
    if (group == 64) {
        if (lpr == 16) JM_ROWS(64, 16); else if (lpr == 32) JM_ROWS(64, 32); else JM_ROWS(64, 64);
    } else {
        if (lpr == 16) JM_ROWS(32, 16); else if (lpr == 32) JM_ROWS(32, 32); else JM_ROWS(32, 64);
    }
#undef JM_ROWS
    return hipGetLastError();
}

}  // namespace jm
