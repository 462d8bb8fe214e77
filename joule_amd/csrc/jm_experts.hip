// Grouped Q4 expert product of the MoE block (gfx950), three launches:
//
//   k_gateup   per (active expert, block of 64 intermediate rows):
//              g = gate_row . x, u = up_row . x for every token routed to the
//              expert, act = (g / (1 + expf_fast(-g))) * u
//              (decode_kernel.c:1365-1375), and the act groups re-encoded as
//              digits for the down pass
//   k_down     per (active expert, block of 128 hidden rows):
//              y[slot][r] = w_slot * (down_row . act_slot) (:1376-1383)
//   k_combine  out[b] = the token's k expert rows summed in the reference's
//              union order (:1502-1507)
//
// Lane layout: one Q4 group per lane.  A row of C columns is spread over
// LPR = next_pow2(C / G) lanes (lanes past C / G idle), a wave covers
// 64 / LPR rows per step, and the lanes' partial sums are reduced with DPP.
// A lane's G/2 packed bytes are one or two 16-byte loads.  Every weight load
// of a work item is issued before any arithmetic, so a wave has all of its
// rows in flight at once; the registers then serve every token of the
// segment in turn.  A block finds its expert, segment and record offsets in
// one load of the work table written by the dispatch.
//
// The group dot runs on v_dot8_i32_i4: the packed nibbles XOR 0x8 are the
// signed values q - 8, and each activation group is given as NDIG signed
// base-16 digits (exact integers a = rint(x / s)), so sum (q - 8) * a is
// computed exactly and scaled by s * fp16 scale in fp32.
#include "jm_device.h"
#include "jm_kernels.h"
#include "jm_q4dot.h"

namespace jm {

__device__ __forceinline__ uint4 flip_nibbles(uint4 v) {
    return make_uint4(v.x ^ 0x88888888u, v.y ^ 0x88888888u, v.z ^ 0x88888888u, v.w ^ 0x88888888u);
}

// ------------------------------------------------------------------ gate/up

template <int G, int NDIG, int LPR, int WAVES = 8>
__global__ void __launch_bounds__(WAVES * 64)
k_gateup(ExpertArgs a) {
    constexpr int RB = 64;
    constexpr int ROWS_PER_WAVE = RB / WAVES;
    constexpr int RPW = JM_WAVE / LPR;
    constexpr int STEPS = ROWS_PER_WAVE / RPW;
    constexpr int Q = G / 32;                          // uint4 per lane per row
    const int nblk = a.m / RB;
    const int u = blockIdx.x / nblk, rb = blockIdx.x % nblk;
    const ExpertWork wk = a.work[u];
    if (wk.n == 0) return;
    int slot = a.seg_slot[wk.s0];            // requested before the weights
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane & (LPR - 1), rsub = lane / LPR;
    const int ngroups = a.d / G;
    const uint8_t* pk_g = a.blob + wk.pk[0];
    const uint16_t* sc_g = (const uint16_t*)(a.blob + wk.sc[0]);
    const uint8_t* pk_u = a.blob + wk.pk[1];
    const uint16_t* sc_u = (const uint16_t*)(a.blob + wk.sc[1]);
    const int row0 = rb * RB + wave * ROWS_PER_WAVE + rsub;

    // every weight load of this wave's rows is issued before any arithmetic;
    // the token's digits are requested between the two halves so that the
    // first steps can start while the later rows are still in flight
    uint4 wg[STEPS][Q], wu[STEPS][Q];
    uint16_t hg[STEPS], hu[STEPS];
    TokDigits<G, NDIG> td;
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
        if (s == STEPS / 2)
            load_digits<G, NDIG>(td, a.xdig, a.xscale, (size_t)(slot / a.topk) * ngroups + g, true);
        const int row = row0 + s * RPW;
        const uint4* pg = (const uint4*)(pk_g + (size_t)row * (a.d / 2) + (size_t)g * (G / 2));
        const uint4* pu = (const uint4*)(pk_u + (size_t)row * (a.d / 2) + (size_t)g * (G / 2));
#pragma unroll
        for (int q = 0; q < Q; q++) { wg[s][q] = pg[q]; wu[s][q] = pu[q]; }
        hg[s] = sc_g[(size_t)row * ngroups + g];
        hu[s] = sc_u[(size_t)row * ngroups + g];
    }
    if (STEPS == 1) load_digits<G, NDIG>(td, a.xdig, a.xscale, (size_t)(slot / a.topk) * ngroups + g, true);

    __shared__ float act_lds[RB];
    for (int t = 0; t < wk.n; t++) {
        const int next = t + 1 < wk.n ? a.seg_slot[wk.s0 + t + 1] : 0;
#pragma unroll
        for (int s = 0; s < STEPS; s++) {
            const float sg = fp16_hw(hg[s]), su = fp16_hw(hu[s]);
            uint4 fg[Q], fu[Q];
#pragma unroll
            for (int q = 0; q < Q; q++) { fg[q] = flip_nibbles(wg[s][q]); fu[q] = flip_nibbles(wu[s][q]); }
            const int ig = group_dot_flipped<G, NDIG>(fg, td);
            const int iu = group_dot_flipped<G, NDIG>(fu, td);
            const float vg = seg_sum<LPR>(__fmul_rn((float)ig, __fmul_rn(td.s, sg)));
            const float vu = seg_sum<LPR>(__fmul_rn((float)iu, __fmul_rn(td.s, su)));
            if (g == 0) {
                const int row_local = wave * ROWS_PER_WAVE + s * RPW + rsub;
                const float av = swiglu(vg, vu);
                act_lds[row_local] = av;
                a.act[(size_t)slot * a.m + rb * RB + row_local] = av;
            }
        }
        __syncthreads();
        // digits of this token's act groups in the row block: one segment of
        // G lanes per group
        constexpr int GPB = RB / G;
        constexpr int PPW = JM_WAVE / G;
        if (wave * PPW < GPB) {
            const int grp = wave * PPW + lane / G;
            const bool ok = grp < GPB;
            const float v = act_lds[(ok ? grp : 0) * G + (lane & (G - 1))];
            const size_t gi = (size_t)slot * (a.m / G) + (size_t)rb * GPB + (ok ? grp : 0);
            encode_group_wave<G, NDIG>(v, ok, a.adig + gi * (NDIG * (G / 8)), a.ascale + gi);
        }
        if (t + 1 < wk.n) {
            slot = next;
            load_digits<G, NDIG>(td, a.xdig, a.xscale, (size_t)(slot / a.topk) * ngroups + g, true);
        }
        __syncthreads();
    }
}

// -------------------------------------------------------------------- down

template <int G, int NDIG, int LPR, int WAVES = 8, int RBD = 128>
__global__ void __launch_bounds__(WAVES * 64)
k_down(ExpertArgs a) {
    constexpr int ROWS_PER_WAVE = RBD / WAVES;
    constexpr int RPW = JM_WAVE / LPR;
    constexpr int STEPS = ROWS_PER_WAVE / RPW;
    constexpr int Q = G / 32;
    const int nblk = a.d / RBD;
    const int u = blockIdx.x / nblk, rb = blockIdx.x % nblk;
    const ExpertWork wk = a.work[u];
    if (wk.n == 0) return;
    int slot = a.seg_slot[wk.s0];            // requested before the weights
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane & (LPR - 1), rsub = lane / LPR;
    const int ngroups = a.m / G;
    const bool glive = g < ngroups;
    const uint8_t* pk_d = a.blob + wk.pk[2];
    const uint16_t* sc_d = (const uint16_t*)(a.blob + wk.sc[2]);
    const int row0 = rb * RBD + wave * ROWS_PER_WAVE + rsub;

    uint4 wd[STEPS][Q];
    uint16_t hd[STEPS];
    float wt = 0.0f;
    TokDigits<G, NDIG> td;
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
        if (s == STEPS / 2) {
            wt = a.tw[slot];
            load_digits<G, NDIG>(td, a.adig, a.ascale, (size_t)slot * ngroups + g, glive);
        }
        const int row = row0 + s * RPW;
        if (glive) {
            const uint4* p = (const uint4*)(pk_d + (size_t)row * (a.m / 2) + (size_t)g * (G / 2));
#pragma unroll
            for (int q = 0; q < Q; q++) wd[s][q] = p[q];
            hd[s] = sc_d[(size_t)row * ngroups + g];
        } else {
#pragma unroll
            for (int q = 0; q < Q; q++) wd[s][q] = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
            hd[s] = 0;
        }
    }
    if (STEPS == 1) {
        wt = a.tw[slot];
        load_digits<G, NDIG>(td, a.adig, a.ascale, (size_t)slot * ngroups + g, glive);
    }

    for (int t = 0; t < wk.n; t++) {
        const int next = t + 1 < wk.n ? a.seg_slot[wk.s0 + t + 1] : 0;
#pragma unroll
        for (int s = 0; s < STEPS; s++) {
            uint4 f[Q];
#pragma unroll
            for (int q = 0; q < Q; q++) f[q] = flip_nibbles(wd[s][q]);
            const int iv = group_dot_flipped<G, NDIG>(f, td);
            const float v = seg_sum<LPR>(glive ? __fmul_rn((float)iv, __fmul_rn(td.s, fp16_hw(hd[s]))) : 0.0f);
            if (g == 0) a.y[(size_t)slot * a.d + row0 + s * RPW] = __fmul_rn(wt, v);
        }
        if (t + 1 < wk.n) {
            slot = next;
            wt = a.tw[slot];
            load_digits<G, NDIG>(td, a.adig, a.ascale, (size_t)slot * ngroups + g, glive);
        }
    }
}

// ----------------------------------------------------------------- combine

__global__ void __launch_bounds__(256)
k_combine(const float* __restrict__ y, const int* __restrict__ comb, int B, int k, int d,
          float* __restrict__ out) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    const int d4 = d / 4;
    if (idx >= B * d4) return;
    const int b = idx / d4, r = 4 * (idx % d4);
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // no early exit: the loads of all k slots can be in flight together
#pragma unroll 8
    for (int i = 0; i < k; i++) {
        const int s = comb[b * k + i];
        const float4 v = s >= 0 ? *(const float4*)(y + (size_t)s * d + r) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (s >= 0) {
            acc.x = __fadd_rn(acc.x, v.x); acc.y = __fadd_rn(acc.y, v.y);
            acc.z = __fadd_rn(acc.z, v.z); acc.w = __fadd_rn(acc.w, v.w);
        }
    }
    *(float4*)(out + (size_t)b * d + r) = acc;
}

hipError_t launch_gateup(const ExpertArgs& a, int umax, hipStream_t st) {
    const dim3 grid(umax * (a.m / 64));
    const int lpr = a.d / a.group;
#define JM_GU(GG, L) hipLaunchKernelGGL((k_gateup<GG, JM_NDIG, L>), grid, dim3(512), 0, st, a)
    if (a.group == 64) {
        if (lpr == 16) JM_GU(64, 16); else if (lpr == 32) JM_GU(64, 32); else JM_GU(64, 64);
    } else {
        if (lpr == 16) JM_GU(32, 16); else if (lpr == 32) JM_GU(32, 32); else JM_GU(32, 64);
    }
#undef JM_GU
    return hipGetLastError();
}

hipError_t launch_down(const ExpertArgs& a, int umax, hipStream_t st) {
    const dim3 grid(umax * (a.d / 128));
    const int ng = a.m / a.group;
    const int lpr = ng <= 16 ? 16 : ng <= 32 ? 32 : 64;
#define JM_DN(GG, L) hipLaunchKernelGGL((k_down<GG, JM_NDIG, L>), grid, dim3(512), 0, st, a)
    if (a.group == 64) {
        if (lpr == 16) JM_DN(64, 16); else if (lpr == 32) JM_DN(64, 32); else JM_DN(64, 64);
    } else {
        if (lpr == 16) JM_DN(32, 16); else if (lpr == 32) JM_DN(32, 32); else JM_DN(32, 64);
    }
#undef JM_DN
    return hipGetLastError();
}

hipError_t launch_combine(const float* y, const int* comb, int B, int k, int d, float* out, hipStream_t st) {
    const long long n = (long long)B * (d / 4);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, y, comb, B, k, d, out);
    return hipGetLastError();
}

}  // namespace jm
