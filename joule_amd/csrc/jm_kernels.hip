// Stage kernels behind the test entry points of the C ABI (jm_router,
// jm_dispatch, jm_q4_dequant) and the plain Q4 products of the
// KernelBackend API (jm_q4_gemv_f32 / jm_q4_gemm_f32).  They share the
// device functions of the fused MoE block (jm_device.h, jm_q4dot.h), so a
// stage computes exactly what the corresponding part of the block computes.
#include "jm_device.h"
#include "jm_kernels.h"
#include "jm_q4dot.h"

namespace jm {

// Router scores from the table in its natural [E][d] layout: one thread per
// (token, expert, chain r); chains and horizontal sum as in k_route.
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

// Digits of `rows` vectors of `cols` floats: one G-lane segment per group.
template <int G, int NDIG>
__global__ void __launch_bounds__(256)
k_prep_digits(const float* __restrict__ src, int src_stride, int rows, int ngroups,
              uint32_t* __restrict__ dig, float* __restrict__ scale) {
    const long long seg = ((long long)blockIdx.x * blockDim.x + threadIdx.x) / G;
    const bool ok = seg < (long long)rows * ngroups;
    const int row = ok ? (int)(seg / ngroups) : 0, g = ok ? (int)(seg % ngroups) : 0;
    const float v = ok ? src[(size_t)row * src_stride + (size_t)g * G + (threadIdx.x & (G - 1))] : 0.0f;
    const size_t gi = (size_t)row * ngroups + g;
    encode_group_wave<G, NDIG>(v, ok, dig + gi * (NDIG * (G / 8)), scale + gi);
}

template <int EPL>
__global__ void __launch_bounds__(64)
k_topk(const float* __restrict__ logits, int E, int k, int renorm, int* __restrict__ top,
       float* __restrict__ tw) {
    __shared__ float p_lds[64 * EPL];
    const int b = blockIdx.x;
    topk_wave<EPL>(logits + (size_t)b * E, E, k, renorm, p_lds, top + (size_t)b * k, tw + (size_t)b * k);
}

__global__ void __launch_bounds__(1024)
k_dispatch(const int* __restrict__ top, int nslot, int E, int k, int* __restrict__ seg_off,
           int* __restrict__ seg_slot, int* __restrict__ active, int* __restrict__ n_active,
           int* __restrict__ first_slot, int* __restrict__ comb) {
    extern __shared__ int lds_i[];
    dispatch_block(top, nslot, E, k, lds_i, seg_off, seg_slot, active, n_active, first_slot, comb);
}

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
// stride ostride).  256 threads; LPR lanes per row.
template <int G, int NDIG, int LPR>
__global__ void __launch_bounds__(256)
k_q4_rows(const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales,
          int rows, int cols, const uint32_t* __restrict__ dig, const float* __restrict__ dscale,
          int T, float* __restrict__ out, int ostride) {
    constexpr int RPW = JM_WAVE / LPR;
    constexpr int Q = G / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane & (LPR - 1), rsub = lane / LPR;
    const int ngroups = cols / G;
    const bool glive = g < ngroups;
    const int row = (blockIdx.x * 4 + wave) * RPW + rsub;
    const bool rlive = row < rows;
    uint4 wq[Q];
    float sw = 0.0f;
    if (glive && rlive) {
        const uint4* p = (const uint4*)(packed + (size_t)row * (cols / 2) + (size_t)g * (G / 2));
#pragma unroll
        for (int q = 0; q < Q; q++) {
            const uint4 v = p[q];
            wq[q] = make_uint4(v.x ^ 0x88888888u, v.y ^ 0x88888888u, v.z ^ 0x88888888u, v.w ^ 0x88888888u);
        }
        sw = fp16_hw(scales[(size_t)row * ngroups + g]);
    } else {
#pragma unroll
        for (int q = 0; q < Q; q++) wq[q] = make_uint4(0, 0, 0, 0);
    }
    for (int t = 0; t < T; t++) {
        TokDigits<G, NDIG> td;
        load_digits<G, NDIG>(td, dig, dscale, (size_t)t * ngroups + g, glive);
        const int iv = group_dot_flipped<G, NDIG>(wq, td);
        const float v = seg_sum<LPR>((glive && rlive) ? __fmul_rn((float)iv, __fmul_rn(td.s, sw)) : 0.0f);
        if (g == 0 && rlive) out[(size_t)t * ostride + row] = v;
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
                              uint32_t* dig, float* scale, hipStream_t st, int ndig) {
    const int ng = cols / group;
    const long long lanes = (long long)rows * ng * group;
    if (lanes == 0) return hipSuccess;
    if (ndig != 4 && ndig != 5) return hipErrorInvalidValue;
#define JM_PD(GG, N) hipLaunchKernelGGL((k_prep_digits<GG, N>), grid1(lanes, 256), dim3(256), 0, st, src, stride, rows, ng, dig, scale)
    if (group == 64) { if (ndig == 5) JM_PD(64, 5); else JM_PD(64, 4); }
    else { if (ndig == 5) JM_PD(32, 5); else JM_PD(32, 4); }
#undef JM_PD
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

hipError_t launch_dispatch(const int* top, int nslot, int E, int k, int* seg_off, int* seg_slot,
                           int* active, int* n_active, int* first_slot, int* comb, hipStream_t st) {
    const size_t lds = (size_t)dispatch_lds_ints(nslot, E) * 4;
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), lds, st, top, nslot, E, k, seg_off, seg_slot,
                       active, n_active, first_slot, comb);
    return hipGetLastError();
}

hipError_t launch_dequant(const uint8_t* packed, const uint16_t* scales, long long numel, int group,
                          float* out, hipStream_t st) {
    if (numel == 0) return hipSuccess;
    if (group == 64) hipLaunchKernelGGL(k_dequant<64>, grid1(numel, 256), dim3(256), 0, st, packed, scales, numel, out);
    else hipLaunchKernelGGL(k_dequant<32>, grid1(numel, 256), dim3(256), 0, st, packed, scales, numel, out);
    return hipGetLastError();
}

// act[i] = SiLU(g[i]) * u[i] for gu = [g; u], as the reference writes it
__global__ void __launch_bounds__(256)
k_swiglu_vec(const float* __restrict__ gu, int m, float* __restrict__ act) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < m) act[i] = swiglu(gu[i], gu[m + i]);
}

// v[i] = v[i] * s
__global__ void __launch_bounds__(256)
k_scale_vec(float* __restrict__ v, int n, float s) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) v[i] = __fmul_rn(v[i], s);
}

hipError_t launch_swiglu_vec(const float* gu, int m, float* act, hipStream_t st) {
    hipLaunchKernelGGL(k_swiglu_vec, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, st, gu, m, act);
    return hipGetLastError();
}

hipError_t launch_scale_vec(float* v, int n, float s, hipStream_t st) {
    hipLaunchKernelGGL(k_scale_vec, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, v, n, s);
    return hipGetLastError();
}

hipError_t launch_q4_rows(const uint8_t* packed, const uint16_t* scales, int rows, int cols, int group,
                          const uint32_t* dig, const float* dscale, int T, float* out, int ostride,
                          hipStream_t st) {
    const int ng = cols / group;
    const int lpr = ng <= 16 ? 16 : ng <= 32 ? 32 : 64;
    const int rows_per_block = 4 * (64 / lpr);
    const dim3 grid((unsigned)((rows + rows_per_block - 1) / rows_per_block));
#define JM_ROWS(GG, L) hipLaunchKernelGGL((k_q4_rows<GG, JM_NDIG, L>), grid, dim3(256), 0, st, \
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
