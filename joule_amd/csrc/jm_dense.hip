// The dense FFN of layer_ffn_batch's E == 0 branch (decode_kernel.c:1393-1422):
// act = silu(x W1^T) * (x W2^T), out = act W3^T, bf16 weights shared by the
// batch.  The products are the decoder's split-K projections (k_gemv_part,
// or k_gemm_bf16 for many tokens); two small kernels sum their slices:
//
//   k_swiglu_slices  the gate and up slices summed (times the RMSNorm row
//                    scale of the input, which the projection leaves out),
//                    then silu(g) * u                       (:1412-1415)
//   k_sum_slices     out = resid + the down slices summed  (:1416-1421, and
//                    the residual of decode_layers_batch, :1546-1552)
#include "jm_device.h"
#include "jm_kernels.h"

namespace jm {

// out[b][j] = (resid ? resid[b][j] : 0) + (part[0][b][j] + part[1][b][j] +
// ... ), the ns slices of part [ns][B][n] added in slice order; thread: 4
// consecutive values of one row.
__global__ void __launch_bounds__(256)
k_sum_slices(const float* __restrict__ resid, const float* __restrict__ part, int ns, int B, int n,
             float* __restrict__ out) {
    const int b = blockIdx.y;
    const int j4 = blockIdx.x * 256 + threadIdx.x;
    if (4 * j4 >= n) return;
    const size_t stride = (size_t)B * n / 4;
    const float4* p = (const float4*)(part + (size_t)b * n) + j4;
    float4 acc = p[0];
#pragma unroll 4
    for (int s = 1; s < ns; s++) {
        const float4 u = p[s * stride];
        acc = make_float4(__fadd_rn(acc.x, u.x), __fadd_rn(acc.y, u.y), __fadd_rn(acc.z, u.z), __fadd_rn(acc.w, u.w));
    }
    if (resid) {
        const float4 r = ((const float4*)(resid + (size_t)b * n))[j4];
        acc = make_float4(__fadd_rn(r.x, acc.x), __fadd_rn(r.y, acc.y), __fadd_rn(r.z, acc.z), __fadd_rn(r.w, acc.w));
    }
    ((float4*)(out + (size_t)b * n))[j4] = acc;
}

// act[b][i] = (g / (1 + expf_fast(-g))) * u (decode_kernel.c:1412-1415)
// with g, u the sums over the ns slices of gu [ns][B][2m] (gate rows
// 0..m-1, up rows m..2m-1), each times inv = 1 / sqrtf_fast(sum x^2 / d +
// eps) of the input row when rss [nrs][B] holds its sums of squares per
// slice (the projection took x * norm weight; the row scale comes after).
__global__ void __launch_bounds__(256)
k_swiglu_slices(const float* __restrict__ gu, int ns, const float* __restrict__ rss, int nrs, int d, float eps,
                int B, int m, float* __restrict__ act) {
    const int b = blockIdx.y;
    const int i4 = blockIdx.x * 256 + threadIdx.x;
    if (4 * i4 >= m) return;
    float inv = 1.0f;
    if (rss) {
        float ss = rss[b];
        for (int s = 1; s < nrs; s++) ss = __fadd_rn(ss, rss[(size_t)s * B + b]);
        inv = rms_inv(ss, d, eps);
    }
    const size_t stride = (size_t)B * 2 * m / 4;
    const float4* pg = (const float4*)(gu + (size_t)b * 2 * m) + i4;
    const float4* pu = (const float4*)(gu + (size_t)b * 2 * m + m) + i4;
    float4 g = pg[0], u = pu[0];
#pragma unroll 4
    for (int s = 1; s < ns; s++) {
        const float4 a = pg[s * stride], c = pu[s * stride];
        g = make_float4(__fadd_rn(g.x, a.x), __fadd_rn(g.y, a.y), __fadd_rn(g.z, a.z), __fadd_rn(g.w, a.w));
        u = make_float4(__fadd_rn(u.x, c.x), __fadd_rn(u.y, c.y), __fadd_rn(u.z, c.z), __fadd_rn(u.w, c.w));
    }
    const float gv[4] = {g.x, g.y, g.z, g.w}, uv[4] = {u.x, u.y, u.z, u.w};
    float r[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float gg = __fmul_rn(gv[e], inv), uu = __fmul_rn(uv[e], inv);
        r[e] = __fmul_rn(__fdiv_rn(gg, __fadd_rn(1.0f, expf_fast(-gg))), uu);
    }
    ((float4*)(act + (size_t)b * m))[i4] = make_float4(r[0], r[1], r[2], r[3]);
}

bool dense_shape_ok(int d, int m) { return gemv_shape_ok(d) && m >= 512 && m % 512 == 0 && m <= JM_DENSE_MAX_M; }

// The two products' shapes, and whether launch_dense_ffn takes the GEMM
// (from JM_GEMM_MIN_B tokens, when its shape allows) or the GEMV for them:
// the workspace sizing and the launcher make the same decision here.
static GemvArgs gu_shape(int d, int m, int B) {
    GemvArgs g{};
    g.rows[0] = m; g.rows[1] = m; g.rows[2] = 0;
    g.K = d; g.N = 2 * m; g.B = B;
    return g;
}

static GemvArgs dn_shape(int d, int m, int B) {
    GemvArgs o{};
    o.rows[0] = d;
    o.K = m; o.N = d; o.B = B;
    return o;
}

static bool gu_gemm(int d, int m, int B) { return B >= JM_GEMM_MIN_B && gemm_shape_ok(gu_shape(d, m, B)); }
static bool dn_gemm(int d, int m, int B) { return B >= JM_GEMM_MIN_B && gemm_shape_ok(dn_shape(d, m, B)); }

// the most slices the gate/up and down outputs hold at B tokens (the
// GEMM's K slices, at most 4, or the GEMV's K / slice columns)
int dense_gu_slices(int d, int m, int B) { return gu_gemm(d, m, B) ? 4 : d / gemv_slice_cols(d); }

int dense_dn_slices(int d, int m, int B) { return dn_gemm(d, m, B) ? 4 : m / gemv_slice_cols(m); }

hipError_t launch_dense_ffn(const DenseFfn& f, hipStream_t st) {
    if (f.B == 0) return hipSuccess;
    if (!dense_shape_ok(f.d, f.m)) return hipErrorInvalidValue;
    GemvArgs g = gu_shape(f.d, f.m, f.B);
    g.x = f.x;
    g.norm_w = f.norm_w;
    g.w[0] = f.w1; g.w[1] = f.w2; g.w[2] = nullptr;
    g.part = f.gu;
    g.rss = f.norm_w ? f.rss : nullptr;
    const bool gq = gu_gemm(f.d, f.m, f.B);
    hipError_t e = gq ? launch_gemm_bf16(g, st) : launch_gemv_part(g, st);
    if (e != hipSuccess) return e;
    const int ng = gq ? gemm_slices(g) : f.d / gemv_slice_cols(f.d);
    const dim3 ga((unsigned)((f.m / 4 + 255) / 256), (unsigned)f.B);
    hipLaunchKernelGGL(k_swiglu_slices, ga, dim3(256), 0, st, f.gu, ng, g.rss, ng, f.d, f.eps, f.B, f.m, f.act);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    GemvArgs o = dn_shape(f.d, f.m, f.B);
    o.x = f.act;
    o.w[0] = f.w3;
    o.part = f.dn;
    const bool go = dn_gemm(f.d, f.m, f.B);
    e = go ? launch_gemm_bf16(o, st) : launch_gemv_part(o, st);
    if (e != hipSuccess) return e;
    const int nd = go ? gemm_slices(o) : f.m / gemv_slice_cols(f.m);
    const dim3 gs((unsigned)((f.d / 4 + 255) / 256), (unsigned)f.B);
    hipLaunchKernelGGL(k_sum_slices, gs, dim3(256), 0, st, f.resid, f.dn, nd, f.B, f.d, f.out);
    return hipGetLastError();
}

hipError_t launch_sum_slices(const float* resid, const float* part, int ns, int B, int n, float* out,
                             hipStream_t st) {
    if (B == 0) return hipSuccess;
    const dim3 gs((unsigned)((n / 4 + 255) / 256), (unsigned)B);
    hipLaunchKernelGGL(k_sum_slices, gs, dim3(256), 0, st, resid, part, ns, B, n, out);
    return hipGetLastError();
}

}  // namespace jm
