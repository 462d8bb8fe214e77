// Q4 group dot on v_dot8_i32_i4 shared by the expert kernels and the plain
// Q4 products.
#pragma once

#include "jm_device.h"

namespace jm {

// Digits of one token for one Q4 group: NDIG words per 8 values, and the
// group's activation scale.
template <int G, int NDIG>
struct TokDigits {
    uint32_t w[NDIG][G / 8];
    float s;
};

template <int G, int NDIG>
__device__ __forceinline__ void load_digits(TokDigits<G, NDIG>& td, const uint32_t* __restrict__ dig,
                                            const float* __restrict__ scale, size_t gi, bool live) {
    if (!live) {
#pragma unroll
        for (int k = 0; k < NDIG; k++)
#pragma unroll
            for (int w = 0; w < G / 8; w++) td.w[k][w] = 0;
        td.s = 0.0f;
        return;
    }
    const uint4* p = (const uint4*)(dig + gi * (NDIG * (G / 8)));
#pragma unroll
    for (int k = 0; k < NDIG; k++)
#pragma unroll
        for (int q = 0; q < G / 32; q++) {
            const uint4 v = p[k * (G / 32) + q];
            td.w[k][4 * q] = v.x; td.w[k][4 * q + 1] = v.y;
            td.w[k][4 * q + 2] = v.z; td.w[k][4 * q + 3] = v.w;
        }
    td.s = scale[gi];
}

// sum_j (q_j - 8) * a_j over one group; wq holds the packed words already
// XOR 0x88888888, i.e. the signed nibbles q - 8.
template <int G, int NDIG>
__device__ __forceinline__ int group_dot_flipped(const uint4* wq, const TokDigits<G, NDIG>& td) {
    int acc = 0;
#pragma unroll
    for (int k = NDIG - 1; k >= 0; k--) {
        acc <<= 4;
#pragma unroll
        for (int q = 0; q < G / 32; q++) {
            acc = dot8(wq[q].x, td.w[k][4 * q], acc);
            acc = dot8(wq[q].y, td.w[k][4 * q + 1], acc);
            acc = dot8(wq[q].z, td.w[k][4 * q + 2], acc);
            acc = dot8(wq[q].w, td.w[k][4 * q + 3], acc);
        }
    }
    return acc;
}

}  // namespace jm
