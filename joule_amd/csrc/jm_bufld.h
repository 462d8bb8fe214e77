// Raw buffer loads with per-range descriptors (gfx950), shared by the
// small-batch kernels.  A load whose offset lies outside the descriptor's
// range returns zero without touching memory: an item past the end of a
// wave's list is given a zero-length range, so that every wave issues the
// same loads in the same order and the compiler's memory-counter waits stay
// exact.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jm_device.h"

namespace jm {

constexpr unsigned RSRC_W3 = 0x00020000u;   // buffer descriptor word 3 (gfx9: 32-bit data format)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(unsigned long long addr, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)addr, (short)0, bytes, (int)RSRC_W3);
}

__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, unsigned off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint2 bload8(__amdgpu_buffer_rsrc_t r, unsigned off) {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return make_uint2(v.x, v.y);
}

__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

__device__ __forceinline__ uint32_t bload2(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// a wave-uniform 64-bit value (an address read from LDS) in scalar registers
__device__ __forceinline__ unsigned long long uniform64(unsigned long long v) {
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    return ((unsigned long long)hi << 32) | lo;
}

}  // namespace jm
