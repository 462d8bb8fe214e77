// Launch and hand-off cost probes (libjoule_probe.so; bench.py --probe).
//
// Not part of the MoE block: these measure the two costs that decide
// whether a cross-block dependency inside the block should be a kernel
// boundary or an in-kernel hand-off.
//
//   jmp_launch_chain  n launches of a one-wave kernel on one stream, each
//                     reading what the previous one wrote (a dependent chain,
//                     as the block's router -> gate/up -> down), timed with
//                     HIP events; optionally captured once into a HIP graph
//                     and replayed.  Result: microseconds per launch.
//   jmp_stream        a plain read stream of nbytes, each wave reading its
//                     own contiguous piece (the expert kernels' pattern),
//                     rotating over regions copies so that no launch finds
//                     its bytes in a cache; microseconds per launch.
//   jmp_handoff       one launch of nblk blocks of 256 threads.  Each block
//                     sums its slice of a buffer and stores its partial; with
//                     the hand-off on, each block then issues a release fence
//                     and takes a ticket from one device-scope counter, and
//                     the block that takes the last ticket reads every
//                     partial (device-scope loads) and writes the total: the
//                     "last block finishes the work" pattern.  Result:
//                     microseconds per launch, averaged over reps launches;
//                     the difference of the two settings is the hand-off.
//
// Every kernel ends after a fixed amount of work: no block waits on
// another; the last-ticket block only reads what the other blocks already
// stored before taking their tickets.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "joule_probe.h"

namespace {

__global__ void k_touch(unsigned* p) {
    // one wave; lane 0 reads the previous launch's value and writes the next
    if (threadIdx.x == 0) p[0] = p[0] + 1u;
}

constexpr int HT = 256;

template <bool HANDOFF>
__global__ void __launch_bounds__(HT) k_handoff(const float* __restrict__ src, int per_block, float* part,
                                                 unsigned* ticket, float* out, int nblk) {
    __shared__ float red[HT / 64];
    __shared__ int last;
    const float* s = src + (size_t)blockIdx.x * per_block;
    float acc = 0.0f;
    for (int i = threadIdx.x; i < per_block; i += HT) acc += s[i];
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
        for (int w = 0; w < HT / 64; w++) t += red[w];
        if (!HANDOFF) {
            part[blockIdx.x] = t;
        } else {
            __hip_atomic_store(&part[blockIdx.x], t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __atomic_thread_fence(__ATOMIC_RELEASE);
            const unsigned k = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            last = (k == (unsigned)nblk - 1u);
        }
    }
    if (!HANDOFF) return;
    __syncthreads();
    if (!last) return;
    __atomic_thread_fence(__ATOMIC_ACQUIRE);
    float t = 0.0f;
    for (int b = threadIdx.x; b < nblk; b += HT)
        t += __hip_atomic_load(&part[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = t;
    __syncthreads();
    if (threadIdx.x == 0) {
        float u = 0.0f;
        for (int w = 0; w < HT / 64; w++) u += red[w];
        out[0] = u;
        // every block has taken its ticket: reset it for the next launch
        __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Stream: each wave reads its WB-byte piece of src (64 lanes x 16 bytes
// per load, every load issued before any is used) and stores one word, so
// that the loads stay live.  The plain read stream of a kernel whose waves
// each own a contiguous piece, as the expert kernels' wave items do.
template <int NLD>
__global__ void __launch_bounds__(256) k_stream(const uint4* __restrict__ src, unsigned* __restrict__ out) {
    const size_t wave = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const uint4* p = src + wave * NLD * 64 + lane;
    uint4 v[NLD];
#pragma unroll
    for (int i = 0; i < NLD; i++) v[i] = p[(size_t)i * 64];
    unsigned x = 0;
#pragma unroll
    for (int i = 0; i < NLD; i++) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    // every lane's loads feed the stored word (a word stored by lane 0 of
    // its own loads only would let the compiler sink the loads into the
    // store's branch)
    for (int o = 32; o > 0; o >>= 1) x ^= (unsigned)__shfl_xor((int)x, o);
    if (lane == 0) out[wave] = x;
}

// distinct words everywhere (a multiplicative hash of the index)
__global__ void k_fill(unsigned* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = (unsigned)(i * 2654435761ull) ^ (unsigned)(i >> 29);
}

thread_local char g_err[256];

int fail(const char* what, hipError_t e) {
    snprintf(g_err, sizeof g_err, "%s: %s", what, hipGetErrorString(e));
    return -3;
}

#define PCHECK(x)                                   \
    do {                                            \
        hipError_t e_ = (x);                        \
        if (e_ != hipSuccess) return fail(#x, e_);  \
    } while (0)

}  // namespace

extern "C" {

const char* jmp_last_error(void) { return g_err; }

int jmp_launch_chain(int n, int use_graph, int reps, float* us_per_launch) {
    if (n < 1 || n > 4096 || reps < 1 || !us_per_launch) {
        snprintf(g_err, sizeof g_err, "bad arguments");
        return -1;
    }
    unsigned* p = nullptr;
    hipStream_t st = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    int rc = 0;
    float ms = 0.0f;
    auto run = [&]() -> int {
        PCHECK(hipMalloc(&p, 256));
        PCHECK(hipMemset(p, 0, 256));
        PCHECK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
        PCHECK(hipEventCreate(&e0));
        PCHECK(hipEventCreate(&e1));
        if (use_graph) {
            PCHECK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
            for (int i = 0; i < n; i++) hipLaunchKernelGGL(k_touch, dim3(1), dim3(64), 0, st, p);
            PCHECK(hipStreamEndCapture(st, &g));
            PCHECK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
            PCHECK(hipGraphLaunch(ge, st));                 // warm-up
        } else {
            for (int i = 0; i < n; i++) hipLaunchKernelGGL(k_touch, dim3(1), dim3(64), 0, st, p);
            PCHECK(hipGetLastError());
        }
        PCHECK(hipStreamSynchronize(st));
        PCHECK(hipEventRecord(e0, st));
        for (int r = 0; r < reps; r++) {
            if (use_graph) {
                PCHECK(hipGraphLaunch(ge, st));
            } else {
                for (int i = 0; i < n; i++) hipLaunchKernelGGL(k_touch, dim3(1), dim3(64), 0, st, p);
            }
        }
        PCHECK(hipEventRecord(e1, st));
        PCHECK(hipEventSynchronize(e1));
        PCHECK(hipEventElapsedTime(&ms, e0, e1));
        *us_per_launch = ms * 1e3f / (float)(n * reps);
        return 0;
    };
    rc = run();
    if (ge) (void)hipGraphExecDestroy(ge);
    if (g) (void)hipGraphDestroy(g);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (st) (void)hipStreamDestroy(st);
    if (p) (void)hipFree(p);
    return rc;
}

int jmp_handoff(int nblk, int per_block, int handoff, int reps, float* us_per_launch, float* total) {
    if (nblk < 1 || nblk > 65536 || per_block < 1 || per_block > (1 << 20) || reps < 1 || !us_per_launch) {
        snprintf(g_err, sizeof g_err, "bad arguments");
        return -1;
    }
    float *src = nullptr, *part = nullptr, *out = nullptr;
    unsigned* ticket = nullptr;
    hipStream_t st = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0.0f;
    auto run = [&]() -> int {
        const size_t n = (size_t)nblk * per_block;
        PCHECK(hipMalloc(&src, n * sizeof(float)));
        PCHECK(hipMalloc(&part, nblk * sizeof(float)));
        PCHECK(hipMalloc(&out, sizeof(float)));
        PCHECK(hipMalloc(&ticket, sizeof(unsigned)));
        std::vector<float> ones(n, 1.0f);
        PCHECK(hipMemcpy(src, ones.data(), n * sizeof(float), hipMemcpyHostToDevice));
        PCHECK(hipMemset(ticket, 0, sizeof(unsigned)));
        PCHECK(hipMemset(out, 0, sizeof(float)));
        PCHECK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
        PCHECK(hipEventCreate(&e0));
        PCHECK(hipEventCreate(&e1));
        auto launch = [&]() {
            if (handoff)
                hipLaunchKernelGGL(k_handoff<true>, dim3(nblk), dim3(HT), 0, st, src, per_block, part, ticket, out, nblk);
            else
                hipLaunchKernelGGL(k_handoff<false>, dim3(nblk), dim3(HT), 0, st, src, per_block, part, ticket, out, nblk);
        };
        launch();
        PCHECK(hipGetLastError());
        PCHECK(hipStreamSynchronize(st));
        PCHECK(hipEventRecord(e0, st));
        for (int r = 0; r < reps; r++) launch();
        PCHECK(hipEventRecord(e1, st));
        PCHECK(hipEventSynchronize(e1));
        PCHECK(hipEventElapsedTime(&ms, e0, e1));
        *us_per_launch = ms * 1e3f / (float)reps;
        if (total) PCHECK(hipMemcpy(total, out, sizeof(float), hipMemcpyDeviceToHost));
        return 0;
    };
    const int rc = run();
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (st) (void)hipStreamDestroy(st);
    if (src) (void)hipFree(src);
    if (part) (void)hipFree(part);
    if (out) (void)hipFree(out);
    if (ticket) (void)hipFree(ticket);
    return rc;
}

int jmp_stream(unsigned long long nbytes, int wave_bytes, int regions, int reps, float* us_per_launch) {
    if (wave_bytes != 4096 && wave_bytes != 8192 && wave_bytes != 16384) {
        snprintf(g_err, sizeof g_err, "wave_bytes must be 4096, 8192 or 16384");
        return -1;
    }
    const unsigned long long per_block = 4ull * (unsigned long long)wave_bytes;
    if (nbytes == 0 || nbytes % per_block || nbytes > (1ull << 32) || regions < 1 || regions > 16 ||
        nbytes * (unsigned long long)regions > (6ull << 30) || reps < 1 || !us_per_launch) {
        snprintf(g_err, sizeof g_err, "bad arguments");
        return -1;
    }
    const unsigned nblk = (unsigned)(nbytes / per_block);
    char* src = nullptr;
    unsigned* out = nullptr;
    hipStream_t st = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0.0f;
    auto run = [&]() -> int {
        PCHECK(hipMalloc(&src, nbytes * regions));
        PCHECK(hipMalloc(&out, (size_t)nblk * 4 * sizeof(unsigned)));
        hipLaunchKernelGGL(k_fill, dim3(4096), dim3(256), 0, nullptr, (unsigned*)src, (size_t)(nbytes * regions / 4));
        PCHECK(hipGetLastError());
        PCHECK(hipDeviceSynchronize());
        PCHECK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
        PCHECK(hipEventCreate(&e0));
        PCHECK(hipEventCreate(&e1));
        auto launch = [&](int r) {
            const uint4* s4 = (const uint4*)(src + (size_t)(r % regions) * nbytes);
            if (wave_bytes == 4096) hipLaunchKernelGGL(k_stream<4>, dim3(nblk), dim3(256), 0, st, s4, out);
            else if (wave_bytes == 8192) hipLaunchKernelGGL(k_stream<8>, dim3(nblk), dim3(256), 0, st, s4, out);
            else hipLaunchKernelGGL(k_stream<16>, dim3(nblk), dim3(256), 0, st, s4, out);
        };
        for (int r = 0; r < regions; r++) launch(r);
        PCHECK(hipGetLastError());
        PCHECK(hipStreamSynchronize(st));
        PCHECK(hipEventRecord(e0, st));
        for (int r = 0; r < reps; r++) launch(r);
        PCHECK(hipEventRecord(e1, st));
        PCHECK(hipEventSynchronize(e1));
        PCHECK(hipEventElapsedTime(&ms, e0, e1));
        *us_per_launch = ms * 1e3f / (float)reps;
        return 0;
    };
    const int rc = run();
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (st) (void)hipStreamDestroy(st);
    if (src) (void)hipFree(src);
    if (out) (void)hipFree(out);
    return rc;
}

}  // extern "C"
