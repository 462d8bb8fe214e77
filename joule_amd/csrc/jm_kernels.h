// Internal launch interface between the C ABI (jm_api.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Signed base-16 digits per activation value in the Q4 dot (see jm_device.h).
#ifndef JM_NDIG
#define JM_NDIG 4
#endif
// Tokens of one expert segment processed per pass over the expert's rows.
#ifndef JM_NT
#define JM_NT 4
#endif

// Limits of the kernels: experts per layer (top-k keeps E/64 values per lane,
// dispatch keeps per-expert counts in LDS) and slots (B*topk) per call.
#define JM_MAX_E 512
#define JM_MAX_SLOTS 65536
#define JM_MAX_TOPK 32

namespace jm {

struct ExpertArgs {
    const uint8_t* blob;      // HBM copy of experts_q4.bin
    const uint64_t* off;      // [3][L*E][2] (scales offset, packed offset)
    int LE;                   // L * E
    int layer, E, d, m, topk, group;
    const int* n_active;      // number of experts with a non-empty segment
    const int* active;        // their ids, ascending
    const int* seg_off;       // [E+1] segment starts in seg_slot
    const int* seg_slot;      // [B*k] slot ids (b*k+i) grouped by expert, stable
    const float* tw;          // [B*k] routing weight of each slot
    const uint32_t* xdig;     // [B][d/G][NDIG][G/8] token digits
    const float* xscale;      // [B][d/G]
    float* act;               // [B*k][m]   SiLU(gate)*up per slot
    uint32_t* adig;           // [B*k][m/G][NDIG][G/8]
    float* ascale;            // [B*k][m/G]
    float* y;                 // [B*k][d]   weighted expert output per slot
};

hipError_t launch_router(const void* gate_w, int bf16, const float* x, float* logits,
                         int B, int E, int d, hipStream_t st);
hipError_t launch_prep_digits(const float* src, int stride, int rows, int cols, int group,
                              uint32_t* dig, float* scale, hipStream_t st);
hipError_t launch_topk(const float* logits, int B, int E, int k, int renorm, int* top, float* tw,
                       hipStream_t st);
// E <= JM_MAX_E, nslot <= JM_MAX_SLOTS
hipError_t launch_dispatch(const int* top, int nslot, int E, int* seg_off, int* seg_slot,
                           int* active, int* n_active, int* first_slot, int* rank_scratch,
                           hipStream_t st);
hipError_t launch_experts(const ExpertArgs& a, int umax, hipStream_t st);
hipError_t launch_combine(const float* y, const int* top, const int* first_slot, int B, int k, int d,
                          float* out, hipStream_t st);
hipError_t launch_dequant(const uint8_t* packed, const uint16_t* scales, long long numel, int group,
                          float* out, hipStream_t st);
hipError_t launch_q4_rows(const uint8_t* packed, const uint16_t* scales, int rows, int cols, int group,
                          const uint32_t* dig, const float* dscale, int T, float* out, int ostride,
                          hipStream_t st);

}  // namespace jm
