// The greedy choice's order on (logit, index) pairs, shared by the choice kernel (choose.hip) and the one-launch decode
// step's tail (token_step.hip): the first maximum wins (ties → the lower index), NaN never wins (sampling.rs:49-61).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "wave.h"

__device__ __forceinline__ bool better(float v, uint32_t i, float w, uint32_t j) { return v > w || (v == w && i < j); }

// (value, index) → a key whose unsigned order is `better`'s: the value's bits made order-preserving (−0 taken as +0,
// so the two compare equal as in IEEE), then the complemented index (the lower index wins a tie). The workgroup's
// placeholder (−inf, 0xffffffff) maps below every real logit.
__device__ __forceinline__ uint64_t choose_key(float v, uint32_t i) {
    uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)b << 32) | (uint64_t)(~i);
}

__device__ __forceinline__ void wave_best(float &v, uint32_t &i, int lane) {
    // the partner moves of wave.h (for bits 4 and 8 the partner also differs in lower bits: `better` is a total order
    // on (value, index) pairs without NaN, so the order in which lanes meet does not matter)
#define HTR_BEST_STEP(M)                                                                                               \
    {                                                                                                                  \
        const float ov = lane_swap<M>(v, lane);                                                                        \
        const uint32_t oi = lane_swap_u32<M>(i, lane);                                                                 \
        if (better(ov, oi, v, i)) {                                                                                    \
            v = ov;                                                                                                    \
            i = oi;                                                                                                    \
        }                                                                                                              \
    }
    HTR_BEST_STEP(32) HTR_BEST_STEP(16) HTR_BEST_STEP(8) HTR_BEST_STEP(4) HTR_BEST_STEP(2) HTR_BEST_STEP(1)
#undef HTR_BEST_STEP
}

