// The hand-over the one-launch decode step (token_step.hip) rests on, measured on the device it runs on: tagged 64-bit
// words passed between the workgroups of one 256-workgroup launch, the same loads and stores as the step's.
//
//   pair      one word passed back and forth between workgroups a and b, stored at workgroup scope (it stays in the
//             writer XCD's L2) or at agent scope (written through to the coherence point), read with agent-scope
//             loads: the round trip's time, and whether every wait saw its word (a workgroup-scope store is seen by
//             a reader on its own XCD only — the premise of the step's two XCD-local hand-overs);
//   all       every workgroup passes words / 256 tagged words to all the others, iters times in turn over two word
//             areas (an area is rewritten only after every reader has taken it: a workgroup writes area i % 2 of
//             round i after taking every word of round i − 1, which every writer wrote after taking round i − 2),
//             its first poll `pause` × 64 clocks after its own words, polled as the step's take<NP> polls (NP words
//             a thread, each loaded again until it carries its tag): the time an exchange takes.
// Every wait is bounded (max_polls loads of a word); a wait that runs out marks the call unseen and its workgroup
// stops, so the launch always ends. No reference counterpart: a measurement of this device.
#include "htr_internal.h"

namespace {

__device__ __forceinline__ uint64_t ld_agent(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool LOCAL>
__global__ __launch_bounds__(64) void k_handover_pair(uint64_t *w, int a, int b, int iters, int max_polls,
                                                      long long *t, int *unseen) {
    const int g = blockIdx.x;
    if ((g != a && g != b) || threadIdx.x != 0) return;
    uint64_t *mine = w + (g == a ? 0 : 16), *theirs = w + (g == a ? 16 : 0);  // 128 bytes apart
    const long long t0 = wall_clock64();
    bool ok = true;
    for (int i = 1; i <= iters && ok; i++) {
        if (g == a) {
            if (LOCAL) __hip_atomic_store(mine, (uint64_t)i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            else __hip_atomic_store(mine, (uint64_t)i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        int n = 0;
        while (ld_agent(theirs) != (uint64_t)i)
            if (++n > max_polls) {
                ok = false;
                break;
            }
        if (ok && g == b) {
            if (LOCAL) __hip_atomic_store(mine, (uint64_t)i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            else __hip_atomic_store(mine, (uint64_t)i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    const long long t1 = wall_clock64();
    if (g == a) *t = t1 - t0;
    if (!ok) __hip_atomic_store(unseen, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int A2A_MAX_NP = 12;  // words a thread: up to 3072 words an exchange

// the first poll's pause, in s_sleep units of 64 clocks (an immediate operand: the values the probe offers)
__device__ __forceinline__ void pause_for(int pause) {
    switch (pause) {
    case 0: break;
    case 4: __builtin_amdgcn_s_sleep(4); break;
    case 8: __builtin_amdgcn_s_sleep(8); break;
    case 12: __builtin_amdgcn_s_sleep(12); break;
    case 16: __builtin_amdgcn_s_sleep(16); break;
    case 20: __builtin_amdgcn_s_sleep(20); break;
    case 24: __builtin_amdgcn_s_sleep(24); break;
    default: __builtin_amdgcn_s_sleep(32); break;
    }
}

// NP words a thread, polled as the step's take<NP> polls them
template <int NP>
__global__ __launch_bounds__(256) void k_handover_all(uint64_t *area, int pause, int iters, int max_polls,
                                                      long long *t, int *unseen) {
    constexpr int WORDS = 256 * NP;
    const int g = blockIdx.x, tid = threadIdx.x;
    bool ok = true;
    const long long t0 = wall_clock64();
    for (int i = 1; i <= iters && ok; i++) {
        uint64_t *ar = area + (size_t)(i & 1) * WORDS;
        const uint32_t tag = (uint32_t)i;
        if (tid < NP)
            __hip_atomic_store(ar + NP * g + tid, ((uint64_t)tag << 32) | (uint32_t)(NP * g + tid), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        pause_for(pause);
        uint64_t v[NP];
#pragma unroll
        for (int k = 0; k < NP; k++) v[k] = ld_agent(ar + tid + 256 * k);
        int n = 0;
        for (;;) {
            bool all = true;
#pragma unroll
            for (int k = 0; k < NP; k++) all = all && (uint32_t)(v[k] >> 32) == tag;
            if (all) break;
            if (++n > max_polls) {
                ok = false;
                break;
            }
#pragma unroll
            for (int k = 0; k < NP; k++)
                if ((uint32_t)(v[k] >> 32) != tag) v[k] = ld_agent(ar + tid + 256 * k);
        }
        ok = __syncthreads_and(ok);
    }
    const long long t1 = wall_clock64();
    if (tid == 0) {
        if (g == 0) *t = t1 - t0;
        if (!ok) __hip_atomic_store(unseen, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int NP>
void launch_all(hipStream_t st, uint64_t *w, int pause, int iters, int max_polls, long long *t, int *unseen) {
    hipLaunchKernelGGL(k_handover_all<NP>, dim3(256), dim3(256), 0, st, w, pause, iters, max_polls, t, unseen);
}

}  // namespace

extern "C" int htr_debug_handover(htr_device *dev, int kind, int a, int b, int words, int pause, int iters,
                                  int max_polls, double *us, int *seen) {
    if (!dev || !us || !seen) return htr_fail("htr_debug_handover: null argument");
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(htr_check_not_capturing(dev, "htr_debug_handover"));
    if (kind < 0 || kind > 2) return htr_fail("htr_debug_handover: kind %d (0, 1 or 2)", kind);
    if (iters < 1 || iters > 1000000 || max_polls < 1) return htr_fail("htr_debug_handover: %d rounds, %d polls", iters, max_polls);
    if (kind < 2 && (a < 0 || a > 255 || b < 0 || b > 255 || a == b))
        return htr_fail("htr_debug_handover: workgroups %d and %d (two of 0 … 255)", a, b);
    if (kind == 2 && (words < 256 || words > 256 * A2A_MAX_NP || words % 256 ||
                      (pause != 0 && pause != 4 && pause != 8 && pause != 12 && pause != 16 && pause != 20 &&
                       pause != 24 && pause != 32)))
        return htr_fail("htr_debug_handover: %d words (256 … %d, a multiple of 256), pause %d (0, 4, 8, 12, 16, 20, 24 "
                        "or 32)", words, 256 * A2A_MAX_NP, pause);
    // [t, unseen | 128 bytes] then the words: the pair's two 128 bytes apart, or the two areas
    const size_t area_bytes = kind == 2 ? (size_t)2 * words * 8 : 256;
    void *scr = nullptr;
    HTR_TRY(htr_scratch(dev, SCR_HANDOVER, 128 + area_bytes, &scr));
    long long *t = (long long *)scr;
    int *unseen = (int *)((char *)scr + 8);
    uint64_t *w = (uint64_t *)((char *)scr + 128);
    HTR_TRY(htr_hip(dev, hipMemsetAsync(scr, 0, 128 + area_bytes, dev->stream), "hipMemsetAsync"));
    if (kind == 0)
        hipLaunchKernelGGL(k_handover_pair<true>, dim3(256), dim3(64), 0, dev->stream, w, a, b, iters, max_polls, t,
                           unseen);
    else if (kind == 1)
        hipLaunchKernelGGL(k_handover_pair<false>, dim3(256), dim3(64), 0, dev->stream, w, a, b, iters, max_polls, t,
                           unseen);
    else
        switch (words / 256) {
        case 1: launch_all<1>(dev->stream, w, pause, iters, max_polls, t, unseen); break;
        case 2: launch_all<2>(dev->stream, w, pause, iters, max_polls, t, unseen); break;
        case 3: launch_all<3>(dev->stream, w, pause, iters, max_polls, t, unseen); break;
        case 4: launch_all<4>(dev->stream, w, pause, iters, max_polls, t, unseen); break;
        case 5: launch_all<5>(dev->stream, w, pause, iters, max_polls, t, unseen); break;
        case 6: launch_all<6>(dev->stream, w, pause, iters, max_polls, t, unseen); break;
        case 7: launch_all<7>(dev->stream, w, pause, iters, max_polls, t, unseen); break;
        case 8: launch_all<8>(dev->stream, w, pause, iters, max_polls, t, unseen); break;
        case 9: launch_all<9>(dev->stream, w, pause, iters, max_polls, t, unseen); break;
        case 10: launch_all<10>(dev->stream, w, pause, iters, max_polls, t, unseen); break;
        case 11: launch_all<11>(dev->stream, w, pause, iters, max_polls, t, unseen); break;
        default: launch_all<12>(dev->stream, w, pause, iters, max_polls, t, unseen); break;
        }
    HTR_TRY(htr_launched(dev, kind == 2 ? "k_handover_all" : "k_handover_pair"));
    long long ticks = 0;
    int un = 0;
    HTR_TRY(htr_download(dev, &ticks, t, 8));
    HTR_TRY(htr_download(dev, &un, unseen, 4));
    int khz = 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev->ordinal) != hipSuccess || khz <= 0)
        khz = 100000;
    *us = (double)ticks / khz * 1e3 / iters;
    *seen = !un;
    return 0;
}
