// Cross-lane moves and reductions within one wave64 on gfx950, on the VALU (DPP and the gfx950 permlane swaps)
// instead of the LDS unit (ds_bpermute): a reduction step costs a few cycles instead of an LDS round trip.
//
// lane_swap<M>(v) returns the value of the lane's partner across lane bit M:
//   M = 1, 2     the lane ℓ ^ M           (DPP quad_perm)
//   M = 4        the lane ℓ ^ 7            (DPP row_half_mirror: lanes 8k+i ↔ 8k+7−i)
//   M = 8        the lane ℓ ^ 15           (DPP row_mirror: lanes 16k+i ↔ 16k+15−i)
//   M = 16, 32   the lane ℓ ^ M           (v_permlane16_swap / v_permlane32_swap)
// For M = 4 and 8 the partner also differs in the lower bits. Every use below is a butterfly whose steps run from the
// high bit to the low one; there the partner's lower bits are covered by the later steps, so each step still joins two
// disjoint lane sets that differ in bit M, and the lane bits keep deciding which half a lane keeps.
#pragma once

#include <hip/hip_runtime.h>

template <int M> __device__ __forceinline__ float lane_swap(float v, int lane) {
    const int i = __float_as_int(v);
    if constexpr (M == 1) return __int_as_float(__builtin_amdgcn_update_dpp(i, i, 0xB1, 0xF, 0xF, false));
    if constexpr (M == 2) return __int_as_float(__builtin_amdgcn_update_dpp(i, i, 0x4E, 0xF, 0xF, false));
    if constexpr (M == 4) return __int_as_float(__builtin_amdgcn_update_dpp(i, i, 0x141, 0xF, 0xF, false));
    if constexpr (M == 8) return __int_as_float(__builtin_amdgcn_update_dpp(i, i, 0x140, 0xF, 0xF, false));
    if constexpr (M == 16) {
        // odd rows of the first result hold the even rows' values, even rows of the second the odd rows'
        const auto r = __builtin_amdgcn_permlane16_swap((unsigned)i, (unsigned)i, false, false);
        return __uint_as_float((lane & 16) ? r[0] : r[1]);
    }
    if constexpr (M == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap((unsigned)i, (unsigned)i, false, false);
        return __uint_as_float((lane & 32) ? r[0] : r[1]);
    }
    static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "lane bit");
    return v;
}

// the same for a 32-bit integer
template <int M> __device__ __forceinline__ uint32_t lane_swap_u32(uint32_t v, int lane) {
    return __float_as_uint(lane_swap<M>(__uint_as_float(v), lane));
}

// max / sum of a value and its partner across lane bit M (16 or 32), the same in both lanes. The permlane swap of v
// with itself returns, in every lane, its own value in one result and the partner's in the other (which one depends
// on the lane), so the symmetric op takes both without selecting.
template <int M> __device__ __forceinline__ float pair_max(float v) {
    static_assert(M == 16 || M == 32, "lane bit");
    const unsigned u = __float_as_uint(v);
    const auto r = M == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                           : __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
template <int M> __device__ __forceinline__ float pair_sum(float v) {
    static_assert(M == 16 || M == 32, "lane bit");
    const unsigned u = __float_as_uint(v);
    const auto r = M == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                           : __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Σ over the lanes that differ in bits [0, log2(2·M0)): masks M0, M0/2, …, 1
template <int M0> __device__ __forceinline__ float group_sum(float v, int lane) {
    if constexpr (M0 >= 32) v += lane_swap<32>(v, lane);
    if constexpr (M0 >= 16) v += lane_swap<16>(v, lane);
    if constexpr (M0 >= 8) v += lane_swap<8>(v, lane);
    if constexpr (M0 >= 4) v += lane_swap<4>(v, lane);
    if constexpr (M0 >= 2) v += lane_swap<2>(v, lane);
    if constexpr (M0 >= 1) v += lane_swap<1>(v, lane);
    return v;
}
template <int M0> __device__ __forceinline__ float group_max(float v, int lane) {
    if constexpr (M0 >= 32) v = fmaxf(v, lane_swap<32>(v, lane));
    if constexpr (M0 >= 16) v = fmaxf(v, lane_swap<16>(v, lane));
    if constexpr (M0 >= 8) v = fmaxf(v, lane_swap<8>(v, lane));
    if constexpr (M0 >= 4) v = fmaxf(v, lane_swap<4>(v, lane));
    if constexpr (M0 >= 2) v = fmaxf(v, lane_swap<2>(v, lane));
    if constexpr (M0 >= 1) v = fmaxf(v, lane_swap<1>(v, lane));
    return v;
}
__device__ __forceinline__ float wave_sum(float v, int lane) { return group_sum<32>(v, lane); }
__device__ __forceinline__ float wave_max(float v, int lane) { return group_max<32>(v, lane); }

// one exchange-and-halve step across lane bit M: v[0 … 2n) → v[0 … n); a lane with bit M set keeps the upper half
// and adds its partner's upper half, a lane without keeps the lower
template <int M, int N>
__device__ __forceinline__ void halve_step(float (&v)[N], int n, int lane) {
    const bool hi = (lane & M) != 0;
#pragma unroll
    for (int i = 0; i < (N > 1 ? N / 2 : 1); i++) {
        if (i < n) {
            const float send = hi ? v[i] : v[i + n];
            const float keep = hi ? v[i + n] : v[i];
            v[i] = keep + lane_swap<M>(send, lane);
        }
    }
}

// S exchange-and-halve steps across lane bits M0, M0/2, … (S of them): each lane keeps N / 2^S values, summed over
// the 2^S lanes that differ in those bits; with S steps from bit M0 the lane's kept values are
// v[r] = Σ original v[off + r], off = Σ_s bit_s(lane) · N / 2^(s+1).
template <int N, int M0, int S> __device__ __forceinline__ void halve(float (&v)[N], int lane) {
    if constexpr (S >= 1) halve_step<M0, N>(v, N / 2, lane);
    if constexpr (S >= 2) halve_step<(M0 >> 1), N>(v, N / 4, lane);
    if constexpr (S >= 3) halve_step<(M0 >> 2), N>(v, N / 8, lane);
    if constexpr (S >= 4) halve_step<(M0 >> 3), N>(v, N / 16, lane);
    if constexpr (S >= 5) halve_step<(M0 >> 4), N>(v, N / 32, lane);
    if constexpr (S >= 6) halve_step<(M0 >> 5), N>(v, N / 64, lane);
}

// Sums v[r] over the wave for every r < N (a power of two ≤ 64). On return the lanes whose low log2(64/N) bits are
// zero hold a total: lane ℓ holds row ℓ / (64/N) (exchange-and-halve over bits 32 … 64/N, then a plain butterfly).
template <int N> __device__ __forceinline__ float wave_sum_rows(float (&v)[N], int lane) {
    constexpr int S = N == 1 ? 0 : N == 2 ? 1 : N == 4 ? 2 : N == 8 ? 3 : N == 16 ? 4 : N == 32 ? 5 : 6;
    halve<N, 32, S>(v, lane);
    return group_sum<(32 >> S)>(v[0], lane);
}
