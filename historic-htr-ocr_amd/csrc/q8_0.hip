// q8_0 dequant-matvec family for gfx950 (wave64): the decode step's projections and the LM head.
//
// Reference semantics: dmv.wgsl:22-52 (y (+)= W·x, dmv_norm), dmv_qkv.wgsl:23-65, dmv_ffn.wgsl:22-51,
// dmv_common.wgsl:23-30 (the fused RMS norm), embed_q8_0.wgsl:19-38. Layout and schedule are this library's own:
//
//   weights   repacked at load (runtime.hip) into an int8 plane q[rows][K] and an f16 scale plane d[rows][K/32];
//   lanes     a row is cut into groups of 16 quants (16 bytes); lane ℓ of a wave takes the groups ℓ, ℓ+64, … of every
//             row the wave computes, so one wave-wide load instruction reads 1 KiB of contiguous quants (a whole row
//             at K = 1024); the lane's 16·NG inputs sit in registers for all its rows (loaded once per wave);
//   tile      a 256-thread workgroup (4 waves) owns 4·RW consecutive output rows, RW per wave. Every quant load of
//             the wave's rows is issued before the first use; the tile's f16 scales (contiguous: rows are back to
//             back) are copied into LDS by the whole workgroup while those loads are in flight;
//   reduce    the RW per-lane partials of a wave are summed across the 64 lanes by one transposing butterfly:
//             exchange-and-halve steps (lane bits 32, 16, …) leave one row per lane group, then a plain butterfly over
//             the rest — RW−1 + log2(64/RW) cross-lane moves instead of 6·RW, each a DPP / permlane VALU move
//             (wave.h);
//   norm      the fused RMS norm is computed on the registers: the wave's lanes hold all K inputs, so Σx² is one
//             wave sum (no workgroup barrier, no second read of x);
//   math      f32 (the reference's numbers: exact int8·f16-scale dequant, f32 products and sums): the 16 products
//             of a group are an fma chain, times the block's scale into the row's accumulator. The int8 → f32
//             conversion is one v_cvt_f32_i32 with a sign-extended byte select per quant.
#include <cstdio>

#include "htr_internal.h"
#include "wave.h"

namespace {

constexpr int WG = 256;
constexpr int WAVES = WG / 64;
constexpr int MAX_MANY = 128;

struct DmvK {
    DmvMat m[3];
    int n_rows;  // output rows (QKV: the three matrices' rows back to back)
    int k;
    const float *x;
    const float *nw;
    float eps;
    float *y;
    int acc;
};

// n matvecs y_i = W_i · x in one launch: rows of the n matrices back to back (y [n][rows])
struct DmvManyK {
    DmvMat m[MAX_MANY];
    int rows;  // rows of each matrix
    int n_rows;
    int k;
    const float *x;
    float *y;
};

// a kernel argument's pointer as a wave-uniform value (scalar registers): selects between such values stay selects of
// values — a select between argument fields themselves would become one per-lane load from the argument buffer
template <typename T> __device__ __forceinline__ T *uniform_ptr(T *p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (T *)(((uint64_t)hi << 32) | lo);
}
// 16 / 2 bytes from global memory (address space 1: a global_load, not a flat one — pointers that went through
// uniform_ptr have lost their address space)
typedef int gint4 __attribute__((ext_vector_type(4)));
typedef float gfloat4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 gload16(const void *p) {
    const gint4 v = *(const __attribute__((address_space(1))) gint4 *)(uintptr_t)p;
    return make_int4(v.x, v.y, v.z, v.w);
}
// the weight stream: non-temporal (each quant is read once a token; streaming loads that do not allocate in the
// caches measure ≈ 6.9 TB/s on one MI355X against ≈ 6.2 TB/s for plain loads)
__device__ __forceinline__ int4 gload16_stream(const void *p) {
    const gint4 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) gint4 *)(uintptr_t)p);
    return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 gload16u(const void *p) {
    const gint4 v = *(const __attribute__((address_space(1))) gint4 *)(uintptr_t)p;
    return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}
__device__ __forceinline__ float4 gload16f(const float *p) {
    const gfloat4 v = *(const __attribute__((address_space(1))) gfloat4 *)(uintptr_t)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ _Float16 gload2h(const _Float16 *p) {
    return *(const __attribute__((address_space(1))) _Float16 *)(uintptr_t)p;
}
__device__ __forceinline__ DmvMat uniform_mat(const DmvMat &m) {
    return DmvMat{uniform_ptr(m.q), uniform_ptr(m.d), __builtin_amdgcn_readfirstlane(m.rows)};
}

// Σ_j q_j · x_j over the 16 quants of one group (fma chain)
__device__ __forceinline__ float dot16(const int4 q, const float *x) {
    const int w[4] = {q.x, q.y, q.z, q.w};
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int b = 0; b < 4; b++) s = fmaf((float)(int8_t)(w[i] >> (8 * b)), x[4 * i + b], s);
    }
    return s;
}

// the lane's inputs x[16g … 16g+15] for its groups g = lane + 64·i (zero beyond K), and with NORM the norm weights
// of the same positions. The wave's lanes together hold all K inputs. Loads are unconditional (a lane past K reads
// group 0 and drops it) so that no branch separates them from the quant loads that follow.
template <int NG, bool NORM>
__device__ __forceinline__ void load_x(float (&xv)[NG][16], float (&wv)[NG][16], const float *x, const float *nw,
                                       int lane, int ng) {
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const int g = lane + 64 * i;
        const int gg = g < ng ? g : 0;
        const float keep = g < ng ? 1.0f : 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float4 v = gload16f(x + 16 * gg + 4 * j);
            xv[i][4 * j + 0] = v.x * keep;
            xv[i][4 * j + 1] = v.y * keep;
            xv[i][4 * j + 2] = v.z * keep;
            xv[i][4 * j + 3] = v.w * keep;
            if (NORM) {
                const float4 w = gload16f(nw + 16 * gg + 4 * j);
                wv[i][4 * j + 0] = w.x;
                wv[i][4 * j + 1] = w.y;
                wv[i][4 * j + 2] = w.z;
                wv[i][4 * j + 3] = w.w;
            }
        }
    }
}

// the fused RMS norm (dmv_common.wgsl:23-30) on the registers: x · 1/sqrt(Σx²/K + eps) · nw. Σx² is a wave sum: the
// wave holds all of x, so no workgroup barrier.
template <int NG>
__device__ __forceinline__ void norm_x(float (&xv)[NG][16], const float (&wv)[NG][16], float eps, int k, int lane) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NG; i++)
#pragma unroll
        for (int j = 0; j < 16; j++) s = fmaf(xv[i][j], xv[i][j], s);
    const float scale = 1.0f / sqrtf(wave_sum(s, lane) / (float)k + eps);
#pragma unroll
    for (int i = 0; i < NG; i++)
#pragma unroll
        for (int j = 0; j < 16; j++) xv[i][j] = (xv[i][j] * scale) * wv[i][j];
}

// The tile's f16 scales → LDS s_d[r][nb] for rows [row0, row0 + RT). When nb is a multiple of 8 every row is whole
// 16-byte units and a thread moves at most one unit (the host keeps RT·nb/8 ≤ 256): `issue` loads it into a register
// before the quant loads go out, `store` writes it to LDS after. Other K (small reference-test shapes) copy halves.
struct ScaleStage {
    uint4 v;
    int at;  // LDS offset in halves, −1 = none
};

template <typename MatOf>
__device__ __forceinline__ ScaleStage scales_issue(int row0, int rt, int n_rows, int nb, MatOf mat_of) {
    // branch-free (a branch would make the compiler wait for this load before the quant loads): every thread loads
    // 16 bytes; a thread without a unit reads the tile's first row (the scale plane has 16 bytes of slack past its
    // end, so a row of fewer than 8 scales is still a safe read) and stores nothing
    const int per_row = nb % 8 == 0 ? nb / 8 : 1;
    const int u = threadIdx.x;
    const int r = u / per_row, part = u - r * per_row;
    const bool valid = nb % 8 == 0 && u < rt * per_row && row0 + r < n_rows;
    int lr;
    const DmvMat m = mat_of(valid ? row0 + r : row0, lr);
    ScaleStage st;
    st.v = gload16u(m.d + (size_t)lr * nb + (valid ? 8 * part : 0));
    st.at = valid ? r * nb + 8 * part : -1;
    return st;
}

template <typename MatOf>
__device__ __forceinline__ void scales_store(_Float16 *s_d, const ScaleStage &st, int row0, int rt, int n_rows, int nb,
                                             MatOf mat_of) {
    if (nb % 8 == 0) {
        if (st.at >= 0) *reinterpret_cast<uint4 *>(s_d + st.at) = st.v;
        return;
    }
    for (int u = threadIdx.x; u < rt * nb; u += WG) {
        const int r = u / nb, b = u - r * nb;
        const int row = row0 + r;
        if (row < n_rows) {
            int lr;
            const DmvMat m = mat_of(row, lr);
            s_d[u] = gload2h(m.d + (size_t)lr * nb + b);
        }
    }
}

// the lane's quants of one row (lr must be a row of m: callers clamp rows past the end and drop their result)
template <int NG>
__device__ __forceinline__ void load_row(int4 (&qv)[NG], const DmvMat &m, int lr, int k, int lane, int ng) {
    const int8_t *qrow = m.q + (size_t)lr * k;
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const int g = lane + 64 * i;
        const int4 v = gload16_stream(qrow + 16 * (g < ng ? g : 0));
        qv[i] = g < ng ? v : make_int4(0, 0, 0, 0);
    }
}

template <int NG>
__device__ __forceinline__ float row_dot(const int4 (&qv)[NG], const float (&xv)[NG][16], const _Float16 *s_row,
                                         int lane, int ng) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const int g = lane + 64 * i;
        const float d = g < ng ? (float)s_row[g >> 1] : 0.0f;
        s = fmaf(dot16(qv[i], xv[i]), d, s);
    }
    return s;
}

// The general kernel: PLAIN / NORM (dmv, dmv_norm), QKV (three matrices, attn_norm fused), FFN (gate and up, ffn_norm
// and SwiGLU fused). RW output rows per wave. Order: inputs, then the scale loads, then every quant load of the wave's
// rows; the norm and the scales' LDS store overlap the quant loads' flight.
template <int RW, int NG, int MODE> __global__ __launch_bounds__(WG) void k_dmv(const DmvK a) {
    constexpr int NM = MODE == DMV_FFN ? 2 : 1;  // matrices read per output row
    constexpr int RT = WAVES * RW;                 // rows per workgroup
    __shared__ _Float16 s_d[NM][RT * NG * 32];     // scales: RT rows × nb ≤ 32·NG
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int k = a.k, ng = k >> 4, nb = k >> 5;
    const int row0 = blockIdx.x * RT;
    const int wrow0 = row0 + wave * RW;

    // the row's matrix (QKV: rows of q, then k, then v), by selects of the kernel arguments' pointers (a per-thread
    // row must not index the argument array: that would be a vector load and a wait before the quant loads)
    auto mat_of = [&](int row, int &lr) -> DmvMat {
        if (MODE != DMV_QKV) {
            lr = row;
            return a.m[0];
        }
        const DmvMat m0 = uniform_mat(a.m[0]), m1 = uniform_mat(a.m[1]), m2 = uniform_mat(a.m[2]);
        const int r0 = m0.rows, r01 = r0 + m1.rows;
        const bool in1 = row >= r0, in2 = row >= r01;
        lr = row - (in2 ? r01 : in1 ? r0 : 0);
        DmvMat m;
        m.q = in2 ? m2.q : in1 ? m1.q : m0.q;
        m.d = in2 ? m2.d : in1 ? m1.d : m0.d;
        m.rows = in2 ? m2.rows : in1 ? m1.rows : m0.rows;
        return m;
    };
    auto up_of = [&](int row, int &lr) -> DmvMat {
        lr = row;
        return a.m[NM - 1];
    };

    float xv[NG][16], wv[NG][16];
    load_x<NG, MODE != DMV_PLAIN>(xv, wv, a.x, a.nw, lane, ng);
    ScaleStage ss[NM];
    ss[0] = scales_issue(row0, RT, a.n_rows, nb, mat_of);
    if (NM == 2) ss[NM - 1] = scales_issue(row0, RT, a.n_rows, nb, up_of);
    int4 qv[NM][RW][NG];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const int row = min(wrow0 + r, a.n_rows - 1);  // rows past the end repeat the last (their result is dropped)
        int lr;
        const DmvMat m = mat_of(row, lr);
        load_row<NG>(qv[0][r], m, lr, k, lane, ng);
        if (NM == 2) load_row<NG>(qv[NM - 1][r], a.m[1], lr, k, lane, ng);
    }
    if (MODE != DMV_PLAIN) norm_x<NG>(xv, wv, a.eps, k, lane);
    scales_store(s_d[0], ss[0], row0, RT, a.n_rows, nb, mat_of);
    if (NM == 2) scales_store(s_d[NM - 1], ss[NM - 1], row0, RT, a.n_rows, nb, up_of);
    __syncthreads();

    float acc[NM][RW];
#pragma unroll
    for (int t = 0; t < NM; t++) {
#pragma unroll
        for (int r = 0; r < RW; r++) acc[t][r] = row_dot<NG>(qv[t][r], xv, s_d[t] + (wave * RW + r) * nb, lane, ng);
    }
    float v[NM];
#pragma unroll
    for (int t = 0; t < NM; t++) v[t] = wave_sum_rows<RW>(acc[t], lane);
    constexpr int SPREAD = 64 / RW;
    if ((lane & (SPREAD - 1)) == 0) {
        const int row = wrow0 + lane / SPREAD;
        if (row < a.n_rows) {
            float out = v[0];
            if (MODE == DMV_FFN) out = (v[0] / (1.0f + expf(-v[0]))) * v[NM - 1];
            if (a.acc) out = a.y[row] + out;
            a.y[row] = out;
        }
    }
}

// The decoder's own shapes: K = 1024·NG (each lane holds NG whole groups of 16, no lane idle) and rows a multiple of
// the tile, launched as one workgroup per CU with RW = rows / (4·CUs) rows a wave. A decode matvec is latency bound
// (all of its loads go out at once); what is left is the VALU work after the loads land, and one wave per SIMD pays
// the per-wave part (x, the norm, addressing, the reduction) once instead of once per row. No clamps or guards: the
// host checks the shape. Same arithmetic as k_dmv (dot16 per group, fma by the block scale, wave_sum_rows).
template <int RW, int NG, int MODE> __global__ __launch_bounds__(WG) void k_dmv_full(const DmvK a) {
    constexpr int NM = MODE == DMV_FFN ? 2 : 1;
    constexpr int RT = WAVES * RW;
    constexpr int K = 1024 * NG, NB = K / 32, PER_ROW = NB / 8;  // 16-byte scale units a row
    constexpr int RP = RW == 3 ? 4 : RW;                          // rows reduced together (a power of two)
    static_assert(RT * PER_ROW <= WG, "one scale unit per thread");
    __shared__ _Float16 s_d[NM][RT * NB + 8];  // + one 16-byte slot that threads without a unit write
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = blockIdx.x * RT, wrow0 = row0 + wave * RW;
    auto mat_of = [&](int row, int &lr) -> DmvMat {
        if (MODE != DMV_QKV) {
            lr = row;
            return a.m[0];
        }
        const DmvMat m0 = uniform_mat(a.m[0]), m1 = uniform_mat(a.m[1]), m2 = uniform_mat(a.m[2]);
        const int r0 = m0.rows, r01 = r0 + m1.rows;
        const bool in1 = row >= r0, in2 = row >= r01;
        lr = row - (in2 ? r01 : in1 ? r0 : 0);
        DmvMat m;
        m.q = in2 ? m2.q : in1 ? m1.q : m0.q;
        m.d = in2 ? m2.d : in1 ? m1.d : m0.d;
        m.rows = in2 ? m2.rows : in1 ? m1.rows : m0.rows;
        return m;
    };
    float xv[NG][16], wv[NG][16];
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const int g = lane + 64 * i;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float4 v = gload16f(a.x + 16 * g + 4 * j);
            xv[i][4 * j] = v.x, xv[i][4 * j + 1] = v.y, xv[i][4 * j + 2] = v.z, xv[i][4 * j + 3] = v.w;
            if (MODE != DMV_PLAIN) {
                const float4 w = gload16f(a.nw + 16 * g + 4 * j);
                wv[i][4 * j] = w.x, wv[i][4 * j + 1] = w.y, wv[i][4 * j + 2] = w.z, wv[i][4 * j + 3] = w.w;
            }
        }
    }
    // the tile's scales: thread u < RT·PER_ROW moves unit u % PER_ROW of tile row u / PER_ROW (the others repeat
    // unit 0 into the spare slot: no branch, which would hold the loads back until their use)
    const bool has = threadIdx.x < RT * PER_ROW;
    const int su = has ? threadIdx.x : 0, sr = su / PER_ROW, sp = su % PER_ROW;
    uint4 sv[NM];
    {
        int lr;
        const DmvMat m = mat_of(row0 + sr, lr);
        sv[0] = gload16u(m.d + (size_t)lr * NB + 8 * sp);
        if (NM == 2) sv[NM - 1] = gload16u(a.m[1].d + (size_t)lr * NB + 8 * sp);
    }
    int4 qv[NM][RW][NG];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        int lr;
        const DmvMat m = mat_of(wrow0 + r, lr);
#pragma unroll
        for (int i = 0; i < NG; i++) {
            qv[0][r][i] = gload16_stream(m.q + (size_t)lr * K + 16 * (lane + 64 * i));
            if (NM == 2) qv[NM - 1][r][i] = gload16_stream(a.m[1].q + (size_t)lr * K + 16 * (lane + 64 * i));
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load is out before the norm waits for x
    if (MODE != DMV_PLAIN) norm_x<NG>(xv, wv, a.eps, K, lane);
    const int at = has ? sr * NB + 8 * sp : RT * NB;
#pragma unroll
    for (int t = 0; t < NM; t++) *reinterpret_cast<uint4 *>(s_d[t] + at) = sv[t];
    __syncthreads();
    float acc[NM][RP];
#pragma unroll
    for (int t = 0; t < NM; t++)
#pragma unroll
        for (int r = 0; r < RP; r++) {
            float sum = 0.0f;
            if (r < RW) {
                const _Float16 *s_row = s_d[t] + (wave * RW + r) * NB;
#pragma unroll
                for (int i = 0; i < NG; i++)
                    sum = fmaf(dot16(qv[t][r < RW ? r : 0][i], xv[i]), (float)s_row[(lane + 64 * i) >> 1], sum);
            }
            acc[t][r] = sum;
        }
    float v[NM];
#pragma unroll
    for (int t = 0; t < NM; t++) v[t] = wave_sum_rows<RP>(acc[t], lane);
    constexpr int SPREAD = 64 / RP;
    if ((lane & (SPREAD - 1)) == 0 && lane / SPREAD < RW) {
        const int row = wrow0 + lane / SPREAD;
        float out = v[0];
        if (MODE == DMV_FFN) out = (v[0] / (1.0f + expf(-v[0]))) * v[NM - 1];
        if (a.acc) out = a.y[row] + out;
        a.y[row] = out;
    }
}

template <int RW, int NG> __global__ __launch_bounds__(WG) void k_dmv_many(const DmvManyK a) {
    constexpr int RT = WAVES * RW;
    __shared__ _Float16 s_d[RT * NG * 32];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int k = a.k, ng = k >> 4, nb = k >> 5;
    const int row0 = blockIdx.x * RT;
    const int wrow0 = row0 + wave * RW;
    // the row's matrix: one of the tile's two (the host keeps RT ≤ rows, so a tile spans at most two), by selects
    const int mi0 = row0 / a.rows;
    const DmvMat m0 = uniform_mat(a.m[mi0]), m1 = uniform_mat(a.m[min(mi0 + 1, MAX_MANY - 1)]);
    auto mat_of = [&](int row, int &lr) -> DmvMat {
        const bool second = row - mi0 * a.rows >= a.rows;
        lr = row - (mi0 + (second ? 1 : 0)) * a.rows;
        DmvMat m;
        m.q = second ? m1.q : m0.q;
        m.d = second ? m1.d : m0.d;
        m.rows = a.rows;
        return m;
    };
    float xv[NG][16], wv[NG][16];
    load_x<NG, false>(xv, wv, a.x, nullptr, lane, ng);
    const ScaleStage ss = scales_issue(row0, RT, a.n_rows, nb, mat_of);
    int4 qv[RW][NG];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const int row = min(wrow0 + r, a.n_rows - 1);  // rows past the end repeat the last (their result is dropped)
        int lr;
        const DmvMat m = mat_of(row, lr);
        load_row<NG>(qv[r], m, lr, k, lane, ng);
    }
    scales_store(s_d, ss, row0, RT, a.n_rows, nb, mat_of);
    __syncthreads();
    float acc[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) acc[r] = row_dot<NG>(qv[r], xv, s_d + (wave * RW + r) * nb, lane, ng);
    const float v = wave_sum_rows<RW>(acc, lane);
    constexpr int SPREAD = 64 / RW;
    if ((lane & (SPREAD - 1)) == 0) {
        const int row = wrow0 + lane / SPREAD;
        if (row < a.n_rows) a.y[row] = v;
    }
}

// X[t] = dequant(token_embd[tok[t]]) for rows whose id is not 0xffffffff (embed_q8_0.wgsl:28-38)
__global__ __launch_bounds__(WG) void k_embed(const int8_t *q, const _Float16 *d, int dim, const uint32_t *tok,
                                              int n_tok, int n_vocab, float *x) {
    const size_t total = (size_t)n_tok * dim;
    for (size_t i = blockIdx.x * (size_t)WG + threadIdx.x; i < total; i += (size_t)gridDim.x * WG) {
        const size_t t = i / dim, c = i % dim;
        const uint32_t id = tok[t];
        if (id == 0xffffffffu || id >= (uint32_t)n_vocab) continue;
        x[i] = (float)q[(size_t)id * dim + c] * (float)d[((size_t)id * dim + c) >> 5];
    }
}

template <int RW, int MODE> int dispatch_ng(hipStream_t st, int ng_lane, const DmvK &a) {
    const dim3 grid((a.n_rows + WAVES * RW - 1) / (WAVES * RW));
    switch (ng_lane) {
    case 1: hipLaunchKernelGGL((k_dmv<RW, 1, MODE>), grid, dim3(WG), 0, st, a); return 0;
    case 2: hipLaunchKernelGGL((k_dmv<RW, 2, MODE>), grid, dim3(WG), 0, st, a); return 0;
    case 3: hipLaunchKernelGGL((k_dmv<RW, 3, MODE>), grid, dim3(WG), 0, st, a); return 0;
    case 4: hipLaunchKernelGGL((k_dmv<RW, 4, MODE>), grid, dim3(WG), 0, st, a); return 0;
    }
    return -1;
}

template <int MODE> int dispatch_r(hipStream_t st, int rw, int ng_lane, const DmvK &a) {
    switch (rw) {
    case 1: return dispatch_ng<1, MODE>(st, ng_lane, a);
    case 2: return dispatch_ng<2, MODE>(st, ng_lane, a);
    case 4: return dispatch_ng<4, MODE>(st, ng_lane, a);
    case 8: return dispatch_ng<8, MODE>(st, ng_lane, a);
    case 16: return dispatch_ng<16, MODE>(st, ng_lane, a);
    }
    return -1;
}

// Rows per wave: from rw (the caller's measured best for its long matrices) down to the largest that still gives
// every CU two workgroups or more (small decode matrices are latency bound: all their loads go out at once), capped so
// a lane's quant registers stay ≤ 64 (+ x) for occupancy. The cap
// RW·NG ≤ 16 also keeps a tile's scales within one 16-byte unit per thread (RT·nb/8 = RW·nb/2 ≤ 8·RW·NG ≤ 256 halves
// … units), which scales_issue relies on.
int rows_per_wave(int n_rows, int n_cu, int ng_lane, int nm, int rw) {
    while (rw > 1 && (n_rows + WAVES * rw - 1) / (WAVES * rw) < 2 * n_cu) rw >>= 1;
    while (rw > 1 && rw * ng_lane * nm > 16) rw >>= 1;
    return rw;
}

const char *mode_name(int mode) {
    return mode == DMV_PLAIN ? "plain" : mode == DMV_NORM ? "norm" : mode == DMV_QKV ? "qkv" : "ffn";
}

}  // namespace

int dmv_full_rw(htr_device *dev, int mode, const DmvMat *mats, int n_mats, int k) {
    int rows = 0;
    for (int i = 0; i < n_mats; i++) rows += mats[i].rows;
    if (mode == DMV_FFN) rows = mats[0].rows;
    if (k % 1024 != 0 || k > 3072 || rows % (WAVES * dev->n_cu) != 0) return 0;
    const int rw = rows / (WAVES * dev->n_cu);
    return rw <= 4 ? rw : 0;
}

int launch_dmv(htr_device *dev, hipStream_t st, int mode, const DmvMat *mats, int n_mats, int k, const float *x,
               const float *nw, float eps, float *y, int acc) {
    if (k <= 0 || k % 32 != 0 || k > 4096) return htr_fail("matvec: K = %d (a multiple of 32, at most 4096)", k);
    if (mode != DMV_PLAIN && !nw) return htr_fail("matvec: the fused norm needs its weights");
    DmvK a{};
    int rows = 0;
    for (int i = 0; i < n_mats; i++) {
        a.m[i] = mats[i];
        rows += mats[i].rows;
    }
    if (mode == DMV_FFN) {
        if (n_mats != 2 || mats[0].rows != mats[1].rows) return htr_fail("matvec_ffn: gate / up rows differ");
        rows = mats[0].rows;
    }
    a.n_rows = rows;
    a.k = k;
    a.x = x;
    a.nw = nw;
    a.eps = eps;
    a.y = y;
    a.acc = acc;
    const int ng_lane = (k / 16 + 63) / 64;
    const int full_rw = dmv_full_rw(dev, mode, mats, n_mats, k);
    if (full_rw > 0) {
        const dim3 grid(rows / (WAVES * full_rw));
#define HTR_FULL(RW, MODE)                                                                                             \
    switch (k / 1024) {                                                                                                \
    case 1: hipLaunchKernelGGL((k_dmv_full<RW, 1, MODE>), grid, dim3(WG), 0, st, a); break;                            \
    case 2: hipLaunchKernelGGL((k_dmv_full<RW, 2, MODE>), grid, dim3(WG), 0, st, a); break;                            \
    default: hipLaunchKernelGGL((k_dmv_full<RW, 3, MODE>), grid, dim3(WG), 0, st, a); break;                           \
    }
#define HTR_FULL_RW(MODE)                                                                                              \
    switch (full_rw) {                                                                                                 \
    case 1: HTR_FULL(1, MODE) break;                                                                                   \
    case 2: HTR_FULL(2, MODE) break;                                                                                   \
    case 3: HTR_FULL(3, MODE) break;                                                                                   \
    default: HTR_FULL(4, MODE) break;                                                                                  \
    }
        switch (mode) {
        case DMV_PLAIN: HTR_FULL_RW(DMV_PLAIN) break;
        case DMV_NORM: HTR_FULL_RW(DMV_NORM) break;
        case DMV_QKV: HTR_FULL_RW(DMV_QKV) break;
        default: HTR_FULL_RW(DMV_FFN) break;
        }
#undef HTR_FULL_RW
#undef HTR_FULL
        char name[48];
        snprintf(name, sizeof name, "k_dmv_full<%d,%d,%s>", full_rw, std::min(k / 1024, 3), mode_name(mode));
        return htr_launched(dev, name);
    }
    // 8 rows a wave at most: the LM head (151,936 rows) decodes 1638 tokens/s against 1630 with 16 and 1631 with 4
    const int rw = rows_per_wave(rows, dev->n_cu, ng_lane, mode == DMV_FFN ? 2 : 1, 8);
    int rc = -1;
    switch (mode) {
    case DMV_PLAIN: rc = dispatch_r<DMV_PLAIN>(st, rw, ng_lane, a); break;
    case DMV_NORM: rc = dispatch_r<DMV_NORM>(st, rw, ng_lane, a); break;
    case DMV_QKV: rc = dispatch_r<DMV_QKV>(st, rw, ng_lane, a); break;
    case DMV_FFN: rc = dispatch_r<DMV_FFN>(st, rw, ng_lane, a); break;
    }
    if (rc < 0) return htr_fail("matvec: no kernel for mode %d, RW %d, K %d", mode, rw, k);
    char name[48];
    snprintf(name, sizeof name, "k_dmv<%d,%d,%s>", rw, ng_lane, mode_name(mode));
    return htr_launched(dev, name);
}

int launch_dmv_many(htr_device *dev, hipStream_t st, const DmvMat *mats, int n, int k, const float *x, float *y) {
    if (k <= 0 || k % 32 != 0 || k > 4096) return htr_fail("matvec_many: K = %d (a multiple of 32, at most 4096)", k);
    for (int base = 0; base < n; base += MAX_MANY) {
        const int cnt = std::min(MAX_MANY, n - base);
        DmvManyK a{};
        for (int i = 0; i < cnt; i++) a.m[i] = mats[base + i];
        a.rows = mats[0].rows;
        a.n_rows = cnt * a.rows;
        a.k = k;
        a.x = x;
        a.y = y + (size_t)base * mats[0].rows;
        const int ng_lane = (k / 16 + 63) / 64;
        // 4 rows a wave at most: 430 MB in 61.4 µs (7.0 TB/s) against 62.9 µs with 8, 65.7 µs with 16, 79 µs with 2
        int rw = rows_per_wave(a.n_rows, dev->n_cu, ng_lane, 1, 4);
        while (rw > 1 && WAVES * rw > a.rows) rw >>= 1;  // a tile spans at most two matrices
        const dim3 grid((a.n_rows + WAVES * rw - 1) / (WAVES * rw));
#define HTR_MANY(RW)                                                                                                   \
    switch (ng_lane) {                                                                                                 \
    case 1: hipLaunchKernelGGL((k_dmv_many<RW, 1>), grid, dim3(WG), 0, st, a); break;                                  \
    case 2: hipLaunchKernelGGL((k_dmv_many<RW, 2>), grid, dim3(WG), 0, st, a); break;                                  \
    case 3: hipLaunchKernelGGL((k_dmv_many<RW, 3>), grid, dim3(WG), 0, st, a); break;                                  \
    default: hipLaunchKernelGGL((k_dmv_many<RW, 4>), grid, dim3(WG), 0, st, a); break;                                 \
    }
        switch (rw) {
        case 1: HTR_MANY(1) break;
        case 2: HTR_MANY(2) break;
        case 4: HTR_MANY(4) break;
        case 8: HTR_MANY(8) break;
        default: HTR_MANY(16) break;
        }
#undef HTR_MANY
        HTR_TRY(htr_launched(dev, "k_dmv_many"));
    }
    return 0;
}

int launch_embed(htr_device *dev, hipStream_t st, const htr_weight *w, const uint32_t *tok, int n_tok, float *x) {
    const size_t total = (size_t)n_tok * w->cols;
    const int grid = (int)std::min<size_t>((total + WG - 1) / WG, 16384);
    hipLaunchKernelGGL(k_embed, dim3(grid), dim3(WG), 0, st, w->q, w->d, (int)w->cols, tok, n_tok, (int)w->rows, x);
    return htr_launched(dev, "k_embed");
}

// ---- ABI ------------------------------------------------------------------------------------------------------------

static DmvMat mat_of(const htr_weight *w) { return DmvMat{w->q, w->d, (int)w->rows}; }

extern "C" int htr_matvec_q8_0(htr_device *dev, const htr_weight *w, const float *d_x, const float *d_norm_w,
                               float eps, float *d_y, int acc) {
    HTR_TRY(htr_check_alive(dev));
    if (!w || !w->q || !d_x || !d_y) return htr_fail("htr_matvec_q8_0: null argument (or a weight without q8_0 planes)");
    DmvMat m = mat_of(w);
    return launch_dmv(dev, dev->stream, d_norm_w ? DMV_NORM : DMV_PLAIN, &m, 1, (int)w->cols, d_x, d_norm_w, eps, d_y,
                      acc);
}

extern "C" int htr_matvec_q8_0_many(htr_device *dev, const htr_weight *const *ws, size_t n, const float *d_x,
                                    float *d_y) {
    HTR_TRY(htr_check_alive(dev));
    if (!ws || n == 0 || !d_x || !d_y) return htr_fail("htr_matvec_q8_0_many: null argument");
    std::vector<DmvMat> ms(n);
    for (size_t i = 0; i < n; i++) {
        if (!ws[i] || !ws[i]->q) return htr_fail("htr_matvec_q8_0_many: weight %zu is null", i);
        if (ws[i]->rows != ws[0]->rows || ws[i]->cols != ws[0]->cols)
            return htr_fail("htr_matvec_q8_0_many: weight %zu is [%zu x %zu], weight 0 [%zu x %zu]", i, ws[i]->rows,
                            ws[i]->cols, ws[0]->rows, ws[0]->cols);
        ms[i] = mat_of(ws[i]);
    }
    if (ws[0]->rows < (size_t)WAVES)
        return htr_fail("htr_matvec_q8_0_many: %zu rows per matrix (at least %d)", ws[0]->rows, WAVES);
    if (ws[0]->rows * std::min<size_t>(n, MAX_MANY) > (size_t)INT32_MAX)
        return htr_fail("htr_matvec_q8_0_many: %zu rows per launch", ws[0]->rows * std::min<size_t>(n, MAX_MANY));
    return launch_dmv_many(dev, dev->stream, ms.data(), (int)n, (int)ws[0]->cols, d_x, d_y);
}

extern "C" int htr_matvec_qkv(htr_device *dev, const htr_weight *wq, const htr_weight *wk, const htr_weight *wv,
                              const float *d_x, const float *d_norm_w, float eps, float *d_qkv) {
    HTR_TRY(htr_check_alive(dev));
    if (!wq || !wk || !wv || !d_x || !d_norm_w || !d_qkv) return htr_fail("htr_matvec_qkv: null argument");
    if (wq->cols != wk->cols || wq->cols != wv->cols || wk->rows != wv->rows)
        return htr_fail("htr_matvec_qkv: q [%zu x %zu], k [%zu x %zu], v [%zu x %zu]", wq->rows, wq->cols, wk->rows,
                        wk->cols, wv->rows, wv->cols);
    DmvMat m[3] = {mat_of(wq), mat_of(wk), mat_of(wv)};
    return launch_dmv(dev, dev->stream, DMV_QKV, m, 3, (int)wq->cols, d_x, d_norm_w, eps, d_qkv, 0);
}

extern "C" int htr_matvec_ffn(htr_device *dev, const htr_weight *wg, const htr_weight *wu, const float *d_x,
                              const float *d_norm_w, float eps, float *d_g) {
    HTR_TRY(htr_check_alive(dev));
    if (!wg || !wu || !d_x || !d_norm_w || !d_g) return htr_fail("htr_matvec_ffn: null argument");
    if (wg->rows != wu->rows || wg->cols != wu->cols)
        return htr_fail("htr_matvec_ffn: gate [%zu x %zu], up [%zu x %zu]", wg->rows, wg->cols, wu->rows, wu->cols);
    DmvMat m[2] = {mat_of(wg), mat_of(wu)};
    return launch_dmv(dev, dev->stream, DMV_FFN, m, 2, (int)wg->cols, d_x, d_norm_w, eps, d_g, 0);
}
