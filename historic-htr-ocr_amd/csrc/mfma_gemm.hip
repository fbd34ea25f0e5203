// The vision encoder's GEMMs on gfx950's matrix cores: Y[M,N] (+)= X[M,K] · W[N,K]ᵀ with X and W f16 in memory and
// f32 accumulation, and the fused FFN first half G = silu(X·Wgᵀ) · (X·Wuᵀ) · scale → f16.
//
// Reference semantics: matmul_coopd.wgsl (Batch::matmul_f16x, gpu.rs:2019-2042) and ffn_coopd.wgsl (Batch::ffn_f16,
// gpu.rs:2048-2086; out_scale = 1/64, vision.rs:31-35). The schedule is this library's own:
//
//   tile      a 256-thread workgroup owns a 128 × 128 output tile; its 4 waves own 64 × 64 each, as 2 × 2
//             v_mfma_f32_32x32x16_f16 tiles (lane layouts checked on the GPU: A lane ℓ holds A[ℓ%32][8(ℓ/32) …+7],
//             B lane ℓ holds B[8(ℓ/32) …+7][ℓ%32], D lane ℓ register r is row 8(r/4) + 4(ℓ/32) + r%4, column ℓ%32);
//   K         in steps of 32 through LDS, double-buffered: the next step's global loads (16 B a lane) are in flight
//             while the current one feeds the matrix cores; one workgroup barrier per step. LDS rows are padded to
//             80 bytes so the fragment reads (16 B a lane, 32 rows) fall on distinct banks;
//   order     the tiles are dealt to the 8 XCDs in contiguous bands (workgroup b runs on XCD b mod 8), so an XCD's
//             L2 keeps a band of X rows and the W tiles they meet;
//   rows      rows past M read row M−1 and are not stored (no padding required of the caller).
#include "htr_internal.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int GW = 256;
constexpr int BM = 128, BN = 128, BK = 32;
constexpr int LDK = BK + 8;  // LDS row stride in halves (80 bytes)
constexpr int XCDS = 8;

struct GemmK {
    const _Float16 *x;   // [M][K]
    const _Float16 *w;   // [N][K]
    const _Float16 *w2;  // FFN: up [N][K]
    float *y;            // [M][N] f32 (F32 / ACC)
    _Float16 *y16;       // FFN: [M][N] f16
    int m, n, k;
    float scale;  // FFN output scale
    int tiles_m, tiles_n;
};

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// the tile of workgroup b: XCD x = b mod 8 takes the x-th contiguous band of tiles (row-major over (m, n))
__device__ __forceinline__ void tile_of(int b, int tiles_m, int tiles_n, int &tm, int &tn) {
    const int total = tiles_m * tiles_n;
    const int xcd = b % XCDS, i = b / XCDS;
    const int per = total / XCDS, extra = total % XCDS;
    const int t = xcd * per + min(xcd, extra) + i;
    tm = t / tiles_n;
    tn = t - tm * tiles_n;
}

template <int EPI> __global__ __launch_bounds__(GW) void k_gemm_f16(const GemmK a) {
    constexpr int NB = EPI == GEMM_FFN ? 2 : 1;  // weight matrices
    __shared__ __attribute__((aligned(16))) _Float16 s_a[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) _Float16 s_b[2][NB][BN * LDK];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    tile_of(blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
    const int row0 = tm * BM, col0 = tn * BN;
    const int k = a.k, nk = k / BK;

    // global → registers: thread t moves the 16-byte chunks (row t/4 + 64·i, chunk t%4) of the A and B tiles
    const int lr = tid >> 2, lc = tid & 3;
    const size_t xo0 = (size_t)min(row0 + lr, a.m - 1) * k + 8 * lc;
    const size_t xo1 = (size_t)min(row0 + lr + 64, a.m - 1) * k + 8 * lc;
    const size_t wo0 = (size_t)(col0 + lr) * k + 8 * lc;
    const size_t wo1 = (size_t)(col0 + lr + 64) * k + 8 * lc;
    int4 ra0, ra1, rb0[NB], rb1[NB];
#define HTR_GEMM_LOAD(kt)                                                                                              \
    {                                                                                                                  \
        const size_t kk_ = (size_t)(kt) * BK;                                                                          \
        ra0 = *reinterpret_cast<const int4 *>(a.x + xo0 + kk_);                                                        \
        ra1 = *reinterpret_cast<const int4 *>(a.x + xo1 + kk_);                                                        \
        rb0[0] = *reinterpret_cast<const int4 *>(a.w + wo0 + kk_);                                                     \
        rb1[0] = *reinterpret_cast<const int4 *>(a.w + wo1 + kk_);                                                     \
        if (NB == 2) {                                                                                                 \
            rb0[NB - 1] = *reinterpret_cast<const int4 *>(a.w2 + wo0 + kk_);                                           \
            rb1[NB - 1] = *reinterpret_cast<const int4 *>(a.w2 + wo1 + kk_);                                           \
        }                                                                                                              \
    }
#define HTR_GEMM_STORE(buf)                                                                                            \
    {                                                                                                                  \
        *reinterpret_cast<int4 *>(&s_a[buf][lr * LDK + 8 * lc]) = ra0;                                                 \
        *reinterpret_cast<int4 *>(&s_a[buf][(lr + 64) * LDK + 8 * lc]) = ra1;                                          \
        _Pragma("unroll") for (int t = 0; t < NB; t++) {                                                               \
            *reinterpret_cast<int4 *>(&s_b[buf][t][lr * LDK + 8 * lc]) = rb0[t];                                       \
            *reinterpret_cast<int4 *>(&s_b[buf][t][(lr + 64) * LDK + 8 * lc]) = rb1[t];                                \
        }                                                                                                              \
    }

    f32x16 acc[NB][2][2];
#pragma unroll
    for (int t = 0; t < NB; t++)
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[t][i][j][r] = 0.0f;

    HTR_GEMM_LOAD(0)
    HTR_GEMM_STORE(0)
    __syncthreads();
    const int fr = lane & 31, fk = 8 * (lane >> 5);  // fragment row within a 32-block, k offset
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) HTR_GEMM_LOAD(kt + 1)
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            half8 af[2], bf[NB][2];
#pragma unroll
            for (int i = 0; i < 2; i++)
                af[i] = *reinterpret_cast<const half8 *>(&s_a[cur][(wm * 64 + 32 * i + fr) * LDK + 16 * ks + fk]);
#pragma unroll
            for (int t = 0; t < NB; t++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    bf[t][j] =
                        *reinterpret_cast<const half8 *>(&s_b[cur][t][(wn * 64 + 32 * j + fr) * LDK + 16 * ks + fk]);
#pragma unroll
            for (int t = 0; t < NB; t++)
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[t][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[t][j], acc[t][i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) HTR_GEMM_STORE(cur ^ 1)
        __syncthreads();
    }

#undef HTR_GEMM_LOAD
#undef HTR_GEMM_STORE

    // epilogue: lane ℓ, register r → row 8(r/4) + 4(ℓ/32) + r%4, column ℓ%32 of each 32 × 32 tile
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = col0 + wn * 64 + 32 * j + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = row0 + wm * 64 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row >= a.m) continue;
                const size_t o = (size_t)row * a.n + col;
                if (EPI == GEMM_F32) a.y[o] = acc[0][i][j][r];
                if (EPI == GEMM_ACC) a.y[o] = a.y[o] + acc[0][i][j][r];
                if (EPI == GEMM_FFN) {
                    const float g = acc[0][i][j][r], u = acc[NB - 1][i][j][r];
                    a.y16[o] = (_Float16)(silu(g) * u * a.scale);
                }
            }
        }
    }
}

}  // namespace

int launch_gemm_f16(htr_device *dev, hipStream_t st, int epi, const _Float16 *x, int m, const htr_weight *w,
                    const htr_weight *w2, float *y, _Float16 *y16, float scale) {
    if (!w || !w->h) return htr_fail("gemm_f16: the weight has no f16 plane (htr_weight_q8_0_f16)");
    const int n = (int)w->rows, k = (int)w->cols;
    if (m < 1) return htr_fail("gemm_f16: %d rows", m);
    if (n % BN || k % BK)
        return htr_fail("gemm_f16: W [%d x %d]: rows a multiple of %d, columns a multiple of %d", n, k, BN, BK);
    if (epi == GEMM_FFN && (!w2 || !w2->h || (int)w2->rows != n || (int)w2->cols != k))
        return htr_fail("gemm_f16: the FFN's up weight must match the gate weight [%d x %d]", n, k);
    GemmK a{};
    a.x = x;
    a.w = w->h;
    a.w2 = epi == GEMM_FFN ? w2->h : nullptr;
    a.y = y;
    a.y16 = y16;
    a.m = m;
    a.n = n;
    a.k = k;
    a.scale = scale;
    a.tiles_m = (m + BM - 1) / BM;
    a.tiles_n = n / BN;
    const dim3 grid(a.tiles_m * a.tiles_n);
    switch (epi) {
    case GEMM_F32: hipLaunchKernelGGL(k_gemm_f16<GEMM_F32>, grid, dim3(GW), 0, st, a); break;
    case GEMM_ACC: hipLaunchKernelGGL(k_gemm_f16<GEMM_ACC>, grid, dim3(GW), 0, st, a); break;
    case GEMM_FFN: hipLaunchKernelGGL(k_gemm_f16<GEMM_FFN>, grid, dim3(GW), 0, st, a); break;
    default: return htr_fail("gemm_f16: epilogue %d", epi);
    }
    return htr_launched(dev, "k_gemm_f16");
}

// ---- ABI ------------------------------------------------------------------------------------------------------------

extern "C" int htr_gemm_f16(htr_device *dev, const uint16_t *d_x, size_t m, const htr_weight *w, float *d_y, int acc) {
    HTR_TRY(htr_check_alive(dev));
    if (!d_x || !d_y || !w) return htr_fail("htr_gemm_f16: null argument");
    if (m > (size_t)INT32_MAX / 2) return htr_fail("htr_gemm_f16: %zu rows", m);
    return launch_gemm_f16(dev, dev->stream, acc ? GEMM_ACC : GEMM_F32, (const _Float16 *)d_x, (int)m, w, nullptr, d_y,
                           nullptr, 1.0f);
}

extern "C" int htr_gemm_ffn_f16(htr_device *dev, const uint16_t *d_x, size_t m, const htr_weight *w_gate,
                                const htr_weight *w_up, float scale, uint16_t *d_g) {
    HTR_TRY(htr_check_alive(dev));
    if (!d_x || !d_g || !w_gate || !w_up) return htr_fail("htr_gemm_ffn_f16: null argument");
    if (m > (size_t)INT32_MAX / 2) return htr_fail("htr_gemm_ffn_f16: %zu rows", m);
    return launch_gemm_f16(dev, dev->stream, GEMM_FFN, (const _Float16 *)d_x, (int)m, w_gate, w_up, nullptr,
                           (_Float16 *)d_g, scale);
}
