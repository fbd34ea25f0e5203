// Dense kernels of the prefill for gfx950: Y[M,N] (+)= X[M,K]·Wᵀ with q8_0 weights, RMS norm over rows, SwiGLU.
//
// Reference semantics: matmul.wgsl:47-91 (F32 path: W dequantised exactly — q·d is exact in f32 — and f32 fma
// accumulation; acc = 1 adds onto Y, the residual stream), rms_norm.wgsl:21-41, swiglu.wgsl:18-24 (text.rs:484-518).
//
// The GEMM: 64×64 output tiles, 256 threads with 4×4 outputs each, K in steps of 32 = one q8_0 block, so a tile's
// column needs one scale; X and the dequantised W tile are staged in LDS as f32.
#include "htr_internal.h"

namespace {

constexpr int BM = 64, BN = 64, BK = 32;

__global__ __launch_bounds__(256) void k_gemm_q8_0_f32(const float *x, const int8_t *wq, const _Float16 *wd, float *y,
                                                       int m, int n, int k, int acc) {
    __shared__ float s_a[BK][BM + 4];
    __shared__ float s_b[BK][BN + 4];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int row0 = blockIdx.y * BM, col0 = blockIdx.x * BN;
    const int nb = k / 32;
    float c[4][4] = {};
    for (int k0 = 0; k0 < k; k0 += BK) {
        // X tile: 64 rows × 32 k (8 per thread, k fastest for coalescing)
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int e = tid + 256 * i, r = e / BK, cc = e % BK;
            const int gr = row0 + r;
            s_a[cc][r] = gr < m ? x[(size_t)gr * k + k0 + cc] : 0.0f;
        }
        // W tile: 64 columns × 32 quants of one block each, times that block's scale
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int e = tid + 256 * i, r = e / BK, cc = e % BK;
            const int gc = col0 + r;
            float v = 0.0f;
            if (gc < n) v = (float)wq[(size_t)gc * k + k0 + cc] * (float)wd[(size_t)gc * nb + k0 / 32];
            s_b[cc][r] = v;
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < BK; kk++) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                a[i] = s_a[kk][ty + 16 * i];
                b[i] = s_b[kk][tx + 16 * i];
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) c[i][j] = fmaf(a[i], b[j], c[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = row0 + ty + 16 * i;
        if (r >= m) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int cc = col0 + tx + 16 * j;
            if (cc >= n) continue;
            float *o = y + (size_t)r * n + cc;
            *o = acc ? *o + c[i][j] : c[i][j];
        }
    }
}

// one workgroup per row: y = x · 1/sqrt(mean(x²) + eps) · w
__global__ __launch_bounds__(256) void k_rms_norm(const float *x, const float *w, float *y, int dim, float eps) {
    __shared__ float red[4];
    const size_t base = (size_t)blockIdx.x * dim;
    const int tid = threadIdx.x;
    float s = 0.0f;
    for (int i = tid; i < dim; i += 256) s = fmaf(x[base + i], x[base + i], s);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    const float scale = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)dim + eps);
    for (int i = tid; i < dim; i += 256) y[base + i] = (x[base + i] * scale) * w[i];
}

__global__ __launch_bounds__(256) void k_swiglu(float *g, const float *u, size_t n) {
    for (size_t i = blockIdx.x * (size_t)256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const float v = g[i];
        g[i] = (v / (1.0f + expf(-v))) * u[i];
    }
}

}  // namespace

int launch_gemm_q8_0_f32(htr_device *dev, hipStream_t st, const float *x, const htr_weight *w, float *y, int m,
                         int acc) {
    if (!w->q) return htr_fail("gemm: weight has no q8_0 planes");
    dim3 grid(((int)w->rows + BN - 1) / BN, (m + BM - 1) / BM);
    hipLaunchKernelGGL(k_gemm_q8_0_f32, grid, dim3(256), 0, st, x, w->q, w->d, y, m, (int)w->rows, (int)w->cols, acc);
    return htr_launched(dev, "k_gemm_q8_0_f32");
}

int launch_rms_norm(htr_device *dev, hipStream_t st, const float *x, const float *w, float *y, int rows, int dim,
                    float eps) {
    hipLaunchKernelGGL(k_rms_norm, dim3(rows), dim3(256), 0, st, x, w, y, dim, eps);
    return htr_launched(dev, "k_rms_norm");
}

int launch_swiglu(htr_device *dev, hipStream_t st, float *g, const float *u, size_t n) {
    const int grid = (int)std::min<size_t>((n + 255) / 256, 16384);
    hipLaunchKernelGGL(k_swiglu, dim3(grid), dim3(256), 0, st, g, u, n);
    return htr_launched(dev, "k_swiglu");
}
