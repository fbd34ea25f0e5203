// Dense kernels of the prefill for gfx950: Y[M,N] (+)= X[M,K]·Wᵀ with q8_0 weights, RMS norm over rows, SwiGLU.
//
// Reference semantics: matmul.wgsl:47-91 (F32 path: W dequantised exactly — q·d is exact in f32 — and f32 fma
// accumulation; acc = 1 adds onto Y, the residual stream), rms_norm.wgsl:21-41, swiglu.wgsl:18-24 (text.rs:484-518).
//
// The GEMM on the matrix cores (k_gemm_q8_0_mfma; N a multiple of 64): v_mfma_f32_32x32x2_f32 keeps the F32 path's
// f32 products and sums (the order is the matrix unit's). 64×64 output tiles (M is the prompt length, ~1000, so small
// tiles keep 256+ workgroups busy), 4 waves of one 32×32 MFMA tile each, K in steps of 32 = one q8_0 block: X and the
// exactly dequantised W tile are staged in LDS as f32 (double-buffered, the next step's global loads in flight),
// 16-byte chunks placed at chunk ^ (row/2 % 8) so 16 lanes' 16-byte reads fall on 16 bank groups. Lane half h takes
// the 16 consecutive k of 16h … 16h + 15 over the step's 16 MFMAs (k-slot h of each), so a lane's fragments are 4
// contiguous 16-byte reads. Measured (1023 rows): see the bench's prefill. Other shapes: k_gemm_q8_0_f32, 64×64
// tiles, 256 threads with 4×4 outputs each in f32 fma.
//
// The f16 compute path (matmul_coop_q8_0 / matmul128h_q8_0, gpu.rs:1976-1995) rounds X and the dequantised W to f16
// where they enter the tiles and accumulates in f32: k_gemm_q8_0_f32<true> does that for any shape (the MFMA kernels
// of that path, on f16 planes made by k_q8_to_f16, are in mfma_gemm.hip).
#include <algorithm>

#include "htr_internal.h"

namespace {

constexpr int BM = 64, BN = 64, BK = 32;

// R16: X and W values rounded to f16 (round to nearest even) as they enter the tiles
template <bool R16> __device__ __forceinline__ float tile_val(float v) { return R16 ? (float)(_Float16)v : v; }

template <bool R16>
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
            s_a[cc][r] = gr < m ? tile_val<R16>(x[(size_t)gr * k + k0 + cc]) : 0.0f;
        }
        // W tile: 64 columns × 32 quants of one block each, times that block's scale
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int e = tid + 256 * i, r = e / BK, cc = e % BK;
            const int gc = col0 + r;
            float v = 0.0f;
            if (gc < n) v = tile_val<R16>((float)wq[(size_t)gc * k + k0 + cc] * (float)wd[(size_t)gc * nb + k0 / 32]);
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


typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ int mf_slot(int r, int q) { return 8 * r + (q ^ ((r >> 1) & 7)); }

__global__ __launch_bounds__(256) void k_gemm_q8_0_mfma(const float *x, const int8_t *wq, const _Float16 *wd, float *y,
                                                        int m, int n, int k, int acc) {
    __shared__ __attribute__((aligned(16))) float4 s_a[2][64 * 8];  // [row][chunk] f32, 8 KB a buffer
    __shared__ __attribute__((aligned(16))) float4 s_b[2][64 * 8];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int row0 = blockIdx.y * 64, col0 = blockIdx.x * 64;
    const int nb = k / 32;
    // staging: thread t moves row t/4, k 8·(t%4) … + 7 of the X tile and of the W tile
    const int lr = tid >> 2, lq = tid & 3;
    const float *xr = x + (size_t)min(row0 + lr, m - 1) * k + 8 * lq;
    const int8_t *wr = wq + (size_t)(col0 + lr) * k + 8 * lq;
    const _Float16 *dr = wd + (size_t)(col0 + lr) * nb;
    float4 ra0, ra1;
    int2 rq;
    float rd;
    auto gload = [&](int kb) {
        const float4 *xs = reinterpret_cast<const float4 *>(xr + 32 * kb);
        ra0 = xs[0];
        ra1 = xs[1];
        rq = *reinterpret_cast<const int2 *>(wr + 32 * kb);
        rd = (float)dr[kb];
    };
    auto lstore = [&](int buf) {
        s_a[buf][mf_slot(lr, 2 * lq)] = ra0;
        s_a[buf][mf_slot(lr, 2 * lq + 1)] = ra1;
        const uint32_t u0 = (uint32_t)rq.x, u1 = (uint32_t)rq.y;
        s_b[buf][mf_slot(lr, 2 * lq)] = make_float4((float)(int8_t)u0 * rd, (float)(int8_t)(u0 >> 8) * rd,
                                                    (float)(int8_t)(u0 >> 16) * rd, (float)(int8_t)(u0 >> 24) * rd);
        s_b[buf][mf_slot(lr, 2 * lq + 1)] = make_float4((float)(int8_t)u1 * rd, (float)(int8_t)(u1 >> 8) * rd,
                                                        (float)(int8_t)(u1 >> 16) * rd, (float)(int8_t)(u1 >> 24) * rd);
    };
    f32x16 c;
#pragma unroll
    for (int r = 0; r < 16; r++) c[r] = 0.0f;
    const int fr_a = wm * 32 + (lane & 31), fr_b = wn * 32 + (lane & 31), h = lane >> 5;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kb = 0; kb < nb; kb++) {
        const int cur = kb & 1;
        if (kb + 1 < nb) gload(kb + 1);
        float a[16], b[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 va = s_a[cur][mf_slot(fr_a, 4 * h + q)], vb = s_b[cur][mf_slot(fr_b, 4 * h + q)];
            a[4 * q] = va.x, a[4 * q + 1] = va.y, a[4 * q + 2] = va.z, a[4 * q + 3] = va.w;
            b[4 * q] = vb.x, b[4 * q + 1] = vb.y, b[4 * q + 2] = vb.z, b[4 * q + 3] = vb.w;
        }
#pragma unroll
        for (int s2 = 0; s2 < 16; s2++) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s2], b[s2], c, 0, 0, 0);
        if (kb + 1 < nb) lstore(cur ^ 1);
        __syncthreads();
    }
    const int col = col0 + wn * 32 + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int row = row0 + wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row >= m) continue;
        float *o = y + (size_t)row * n + col;
        *o = acc ? *o + c[r] : c[r];
    }
}

// the f16 plane of a q8_0 weight: h = f16(q · d) (round to nearest even), 8 values a thread
__global__ __launch_bounds__(256) void k_q8_to_f16(const int8_t *q, const _Float16 *d, _Float16 *h, size_t n8,
                                                    int cols) {
    for (size_t i = blockIdx.x * (size_t)256 + threadIdx.x; i < n8; i += (size_t)gridDim.x * 256) {
        const size_t e = 8 * i, r = e / cols, c = e % cols;
        const float s = (float)d[r * (cols / 32) + c / 32];
        const int2 v = *reinterpret_cast<const int2 *>(q + e);
        const uint32_t u[2] = {(uint32_t)v.x, (uint32_t)v.y};
        _Float16 o[8];
#pragma unroll
        for (int j = 0; j < 8; j++) o[j] = (_Float16)((float)(int8_t)(u[j / 4] >> (8 * (j % 4))) * s);
        int4 out;
        __builtin_memcpy(&out, o, 16);
        *reinterpret_cast<int4 *>(h + e) = out;
    }
}

}  // namespace

int weight_attach_f16(htr_device *dev, hipStream_t st, htr_weight *w) {
    if (w->h) return 0;
    if (!w->q) return htr_fail("weight_attach_f16: the weight has no q8_0 planes");
    HTR_TRY(htr_dev_alloc(dev, w->rows * w->cols * 2, HTR_MEM_WEIGHTS, (void **)&w->h));
    const size_t n8 = w->rows * w->cols / 8;  // cols is a multiple of 32
    const int grid = (int)std::min<size_t>((n8 + 255) / 256, (size_t)dev->n_cu * 16);
    hipLaunchKernelGGL(k_q8_to_f16, dim3(grid), dim3(256), 0, st, w->q, w->d, w->h, n8, (int)w->cols);
    return htr_launched(dev, "k_q8_to_f16");
}

int launch_gemm_q8_0_f32(htr_device *dev, hipStream_t st, const float *x, const htr_weight *w, float *y, int m,
                         int acc) {
    if (!w->q) return htr_fail("gemm: weight has no q8_0 planes");
    dim3 grid(((int)w->rows + BN - 1) / BN, (m + BM - 1) / BM);
    if (w->rows % 64 == 0 && w->cols % 32 == 0) {
        hipLaunchKernelGGL(k_gemm_q8_0_mfma, grid, dim3(256), 0, st, x, w->q, w->d, y, m, (int)w->rows, (int)w->cols,
                           acc);
        return htr_launched(dev, "k_gemm_q8_0_mfma");
    }
    hipLaunchKernelGGL(k_gemm_q8_0_f32<false>, grid, dim3(256), 0, st, x, w->q, w->d, y, m, (int)w->rows,
                       (int)w->cols, acc);
    return htr_launched(dev, "k_gemm_q8_0_f32");
}

int launch_gemm_q8_0_r16(htr_device *dev, hipStream_t st, const float *x, const htr_weight *w, float *y, int m,
                         int acc) {
    if (!w->q) return htr_fail("gemm: weight has no q8_0 planes");
    dim3 grid(((int)w->rows + BN - 1) / BN, (m + BM - 1) / BM);
    hipLaunchKernelGGL(k_gemm_q8_0_f32<true>, grid, dim3(256), 0, st, x, w->q, w->d, y, m, (int)w->rows,
                       (int)w->cols, acc);
    return htr_launched(dev, "k_gemm_q8_0_f32<r16>");
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

// ---- ABI ------------------------------------------------------------------------------------------------------------

extern "C" int htr_matmul_q8_0(htr_device *dev, const float *d_x, size_t m, const htr_weight *w, float *d_y, int acc) {
    HTR_TRY(htr_check_alive(dev));
    if (!d_x || !d_y || !w) return htr_fail("htr_matmul_q8_0: null argument");
    if (m == 0) return 0;
    if (m > (size_t)INT32_MAX / 2) return htr_fail("htr_matmul_q8_0: %zu rows", m);
    return dev->compute == HTR_COMPUTE_F32 ? launch_gemm_q8_0_f32(dev, dev->stream, d_x, w, d_y, (int)m, acc)
                                           : launch_gemm_q8_0_r16(dev, dev->stream, d_x, w, d_y, (int)m, acc);
}
