// The vision encoder's non-GEMM kernels for gfx950 and the f32 GEMM of its patch embedding and projector.
//
// Reference semantics (the f16 compute path, vision.rs:328-423): patchify.wgsl (normalise + im2col), rms_norm.wgsl /
// rms_norm_h (gpu.rs:268-275), rope2d.wgsl (+ vision.rs:159-175), heads_f16.wgsl, attention_coop.wgsl (flash attention
// with q·scale, K, V and P rounded to f16, f32 sums, the output rounded to f16), unfold2x2.wgsl, gelu.wgsl, and the
// f32 matmul of the patch embedding (K = 588) and the projector (f32 activations, f16-valued weights).
#include <cmath>

#include "htr_internal.h"
#include "wave.h"

namespace {

constexpr int VW = 256;

__device__ __forceinline__ size_t gsize() { return (size_t)gridDim.x * VW; }
__device__ __forceinline__ size_t gid() { return blockIdx.x * (size_t)VW + threadIdx.x; }

// patchify.wgsl: P[t][c·p·p + ky·p + kx] = lut[c·256 + rgb[((ty·p + ky)·w + tx·p + kx)·3 + c]]
__global__ __launch_bounds__(VW) void k_patchify(const uint8_t *rgb, const float *lut, int w, int px, int n, int side,
                                                 float *P) {
    const int pp = side * side;
    const size_t total = (size_t)n * 3 * pp;
    for (size_t i = gid(); i < total; i += gsize()) {
        const int t = (int)(i / (3 * pp)), r = (int)(i % (3 * pp));
        const int c = r / pp, ky = (r % pp) / side, kx = r % side;
        const int x = (t % px) * side + kx, y = (t / px) * side + ky;
        P[i] = lut[c * 256 + rgb[((size_t)y * w + x) * 3 + c]];
    }
}

// one workgroup per row: y = x·1/sqrt(mean(x²) + eps)·w, as f32 or rounded to f16
template <typename T>
__global__ __launch_bounds__(VW) void k_rms_norm_rows(const float *x, const float *w, T *y, int dim, float eps) {
    __shared__ float red[VW / 64];
    const size_t base = (size_t)blockIdx.x * dim;
    const int tid = threadIdx.x, lane = tid & 63;
    float s = 0.0f;
    for (int i = tid; i < dim; i += VW) s = fmaf(x[base + i], x[base + i], s);
    s = wave_sum(s, lane);
    if (lane == 0) red[tid >> 6] = s;
    __syncthreads();
    const float scale = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)dim + eps);
    for (int i = tid; i < dim; i += VW) y[base + i] = (T)((x[base + i] * scale) * w[i]);
}

// rope2d.wgsl in place: pairs (2k, 2k+1) of each half of a head; half 0 at the row t / px, half 1 at the column
__global__ __launch_bounds__(VW) void k_rope2d(float *Q, const float *cs, int n_tok, int n_head, int d_head, int px,
                                               int max_pos) {
    const int nk = d_head / 4;
    const size_t total = (size_t)n_tok * n_head * 2 * nk;
    for (size_t i = gid(); i < total; i += gsize()) {
        const int k = (int)(i % nk), half = (int)((i / nk) % 2), h = (int)((i / (2 * nk)) % n_head);
        const int t = (int)(i / (2 * nk * n_head));
        const int pos = half == 0 ? t / px : t % px;
        const float c = cs[2 * (((size_t)half * max_pos + pos) * nk + k)];
        const float s = cs[2 * (((size_t)half * max_pos + pos) * nk + k) + 1];
        float *x = Q + (size_t)t * n_head * d_head + h * d_head + half * (d_head / 2) + 2 * k;
        const float x0 = x[0], x1 = x[1];
        x[0] = x0 * c - x1 * s;
        x[1] = x0 * s + x1 * c;
    }
}

// heads_f16.wgsl: K, V f32 [n][H·64] → f16 [H][n_pad][64] (rows n … n_pad − 1 zero)
__global__ __launch_bounds__(VW) void k_heads_f16(const float *K, const float *V, _Float16 *Kh, _Float16 *Vh, int n_tok,
                                                  int n_head, int n_pad) {
    const size_t total = (size_t)n_head * n_pad * 64;
    for (size_t i = gid(); i < total; i += gsize()) {
        const int d = (int)(i % 64), t = (int)((i / 64) % n_pad), h = (int)(i / (64 * (size_t)n_pad));
        float kv = 0.0f, vv = 0.0f;
        if (t < n_tok) {
            const size_t src = (size_t)t * n_head * 64 + h * 64 + d;
            kv = K[src];
            vv = V[src];
        }
        Kh[i] = (_Float16)kv;
        Vh[i] = (_Float16)vv;
    }
}

// attention_coop.wgsl's arithmetic: O[t][h] = softmax(q16·K16ᵀ)·V16 with q16 = f16(q·scale), keys in blocks of 32
// with the running max (start −3e38), P = f16(e^(S − max)), l = l·corr + Σ P, O = O·corr + Σ P·v; O / l → f16.
// grid (⌈n/64⌉, H), 256 threads = 64 queries × 4 lanes (16 dims each, adjacent lanes); the key block staged in LDS.
constexpr int AQ = 64, AB = 32;
__global__ __launch_bounds__(VW) void k_attn_vision(const float *Q, const _Float16 *Kh, const _Float16 *Vh,
                                                    _Float16 *O, int n_tok, int n_head, int n_pad, float scale) {
    __shared__ __attribute__((aligned(16))) _Float16 s_k[AB * 64];
    __shared__ __attribute__((aligned(16))) _Float16 s_v[AB * 64];
    const int h = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int ql = tid >> 2, part = tid & 3;  // query within the tile, 16-dim part
    const int qi = min(blockIdx.x * AQ + ql, n_tok - 1);
    const int row = n_head * 64;
    float q[16], acc[16];
#pragma unroll
    for (int d = 0; d < 16; d++) {
        q[d] = (float)(_Float16)(Q[(size_t)qi * row + h * 64 + 16 * part + d] * scale);
        acc[d] = 0.0f;
    }
    float m = -3.0e38f, l = 0.0f;
    const _Float16 *kb = Kh + (size_t)h * n_pad * 64, *vb = Vh + (size_t)h * n_pad * 64;
    for (int k0 = 0; k0 < n_tok; k0 += AB) {
        __syncthreads();
        // the block's keys / values: 32 × 64 halves each = 256 × 16 bytes
        reinterpret_cast<int4 *>(s_k)[tid] = reinterpret_cast<const int4 *>(kb + (size_t)k0 * 64)[tid];
        reinterpret_cast<int4 *>(s_v)[tid] = reinterpret_cast<const int4 *>(vb + (size_t)k0 * 64)[tid];
        __syncthreads();
        const int nb = min(AB, n_tok - k0);
        float s[AB];
        float mx = m;
#pragma unroll
        for (int j = 0; j < AB; j++) {
            float d_ = 0.0f;
#pragma unroll
            for (int d = 0; d < 16; d++) d_ = fmaf(q[d], (float)s_k[j * 64 + 16 * part + d], d_);
            d_ += lane_swap<1>(d_, lane);
            d_ += lane_swap<2>(d_, lane);
            s[j] = d_;
            if (j < nb) mx = fmaxf(mx, d_);
        }
        const float corr = expf(m - mx);
        float ps = 0.0f;
#pragma unroll
        for (int d = 0; d < 16; d++) acc[d] *= corr;
#pragma unroll
        for (int j = 0; j < AB; j++) {
            const float p = j < nb ? (float)(_Float16)expf(s[j] - mx) : 0.0f;
            ps += p;
#pragma unroll
            for (int d = 0; d < 16; d++) acc[d] = fmaf(p, (float)s_v[j * 64 + 16 * part + d], acc[d]);
        }
        l = l * corr + ps;
        m = mx;
    }
    if (blockIdx.x * AQ + ql < n_tok) {
        const float inv = 1.0f / l;
#pragma unroll
        for (int d = 0; d < 16; d++) O[(size_t)qi * row + h * 64 + 16 * part + d] = (_Float16)(acc[d] * inv);
    }
}

// unfold2x2.wgsl: Z[o][c·4 + ky·2 + kx] = X[(2·oy + ky)·px + 2·ox + kx][c]
__global__ __launch_bounds__(VW) void k_unfold2x2(const float *X, float *Z, int px, int py, int dim) {
    const int ox_n = px / 2;
    const size_t total = (size_t)(px / 2) * (py / 2) * dim * 4;
    for (size_t i = gid(); i < total; i += gsize()) {
        const int kx = (int)(i % 2), ky = (int)((i / 2) % 2), c = (int)((i / 4) % dim);
        const int o = (int)(i / (4 * (size_t)dim));
        const int ox = o % ox_n, oy = o / ox_n;
        Z[i] = X[((size_t)(2 * oy + ky) * px + 2 * ox + kx) * dim + c];
    }
}

// gelu.wgsl in place (tanh form, argument clamped to ±15)
__global__ __launch_bounds__(VW) void k_gelu(float *X, size_t n) {
    for (size_t i = gid(); i < n; i += gsize()) {
        const float x = X[i];
        const float t = fminf(fmaxf(0.7978845608028654f * x * (1.0f + 0.044715f * x * x), -15.0f), 15.0f);
        X[i] = 0.5f * x * (1.0f + tanhf(t));
    }
}

// Y[M,N] (+)= X[M,K]·Wᵀ with f32 X and W of type WT (f32, or f16 read as f32), f32 fma in k order per output;
// 64 × 64 tiles, K in steps of 16 through LDS, 4 × 4 outputs a thread
template <typename WT>
__global__ __launch_bounds__(VW) void k_gemm_f32w(const float *X, const WT *W, float *Y, int m, int n, int k, int acc) {
    __shared__ float s_x[16][64 + 4];
    __shared__ float s_w[16][64 + 4];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int row0 = blockIdx.y * 64, col0 = blockIdx.x * 64;
    float c[4][4] = {};
    for (int k0 = 0; k0 < k; k0 += 16) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = tid + VW * i, r = e >> 4, kk = e & 15;
            const int gr = row0 + r, gc = col0 + r, gk = k0 + kk;
            s_x[kk][r] = gr < m && gk < k ? X[(size_t)gr * k + gk] : 0.0f;
            s_w[kk][r] = gc < n && gk < k ? (float)W[(size_t)gc * k + gk] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; kk++) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                a[i] = s_x[kk][ty + 16 * i];
                b[i] = s_w[kk][tx + 16 * i];
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
            float *o = Y + (size_t)r * n + cc;
            *o = acc ? *o + c[i][j] : c[i][j];
        }
    }
}

int grid_for(size_t total) { return (int)std::max<size_t>(1, std::min<size_t>((total + VW - 1) / VW, 65536)); }

}  // namespace

int launch_patchify(htr_device *dev, hipStream_t st, const uint8_t *rgb, const float *lut, int w, int px, int n,
                    int side, float *P) {
    hipLaunchKernelGGL(k_patchify, dim3(grid_for((size_t)n * 3 * side * side)), dim3(VW), 0, st, rgb, lut, w, px, n,
                       side, P);
    return htr_launched(dev, "k_patchify");
}

int launch_rms_norm_f16(htr_device *dev, hipStream_t st, const float *x, const float *w, _Float16 *y, int rows, int dim,
                        float eps) {
    hipLaunchKernelGGL(k_rms_norm_rows<_Float16>, dim3(rows), dim3(VW), 0, st, x, w, y, dim, eps);
    return htr_launched(dev, "k_rms_norm_rows<f16>");
}

int launch_rope2d(htr_device *dev, hipStream_t st, float *q, const float *cs, int n_tok, int n_head, int d_head, int px,
                  int max_pos) {
    hipLaunchKernelGGL(k_rope2d, dim3(grid_for((size_t)n_tok * n_head * d_head / 2)), dim3(VW), 0, st, q, cs, n_tok,
                       n_head, d_head, px, max_pos);
    return htr_launched(dev, "k_rope2d");
}

int launch_heads_f16(htr_device *dev, hipStream_t st, const float *k, const float *v, _Float16 *kh, _Float16 *vh,
                     int n_tok, int n_head, int n_pad) {
    hipLaunchKernelGGL(k_heads_f16, dim3(grid_for((size_t)n_head * n_pad * 64)), dim3(VW), 0, st, k, v, kh, vh, n_tok,
                       n_head, n_pad);
    return htr_launched(dev, "k_heads_f16");
}

int launch_attn_vision(htr_device *dev, hipStream_t st, const float *q, const _Float16 *kh, const _Float16 *vh,
                       _Float16 *o, int n_tok, int n_head, int n_pad, float scale) {
    if (n_pad % AB || n_pad < n_tok) return htr_fail("vision attention: %d padded keys for %d tokens", n_pad, n_tok);
    hipLaunchKernelGGL(k_attn_vision, dim3((n_tok + AQ - 1) / AQ, n_head), dim3(VW), 0, st, q, kh, vh, o, n_tok, n_head,
                       n_pad, scale);
    return htr_launched(dev, "k_attn_vision");
}

int launch_unfold2x2(htr_device *dev, hipStream_t st, const float *x, float *z, int px, int py, int dim) {
    hipLaunchKernelGGL(k_unfold2x2, dim3(grid_for((size_t)px * py * dim)), dim3(VW), 0, st, x, z, px, py, dim);
    return htr_launched(dev, "k_unfold2x2");
}

int launch_gelu(htr_device *dev, hipStream_t st, float *x, size_t n) {
    hipLaunchKernelGGL(k_gelu, dim3(grid_for(n)), dim3(VW), 0, st, x, n);
    return htr_launched(dev, "k_gelu");
}

int launch_gemm_f32w(htr_device *dev, hipStream_t st, const float *x, const void *w, bool w_f16, float *y, int m, int n,
                     int k, int acc) {
    const dim3 grid((n + 63) / 64, (m + 63) / 64);
    if (w_f16)
        hipLaunchKernelGGL(k_gemm_f32w<_Float16>, grid, dim3(VW), 0, st, x, (const _Float16 *)w, y, m, n, k, acc);
    else
        hipLaunchKernelGGL(k_gemm_f32w<float>, grid, dim3(VW), 0, st, x, (const float *)w, y, m, n, k, acc);
    return htr_launched(dev, "k_gemm_f32w");
}
