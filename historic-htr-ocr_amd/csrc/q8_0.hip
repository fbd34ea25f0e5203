// q8_0 dequant-matvec family for gfx950 (wave64): the decode step's projections and the LM head.
//
// Reference semantics: dmv.wgsl:22-52 (y (+)= W·x, dmv_norm), dmv_qkv.wgsl:23-65, dmv_ffn.wgsl:22-51,
// dmv_common.wgsl:23-30 (the fused RMS norm), embed_q8_0.wgsl:19-38. Layout and schedule are this library's own:
//
//   weights   repacked at load (runtime.hip) into an int8 plane q[rows][K] and an f16 scale plane d[rows][K/32];
//   lanes     a row is cut into groups of 16 quants (16 bytes); lane ℓ of a wave takes the groups ℓ, ℓ+64, … of every
//             row the wave computes, so one wave-wide load instruction reads 1 KiB of contiguous quants (a whole row
//             at K = 1024); the lane's 16 inputs x[16g…16g+15] sit in registers for all its rows;
//   schedule  a wave computes R consecutive rows; all R·NG 16-byte loads (and their scales) are issued before the
//             first use; a 256-thread workgroup = 4 waves = 4R rows;
//   reduce    per row, the 64 lane partials are summed across the wave (cross-lane butterfly);
//   norm      the fused RMS norm computes Σx² once per workgroup (x is ≤ 16 KiB and L2-resident);
//   math      f32: the 16 int8·x products of a group are an fma chain, times the block's f16 scale into the row's
//             accumulator (the scale is exact in f32).
#include "htr_internal.h"

namespace {

constexpr int WG = 256;
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

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
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

// 1/sqrt(mean(x²) + eps) over k inputs, the whole workgroup
__device__ __forceinline__ float norm_scale(const float *x, int k, float eps) {
    __shared__ float red[WG / 64];
    const int tid = threadIdx.x;
    float s = 0.0f;
    for (int i = tid; i < k / 4; i += WG) {
        float4 v = reinterpret_cast<const float4 *>(x)[i];
        s = fmaf(v.x, v.x, s);
        s = fmaf(v.y, v.y, s);
        s = fmaf(v.z, v.z, s);
        s = fmaf(v.w, v.w, s);
    }
    s = wave_sum(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    float t = (red[0] + red[1]) + (red[2] + red[3]);
    return 1.0f / sqrtf(t / (float)k + eps);
}

template <int R, int NG, int MODE> __global__ __launch_bounds__(WG) void k_dmv(const DmvK a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int k = a.k, ng = k >> 4, nb = k >> 5;
    float scale = 1.0f;
    if (MODE != DMV_PLAIN) scale = norm_scale(a.x, k, a.eps);

    // the lane's inputs: groups lane + 64·i
    float xv[NG][16];
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const int g = lane + 64 * i;
#pragma unroll
        for (int j = 0; j < 16; j++) xv[i][j] = 0.0f;
        if (g < ng) {
            const float4 *xp = reinterpret_cast<const float4 *>(a.x + 16 * g);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float4 v = xp[j];
                xv[i][4 * j + 0] = v.x;
                xv[i][4 * j + 1] = v.y;
                xv[i][4 * j + 2] = v.z;
                xv[i][4 * j + 3] = v.w;
            }
            if (MODE != DMV_PLAIN) {
                const float4 *wp = reinterpret_cast<const float4 *>(a.nw + 16 * g);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float4 w = wp[j];
                    xv[i][4 * j + 0] = (xv[i][4 * j + 0] * scale) * w.x;
                    xv[i][4 * j + 1] = (xv[i][4 * j + 1] * scale) * w.y;
                    xv[i][4 * j + 2] = (xv[i][4 * j + 2] * scale) * w.z;
                    xv[i][4 * j + 3] = (xv[i][4 * j + 3] * scale) * w.w;
                }
            }
        }
    }

    constexpr int NM = MODE == DMV_FFN ? 2 : 1;  // matrices read per output row
    const int row0 = (blockIdx.x * (WG / 64) + wave) * R;
    int4 qv[NM][R][NG];
    float dv[NM][R][NG];
    // issue every load of the wave's rows first
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = row0 + r;
        const bool ok = row < a.n_rows;
        int mi = 0, lr = row;
        if (MODE == DMV_QKV) {
            if (lr >= a.m[0].rows) {
                lr -= a.m[0].rows;
                mi = 1;
                if (lr >= a.m[1].rows) {
                    lr -= a.m[1].rows;
                    mi = 2;
                }
            }
        }
#pragma unroll
        for (int t = 0; t < NM; t++) {
            const DmvMat &m = a.m[MODE == DMV_FFN ? t : mi];
            const int8_t *qrow = m.q + (size_t)lr * k;
            const _Float16 *drow = m.d + (size_t)lr * nb;
#pragma unroll
            for (int i = 0; i < NG; i++) {
                const int g = lane + 64 * i;
                if (ok && g < ng) {
                    qv[t][r][i] = *reinterpret_cast<const int4 *>(qrow + 16 * g);
                    dv[t][r][i] = (float)drow[g >> 1];
                } else {
                    qv[t][r][i] = make_int4(0, 0, 0, 0);
                    dv[t][r][i] = 0.0f;
                }
            }
        }
    }
    float acc[NM][R];
#pragma unroll
    for (int t = 0; t < NM; t++) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < NG; i++) s = fmaf(dot16(qv[t][r][i], xv[i]), dv[t][r][i], s);
            acc[t][r] = wave_sum(s);
        }
    }
    if (lane < R) {
        // lane r writes row r (a select chain keeps the accumulators in registers)
        float v[NM];
#pragma unroll
        for (int t = 0; t < NM; t++) {
            v[t] = acc[t][0];
#pragma unroll
            for (int r = 1; r < R; r++) v[t] = lane == r ? acc[t][r] : v[t];
        }
        const int row = row0 + lane;
        if (row < a.n_rows) {
            float out = v[0];
            if (MODE == DMV_FFN) out = (v[0] / (1.0f + expf(-v[0]))) * v[1];
            if (a.acc) out = a.y[row] + out;
            a.y[row] = out;
        }
    }
}

// n matvecs y_i = W_i · x in one launch (blockIdx.y = i), the plain kernel's schedule
struct DmvManyK {
    DmvMat m[MAX_MANY];
    int k;
    const float *x;
    float *y;
};

template <int R, int NG> __global__ __launch_bounds__(WG) void k_dmv_many(const DmvManyK a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int k = a.k, ng = k >> 4, nb = k >> 5;
    const DmvMat m = a.m[blockIdx.y];
    float xv[NG][16];
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const int g = lane + 64 * i;
#pragma unroll
        for (int j = 0; j < 16; j++) xv[i][j] = g < ng ? a.x[16 * g + j] : 0.0f;
    }
    const int row0 = (blockIdx.x * (WG / 64) + wave) * R;
    int4 qv[R][NG];
    float dv[R][NG];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = row0 + r;
#pragma unroll
        for (int i = 0; i < NG; i++) {
            const int g = lane + 64 * i;
            if (row < m.rows && g < ng) {
                qv[r][i] = *reinterpret_cast<const int4 *>(m.q + (size_t)row * k + 16 * g);
                dv[r][i] = (float)m.d[(size_t)row * nb + (g >> 1)];
            } else {
                qv[r][i] = make_int4(0, 0, 0, 0);
                dv[r][i] = 0.0f;
            }
        }
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < NG; i++) s = fmaf(dot16(qv[r][i], xv[i]), dv[r][i], s);
        acc[r] = wave_sum(s);
    }
    if (lane < R) {
        float v = acc[0];
#pragma unroll
        for (int r = 1; r < R; r++) v = lane == r ? acc[r] : v;
        const int row = row0 + lane;
        if (row < m.rows) a.y[(size_t)blockIdx.y * m.rows + row] = v;
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

template <int R, int MODE> int dispatch_ng(hipStream_t st, int ng_lane, dim3 grid, const DmvK &a) {
    switch (ng_lane) {
    case 1: hipLaunchKernelGGL((k_dmv<R, 1, MODE>), grid, dim3(WG), 0, st, a); return 0;
    case 2: hipLaunchKernelGGL((k_dmv<R, 2, MODE>), grid, dim3(WG), 0, st, a); return 0;
    case 3: hipLaunchKernelGGL((k_dmv<R, 3, MODE>), grid, dim3(WG), 0, st, a); return 0;
    case 4: hipLaunchKernelGGL((k_dmv<R, 4, MODE>), grid, dim3(WG), 0, st, a); return 0;
    }
    return -1;
}

template <int MODE> int dispatch_r(hipStream_t st, int r, int ng_lane, const DmvK &a) {
    dim3 grid((a.n_rows + 4 * r - 1) / (4 * r));
    switch (r) {
    case 1: return dispatch_ng<1, MODE>(st, ng_lane, grid, a);
    case 2: return dispatch_ng<2, MODE>(st, ng_lane, grid, a);
    case 4: return dispatch_ng<4, MODE>(st, ng_lane, grid, a);
    }
    return -1;
}

// rows per wave: enough workgroups to cover the chip several times over before rows are batched per wave
int rows_per_wave(int n_rows) {
    if (n_rows >= 16 * 4096) return 4;
    if (n_rows >= 8 * 2048) return 2;
    return 1;
}

}  // namespace

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
    const int r = rows_per_wave(rows);
    int rc = -1;
    switch (mode) {
    case DMV_PLAIN: rc = dispatch_r<DMV_PLAIN>(st, r, ng_lane, a); break;
    case DMV_NORM: rc = dispatch_r<DMV_NORM>(st, r, ng_lane, a); break;
    case DMV_QKV: rc = dispatch_r<DMV_QKV>(st, r, ng_lane, a); break;
    case DMV_FFN: rc = dispatch_r<DMV_FFN>(st, r, ng_lane, a); break;
    }
    if (rc < 0) return htr_fail("matvec: no kernel for mode %d, R %d, K %d", mode, r, k);
    return htr_launched(dev, "k_dmv");
}

int launch_dmv_many(htr_device *dev, hipStream_t st, const DmvMat *mats, int n, int k, const float *x, float *y) {
    if (k <= 0 || k % 32 != 0 || k > 4096) return htr_fail("matvec_many: K = %d (a multiple of 32, at most 4096)", k);
    for (int base = 0; base < n; base += MAX_MANY) {
        const int cnt = std::min(MAX_MANY, n - base);
        DmvManyK a{};
        for (int i = 0; i < cnt; i++) a.m[i] = mats[base + i];
        a.k = k;
        a.x = x;
        a.y = y + (size_t)base * mats[0].rows;
        const int rows = mats[0].rows;
        const int ng_lane = (k / 16 + 63) / 64;
        const int r = 2;
        dim3 grid((rows + 4 * r - 1) / (4 * r), cnt);
        switch (ng_lane) {
        case 1: hipLaunchKernelGGL((k_dmv_many<2, 1>), grid, dim3(WG), 0, st, a); break;
        case 2: hipLaunchKernelGGL((k_dmv_many<2, 2>), grid, dim3(WG), 0, st, a); break;
        case 3: hipLaunchKernelGGL((k_dmv_many<2, 3>), grid, dim3(WG), 0, st, a); break;
        default: hipLaunchKernelGGL((k_dmv_many<2, 4>), grid, dim3(WG), 0, st, a); break;
        }
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
