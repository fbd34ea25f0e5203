// Attention for gfx950: the decode step's q/k post-processing and split-K GQA decode attention, and the prefill's
// per-head norm + RoPE + KV store and causal flash attention.
//
// Reference semantics: qkv_post.wgsl:31-83, attn_decode.wgsl:34-100 + attn_merge.wgsl:22-39 (text.rs:639-641),
// rms_norm.wgsl / rope_neox.wgsl / kv_store.wgsl / attention_causal.wgsl (text.rs:484-499). Head dim 128.
//
// KV cache layout (this library's): f16, head-major per layer, [n_kv][n_ctx][128] — one KV head's keys are
// contiguous, so a workgroup working on (kv head, key chunk) reads one contiguous range (256 bytes per key).
#include "htr_internal.h"

namespace {

constexpr int D = 128;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// one head's 128 values held as (lane, lane + 64) by a 64-lane wave: RMS norm with w, then RoPE NEOX with (c, s)
__device__ __forceinline__ void norm_rope(float &x0, float &x1, const float *w, const float *rope_row, int lane,
                                          float eps) {
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float scale = 1.0f / sqrtf(ss / (float)D + eps);
    const float y0 = (x0 * scale) * w[lane], y1 = (x1 * scale) * w[lane + 64];
    const float c = rope_row[2 * lane], s = rope_row[2 * lane + 1];
    x0 = y0 * c - y1 * s;
    x1 = y0 * s + y1 * c;
}

// qkv_post: block h < n_head: q head (norm, rope, in place); < n_head + n_kv: k head (norm, rope, f16 cache);
// else v head (f16 cache). One wave per head.
__global__ __launch_bounds__(64) void k_qkv_post(float *qkv, const float *qn, const float *kn, const float *rope,
                                                 int n_head, int n_kv, const int *pos_dev, int pos_arg, int n_ctx,
                                                 float eps, _Float16 *kc, _Float16 *vc) {
    const int h = blockIdx.x, lane = threadIdx.x;
    const int pos = pos_dev ? *pos_dev : pos_arg;
    float *x = qkv + (size_t)h * D;
    float x0 = x[lane], x1 = x[lane + 64];
    if (h >= n_head + n_kv) {
        _Float16 *o = vc + ((size_t)(h - n_head - n_kv) * n_ctx + pos) * D;
        o[lane] = (_Float16)x0;
        o[lane + 64] = (_Float16)x1;
        return;
    }
    norm_rope(x0, x1, h < n_head ? qn : kn, rope + (size_t)pos * D, lane, eps);
    if (h < n_head) {
        x[lane] = x0;
        x[lane + 64] = x1;
    } else {
        _Float16 *o = kc + ((size_t)(h - n_head) * n_ctx + pos) * D;
        o[lane] = (_Float16)x0;
        o[lane + 64] = (_Float16)x1;
    }
}

// prefill rows: block (t, h): q heads, k heads (→ f16 cache rows pos0 + t), v heads (→ f16 cache)
__global__ __launch_bounds__(64) void k_qk_rows(float *q, float *k, const float *v, const float *qn, const float *kn,
                                                const float *rope, int n_head, int n_kv, int pos0, int n_ctx,
                                                float eps, _Float16 *kc, _Float16 *vc) {
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int pos = pos0 + t;
    if (h < n_head) {
        float *x = q + ((size_t)t * n_head + h) * D;
        float x0 = x[lane], x1 = x[lane + 64];
        norm_rope(x0, x1, qn, rope + (size_t)pos * D, lane, eps);
        x[lane] = x0;
        x[lane + 64] = x1;
    } else if (h < n_head + n_kv) {
        const int j = h - n_head;
        float *x = k + ((size_t)t * n_kv + j) * D;
        float x0 = x[lane], x1 = x[lane + 64];
        norm_rope(x0, x1, kn, rope + (size_t)pos * D, lane, eps);
        _Float16 *o = kc + ((size_t)j * n_ctx + pos) * D;
        o[lane] = (_Float16)x0;
        o[lane + 64] = (_Float16)x1;
    } else {
        const int j = h - n_head - n_kv;
        const float *x = v + ((size_t)t * n_kv + j) * D;
        _Float16 *o = vc + ((size_t)j * n_ctx + pos) * D;
        o[lane] = (_Float16)x[lane];
        o[lane + 64] = (_Float16)x[lane + 64];
    }
}

// ---- split-K decode attention -----------------------------------------------------------------------------------------
//
// grid (chunks, n_kv), 256 threads = 4 waves. A workgroup takes `chunk` keys of one KV head and both of its q heads
// (GQA group 2): every K / V byte is read once. Within a wave, 16 lanes share a key (8 dims = 16 bytes each), so a
// wave reads 4 keys (1 KiB) per load instruction.
//   1. scores s[h][t] = (q_h·scale)·k_t      → LDS
//   2. m = max s, e = exp(s − m), l = Σ e     (per head, over the chunk)
//   3. o[h][·] = Σ_t e[h][t]·v_t              → lane partials, summed across the wave's 4 key groups and the 4 waves
//      in LDS
//   4. the chunk's (m, l, o) → part; the last workgroup of the KV head (atomic ticket) merges every chunk's partials
//      in LDS: M = max m_c, L = Σ l_c e^(m_c − M), O = Σ o_c e^(m_c − M) / L — no second launch.
constexpr int AW = 256;
constexpr int MAX_CHUNK_KEYS = 256;

__global__ __launch_bounds__(AW) void k_attn_decode(const float *q, const _Float16 *kc, const _Float16 *vc, int n_kv,
                                                    int n_ctx, const int *pos_dev, int n_keys_arg, int chunk,
                                                    int max_chunk, float scale, float *part, uint32_t *counters,
                                                    float *out) {
    __shared__ float s_sc[2][MAX_CHUNK_KEYS];
    __shared__ float s_red[2][4];
    __shared__ float s_o[4][2][D];
    __shared__ int s_last;
    const int c = blockIdx.x, kvh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n_keys = pos_dev ? *pos_dev + 1 : n_keys_arg;
    const int n_chunk = (n_keys + chunk - 1) / chunk;
    if (c >= n_chunk) return;  // uniform per workgroup
    const int k0 = c * chunk;
    const int nk = min(chunk, n_keys - k0);
    const int h0 = 2 * kvh;
    const int j = lane & 15, grp = lane >> 4;  // dims 8j … 8j+7; key group within the wave

    // 1. scores
    float qa[8], qb[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        qa[e] = q[h0 * D + 8 * j + e] * scale;
        qb[e] = q[(h0 + 1) * D + 8 * j + e] * scale;
    }
    const _Float16 *kbase = kc + ((size_t)kvh * n_ctx + k0) * D;
    for (int t0 = wave * 4; t0 < nk; t0 += 16) {
        const int t = t0 + grp;
        float da = 0.0f, db = 0.0f;
        if (t < nk) {
            const uint4 w = *reinterpret_cast<const uint4 *>(kbase + (size_t)t * D + 8 * j);
            const _Float16 *kh = reinterpret_cast<const _Float16 *>(&w);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float kv = (float)kh[e];
                da = fmaf(qa[e], kv, da);
                db = fmaf(qb[e], kv, db);
            }
        }
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {
            da += __shfl_xor(da, off, 64);
            db += __shfl_xor(db, off, 64);
        }
        if (j == 0 && t < nk) {
            s_sc[0][t] = da;
            s_sc[1][t] = db;
        }
    }
    __syncthreads();

    // 2. max, exp, sum per head (threads over keys)
    float ma = -INFINITY, mb = -INFINITY;
    for (int t = tid; t < nk; t += AW) {
        ma = fmaxf(ma, s_sc[0][t]);
        mb = fmaxf(mb, s_sc[1][t]);
    }
    ma = wave_max(ma);
    mb = wave_max(mb);
    if (lane == 0) {
        s_red[0][wave] = ma;
        s_red[1][wave] = mb;
    }
    __syncthreads();
    ma = fmaxf(fmaxf(s_red[0][0], s_red[0][1]), fmaxf(s_red[0][2], s_red[0][3]));
    mb = fmaxf(fmaxf(s_red[1][0], s_red[1][1]), fmaxf(s_red[1][2], s_red[1][3]));
    __syncthreads();
    float la = 0.0f, lb = 0.0f;
    for (int t = tid; t < nk; t += AW) {
        const float ea = expf(s_sc[0][t] - ma), eb = expf(s_sc[1][t] - mb);
        s_sc[0][t] = ea;
        s_sc[1][t] = eb;
        la += ea;
        lb += eb;
    }
    la = wave_sum(la);
    lb = wave_sum(lb);
    if (lane == 0) {
        s_red[0][wave] = la;
        s_red[1][wave] = lb;
    }
    __syncthreads();
    la = (s_red[0][0] + s_red[0][1]) + (s_red[0][2] + s_red[0][3]);
    lb = (s_red[1][0] + s_red[1][1]) + (s_red[1][2] + s_red[1][3]);

    // 3. values
    float oa[8], ob[8];
#pragma unroll
    for (int e = 0; e < 8; e++) oa[e] = ob[e] = 0.0f;
    const _Float16 *vbase = vc + ((size_t)kvh * n_ctx + k0) * D;
    for (int t0 = wave * 4; t0 < nk; t0 += 16) {
        const int t = t0 + grp;
        if (t < nk) {
            const uint4 w = *reinterpret_cast<const uint4 *>(vbase + (size_t)t * D + 8 * j);
            const _Float16 *vh = reinterpret_cast<const _Float16 *>(&w);
            const float ea = s_sc[0][t], eb = s_sc[1][t];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float vv = (float)vh[e];
                oa[e] = fmaf(ea, vv, oa[e]);
                ob[e] = fmaf(eb, vv, ob[e]);
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 8; e++) {
        oa[e] += __shfl_xor(oa[e], 16, 64);
        oa[e] += __shfl_xor(oa[e], 32, 64);
        ob[e] += __shfl_xor(ob[e], 16, 64);
        ob[e] += __shfl_xor(ob[e], 32, 64);
    }
    if (grp == 0) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            s_o[wave][0][8 * j + e] = oa[e];
            s_o[wave][1][8 * j + e] = ob[e];
        }
    }
    __syncthreads();
    {
        const int hh = tid >> 7, d = tid & 127;  // 256 threads = 2 heads × 128 dims
        const float o = (s_o[0][hh][d] + s_o[1][hh][d]) + (s_o[2][hh][d] + s_o[3][hh][d]);
        float *p = part + ((size_t)(h0 + hh) * max_chunk + c) * (D + 2);
        p[2 + d] = o;
        if (d == 0) {
            p[0] = hh ? mb : ma;
            p[1] = hh ? lb : la;
        }
    }

    // 4. the last chunk of this KV head merges
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(&counters[kvh], 1u) == (uint32_t)(n_chunk - 1);
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    {
        const int hh = tid >> 7, d = tid & 127;
        const float *p = part + (size_t)(h0 + hh) * max_chunk * (D + 2);
        float m = -INFINITY;
        for (int cc = 0; cc < n_chunk; cc++) m = fmaxf(m, __builtin_nontemporal_load(p + (size_t)cc * (D + 2)));
        float l = 0.0f, o = 0.0f;
        for (int cc = 0; cc < n_chunk; cc++) {
            const float *pc = p + (size_t)cc * (D + 2);
            const float w = expf(__builtin_nontemporal_load(pc) - m);
            l = fmaf(__builtin_nontemporal_load(pc + 1), w, l);
            o = fmaf(__builtin_nontemporal_load(pc + 2 + d), w, o);
        }
        out[(h0 + hh) * D + d] = o / l;
    }
    if (tid == 0) counters[kvh] = 0;  // ready for the next launch
}

// ---- prefill causal attention --------------------------------------------------------------------------------------
//
// grid (⌈n_q/64⌉, n_head), 128 threads = 64 queries × 2 halves of the head dim (adjacent lanes). K / V tiles of 32 keys
// are staged in LDS as f32; online softmax per query (f32).
constexpr int CQ = 64, CT = 32;

__global__ __launch_bounds__(128) void k_attn_causal(const float *q, const _Float16 *kc, const _Float16 *vc, int n_q,
                                                     int pos0, int n_head, int n_kv, int n_ctx, float scale,
                                                     float *out) {
    __shared__ float s_k[CT][D];
    __shared__ float s_v[CT][D];
    const int h = blockIdx.y, kvh = h / (n_head / n_kv);
    const int tid = threadIdx.x, ql = tid >> 1, half = tid & 1;
    const int qi_raw = blockIdx.x * CQ + ql;
    const int qi = min(qi_raw, n_q - 1);
    const int qpos = pos0 + qi;
    const int last_q = min(blockIdx.x * CQ + CQ - 1, n_q - 1);
    const int kend = pos0 + last_q + 1;
    float qv[64], acc[64];
    const float *qr = q + ((size_t)qi * n_head + h) * D + half * 64;
#pragma unroll
    for (int i = 0; i < 64; i++) {
        qv[i] = qr[i] * scale;
        acc[i] = 0.0f;
    }
    float m = -INFINITY, l = 0.0f;
    const _Float16 *kb = kc + (size_t)kvh * n_ctx * D, *vb = vc + (size_t)kvh * n_ctx * D;
    for (int k0 = 0; k0 < kend; k0 += CT) {
        __syncthreads();
        for (int e = tid; e < CT * D; e += 128) {
            const int t = e / D, d = e % D;
            const int kj = min(k0 + t, kend - 1);
            s_k[t][d] = (float)kb[(size_t)kj * D + d];
            s_v[t][d] = (float)vb[(size_t)kj * D + d];
        }
        __syncthreads();
        const int nk = min(CT, max(0, qpos + 1 - k0));
        for (int t = 0; t < nk; t++) {
            float dp = 0.0f;
#pragma unroll
            for (int i = 0; i < 64; i++) dp = fmaf(qv[i], s_k[t][half * 64 + i], dp);
            const float sc = dp + __shfl_xor(dp, 1, 64);
            const float mn = fmaxf(m, sc);
            const float corr = expf(m - mn), p = expf(sc - mn);
            l = fmaf(l, corr, p);
#pragma unroll
            for (int i = 0; i < 64; i++) acc[i] = fmaf(p, s_v[t][half * 64 + i], acc[i] * corr);
            m = mn;
        }
    }
    if (qi_raw < n_q) {
        const float inv = 1.0f / l;
        float *o = out + ((size_t)qi * n_head + h) * D + half * 64;
#pragma unroll
        for (int i = 0; i < 64; i++) o[i] = acc[i] * inv;
    }
}

}  // namespace

int attn_chunk_for(int n_ctx) {
    // chunks of 64 keys up to 2048 positions, then longer chunks so the chunk count (the grid's x) stays ≤ 64
    int chunk = 64;
    while ((n_ctx + chunk - 1) / chunk > 64 && chunk < MAX_CHUNK_KEYS) chunk *= 2;
    return chunk;
}

int launch_qkv_post(htr_device *dev, hipStream_t st, float *qkv, const float *qn, const float *kn, const float *rope,
                    int n_head, int n_kv, const int *pos_dev, int pos, int n_ctx, float eps, uint16_t *kc,
                    uint16_t *vc) {
    hipLaunchKernelGGL(k_qkv_post, dim3(n_head + 2 * n_kv), dim3(64), 0, st, qkv, qn, kn, rope, n_head, n_kv, pos_dev,
                       pos, n_ctx, eps, (_Float16 *)kc, (_Float16 *)vc);
    return htr_launched(dev, "k_qkv_post");
}

int launch_attn_decode(htr_device *dev, hipStream_t st, const float *q, const uint16_t *kc, const uint16_t *vc,
                       int n_head, int n_kv, int n_ctx, const int *pos_dev, int n_keys, float scale,
                       const AttnScratch &sc, float *out) {
    if (n_head != 2 * n_kv) return htr_fail("decode attention: %d q heads on %d kv heads (groups of 2)", n_head, n_kv);
    if (sc.chunk > MAX_CHUNK_KEYS || sc.chunk % 16) return htr_fail("decode attention: chunk %d", sc.chunk);
    if (!pos_dev && (n_keys < 1 || n_keys > n_ctx)) return htr_fail("decode attention: %d keys, cache %d", n_keys, n_ctx);
    const int grid_x = pos_dev ? sc.max_chunk : (n_keys + sc.chunk - 1) / sc.chunk;
    if (grid_x > sc.max_chunk) return htr_fail("decode attention: %d chunks, scratch for %d", grid_x, sc.max_chunk);
    hipLaunchKernelGGL(k_attn_decode, dim3(grid_x, n_kv), dim3(AW), 0, st, q, (const _Float16 *)kc,
                       (const _Float16 *)vc, n_kv, n_ctx, pos_dev, n_keys, sc.chunk, sc.max_chunk, scale, sc.part,
                       sc.counters, out);
    return htr_launched(dev, "k_attn_decode");
}

int launch_qk_norm_rope_rows(htr_device *dev, hipStream_t st, float *q, float *k, const float *v, const float *qn,
                             const float *kn, const float *rope, int n_tok, int n_head, int n_kv, int pos0, int n_ctx,
                             float eps, uint16_t *kc, uint16_t *vc) {
    hipLaunchKernelGGL(k_qk_rows, dim3(n_tok, n_head + 2 * n_kv), dim3(64), 0, st, q, k, v, qn, kn, rope, n_head, n_kv,
                       pos0, n_ctx, eps, (_Float16 *)kc, (_Float16 *)vc);
    return htr_launched(dev, "k_qk_rows");
}

int launch_attn_causal(htr_device *dev, hipStream_t st, const float *q, const uint16_t *kc, const uint16_t *vc,
                       int n_q, int pos0, int n_head, int n_kv, int n_ctx, float scale, float *out) {
    hipLaunchKernelGGL(k_attn_causal, dim3((n_q + CQ - 1) / CQ, n_head), dim3(128), 0, st, q, (const _Float16 *)kc,
                       (const _Float16 *)vc, n_q, pos0, n_head, n_kv, n_ctx, scale, out);
    return htr_launched(dev, "k_attn_causal");
}

// ---- ABI ------------------------------------------------------------------------------------------------------------

extern "C" int htr_qkv_post(htr_device *dev, float *d_qkv, const float *d_q_norm, const float *d_k_norm,
                            const float *d_rope, int n_head, int n_kv, int pos, int n_ctx, float eps, uint16_t *d_k,
                            uint16_t *d_v) {
    HTR_TRY(htr_check_alive(dev));
    if (!d_qkv || !d_q_norm || !d_k_norm || !d_rope || !d_k || !d_v) return htr_fail("htr_qkv_post: null argument");
    if (pos < 0 || pos >= n_ctx || n_head <= 0 || n_kv <= 0)
        return htr_fail("htr_qkv_post: position %d of a %d-row cache, %d / %d heads", pos, n_ctx, n_head, n_kv);
    return launch_qkv_post(dev, dev->stream, d_qkv, d_q_norm, d_k_norm, d_rope, n_head, n_kv, nullptr, pos, n_ctx, eps,
                           d_k, d_v);
}

extern "C" int htr_decode_attention(htr_device *dev, const float *d_q, const uint16_t *d_k, const uint16_t *d_v,
                                    int n_head, int n_kv, int n_ctx, int n_keys, float scale, float *d_out) {
    HTR_TRY(htr_check_alive(dev));
    if (!d_q || !d_k || !d_v || !d_out) return htr_fail("htr_decode_attention: null argument");
    if (n_keys < 1 || n_keys > n_ctx) return htr_fail("htr_decode_attention: %d keys in a %d-row cache", n_keys, n_ctx);
    AttnScratch sc{};
    sc.chunk = attn_chunk_for(n_ctx);
    sc.max_chunk = (n_ctx + sc.chunk - 1) / sc.chunk;
    HTR_TRY(htr_scratch(dev, SCR_ATTN_PART, (size_t)n_head * sc.max_chunk * (D + 2) * 4, (void **)&sc.part));
    HTR_TRY(htr_scratch(dev, SCR_ATTN_CNT, (size_t)n_kv * 4, (void **)&sc.counters));
    return launch_attn_decode(dev, dev->stream, d_q, d_k, d_v, n_head, n_kv, n_ctx, nullptr, n_keys, scale, sc, d_out);
}
