/*
 * htr_oracle.c — CPU restatement of the reference engine's LightOnOCR decode path. TEST INFRASTRUCTURE ONLY: it
 * checks the HIP library and is never linked into it. See htr_oracle.h for the function list, the reference lines each
 * one restates and what pins it.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off). f32 arithmetic in the reference kernels' order; every
 * fma written here is one the reference kernel writes (fmaf), every other product / sum is rounded on its own.
 */
#include "htr_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------------------------------------------------- */
/* seeded inputs                                                                                              */

/* text.rs:670-673 */
static inline float lcg_next(uint64_t *s) {
    *s = *s * 6364136223846793005ULL + 1442695040888963407ULL;
    return ((float)(*s >> 40) / 16777216.0f) * 2.0f - 1.0f;
}

void or_lcg_fill(uint64_t *state, float *out, size_t n, float scale) {
    for (size_t i = 0; i < n; i++) {
        float v = lcg_next(state);
        out[i] = scale == 1.0f ? v : v * scale;
    }
}

/* the logits of gpu_choice_matches_choose (text.rs:1021-1027), one LCG draw order per mode: 0 round(lcg·3), 1 lcg·20,
 * 2 −inf when a draw is > 0.9, else a second draw → round(lcg·2) − 1, 3 lcg·1e-3. Rust's f32::round rounds half away
 * from zero, as C's roundf does; the products are f32 */
void or_choice_matrix_logits(uint64_t *state, int mode, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) {
        switch (mode) {
        case 0: out[i] = roundf(lcg_next(state) * 3.0f); break;
        case 1: out[i] = lcg_next(state) * 20.0f; break;
        case 2: {
            const float u = lcg_next(state);
            out[i] = u > 0.9f ? -INFINITY : roundf(lcg_next(state) * 2.0f) - 1.0f;
            break;
        }
        default: out[i] = lcg_next(state) * 1e-3f; break;
        }
    }
}

/* text.rs:1070-1073 */
void or_lcg_bits(uint64_t *state, uint32_t *out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        *state = *state * 6364136223846793005ULL + 1442695040888963407ULL;
        out[i] = (uint32_t)(*state >> 32);
    }
}

/* ---------------------------------------------------------------------------------------------------------- */
/* f16 (IEEE binary16, round to nearest even)                                                                 */

static inline uint32_t fbits(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    return b;
}
static inline float bitsf(uint32_t b) {
    float v;
    memcpy(&v, &b, 4);
    return v;
}

uint16_t or_f16_from_f32(float v) {
    uint32_t x = fbits(v);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / NaN (NaN keeps a quiet payload) */
        return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u | ((ax >> 13) & 0x3ffu) : 0x7c00u));
    }
    if (ax >= 0x477ff000u) { /* ≥ 65520 rounds past the largest finite 65504 */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax >= 0x38800000u) { /* normal f16: rebias the exponent, round 13 bits off */
        uint32_t r = ax - 0x38000000u;
        r += 0xfffu + ((r >> 13) & 1u);
        return (uint16_t)(sign | (r >> 13));
    }
    /* subnormal f16 (units of 2^-24) or zero */
    uint32_t e = ax >> 23;
    if (e == 0) {
        return (uint16_t)sign; /* f32 subnormals are far below 2^-25 */
    }
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e; /* value = m · 2^(e−150) = (m >> shift) units of 2^-24 */
    if (shift > 24u) {
        return (uint16_t)sign;
    }
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) {
        q++;
    }
    return (uint16_t)(sign | q);
}

float or_f32_from_f16(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1fu) {
        return bitsf(sign | 0x7f800000u | (m << 13));
    }
    if (e == 0) {
        if (m == 0) {
            return bitsf(sign);
        }
        float v = (float)m * (1.0f / 16777216.0f); /* exact: m < 2^10 units of 2^-24 */
        return sign ? -v : v;
    }
    return bitsf(sign | ((e + 112u) << 23) | (m << 13));
}

void or_f16_from_f32_n(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        out[i] = or_f16_from_f32(in[i]);
    }
}

/* ---------------------------------------------------------------------------------------------------------- */
/* q8_0                                                                                                       */

/* text.rs:675-691 (ggml quantize_row_q8_0_ref) */
void or_q8_0_quantize(const float *x, size_t n, uint8_t *blocks, float *deq) {
    for (size_t b = 0; b < n / 32; b++) {
        const float *blk = x + 32 * b;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) {
            float a = fabsf(blk[i]);
            amax = a > amax ? a : amax; /* f32::max: a NaN operand loses */
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t dh = or_f16_from_f32(d);
        float df = or_f32_from_f16(dh);
        uint8_t *o = blocks + 34 * b;
        o[0] = (uint8_t)(dh & 0xff);
        o[1] = (uint8_t)(dh >> 8);
        for (int i = 0; i < 32; i++) {
            float r = roundf(blk[i] * id); /* Rust f32::round: half away from zero */
            int q = r != r ? 0 : (r > 127.0f ? 127 : (r < -128.0f ? -128 : (int)r)); /* `as i8` saturates */
            o[2 + i] = (uint8_t)(int8_t)q;
            if (deq) {
                deq[32 * b + i] = (float)q * df;
            }
        }
    }
}

static inline float blk_scale(const uint8_t *blk) {
    return or_f32_from_f16((uint16_t)(blk[0] | (blk[1] << 8)));
}

/* ocr-gguf lib.rs:500-507 */
void or_q8_0_dequant(const uint8_t *blocks, size_t n, float *out) {
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *blk = blocks + 34 * b;
        float d = blk_scale(blk);
        for (int i = 0; i < 32; i++) {
            out[32 * b + i] = (float)(int8_t)blk[2 + i] * d;
        }
    }
}

/* ---------------------------------------------------------------------------------------------------------- */
/* matvec                                                                                                     */

/* WGSL dot(a, b) of two vec4 as the sum of the four rounded products, left to right */
static inline float dot4(const float *a, const float *b) {
    float p0 = a[0] * b[0], p1 = a[1] * b[1], p2 = a[2] * b[2], p3 = a[3] * b[3];
    return ((p0 + p1) + p2) + p3;
}

/* matvec_q8_0.wgsl:29-73 */
void or_matvec_q8_0(const uint8_t *w, size_t n_rows, size_t k, const float *x, float *y, int acc) {
    size_t nb = k / 32;
#pragma omp parallel for schedule(static)
    for (size_t row = 0; row < n_rows; row++) {
        float part[32];
        for (size_t lane = 0; lane < 32; lane++) {
            float s = 0.0f;
            for (size_t b = lane; b < nb; b += 32) {
                const uint8_t *blk = w + 34 * (row * nb + b);
                float d = blk_scale(blk);
                float dot = 0.0f;
                for (int j = 0; j < 8; j++) {
                    const float *xv = x + 32 * b + 4 * j;
                    float v0 = (float)(int8_t)blk[2 + 4 * j + 0] * xv[0];
                    float v1 = (float)(int8_t)blk[2 + 4 * j + 1] * xv[1];
                    float v2 = (float)(int8_t)blk[2 + 4 * j + 2] * xv[2];
                    float v3 = (float)(int8_t)blk[2 + 4 * j + 3] * xv[3];
                    dot += ((v0 + v1) + v2) + v3;
                }
                s = fmaf(dot, d, s);
            }
            part[lane] = s;
        }
        for (int n = 16; n > 0; n >>= 1) {
            for (int l = 0; l < n; l++) {
                part[l] += part[l + n];
            }
        }
        y[row] = acc ? y[row] + part[0] : part[0];
    }
}

/* dmv_common.wgsl:23-30 with dmv_reduce_wg.wgsl:8-20: 256 threads, thread li sums dot(v, v) over the vec4s
 * li, li + 256, …; the 256 partials summed by a 128/64/…/1 tree */
static float norm_scale(const float *x, size_t k, float eps) {
    float red[256];
    for (size_t li = 0; li < 256; li++) {
        float s = 0.0f;
        for (size_t i = li; i < k / 4; i += 256) {
            s += dot4(x + 4 * i, x + 4 * i);
        }
        red[li] = s;
    }
    for (int n = 128; n > 0; n >>= 1) {
        for (int l = 0; l < n; l++) {
            red[l] += red[l + n];
        }
    }
    return 1.0f / sqrtf(red[0] / (float)k + eps);
}

/* dmv_dot.wgsl:7-30: (Σ_j dot(i8x4(q_j), xs_j)) · d */
static inline float dmv_dot(const uint8_t *blk, const float *xs) {
    float d = blk_scale(blk);
    float s = 0.0f;
    for (int j = 0; j < 8; j++) {
        float q[4] = {(float)(int8_t)blk[2 + 4 * j], (float)(int8_t)blk[3 + 4 * j], (float)(int8_t)blk[4 + 4 * j],
                      (float)(int8_t)blk[5 + 4 * j]};
        float t = dot4(q, xs + 4 * j);
        s = j == 0 ? t : s + t;
    }
    return s * d;
}

/* one row of dmv.wgsl:29-41 on the prepared input xs: 32 lanes over the blocks, then dmv_reduce_wg.wgsl:23-38's
 * sequential 32-lane sum */
static float dmv_row(const uint8_t *w, size_t row, size_t nb, const float *xs) {
    float acc[32];
    for (size_t lane = 0; lane < 32; lane++) {
        float a = 0.0f;
        for (size_t b = lane; b < nb; b += 32) {
            a += dmv_dot(w + 34 * (row * nb + b), xs + 32 * b);
        }
        acc[lane] = a;
    }
    float s = 0.0f;
    for (int l = 0; l < 32; l++) {
        s += acc[l];
    }
    return s;
}

/* xs = X · scale · NW (dmv.wgsl:33, dmv_qkv.wgsl:46) */
static float *normed(const float *x, const float *nw, size_t k, float eps) {
    float *xs = (float *)malloc(k * sizeof(float));
    if (!nw) {
        memcpy(xs, x, k * sizeof(float));
        return xs;
    }
    float scale = norm_scale(x, k, eps);
    for (size_t i = 0; i < k; i++) {
        xs[i] = (x[i] * scale) * nw[i];
    }
    return xs;
}

/* dmv.wgsl:22-52 */
void or_dmv(const uint8_t *w, size_t n_rows, size_t k, const float *x, const float *nw, float eps, float *y, int acc) {
    float *xs = normed(x, nw, k, eps);
    size_t nb = k / 32;
#pragma omp parallel for schedule(static)
    for (size_t row = 0; row < n_rows; row++) {
        float s = dmv_row(w, row, nb, xs);
        y[row] = acc ? y[row] + s : s;
    }
    free(xs);
}

/* dmv_qkv.wgsl:23-65 */
void or_dmv_qkv(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, size_t nq, size_t nkv, size_t k,
                const float *x, const float *nw, float eps, float *y) {
    float *xs = normed(x, nw, k, eps);
    size_t nb = k / 32;
    size_t total = nq + 2 * nkv;
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < total; r++) {
        if (r < nq) {
            y[r] = dmv_row(wq, r, nb, xs);
        } else if (r < nq + nkv) {
            y[r] = dmv_row(wk, r - nq, nb, xs);
        } else {
            y[r] = dmv_row(wv, r - nq - nkv, nb, xs);
        }
    }
    free(xs);
}

/* dmv_ffn.wgsl:22-51 */
void or_dmv_ffn(const uint8_t *wg, const uint8_t *wu, size_t n_rows, size_t k, const float *x, const float *nw,
                float eps, float *g) {
    float *xs = normed(x, nw, k, eps);
    size_t nb = k / 32;
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < n_rows; r++) {
        float gv = dmv_row(wg, r, nb, xs);
        float uv = dmv_row(wu, r, nb, xs);
        g[r] = (gv / (1.0f + expf(-gv))) * uv;
    }
    free(xs);
}

void or_matvec_q8_0_f64(const uint8_t *w, size_t n_rows, size_t k, const float *x, double *y) {
    size_t nb = k / 32;
#pragma omp parallel for schedule(static)
    for (size_t row = 0; row < n_rows; row++) {
        double s = 0.0;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = w + 34 * (row * nb + b);
            double d = (double)blk_scale(blk);
            for (int i = 0; i < 32; i++) {
                s += (double)(int8_t)blk[2 + i] * d * (double)x[32 * b + i];
            }
        }
        y[row] = s;
    }
}

/* ---------------------------------------------------------------------------------------------------------- */
/* norms, RoPE                                                                                                */

/* rms_norm.wgsl:21-41 */
static void rms_norm_row(const float *x, const float *w, float *y, size_t dim, float eps) {
    float part[256];
    for (size_t li = 0; li < 256; li++) {
        float s = 0.0f;
        for (size_t i = li; i < dim; i += 256) {
            s = fmaf(x[i], x[i], s);
        }
        part[li] = s;
    }
    for (int n = 128; n > 0; n >>= 1) {
        for (int l = 0; l < n; l++) {
            part[l] += part[l + n];
        }
    }
    float scale = 1.0f / sqrtf(part[0] / (float)dim + eps);
    for (size_t i = 0; i < dim; i++) {
        y[i] = (x[i] * scale) * w[i];
    }
}

void or_rms_norm(const float *x, const float *w, float *y, size_t rows, size_t dim, float eps) {
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; r++) {
        rms_norm_row(x + r * dim, w, y + r * dim, dim, eps);
    }
}

/* text.rs:132-142 */
void or_rope_table(float base, size_t d_head, size_t n_pos, float *out) {
    size_t half = d_head / 2;
    for (size_t pos = 0; pos < n_pos; pos++) {
        for (size_t i = 0; i < half; i++) {
            float theta = (float)pos * powf(base, -((float)(2 * i)) / (float)d_head);
            out[2 * (pos * half + i)] = cosf(theta);
            out[2 * (pos * half + i) + 1] = sinf(theta);
        }
    }
}

/* qkv_post.wgsl:31-83 (head dim 128) */
void or_qkv_post(float *qkv, const float *qn, const float *kn, const float *cs, int n_head, int n_kv, int pos,
                 float eps, uint16_t *k_row, uint16_t *v_row) {
    const int D = 128, HALF = 64;
    for (int h = 0; h < n_head + 2 * n_kv; h++) {
        float *x = qkv + (size_t)h * D;
        if (h >= n_head + n_kv) {
            int vh = h - n_head - n_kv;
            for (int i = 0; i < D; i++) {
                v_row[vh * D + i] = or_f16_from_f32(x[i]);
            }
            continue;
        }
        float sh[128];
        for (int i = 0; i < D; i++) {
            sh[i] = x[i] * x[i];
        }
        for (int n = 64; n > 0; n >>= 1) {
            for (int i = 0; i < n; i++) {
                sh[i] += sh[i + n];
            }
        }
        float scale = 1.0f / sqrtf(sh[0] / (float)D + eps);
        const float *w = h < n_head ? qn : kn;
        float y[128], r[128];
        for (int i = 0; i < D; i++) {
            y[i] = (x[i] * scale) * w[i];
        }
        for (int i = 0; i < D; i++) {
            const float *c = cs + 2 * ((size_t)pos * HALF + (i % HALF));
            r[i] = i < HALF ? y[i] * c[0] - y[i + HALF] * c[1] : y[i - HALF] * c[1] + y[i] * c[0];
        }
        if (h < n_head) {
            memcpy(x, r, sizeof r);
        } else {
            int kh = h - n_head;
            for (int i = 0; i < D; i++) {
                k_row[kh * D + i] = or_f16_from_f32(r[i]);
            }
        }
    }
}

/* ---------------------------------------------------------------------------------------------------------- */
/* attention                                                                                                  */

#define DECODE_CHUNK 128

/* attn_decode.wgsl:34-100 (one chunk of one kv head → the partials of its two q heads) */
static void attn_decode_chunk(const float *q, const uint16_t *k, const uint16_t *v, size_t kv_stride, int n_keys,
                              int n_kv, int kvh, int c, float scale, float *part0, float *part1) {
    (void)n_kv;
    const int D = 128;
    int h0 = 2 * kvh;
    float qs[2][128];
    for (int i = 0; i < D; i++) {
        qs[0][i] = q[h0 * D + i] * scale;
        qs[1][i] = q[(h0 + 1) * D + i] * scale;
    }
    float s[2][DECODE_CHUNK], red[2][DECODE_CHUNK], S[2][DECODE_CHUNK];
    for (int li = 0; li < DECODE_CHUNK; li++) {
        int j = c * DECODE_CHUNK + li;
        int valid = j < n_keys;
        for (int hh = 0; hh < 2; hh++) {
            if (!valid) {
                s[hh][li] = -3.0e38f;
                continue;
            }
            float d[4] = {0, 0, 0, 0};
            const uint16_t *kr = k + (size_t)j * kv_stride + (size_t)kvh * D;
            for (int e = 0; e < 32; e++) {
                for (int t = 0; t < 4; t++) {
                    d[t] = fmaf(qs[hh][4 * e + t], or_f32_from_f16(kr[4 * e + t]), d[t]);
                }
            }
            s[hh][li] = ((d[0] + d[1]) + d[2]) + d[3];
        }
        red[0][li] = s[0][li];
        red[1][li] = s[1][li];
    }
    for (int n = 64; n > 0; n >>= 1) {
        for (int li = 0; li < n; li++) {
            for (int hh = 0; hh < 2; hh++) {
                red[hh][li] = fmaxf(red[hh][li], red[hh][li + n]);
            }
        }
    }
    float m[2] = {red[0][0], red[1][0]};
    for (int li = 0; li < DECODE_CHUNK; li++) {
        int valid = c * DECODE_CHUNK + li < n_keys;
        for (int hh = 0; hh < 2; hh++) {
            float e = valid ? expf(s[hh][li] - m[hh]) : 0.0f;
            S[hh][li] = e;
            red[hh][li] = e;
        }
    }
    for (int n = 64; n > 0; n >>= 1) {
        for (int li = 0; li < n; li++) {
            for (int hh = 0; hh < 2; hh++) {
                red[hh][li] += red[hh][li + n];
            }
        }
    }
    int nk = n_keys - c * DECODE_CHUNK;
    nk = nk < DECODE_CHUNK ? nk : DECODE_CHUNK;
    for (int li = 0; li < D; li++) {
        float o0 = 0.0f, o1 = 0.0f;
        for (int t = 0; t < nk; t++) {
            float vv = or_f32_from_f16(v[(size_t)(c * DECODE_CHUNK + t) * kv_stride + (size_t)kvh * D + li]);
            o0 = fmaf(S[0][t], vv, o0);
            o1 = fmaf(S[1][t], vv, o1);
        }
        part0[2 + li] = o0;
        part1[2 + li] = o1;
    }
    part0[0] = m[0];
    part0[1] = red[0][0];
    part1[0] = m[1];
    part1[1] = red[1][0];
}

/* attn_decode.wgsl + attn_merge.wgsl:22-39 */
void or_attn_decode(const float *q, const uint16_t *k, const uint16_t *v, size_t kv_stride, int n_keys, int n_head,
                    int n_kv, float scale, float *out) {
    int n_chunk = (n_keys + DECODE_CHUNK - 1) / DECODE_CHUNK;
    float *part = (float *)malloc((size_t)n_head * n_chunk * 130 * sizeof(float));
#pragma omp parallel for collapse(2) schedule(static)
    for (int kvh = 0; kvh < n_kv; kvh++) {
        for (int c = 0; c < n_chunk; c++) {
            int h0 = 2 * kvh;
            attn_decode_chunk(q, k, v, kv_stride, n_keys, n_kv, kvh, c, scale, part + ((size_t)h0 * n_chunk + c) * 130,
                              part + ((size_t)(h0 + 1) * n_chunk + c) * 130);
        }
    }
    (void)n_head;
    for (int h = 0; h < 2 * n_kv; h++) {
        float mx = -3.0e38f;
        for (int c = 0; c < n_chunk; c++) {
            mx = fmaxf(mx, part[((size_t)h * n_chunk + c) * 130]);
        }
        for (int li = 0; li < 128; li++) {
            float l = 0.0f, o = 0.0f;
            for (int c = 0; c < n_chunk; c++) {
                const float *b = part + ((size_t)h * n_chunk + c) * 130;
                float w = expf(b[0] - mx);
                l = fmaf(b[1], w, l);
                o = fmaf(b[2 + li], w, o);
            }
            out[h * 128 + li] = o / l;
        }
    }
    free(part);
}

/* the F32 path's decode attention, three kernels (text.rs:567-569), one q head at a time:
 *   attn_scores.wgsl:26-38   S[j] = (Σ over the 32 vec4 of the head: d = fma(q4, k4, d) per component;
 *                            then ((d.x + d.y) + d.z) + d.w) · scale
 *   attn_softmax.wgsl:22-60  256 lanes: lane ℓ takes keys ℓ, ℓ + 256, …; max from −3e38; e = exp(S − m) in place;
 *                            lane sums in key order, then the tree part[i] += part[i + n] (n = 128 … 1); S ·= 1 / Σ
 *   attn_values.wgsl:29-45   lane (e, r): vec4 e of the head, keys r, r + 8, … (fma(S_j, v4, acc)); then
 *                            part_0 + part_1 + … + part_7 of vec4 e in order */
void or_attn_decode_f32(const float *q, const uint16_t *k, const uint16_t *v, size_t kv_stride, int n_keys, int n_head,
                        int n_kv, float scale, float *out) {
    int group = n_head / n_kv;
#pragma omp parallel for schedule(static)
    for (int h = 0; h < n_head; h++) {
        int kvh = h / group;
        float *S = (float *)malloc((size_t)n_keys * sizeof(float));
        const float *qh = q + (size_t)h * 128;
        for (int j = 0; j < n_keys; j++) {
            const uint16_t *kr = k + (size_t)j * kv_stride + (size_t)kvh * 128;
            float dv[4] = {0, 0, 0, 0};
            for (int e = 0; e < 32; e++) {
                for (int cc = 0; cc < 4; cc++) {
                    dv[cc] = fmaf(qh[4 * e + cc], or_f32_from_f16(kr[4 * e + cc]), dv[cc]);
                }
            }
            S[j] = (((dv[0] + dv[1]) + dv[2]) + dv[3]) * scale;
        }
        float part[256];
        float m = -3.0e38f;
        for (int j = 0; j < n_keys; j++) {
            m = fmaxf(m, S[j]);
        }
        for (int li = 0; li < 256; li++) {
            float sm = 0.0f;
            for (int j = li; j < n_keys; j += 256) {
                float e = expf(S[j] - m);
                S[j] = e;
                sm += e;
            }
            part[li] = sm;
        }
        for (int n = 128; n > 0; n >>= 1) {
            for (int li = 0; li < n; li++) {
                part[li] += part[li + n];
            }
        }
        float inv = 1.0f / part[0];
        for (int j = 0; j < n_keys; j++) {
            S[j] *= inv;
        }
        for (int e = 0; e < 32; e++) {
            float acc[8][4];
            for (int r = 0; r < 8; r++) {
                for (int cc = 0; cc < 4; cc++) {
                    acc[r][cc] = 0.0f;
                }
                for (int j = r; j < n_keys; j += 8) {
                    const uint16_t *vr = v + (size_t)j * kv_stride + (size_t)kvh * 128 + 4 * e;
                    for (int cc = 0; cc < 4; cc++) {
                        acc[r][cc] = fmaf(S[j], or_f32_from_f16(vr[cc]), acc[r][cc]);
                    }
                }
            }
            for (int cc = 0; cc < 4; cc++) {
                float sm = acc[0][cc];
                for (int r = 1; r < 8; r++) {
                    sm += acc[r][cc];
                }
                out[(size_t)h * 128 + 4 * e + cc] = sm;
            }
        }
        free(S);
    }
}

/* attention_causal.wgsl:42-93 (F32 path, tiles of TK = 8 keys): one query row, one head */
static void attn_causal_row(const float *q, const uint16_t *k, const uint16_t *v, size_t kv_stride, int qpos, int kvh,
                            float scale, float *out) {
    const int TK = 8;
    float qs[128], acc[128];
    for (int i = 0; i < 128; i++) {
        qs[i] = q[i] * scale;
        acc[i] = 0.0f;
    }
    float m = -3.0e38f, l = 0.0f;
    for (int k0 = 0; k0 <= qpos; k0 += TK) {
        int nk = qpos + 1 - k0;
        nk = nk < TK ? nk : TK;
        float P[8];
        for (int j = 0; j < nk; j++) {
            const uint16_t *kr = k + (size_t)(k0 + j) * kv_stride + (size_t)kvh * 128;
            float half[2];
            for (int hf = 0; hf < 2; hf++) {
                float d[4] = {0, 0, 0, 0};
                for (int e = 0; e < 16; e++) {
                    for (int t = 0; t < 4; t++) {
                        int i = hf * 64 + 4 * e + t;
                        d[t] = fmaf(qs[i], or_f32_from_f16(kr[i]), d[t]);
                    }
                }
                half[hf] = ((d[0] + d[1]) + d[2]) + d[3];
            }
            P[j] = half[0] + half[1];
        }
        float tmax = m;
        for (int j = 0; j < nk; j++) {
            tmax = fmaxf(tmax, P[j]);
        }
        float corr = expf(m - tmax);
        l *= corr;
        for (int i = 0; i < 128; i++) {
            acc[i] *= corr;
        }
        for (int j = 0; j < nk; j++) {
            float pj = expf(P[j] - tmax);
            l += pj;
            const uint16_t *vr = v + (size_t)(k0 + j) * kv_stride + (size_t)kvh * 128;
            for (int i = 0; i < 128; i++) {
                acc[i] = fmaf(pj, or_f32_from_f16(vr[i]), acc[i]);
            }
        }
        m = tmax;
    }
    float inv = 1.0f / l;
    for (int i = 0; i < 128; i++) {
        out[i] = acc[i] * inv;
    }
}

void or_attn_causal(const float *q, const uint16_t *k, const uint16_t *v, size_t kv_stride, int n_q, int pos0,
                    int n_head, int n_kv, float scale, float *out) {
    int group = n_head / n_kv;
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
    for (int t = 0; t < n_q; t++) {
        for (int h = 0; h < n_head; h++) {
            size_t o = ((size_t)t * n_head + h) * 128;
            attn_causal_row(q + o, k, v, kv_stride, pos0 + t, h / group, scale, out + o);
        }
    }
}

void or_attn_f64(const float *q, const uint16_t *k, const uint16_t *v, size_t kv_stride, int n_keys, int n_head,
                 int n_kv, double scale, double *out) {
    int group = n_head / n_kv;
    double *sc = (double *)malloc((size_t)n_keys * sizeof(double));
    for (int h = 0; h < n_head; h++) {
        int kvh = h / group;
        double mx = -1e308;
        for (int j = 0; j < n_keys; j++) {
            double s = 0.0;
            for (int i = 0; i < 128; i++) {
                s += (double)q[h * 128 + i] * (double)or_f32_from_f16(k[(size_t)j * kv_stride + kvh * 128 + i]);
            }
            sc[j] = s * scale;
            mx = sc[j] > mx ? sc[j] : mx;
        }
        double z = 0.0;
        for (int j = 0; j < n_keys; j++) {
            sc[j] = exp(sc[j] - mx);
            z += sc[j];
        }
        for (int i = 0; i < 128; i++) {
            double o = 0.0;
            for (int j = 0; j < n_keys; j++) {
                o += sc[j] / z * (double)or_f32_from_f16(v[(size_t)j * kv_stride + kvh * 128 + i]);
            }
            out[h * 128 + i] = o;
        }
    }
    free(sc);
}

/* ---------------------------------------------------------------------------------------------------------- */
/* token choice — sampling.rs:38-62 (greedy presets)                                                          */

int32_t or_choose(float *logits, size_t n_vocab, double rp, size_t window, double fp, const int32_t *history,
                  size_t n_hist, const int32_t *count_tok, const uint32_t *count_n, size_t n_counts) {
    if (rp != 1.0) {
        float r = (float)rp;
        size_t start = n_hist - (window < n_hist ? window : n_hist);
        for (size_t j = start; j < n_hist; j++) {
            int32_t t = history[j];
            int seen = 0;
            for (size_t i = start; i < j; i++) {
                if (history[i] == t) {
                    seen = 1;
                    break;
                }
            }
            if (!seen) {
                float *l = logits + t;
                *l = *l < 0.0f ? *l * r : *l / r;
            }
        }
    }
    if (fp > 0.0) {
        for (size_t i = 0; i < n_counts; i++) {
            logits[count_tok[i]] -= (float)fp * (float)count_n[i];
        }
    }
    size_t best = 0;
    for (size_t i = 0; i < n_vocab; i++) {
        if (logits[i] > logits[best]) {
            best = i;
        }
    }
    return (int32_t)best;
}

/* sampling.rs:23-35 Rng: SplitMix64 (Steele, Lea, Flood 2014); the next double in [0, 1) from the top 53 bits */
double or_rng_next_f64(uint64_t *state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (double)(z >> 11) / 9007199254740992.0; /* 2^53 */
}

typedef struct {
    size_t i;
    double p;
} or_prob;

/* probability descending, index ascending on ties: the order of a stable sort of the vocabulary by probability */
static int prob_order(const void *a, const void *b) {
    const or_prob *x = (const or_prob *)a, *y = (const or_prob *)b;
    if (x->p != y->p) {
        return x->p > y->p ? -1 : 1;
    }
    return x->i < y->i ? -1 : (x->i > y->i);
}

/* sampling.rs:38-89 choose with a sampled preset: the penalties as or_choose, then e^((l − max)/T) in f64 from the
 * f32 (l − max)/T, normalised by their sum over the vocabulary in index order; the smallest prefix of the descending
 * order whose running sum reaches top_p (all of it when top_p ≥ 1); r = next_f64 · Σ kept; the first kept token where
 * r minus the running sum falls to ≤ 0 (the last kept one if none does). temperature 0 → or_choose. */
int32_t or_choose_sampled(float *logits, size_t n_vocab, double temperature, double top_p, double rp, size_t window,
                          double fp, const int32_t *history, size_t n_hist, const int32_t *count_tok,
                          const uint32_t *count_n, size_t n_counts, uint64_t *rng) {
    if (temperature == 0.0) {
        return or_choose(logits, n_vocab, rp, window, fp, history, n_hist, count_tok, count_n, n_counts);
    }
    /* the penalties alone: or_choose with no vocabulary to scan (its argmax over 0 tokens) */
    or_choose(logits, 0, rp, window, fp, history, n_hist, count_tok, count_n, n_counts);
    float t = (float)temperature, mx = -INFINITY;
    for (size_t i = 0; i < n_vocab; i++) {
        mx = logits[i] > mx ? logits[i] : mx;
    }
    or_prob *pr = (or_prob *)malloc(n_vocab * sizeof(or_prob));
    double sum = 0.0;
    for (size_t i = 0; i < n_vocab; i++) {
        pr[i].i = i;
        pr[i].p = exp((double)((logits[i] - mx) / t));
        sum += pr[i].p;
    }
    for (size_t i = 0; i < n_vocab; i++) {
        pr[i].p /= sum;
    }
    qsort(pr, n_vocab, sizeof(or_prob), prob_order);
    size_t keep = n_vocab;
    if (top_p < 1.0) {
        double acc = 0.0;
        for (size_t k = 0; k < n_vocab; k++) {
            acc += pr[k].p;
            if (acc >= top_p) {
                keep = k + 1;
                break;
            }
        }
    }
    double total = 0.0;
    for (size_t k = 0; k < keep; k++) {
        total += pr[k].p;
    }
    double r = or_rng_next_f64(rng) * total;
    int32_t tok = (int32_t)pr[keep - 1].i;
    for (size_t k = 0; k < keep; k++) {
        r -= pr[k].p;
        if (r <= 0.0) {
            tok = (int32_t)pr[k].i;
            break;
        }
    }
    free(pr);
    return tok;
}

/* ---------------------------------------------------------------------------------------------------------- */
/* the text decoder                                                                                           */

struct or_session {
    or_text_cfg c;
    const uint8_t *tok_embd;
    const float *output_norm;
    or_layer *layers;
    int n_ctx, n_past;
    uint16_t *kc, *vc; /* [layer][pos][n_kv·128] f16, the reference's cache layout (kv_store.wgsl) */
    float *rope;       /* [n_ctx][64] × (cos, sin) */
    int r16;           /* the prefill GEMMs on the f16 paths' rounding */
    int step_f32;      /* the decode step of the F32 path (text.rs:555-576) instead of the fused one */
};

void or_session_set_f16(or_session *s, int on) { s->r16 = on != 0; }

void or_session_set_step_f32(or_session *s, int on) { s->step_f32 = on != 0; }

/* the cache rows [pos0, pos0 + n) of one layer in the reference's layout [pos][n_kv·128] f16: copied out of / into the
 * session (a test hands a device's cache over, or reads back what a step stored) */
int or_session_get_kv(const or_session *s, int layer, int pos0, int n, uint16_t *k, uint16_t *v) {
    if (layer < 0 || layer >= s->c.n_layer || pos0 < 0 || n < 0 || pos0 + n > s->n_ctx) {
        return -1;
    }
    size_t kvd = (size_t)s->c.n_kv * 128, off = ((size_t)layer * s->n_ctx + pos0) * kvd;
    memcpy(k, s->kc + off, (size_t)n * kvd * 2);
    memcpy(v, s->vc + off, (size_t)n * kvd * 2);
    return 0;
}

int or_session_set_kv(or_session *s, int layer, int pos0, int n, const uint16_t *k, const uint16_t *v) {
    if (layer < 0 || layer >= s->c.n_layer || pos0 < 0 || n < 0 || pos0 + n > s->n_ctx) {
        return -1;
    }
    size_t kvd = (size_t)s->c.n_kv * 128, off = ((size_t)layer * s->n_ctx + pos0) * kvd;
    memcpy(s->kc + off, k, (size_t)n * kvd * 2);
    memcpy(s->vc + off, v, (size_t)n * kvd * 2);
    return 0;
}

or_session *or_session_new(const or_text_cfg *cfg, const uint8_t *tok_embd, const float *output_norm,
                           const or_layer *layers, int n_ctx) {
    if (cfg->d_head != 128 || cfg->n_head != 2 * cfg->n_kv || cfg->dim % 32 || cfg->n_ff % 32) {
        return NULL;
    }
    or_session *s = (or_session *)calloc(1, sizeof *s);
    s->c = *cfg;
    s->tok_embd = tok_embd;
    s->output_norm = output_norm;
    s->layers = (or_layer *)malloc(sizeof(or_layer) * cfg->n_layer);
    memcpy(s->layers, layers, sizeof(or_layer) * cfg->n_layer);
    s->n_ctx = n_ctx;
    size_t row = (size_t)cfg->n_kv * 128;
    s->kc = (uint16_t *)calloc((size_t)cfg->n_layer * n_ctx * row, 2);
    s->vc = (uint16_t *)calloc((size_t)cfg->n_layer * n_ctx * row, 2);
    s->rope = (float *)malloc((size_t)n_ctx * 64 * 2 * sizeof(float));
    or_rope_table(cfg->rope_base, 128, n_ctx, s->rope);
    return s;
}

void or_session_free(or_session *s) {
    if (!s) {
        return;
    }
    free(s->layers);
    free(s->kc);
    free(s->vc);
    free(s->rope);
    free(s);
}

int or_session_n_past(const or_session *s) { return s->n_past; }

void or_session_rewind(or_session *s, int n_past) { s->n_past = n_past; }

static inline float round_f16(float v) { return or_f32_from_f16(or_f16_from_f32(v)); }

/* matmul.wgsl:47-91 (F32 path): Y[M,N] (+)= X[M,K]·Wᵀ with W dequantised exactly, acc = fma(x_k, w_k, acc) over k in
 * order. Blocked over rows of X and columns of W for the CPU; each output's fma chain runs over k in order.
 * r16: the f16 paths (matmul_coop.wgsl:47-70 with load4_q8_0.wgsl, matmul128h): X and the dequantised W (q·d, exact
 * in f32) rounded to f16 (nearest even) as they enter the tiles, the products summed in f32. */
static void matmul_q8_0(const float *x_in, const uint8_t *w, float *y, size_t m, size_t n, size_t k, int acc, int r16) {
    float *wt = (float *)malloc(k * n * sizeof(float)); /* [k][n] dequantised */
    const float *x = x_in;
    float *xr = NULL;
    if (r16) {
        xr = (float *)malloc(m * k * sizeof(float));
        for (size_t i = 0; i < m * k; i++) {
            xr[i] = round_f16(x_in[i]);
        }
        x = xr;
    }
#pragma omp parallel for schedule(static)
    for (size_t c = 0; c < n; c++) {
        float row[8192];
        or_q8_0_dequant(w + 34 * (c * (k / 32)), k, row);
        for (size_t i = 0; i < k; i++) {
            wt[i * n + c] = r16 ? round_f16(row[i]) : row[i];
        }
    }
    enum { MT = 4, NT = 32 };
    size_t n_mt = (m + MT - 1) / MT, n_nt = (n + NT - 1) / NT;
#pragma omp parallel for collapse(2) schedule(static)
    for (size_t mt = 0; mt < n_mt; mt++) {
        for (size_t nt = 0; nt < n_nt; nt++) {
            size_t m0 = mt * MT, n0 = nt * NT;
            float a[MT][NT];
            memset(a, 0, sizeof a);
            if (m0 + MT <= m && n0 + NT <= n) {
                for (size_t kk = 0; kk < k; kk++) {
                    const float *b = wt + kk * n + n0;
                    for (int i = 0; i < MT; i++) {
                        float xv = x[(m0 + i) * k + kk];
                        for (int j = 0; j < NT; j++) {
                            a[i][j] = fmaf(xv, b[j], a[i][j]);
                        }
                    }
                }
            } else {
                for (size_t kk = 0; kk < k; kk++) {
                    for (int i = 0; i < MT && m0 + i < m; i++) {
                        float xv = x[(m0 + i) * k + kk];
                        for (int j = 0; j < NT && n0 + j < n; j++) {
                            a[i][j] = fmaf(xv, wt[kk * n + n0 + j], a[i][j]);
                        }
                    }
                }
            }
            for (int i = 0; i < MT && m0 + i < m; i++) {
                for (int j = 0; j < NT && n0 + j < n; j++) {
                    float *o = y + (m0 + i) * n + n0 + j;
                    *o = acc ? *o + a[i][j] : a[i][j];
                }
            }
        }
    }
    free(wt);
    free(xr);
}

void or_matmul_q8_0(const float *x, const uint8_t *w, float *y, size_t m, size_t n, size_t k, int acc, int r16) {
    matmul_q8_0(x, w, y, m, n, k, acc, r16);
}

/* embed_q8_0.wgsl:28-38 */
static void embed_row(const or_session *s, int32_t tok, float *x) {
    int d = s->c.dim;
    or_q8_0_dequant(s->tok_embd + (size_t)34 * (d / 32) * tok, d, x);
}

/* rope_neox.wgsl:19-34 on rows [n_tok][n_head·128] at positions pos0 + t */
static void rope_rows(const or_session *s, float *q, int n_tok, int n_head, int pos0) {
    for (int t = 0; t < n_tok; t++) {
        for (int h = 0; h < n_head; h++) {
            float *r = q + ((size_t)t * n_head + h) * 128;
            for (int i = 0; i < 64; i++) {
                const float *c = s->rope + 2 * ((size_t)(pos0 + t) * 64 + i);
                float x0 = r[i], x1 = r[i + 64];
                r[i] = x0 * c[0] - x1 * c[1];
                r[i + 64] = x0 * c[1] + x1 * c[0];
            }
        }
    }
}

/* text.rs:437-521 */
int or_session_prefill(or_session *s, const int32_t *ids, int l, float *logits) {
    const or_text_cfg *c = &s->c;
    if (l <= 0 || s->n_past + l > s->n_ctx) {
        return -1;
    }
    for (int i = 0; i < l; i++) {
        if (ids[i] < 0 || ids[i] >= c->n_vocab) {
            return -1;
        }
    }
    size_t d = c->dim, f = c->n_ff, qd = (size_t)c->n_head * 128, kvd = (size_t)c->n_kv * 128;
    int pos0 = s->n_past;
    float *x = (float *)malloc(l * d * 4), *h = (float *)malloc(l * d * 4);
    float *qr = (float *)malloc(l * qd * 4), *q = (float *)malloc(l * qd * 4);
    float *kr = (float *)malloc(l * kvd * 4), *kn = (float *)malloc(l * kvd * 4), *vr = (float *)malloc(l * kvd * 4);
    float *g = (float *)malloc(l * f * 4), *u = (float *)malloc(l * f * 4);
    for (int t = 0; t < l; t++) {
        embed_row(s, ids[t], x + t * d);
    }
    float scale = 1.0f / sqrtf(128.0f);
    for (int li = 0; li < c->n_layer; li++) {
        const or_layer *ly = &s->layers[li];
        uint16_t *kc = s->kc + (size_t)li * s->n_ctx * kvd, *vc = s->vc + (size_t)li * s->n_ctx * kvd;
        or_rms_norm(x, ly->attn_norm, h, l, d, c->eps);
        matmul_q8_0(h, ly->q, qr, l, qd, d, 0, s->r16);
        matmul_q8_0(h, ly->k, kr, l, kvd, d, 0, s->r16);
        matmul_q8_0(h, ly->v, vr, l, kvd, d, 0, s->r16);
        or_rms_norm(qr, ly->q_norm, q, (size_t)l * c->n_head, 128, c->eps);
        or_rms_norm(kr, ly->k_norm, kn, (size_t)l * c->n_kv, 128, c->eps);
        rope_rows(s, q, l, c->n_head, pos0);
        rope_rows(s, kn, l, c->n_kv, pos0);
        or_f16_from_f32_n(kn, kc + (size_t)pos0 * kvd, l * kvd); /* kv_store.wgsl:18-24 */
        or_f16_from_f32_n(vr, vc + (size_t)pos0 * kvd, l * kvd);
        or_attn_causal(q, kc, vc, kvd, l, pos0, c->n_head, c->n_kv, scale, qr);
        matmul_q8_0(qr, ly->o, x, l, d, qd, 1, s->r16);
        or_rms_norm(x, ly->ffn_norm, h, l, d, c->eps);
        matmul_q8_0(h, ly->gate, g, l, f, d, 0, s->r16);
        matmul_q8_0(h, ly->up, u, l, f, d, 0, s->r16);
        for (size_t i = 0; i < (size_t)l * f; i++) { /* swiglu.wgsl:18-24 */
            g[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
        }
        matmul_q8_0(g, ly->down, x, l, d, f, 1, s->r16);
    }
    /* head (text.rs:655-658): rms_norm + matvec_q8_0 of the last row */
    or_rms_norm(x + (size_t)(l - 1) * d, s->output_norm, h, 1, d, c->eps);
    or_matvec_q8_0(s->tok_embd, c->n_vocab, d, h, logits, 0);
    s->n_past += l;
    free(x), free(h), free(qr), free(q), free(kr), free(kn), free(vr), free(g), free(u);
    return 0;
}

/* record_step on the F32 path (text.rs:555-576): rms_norm → matvec_q8_0 q / k / v → per-head rms_norm of q and k →
 * rope_neox → kv_store → attn_scores / attn_softmax / attn_values → matvec o (+ residual) → rms_norm → matvec gate
 * and up → swiglu → matvec down (+ residual); head (text.rs:655-658): rms_norm + matvec_q8_0 */
static void step_f32(or_session *s, int32_t tok, float *logits) {
    const or_text_cfg *c = &s->c;
    size_t d = c->dim, f = c->n_ff, qd = (size_t)c->n_head * 128, kvd = (size_t)c->n_kv * 128;
    int pos = s->n_past;
    float *x = (float *)malloc(d * 4), *h = (float *)malloc(d * 4);
    float *qr = (float *)malloc(qd * 4), *q = (float *)malloc(qd * 4), *a = (float *)malloc(qd * 4);
    float *kr = (float *)malloc(kvd * 4), *kn = (float *)malloc(kvd * 4), *vr = (float *)malloc(kvd * 4);
    float *g = (float *)malloc(f * 4), *u = (float *)malloc(f * 4);
    embed_row(s, tok, x);
    float scale = 1.0f / sqrtf(128.0f);
    for (int li = 0; li < c->n_layer; li++) {
        const or_layer *ly = &s->layers[li];
        uint16_t *kc = s->kc + (size_t)li * s->n_ctx * kvd, *vc = s->vc + (size_t)li * s->n_ctx * kvd;
        or_rms_norm(x, ly->attn_norm, h, 1, d, c->eps);
        or_matvec_q8_0(ly->q, qd, d, h, qr, 0);
        or_matvec_q8_0(ly->k, kvd, d, h, kr, 0);
        or_matvec_q8_0(ly->v, kvd, d, h, vr, 0);
        or_rms_norm(qr, ly->q_norm, q, c->n_head, 128, c->eps);
        or_rms_norm(kr, ly->k_norm, kn, c->n_kv, 128, c->eps);
        rope_rows(s, q, 1, c->n_head, pos);
        rope_rows(s, kn, 1, c->n_kv, pos);
        or_f16_from_f32_n(kn, kc + (size_t)pos * kvd, kvd); /* kv_store.wgsl:18-24 */
        or_f16_from_f32_n(vr, vc + (size_t)pos * kvd, kvd);
        or_attn_decode_f32(q, kc, vc, kvd, pos + 1, c->n_head, c->n_kv, scale, a);
        or_matvec_q8_0(ly->o, d, qd, a, x, 1);
        or_rms_norm(x, ly->ffn_norm, h, 1, d, c->eps);
        or_matvec_q8_0(ly->gate, f, d, h, g, 0);
        or_matvec_q8_0(ly->up, f, d, h, u, 0);
        for (size_t i = 0; i < f; i++) { /* swiglu.wgsl:18-24 */
            g[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
        }
        or_matvec_q8_0(ly->down, d, f, g, x, 1);
    }
    or_rms_norm(x, s->output_norm, h, 1, d, c->eps);
    or_matvec_q8_0(s->tok_embd, c->n_vocab, d, h, logits, 0);
    free(x), free(h), free(qr), free(q), free(a), free(kr), free(kn), free(vr), free(g), free(u);
}

/* text.rs:540-552 + layers_fused text.rs:630-647 (the f16 paths), or the F32 path's step (or_session_set_step_f32) */
int or_session_step(or_session *s, int32_t tok, float *logits) {
    const or_text_cfg *c = &s->c;
    if (tok < 0 || tok >= c->n_vocab || s->n_past + 1 > s->n_ctx) {
        return -1;
    }
    if (s->step_f32) {
        step_f32(s, tok, logits);
        s->n_past += 1;
        return 0;
    }
    size_t d = c->dim, f = c->n_ff, qd = (size_t)c->n_head * 128, kvd = (size_t)c->n_kv * 128;
    int pos = s->n_past;
    float *x = (float *)malloc(d * 4), *qkv = (float *)malloc((qd + 2 * kvd) * 4);
    float *a = (float *)malloc(qd * 4), *g = (float *)malloc(f * 4);
    embed_row(s, tok, x);
    float scale = 1.0f / sqrtf(128.0f);
    for (int li = 0; li < c->n_layer; li++) {
        const or_layer *ly = &s->layers[li];
        uint16_t *kc = s->kc + (size_t)li * s->n_ctx * kvd, *vc = s->vc + (size_t)li * s->n_ctx * kvd;
        or_dmv_qkv(ly->q, ly->k, ly->v, qd, kvd, d, x, ly->attn_norm, c->eps, qkv);
        or_qkv_post(qkv, ly->q_norm, ly->k_norm, s->rope, c->n_head, c->n_kv, pos, c->eps, kc + (size_t)pos * kvd,
                    vc + (size_t)pos * kvd);
        or_attn_decode(qkv, kc, vc, kvd, pos + 1, c->n_head, c->n_kv, scale, a);
        or_dmv(ly->o, d, qd, a, NULL, 0.0f, x, 1);
        or_dmv_ffn(ly->gate, ly->up, f, d, x, ly->ffn_norm, c->eps, g);
        or_dmv(ly->down, d, f, g, NULL, 0.0f, x, 1);
    }
    or_dmv(s->tok_embd, c->n_vocab, d, x, s->output_norm, c->eps, logits, 0);
    s->n_past += 1;
    free(x), free(qkv), free(a), free(g);
    return 0;
}
