/*
 * htr_vision_oracle.c — CPU restatement of the reference engine's LightOnOCR vision encoder on its f16 compute path
 * (app/crates/ocr-wgpu/src/vision.rs:328-423 run_f16 + project), test infrastructure only (see htr_oracle.h).
 *
 * Arithmetic follows the reference kernels: f32 sums in the stated order, f16 rounding (IEEE RNE) exactly where the
 * f16 path rounds — the normed activations (rms_norm_h), K / V (heads_f16.wgsl), the scaled q and P inside the
 * attention (attention_coop.wgsl), the attention output, the SwiGLU product × 1/64 (ffn_coopd.wgsl), the weights
 * (converted to f16 once at load, vision.rs:122-142; here from q8_0: f16(q·d·scale)).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "htr_oracle.h"

/* vision.rs:143-146 pixel_lut */
void or_pixel_lut(const float mean[3], const float stdv[3], float *lut) {
    for (int c = 0; c < 3; c++)
        for (int v = 0; v < 256; v++) lut[c * 256 + v] = ((float)v / 255.0f - mean[c]) / stdv[c];
}

/* patchify.wgsl:23-37: P[t][c·p·p + ky·p + kx] = lut[c·256 + rgb[((ty·p + ky)·w + tx·p + kx)·3 + c]] */
void or_patchify(const uint8_t *rgb, int w, int px, int n, int side, const float *lut, float *P) {
    const int pp = side * side;
    for (int t = 0; t < n; t++)
        for (int c = 0; c < 3; c++)
            for (int ky = 0; ky < side; ky++)
                for (int kx = 0; kx < side; kx++) {
                    const int x = (t % px) * side + kx, y = (t / px) * side + ky;
                    P[(size_t)t * 3 * pp + c * pp + ky * side + kx] = lut[c * 256 + rgb[((size_t)y * w + x) * 3 + c]];
                }
}

/* vision.rs:159-175 rope_table: [half][pos][k] × (cos, sin); half 0 freq_scale 1, half 1 freq_scale θ^(−2/d); the
 * angle t is multiplied by θ^(−2/(d/2)) step by step in f32 */
void or_rope2d_table(float theta, int d_head, int max_pos, float *out) {
    const int n_dims = d_head / 2;
    const float theta_scale = powf(theta, -2.0f / (float)n_dims);
    size_t o = 0;
    for (int half = 0; half < 2; half++) {
        const float freq_scale = half == 0 ? 1.0f : powf(theta, -2.0f / (float)d_head);
        for (int pos = 0; pos < max_pos; pos++) {
            float t = (float)pos;
            for (int k = 0; k < n_dims / 2; k++) {
                const float a = freq_scale * t;
                out[o++] = cosf(a);
                out[o++] = sinf(a);
                t *= theta_scale;
            }
        }
    }
}

/* rope2d.wgsl:28-44 in place: pairs (2k, 2k+1) of each half; half 0 at the patch row t / px, half 1 at its column */
void or_rope2d(float *Q, int n_tok, int n_head, int d_head, int px, int max_pos, const float *cs) {
    const int nk = d_head / 4;
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n_tok; t++)
        for (int h = 0; h < n_head; h++)
            for (int half = 0; half < 2; half++) {
                const int pos = half == 0 ? t / px : t % px;
                for (int k = 0; k < nk; k++) {
                    const float c = cs[2 * (((size_t)half * max_pos + pos) * nk + k)];
                    const float s = cs[2 * (((size_t)half * max_pos + pos) * nk + k) + 1];
                    float *x = Q + (size_t)t * n_head * d_head + h * d_head + half * (d_head / 2) + 2 * k;
                    const float x0 = x[0], x1 = x[1];
                    x[0] = x0 * c - x1 * s;
                    x[1] = x0 * s + x1 * c;
                }
            }
}

/* rms_norm.wgsl with an f16 output (gpu.rs:268-275 rms_norm_h) */
void or_rms_norm_h(const float *x, const float *w, uint16_t *y, size_t rows, size_t dim, float eps) {
    float *tmp = malloc(rows * dim * sizeof(float));
    or_rms_norm(x, w, tmp, rows, dim, eps);
    or_f16_from_f32_n(tmp, y, rows * dim);
    free(tmp);
}

/* q8_0 blocks → f16 weights f16(q·d·scale) (the f16 paths' load-time conversion) */
void or_q8_0_to_f16(const uint8_t *blocks, size_t n, float scale, uint16_t *out) {
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *blk = blocks + 34 * b;
        const float d = or_f32_from_f16((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int i = 0; i < 32; i++) out[32 * b + i] = or_f16_from_f32((float)(int8_t)blk[2 + i] * d * scale);
    }
}

/* Y[M,N] (+)= X·Wᵀ with every output a f32 fma chain in k order. Eight columns run side by side (W transposed in
 * blocks of 8: wt[c/8][j][c%8]), the same chains in the same order, so that the host vectorises across them. */
static void matmul_f32_rows(const float *x, const float *w, float *y, size_t m, size_t n, size_t k, int acc) {
    const size_t nb = (n + 7) / 8;
    float *wt = calloc(nb * k * 8, sizeof(float));
    for (size_t c = 0; c < n; c++)
        for (size_t j = 0; j < k; j++) wt[((c / 8) * k + j) * 8 + c % 8] = w[c * k + j];
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < m; r++) {
        const float *xr = x + r * k;
        for (size_t b = 0; b < nb; b++) {
            float s[8];
            for (int c = 0; c < 8; c++) s[c] = (acc && b * 8 + c < n) ? y[r * n + b * 8 + c] : 0.0f;
            const float *wb = wt + b * k * 8;
            for (size_t j = 0; j < k; j++) {
                const float xv = xr[j];
#pragma omp simd
                for (int c = 0; c < 8; c++) s[c] = fmaf(xv, wb[j * 8 + c], s[c]);
            }
            for (int c = 0; c < 8; c++)
                if (b * 8 + c < n) y[r * n + b * 8 + c] = s[c];
        }
    }
    free(wt);
}

/* matmul_coopd.wgsl: Y[M,N] (+)= X·Wᵀ, X / W f16, each output a f32 sum in k order */
void or_matmul_f16(const uint16_t *x, const uint16_t *w, float *y, size_t m, size_t n, size_t k, int acc) {
    float *wf = malloc(n * k * sizeof(float)), *xf = malloc(m * k * sizeof(float));
    for (size_t i = 0; i < n * k; i++) wf[i] = or_f32_from_f16(w[i]);
    for (size_t i = 0; i < m * k; i++) xf[i] = or_f32_from_f16(x[i]);
    matmul_f32_rows(xf, wf, y, m, n, k, acc);
    free(wf);
    free(xf);
}

/* ffn_coopd.wgsl: G = f16(silu(X·Wgᵀ) · (X·Wuᵀ) · scale) */
void or_ffn_f16(const uint16_t *x, const uint16_t *wg, const uint16_t *wu, uint16_t *g, size_t m, size_t n, size_t k,
                float scale) {
    float *a = malloc(m * n * sizeof(float)), *u = malloc(m * n * sizeof(float));
    or_matmul_f16(x, wg, a, m, n, k, 0);
    or_matmul_f16(x, wu, u, m, n, k, 0);
    for (size_t i = 0; i < m * n; i++) g[i] = or_f16_from_f32(a[i] / (1.0f + expf(-a[i])) * u[i] * scale);
    free(a);
    free(u);
}

/* the f32 matmul of the patch embedding and the projector: Y (+)= X·Wᵀ, f32 X and W, f32 sums in k order */
void or_matmul_f32(const float *x, const float *w, float *y, size_t m, size_t n, size_t k, int acc) {
    matmul_f32_rows(x, w, y, m, n, k, acc);
}

/* heads_f16.wgsl + attention_coop.wgsl: Q, K, V f32 [n][H·64] → O f16 [n][H·64]. K and V rounded to f16; per query q
 * scaled then rounded to f16; keys in blocks of 32: S = q16·k16 (f32), the running max m (start −3e38), corr =
 * e^(m − mx), P = f16(e^(S − mx)), l = l·corr + Σ f32(P), O = O·corr + Σ P·v16; O / l rounded to f16. */
void or_attention_coop(const float *q, const float *k, const float *v, uint16_t *o, int n_tok, int n_head,
                       float scale) {
    const int D = 64, BKV = 32, row = n_head * D;
    const int n_pad = (n_tok + BKV - 1) / BKV * BKV;
    /* K as f16 values transposed per head: kt[h][d][key] (the score chains of a key block run side by side);
     * V as f16 values [key][h·64] */
    float *kt = calloc((size_t)n_head * D * n_pad, sizeof(float)), *v16 = malloc((size_t)n_tok * row * sizeof(float));
    for (int t = 0; t < n_tok; t++)
        for (int h = 0; h < n_head; h++)
            for (int d = 0; d < D; d++) {
                kt[((size_t)h * D + d) * n_pad + t] = or_f32_from_f16(or_f16_from_f32(k[(size_t)t * row + h * D + d]));
                v16[(size_t)t * row + h * D + d] = or_f32_from_f16(or_f16_from_f32(v[(size_t)t * row + h * D + d]));
            }
#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < n_tok; t++)
        for (int h = 0; h < n_head; h++) {
            float qs[64], acc[64], s[32];
            for (int d = 0; d < D; d++) {
                qs[d] = or_f32_from_f16(or_f16_from_f32(q[(size_t)t * row + h * D + d] * scale));
                acc[d] = 0.0f;
            }
            float m = -3.0e38f, l = 0.0f;
            for (int k0 = 0; k0 < n_tok; k0 += BKV) {
                const int nb = n_tok - k0 < BKV ? n_tok - k0 : BKV;
                /* S = q16·k16 in dim order, the block's 32 chains side by side */
                for (int j = 0; j < BKV; j++) s[j] = 0.0f;
                for (int d = 0; d < D; d++) {
                    const float qd = qs[d];
                    const float *kr = kt + ((size_t)h * D + d) * n_pad + k0;
#pragma omp simd
                    for (int j = 0; j < BKV; j++) s[j] = fmaf(qd, kr[j], s[j]);
                }
                float mx = m;
                for (int j = 0; j < nb; j++) mx = fmaxf(mx, s[j]);
                const float corr = expf(m - mx);
                float ps = 0.0f;
                for (int d = 0; d < D; d++) acc[d] *= corr;
                for (int j = 0; j < nb; j++) {
                    const float p = or_f32_from_f16(or_f16_from_f32(expf(s[j] - mx)));
                    ps += p;
                    const float *vr = v16 + (size_t)(k0 + j) * row + h * D;
#pragma omp simd
                    for (int d = 0; d < D; d++) acc[d] = fmaf(p, vr[d], acc[d]);
                }
                l = l * corr + ps;
                m = mx;
            }
            const float inv = 1.0f / l;
            for (int d = 0; d < D; d++) o[(size_t)t * row + h * D + d] = or_f16_from_f32(acc[d] * inv);
        }
    free(kt);
    free(v16);
}

/* unfold2x2.wgsl: Z[o][c·4 + ky·2 + kx] = X[(2·oy + ky)·px + 2·ox + kx][c] */
void or_unfold2x2(const float *x, float *z, int px, int py, int dim) {
    const int ox_n = px / 2, n_out = (px / 2) * (py / 2);
    for (int o = 0; o < n_out; o++)
        for (int c = 0; c < dim; c++)
            for (int ky = 0; ky < 2; ky++)
                for (int kx = 0; kx < 2; kx++)
                    z[(size_t)o * dim * 4 + c * 4 + ky * 2 + kx] =
                        x[((size_t)(2 * (o / ox_n) + ky) * px + 2 * (o % ox_n) + kx) * dim + c];
}

/* gelu.wgsl: 0.5·x·(1 + tanh(clamp(√(2/π)·x·(1 + 0.044715·x²), ±15))) in place */
void or_gelu(float *x, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const float v = x[i];
        float t = 0.7978845608028654f * v * (1.0f + 0.044715f * v * v);
        t = t < -15.0f ? -15.0f : (t > 15.0f ? 15.0f : t);
        x[i] = 0.5f * v * (1.0f + tanhf(t));
    }
}

/* vision.rs:328-423 run_f16 + project on a baked image: n_layers < 0 → every layer and the projector → out
 * [n/4][proj_dim]; n_layers ≥ 0 → the residual after that many layers → out [n][dim]. Returns 0, −1 on bad sizes. */
/* a weight as the f16 plane its matmul reads: q8_0 blocks dequantised to f16 (× scale: the down projection's 64,
 * vision.rs:31-35), or (W16) an f16 plane as given — the mmproj's bf16 weights, converted at load with the scale
 * already applied (f16_from_bf16.wgsl, vision.rs:124-142) */
static void vision_w(const uint8_t *src, int w16, size_t n, float scale, uint16_t *dst) {
    if (w16) memcpy(dst, src, n * 2);
    else or_q8_0_to_f16(src, n, scale, dst);
}

/* layers[first … first + count) of the encoder on the residual x [n][d] of a px × py patch grid, in place
 * (vision.rs:338-399) */
static void vision_layers(const or_vision_cfg *c, const or_vision_layer *layers, int first, int count, int px, int py,
                          float *x, int w16src) {
    const int n = px * py, d = c->dim, f = c->n_ff;
    float *qb = malloc((size_t)n * d * 4), *kb = malloc((size_t)n * d * 4), *vb = malloc((size_t)n * d * 4);
    uint16_t *h16 = malloc((size_t)n * d * 2), *a16 = malloc((size_t)n * d * 2), *g16 = malloc((size_t)n * f * 2);
    uint16_t *w16 = malloc((size_t)f * d * 2), *w16b = malloc((size_t)f * d * 2);
    const int max_pos = px > py ? px : py;
    float *cs = malloc((size_t)2 * max_pos * (c->d_head / 4) * 2 * 4);
    or_rope2d_table(c->rope_theta, c->d_head, max_pos, cs);
    const float scale = 1.0f / sqrtf((float)c->d_head);
    for (int li = first; li < first + count; li++) {
        const or_vision_layer *L = &layers[li];
        or_rms_norm_h(x, L->ln1, h16, n, d, c->eps);
        vision_w(L->q, w16src, (size_t)d * d, 1.0f, w16);
        or_matmul_f16(h16, w16, qb, n, d, d, 0);
        vision_w(L->k, w16src, (size_t)d * d, 1.0f, w16);
        or_matmul_f16(h16, w16, kb, n, d, d, 0);
        vision_w(L->v, w16src, (size_t)d * d, 1.0f, w16);
        or_matmul_f16(h16, w16, vb, n, d, d, 0);
        or_rope2d(qb, n, c->n_head, c->d_head, px, max_pos, cs);
        or_rope2d(kb, n, c->n_head, c->d_head, px, max_pos, cs);
        or_attention_coop(qb, kb, vb, a16, n, c->n_head, scale);
        vision_w(L->o, w16src, (size_t)d * d, 1.0f, w16);
        or_matmul_f16(a16, w16, x, n, d, d, 1);
        or_rms_norm_h(x, L->ln2, h16, n, d, c->eps);
        vision_w(L->gate, w16src, (size_t)f * d, 1.0f, w16);
        vision_w(L->up, w16src, (size_t)f * d, 1.0f, w16b);
        or_ffn_f16(h16, w16, w16b, g16, n, f, d, 1.0f / 64.0f);
        vision_w(L->down, w16src, (size_t)d * f, 64.0f, w16);
        or_matmul_f16(g16, w16, x, n, d, f, 1);
    }
    free(qb);
    free(kb);
    free(vb);
    free(h16);
    free(a16);
    free(g16);
    free(w16);
    free(w16b);
    free(cs);
}

/* project (vision.rs:405-423): input_norm → unfold 2×2 → merger → mm.1 → gelu → mm.2, f32 activations and f16-valued
 * weights; x [n][d] → out [n/4][proj_dim] */
static void vision_project(const or_vision_cfg *c, const float *x, const float *input_norm, const uint8_t *merger,
                           const uint8_t *mm1, const uint8_t *mm2, int px, int py, float *out, int w16src) {
    const int n = px * py, d = c->dim, n_out = n / 4, pd = c->proj_dim;
    float *tmp = malloc((size_t)n * d * 4);
    float *z = malloc((size_t)n * d * 4), *mg = malloc((size_t)n_out * d * 4), *m1 = malloc((size_t)n_out * pd * 4);
    float *wf = malloc((size_t)d * 4 * d * 4);
    uint16_t *wh = malloc((size_t)d * 4 * d * 2);
    or_rms_norm(x, input_norm, tmp, n, d, c->eps);
    or_unfold2x2(tmp, z, px, py, d);
    vision_w(merger, w16src, (size_t)d * 4 * d, 1.0f, wh);
    for (size_t i = 0; i < (size_t)d * 4 * d; i++) wf[i] = or_f32_from_f16(wh[i]);
    or_matmul_f32(z, wf, mg, n_out, d, 4 * d, 0);
    vision_w(mm1, w16src, (size_t)pd * d, 1.0f, wh);
    for (size_t i = 0; i < (size_t)pd * d; i++) wf[i] = or_f32_from_f16(wh[i]);
    or_matmul_f32(mg, wf, m1, n_out, pd, d, 0);
    or_gelu(m1, (size_t)n_out * pd);
    vision_w(mm2, w16src, (size_t)pd * pd, 1.0f, wh);
    for (size_t i = 0; i < (size_t)pd * pd; i++) wf[i] = or_f32_from_f16(wh[i]);
    or_matmul_f32(m1, wf, out, n_out, pd, pd, 0);
    free(tmp);
    free(z);
    free(mg);
    free(m1);
    free(wf);
    free(wh);
}

static int vision_encode(const or_vision_cfg *c, const float *patch_embd, const float *pre_ln, const or_vision_layer *layers,
                         const float *input_norm, const uint8_t *merger, const uint8_t *mm1, const uint8_t *mm2,
                         const uint8_t *rgb, int w, int h, int n_layers, float *out, int w16src) {
    const int grid = c->patch * c->merge;
    if (w % grid || h % grid || w <= 0 || h <= 0 || c->d_head != 64 || c->merge != 2) return -1;
    if (n_layers > c->n_layer) return -1;
    const int px = w / c->patch, py = h / c->patch, n = px * py, d = c->dim, pp = 3 * c->patch * c->patch;
    const int nl = n_layers < 0 ? c->n_layer : n_layers;
    float lut[768];
    or_pixel_lut(c->mean, c->std, lut);
    float *P = malloc((size_t)n * pp * 4), *x = malloc((size_t)n * d * 4), *tmp = malloc((size_t)n * d * 4);
    or_patchify(rgb, w, px, n, c->patch, lut, P);
    or_matmul_f32(P, patch_embd, tmp, n, d, pp, 0);
    or_rms_norm(tmp, pre_ln, x, n, d, c->eps);
    vision_layers(c, layers, 0, nl, px, py, x, w16src);
    if (n_layers >= 0) memcpy(out, x, (size_t)n * d * 4);
    else vision_project(c, x, input_norm, merger, mm1, mm2, px, py, out, w16src);
    free(P);
    free(x);
    free(tmp);
    return 0;
}

int or_vision_resume(const or_vision_cfg *c, const or_vision_layer *layers, const float *input_norm,
                     const uint8_t *merger, const uint8_t *mm1, const uint8_t *mm2, int px, int py, const float *x_in,
                     int first, int count, int project, float *out) {
    if (px % c->merge || py % c->merge || px <= 0 || py <= 0 || c->d_head != 64 || c->merge != 2) return -1;
    if (first < 0 || count < 0 || first + count > c->n_layer) return -1;
    const size_t nd = (size_t)px * py * c->dim;
    float *x = malloc(nd * 4);
    memcpy(x, x_in, nd * 4);
    vision_layers(c, layers, first, count, px, py, x, 0);
    if (project) vision_project(c, x, input_norm, merger, mm1, mm2, px, py, out, 0);
    else memcpy(out, x, nd * 4);
    free(x);
    return 0;
}

int or_vision_encode(const or_vision_cfg *c, const float *patch_embd, const float *pre_ln, const or_vision_layer *layers,
                     const float *input_norm, const uint8_t *merger, const uint8_t *mm1, const uint8_t *mm2,
                     const uint8_t *rgb, int w, int h, int n_layers, float *out) {
    return vision_encode(c, patch_embd, pre_ln, layers, input_norm, merger, mm1, mm2, rgb, w, h, n_layers, out, 0);
}

int or_vision_encode_w16(const or_vision_cfg *c, const float *patch_embd, const float *pre_ln,
                         const or_vision_layer16 *layers, const float *input_norm, const uint16_t *merger,
                         const uint16_t *mm1, const uint16_t *mm2, const uint8_t *rgb, int w, int h, int n_layers,
                         float *out) {
    or_vision_layer *l8 = malloc((size_t)c->n_layer * sizeof(or_vision_layer));
    if (!l8) return -1;
    for (int i = 0; i < c->n_layer; i++) {
        const or_vision_layer16 *s = &layers[i];
        or_vision_layer t = {s->ln1, s->ln2, (const uint8_t *)s->q, (const uint8_t *)s->k, (const uint8_t *)s->v,
                             (const uint8_t *)s->o, (const uint8_t *)s->gate, (const uint8_t *)s->up,
                             (const uint8_t *)s->down};
        l8[i] = t;
    }
    const int rc = vision_encode(c, patch_embd, pre_ln, l8, input_norm, (const uint8_t *)merger, (const uint8_t *)mm1,
                                 (const uint8_t *)mm2, rgb, w, h, n_layers, out, 1);
    free(l8);
    return rc;
}
