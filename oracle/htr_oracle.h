/*
 * htr_oracle.h — CPU restatement of the reference engine's LightOnOCR decode path (test infrastructure only).
 *
 * This library checks the product and is never part of it: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it. Every function names the reference file:line it restates (paths relative to the reference
 * repository root; the engine lives in app/crates/ocr-wgpu/src, the decoding policy in app/crates/ocr-decode/src).
 *
 * Arithmetic is IEEE-754 f32 in the order of the reference kernels where the order is stated in the reference (lane
 * strides, tree reductions, sequential sums, explicit fma); compiled with -ffp-contract=off so that every fma is the
 * one the reference wrote. Built with OpenMP: rows are independent, so the results do not depend on the thread count.
 *
 * Pinning (what checks each function, see tests/test_oracle.py):
 *   or_lcg_*, or_f16_*, or_q8_0_*     golden vectors of the reference tests (ocr-gguf lib.rs:521-593 q8_0 block
 *                                     −8.0 / 7.5), numpy float16 RNE, brute force over all 65536 f16 codes
 *   or_matvec_q8_0, or_dmv*           fp64 closed form (numpy) on LCG inputs of text.rs:707-741 / 864-905
 *   or_rms_norm, or_rope_table,
 *   or_qkv_post                       fp64 closed form (numpy) as in text.rs:768-792, 943-972
 *   or_attn_decode, or_attn_causal,
 *   or_attn_decode_f32                fp64 softmax attention (numpy) on f16-rounded K / V, text.rs:797-858, 1264-1292
 *   or_choose                         sampling.rs:297-321 unit cases, numpy IEEE division (text.rs:1061-1099 sweep),
 *                                     a brute-force numpy argmax
 *   or_session_prefill / or_session_step (both step forms)
 *                                     an independent numpy float64 forward of the same graph (tiny model shape)
 *   or_session_get_kv / set_kv        round trip, and the rows a prefill stores against the forward's f16 K / V
 *   or_pixel_lut / or_patchify, or_rope2d_table / or_rope2d, or_unfold2x2, or_gelu, or_rms_norm_h, or_matmul_f16,
 *   or_ffn_f16, or_attention_coop, or_vision_encode, or_vision_encode_w16
 *                                     numpy restatements (fp64 closed forms, ggml's rope cache by its own recurrence,
 *                                     torch-unfold index order by brute force), tests/test_vision_oracle.py
 */
#ifndef HTR_ORACLE_H
#define HTR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- seeded inputs ---------------------------------------------------------------------------------------- */
/* the reference tests' 64-bit LCG (text.rs:670-673): s = s·6364136223846793005 + 1442695040888963407 (mod 2^64),
 * value = ((s >> 40) / 2^24)·2 − 1, times `scale` */
void or_lcg_fill(uint64_t *state, float *out, size_t n, float scale);
/* the logits of the reference's GPU-choice test matrix (text.rs:1021-1027), `mode` 0 … 3, n values, LCG draws in its
 * order (mode 2 draws the second value only when the first is ≤ 0.9) */
void or_choice_matrix_logits(uint64_t *state, int mode, size_t n, float *out);
/* the raw 32-bit draws of choose_pen_is_exact (text.rs:1070-1073): (s >> 32) */
void or_lcg_bits(uint64_t *state, uint32_t *out, size_t n);

/* ---- f16 ---------------------------------------------------------------------------------------------------- */
/* IEEE binary16 round-to-nearest-even (half 2.7.1 f16::from_f32 / WGSL pack2x16float; text.rs:971) */
uint16_t or_f16_from_f32(float v);
float or_f32_from_f16(uint16_t h);
void or_f16_from_f32_n(const float *in, uint16_t *out, size_t n);

/* ---- q8_0 (ocr-gguf lib.rs:128-135, 500-507) ------------------------------------------------------------------ */
/* ggml quantize_row_q8_0_ref as the reference tests restate it (text.rs:675-691): 34-byte blocks (f16 d LE + 32 i8);
 * `deq` (optional) receives q · f32(f16(d)) */
void or_q8_0_quantize(const float *x, size_t n, uint8_t *blocks, float *deq);
void or_q8_0_dequant(const uint8_t *blocks, size_t n, float *out);

/* ---- matvec ------------------------------------------------------------------------------------------------- */
/* the F32 path's matvec_q8_0.wgsl:29-73: 32 lanes per row, lane ℓ takes blocks ℓ, ℓ+32, …; per block
 * dot = Σ_j sum4(i8x4(q_j)·x_j), s = fma(dot, d, s); lanes summed by a 16/8/4/2/1 tree; acc = 1 adds onto y */
void or_matvec_q8_0(const uint8_t *w, size_t n_rows, size_t k, const float *x, float *y, int acc);
/* the fused decode matvec dmv.wgsl:22-52 (+ dmv_common.wgsl:23-30 norm, dmv_dot.wgsl:7-30, dmv_reduce_wg.wgsl:23-38):
 * nw == NULL → plain dmv; nw != NULL → dmv_norm (x·scale·nw first). acc = 1 adds onto y */
void or_dmv(const uint8_t *w, size_t n_rows, size_t k, const float *x, const float *nw, float eps, float *y, int acc);
/* dmv_qkv.wgsl:23-65: attn_norm fused → [q | k | v] rows of three matrices into one buffer */
void or_dmv_qkv(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, size_t nq, size_t nkv, size_t k,
                const float *x, const float *nw, float eps, float *y);
/* dmv_ffn.wgsl:22-51: ffn_norm fused → g = silu(Wg·xn)·(Wu·xn) */
void or_dmv_ffn(const uint8_t *wg, const uint8_t *wu, size_t n_rows, size_t k, const float *x, const float *nw,
                float eps, float *g);
/* the fp64 dequantised reference: y = Σ_k f64(q·d)·f64(x) (+ y) */
void or_matvec_q8_0_f64(const uint8_t *w, size_t n_rows, size_t k, const float *x, double *y);

/* ---- norms, RoPE, KV --------------------------------------------------------------------------------------- */
/* rms_norm.wgsl:21-41: per row, 256 strided fma partials, tree sum, scale = 1/sqrt(Σ/dim + eps), y = x·scale·w */
void or_rms_norm(const float *x, const float *w, float *y, size_t rows, size_t dim, float eps);
/* text.rs:132-142: [pos][d/2] × (cos, sin), θ = f32(pos)·powf(base, −2i/d) in f32 */
void or_rope_table(float base, size_t d_head, size_t n_pos, float *out);
/* qkv_post.wgsl:31-83 on the [q | k | v] row at position pos: q heads normed + roped in place; k heads normed, roped
 * and stored f16 into k_row (n_kv·128 halves); v heads stored f16 into v_row */
void or_qkv_post(float *qkv, const float *qn, const float *kn, const float *cs, int n_head, int n_kv, int pos,
                 float eps, uint16_t *k_row, uint16_t *v_row);

/* ---- attention ---------------------------------------------------------------------------------------------- */
/* split-K decode attention attn_decode.wgsl:34-100 + attn_merge.wgsl:22-39 (chunks of 128 keys, GQA group 2):
 * q [n_head·128] f32, K / V f16 rows [key][n_kv·128] (row stride kv_stride halves), out [n_head·128] */
void or_attn_decode(const float *q, const uint16_t *k, const uint16_t *v, size_t kv_stride, int n_keys, int n_head,
                    int n_kv, float scale, float *out);
/* the F32 path's decode attention (attn_scores / attn_softmax / attn_values, text.rs:567-569): the score scaled after
 * its dot product, the softmax normalised before the values; same arguments as or_attn_decode */
void or_attn_decode_f32(const float *q, const uint16_t *k, const uint16_t *v, size_t kv_stride, int n_keys, int n_head,
                        int n_kv, float scale, float *out);
/* causal prefill attention attention_causal.wgsl:42-93 (tiles of 8 keys, online softmax): queries t < n_q at
 * positions pos0 + t, q / out [n_q][n_head·128] */
void or_attn_causal(const float *q, const uint16_t *k, const uint16_t *v, size_t kv_stride, int n_q, int pos0,
                    int n_head, int n_kv, float scale, float *out);
/* fp64 softmax attention of one query row over n_keys keys (the tests' reference, text.rs:812-822) */
void or_attn_f64(const float *q, const uint16_t *k, const uint16_t *v, size_t kv_stride, int n_keys, int n_head,
                 int n_kv, double scale, double *out);

/* ---- token choice (sampling.rs:38-62) --------------------------------------------------------------------- */
/* rp → fp → greedy, in place on logits. rp == 1.0 (f64) skips the penalty. counts: (token, count) pairs of the output
 * so far (n_counts entries, distinct tokens). Returns the token (first maximum; index 0 when logits[0] is NaN or all
 * are −inf / NaN) */
int32_t or_choose(float *logits, size_t n_vocab, double rp, size_t window, double fp, const int32_t *history,
                  size_t n_hist, const int32_t *count_tok, const uint32_t *count_n, size_t n_counts);
/* sampling.rs:23-35 Rng (SplitMix64): the next f64 in [0, 1) */
double or_rng_next_f64(uint64_t *state);
/* sampling.rs:38-89 choose for any preset: temperature 0 → or_choose; else T + top-p sampling with *rng */
int32_t or_choose_sampled(float *logits, size_t n_vocab, double temperature, double top_p, double rp, size_t window,
                          double fp, const int32_t *history, size_t n_hist, const int32_t *count_tok,
                          const uint32_t *count_n, size_t n_counts, uint64_t *rng);

/* ---- the text decoder (text.rs:437-658) -------------------------------------------------------------------- */
typedef struct {
    int n_layer, dim, n_head, n_kv, d_head, n_ff, n_vocab;
    float eps, rope_base;
} or_text_cfg;

/* one layer's tensors: q8_0 GGUF block bytes (row-major [rows][cols/32] blocks) and f32 norms */
typedef struct {
    const uint8_t *q, *k, *v, *o, *gate, *up, *down;
    const float *attn_norm, *q_norm, *k_norm, *ffn_norm;
} or_layer;

typedef struct or_session or_session;

/* a session over n_ctx positions; the weights are borrowed (they must outlive the session) */
or_session *or_session_new(const or_text_cfg *cfg, const uint8_t *tok_embd, const float *output_norm,
                           const or_layer *layers, int n_ctx);
void or_session_free(or_session *s);
int or_session_n_past(const or_session *s);
/* TextModel::prefill (text.rs:437-521), the F32 path's kernels unless or_session_set_f16: ids at positions n_past…,
 * logits of the last row
 * (head: rms_norm + matvec_q8_0, text.rs:655-658). Returns 0, or −1 on a bad id / overflow */
int or_session_prefill(or_session *s, const int32_t *ids, int n, float *logits);
/* the prefill GEMMs with the f16 paths' rounding (matmul_coop_q8_0: X and q·d rounded to f16, f32 sums) when on;
 * the F32 path's (exact) otherwise. The rest of the prefill is the same on both paths. */
void or_session_set_f16(or_session *s, int on);
/* Batch::matmul with a q8_0 weight (gpu.rs:1963-2014): Y[m][n] (+)= X·Wᵀ, W as q8_0 blocks [n][k]; r16: the f16
 * paths' rounding of X and W */
void or_matmul_q8_0(const float *x, const uint8_t *w, float *y, size_t m, size_t n, size_t k, int acc, int r16);
/* record_step (text.rs:540-578) on the f16 paths: embed + layers_fused (text.rs:630-647) + dmv_norm LM head; with
 * or_session_set_step_f32 the F32 path's step (text.rs:555-576: rms_norm, matvec_q8_0 per projection, rope_neox,
 * kv_store, the three-kernel attention or_attn_decode_f32, swiglu; head rms_norm + matvec_q8_0) */
int or_session_step(or_session *s, int32_t tok, float *logits);
void or_session_set_step_f32(or_session *s, int on);
/* cache rows [pos0, pos0 + n) of one layer in the reference's layout [pos][n_kv·128] f16, out of / into the session;
 * −1 outside the session */
int or_session_get_kv(const or_session *s, int layer, int pos0, int n, uint16_t *k, uint16_t *v);
int or_session_set_kv(or_session *s, int layer, int pos0, int n, const uint16_t *k, const uint16_t *v);
/* rewind to n_past positions (the rows beyond are overwritten by later steps) */
void or_session_rewind(or_session *s, int n_past);

/* ---- the vision encoder (vision.rs:266-423, the f16 compute path; htr_vision_oracle.c) ------------------------- */
void or_pixel_lut(const float mean[3], const float stdv[3], float *lut);
void or_patchify(const uint8_t *rgb, int w, int px, int n, int side, const float *lut, float *P);
void or_rope2d_table(float theta, int d_head, int max_pos, float *out);
void or_rope2d(float *Q, int n_tok, int n_head, int d_head, int px, int max_pos, const float *cs);
void or_rms_norm_h(const float *x, const float *w, uint16_t *y, size_t rows, size_t dim, float eps);
void or_q8_0_to_f16(const uint8_t *blocks, size_t n, float scale, uint16_t *out);
void or_matmul_f16(const uint16_t *x, const uint16_t *w, float *y, size_t m, size_t n, size_t k, int acc);
void or_ffn_f16(const uint16_t *x, const uint16_t *wg, const uint16_t *wu, uint16_t *g, size_t m, size_t n, size_t k,
                float scale);
void or_matmul_f32(const float *x, const float *w, float *y, size_t m, size_t n, size_t k, int acc);
void or_attention_coop(const float *q, const float *k, const float *v, uint16_t *o, int n_tok, int n_head,
                       float scale);
void or_unfold2x2(const float *x, float *z, int px, int py, int dim);
void or_gelu(float *x, size_t n);

typedef struct {
    int n_layer, dim, n_head, d_head, n_ff, patch, merge, proj_dim;
    float eps, rope_theta, mean[3], std[3];
} or_vision_cfg;
typedef struct {
    const float *ln1, *ln2;
    const uint8_t *q, *k, *v, *o, *gate, *up, *down; /* q8_0 GGUF blocks */
} or_vision_layer;
int or_vision_encode(const or_vision_cfg *c, const float *patch_embd, const float *pre_ln, const or_vision_layer *layers,
                     const float *input_norm, const uint8_t *merger, const uint8_t *mm1, const uint8_t *mm2,
                     const uint8_t *rgb, int w, int h, int n_layers, float *out);
/* the encoder resumed from a residual: x_in [px·py][dim] (the residual before layer `first`, of a px × py patch grid)
 * through layers first … first + count − 1 → out [px·py][dim], or (project) further through the projector → out
 * [px·py/4][proj_dim]. Pinned by composition: resumed from or_vision_encode's residual after `first` layers it is
 * or_vision_encode after first + count (tests/test_vision_oracle.py). Returns 0, −1 on bad sizes. */
int or_vision_resume(const or_vision_cfg *c, const or_vision_layer *layers, const float *input_norm,
                     const uint8_t *merger, const uint8_t *mm1, const uint8_t *mm2, int px, int py, const float *x_in,
                     int first, int count, int project, float *out);
/* the same with f16 weight planes (an mmproj's bf16 weights as vision.rs:124-142 converts them at load:
 * f16(w · scale), the down projection × 64) */
typedef struct {
    const float *ln1, *ln2;
    const uint16_t *q, *k, *v, *o, *gate, *up, *down;
} or_vision_layer16;
int or_vision_encode_w16(const or_vision_cfg *c, const float *patch_embd, const float *pre_ln,
                         const or_vision_layer16 *layers, const float *input_norm, const uint16_t *merger,
                         const uint16_t *mm1, const uint16_t *mm2, const uint8_t *rgb, int w, int h, int n_layers,
                         float *out);

#ifdef __cplusplus
}
#endif
#endif
