// Internal declarations of libhtr: the device object, the sticky error latch, weights, and the kernel launchers the
// host-side decoder (text_model.hip) composes. Kernels are compiled for gfx950 only.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "htr.h"

// ---- errors ---------------------------------------------------------------------------------------------------------

// sets the calling thread's message; returns -1 (the ABI's error code)
int htr_fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

struct htr_device {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    // sticky health (gpu.rs:900-970): the first failure's kind and message; every later call fails with it
    std::string dead_kind, dead_msg;
    htr_fatal_hook hook = nullptr;
    void *hook_user = nullptr;
    htr_gpu_bytes live{};
    std::unordered_map<void *, std::pair<size_t, int>> allocs;
    char name[256] = {0};
    int n_cu = 0;
    // pinned host staging for small transfers (token ids, positions)
    void *pinned = nullptr;
    size_t pinned_bytes = 0;
    // scratch of the standalone kernel entry points, grown on demand (zero-filled when (re)allocated)
    void *scratch[8] = {nullptr};
    size_t scratch_bytes[8] = {0};
    // the measurement timer's events
    hipEvent_t t0 = nullptr, t1 = nullptr;
    // decode steps replayed as captured HIP graphs (HTR_GRAPHS=0 at open: launched one by one)
    bool use_graphs = true;
    // the compute path of the models created on this device (HTR_COMPUTE_F16 / HTR_COMPUTE_F32)
    int compute = HTR_COMPUTE_F16;
    // the caller is capturing the device's stream (htr_capture_begin … end): nothing may allocate or synchronise
    bool capturing = false;
    // the last kernel launched (its instance: template arguments included), for tests that check the dispatch
    std::string last_kernel;
    // this device's address of the file-scope scratch array of htr_decode_attention_static (attention.hip)
    void *static_scratch = nullptr;
    // htr_phase has a roctx range open on the calling thread
    bool phase_open = false;
    // HTR_POISON=1 at open: fresh and given-back memory is filled with 0xFF (htr_dev_alloc)
    bool poison = false;
    // a 256-workgroup launch spreads its workgroups over 8 XCDs round-robin and a workgroup-scope word is seen across
    // an XCD's workgroups (token_step_xcds; -1: not yet looked at, 1: both hold, 0: the placement does not, 2: the
    // visibility does not)
    int xcd_round_robin = -1;
};

// looks up this device's address of the allocation-free attention's scratch array (the device must be current)
int attn_static_scratch_init(htr_device *dev);

// -1 with a message when the device's stream is being captured by the caller (allocation and synchronisation are not
// part of a graph), else 0
int htr_check_not_capturing(htr_device *dev, const char *what);

enum {
    SCR_CHOOSE_PART = 0,
    SCR_CHOOSE_CNT = 1,
    SCR_ATTN_PART = 2,
    SCR_ATTN_CNT = 3,
    SCR_CAUSAL_BLOCKS = 4,
    SCR_GEMM_PART = 5,  // split-K products [split][M][N]
    SCR_HANDOVER = 6,   // htr_debug_handover's words
};
// the device's scratch buffer `slot` with at least `bytes` bytes (a larger one replaces it: the tickets' and best
// keys' slots zero-filled, the others as htr_dev_alloc fills)
int htr_scratch(htr_device *dev, int slot, size_t bytes, void **out);

// the device is dead: latch the first reason and fire the hook once; returns -1
int htr_latch(htr_device *dev, const char *kind, const char *msg);
// -1 with the sticky reason if the device is dead, else 0
int htr_check_alive(htr_device *dev);
// a HIP error on dev → latched death (kind from the error code); returns -1. ok → 0.
int htr_hip(htr_device *dev, hipError_t e, const char *what);
// after a kernel launch: hipGetLastError → htr_hip
int htr_launched(htr_device *dev, const char *kernel);

// device memory counted in the ledger: zero-filled, or 0xFF under HTR_POISON=1 (for memory written before it is read)
int htr_dev_alloc(htr_device *dev, size_t bytes, int kind, void **out);
// the same, zero-filled in every mode (counters, tickets, self-resetting words that must start at zero)
int htr_dev_alloc_zero(htr_device *dev, size_t bytes, int kind, void **out);
int htr_dev_free(htr_device *dev, void *p);

#define HTR_TRY(expr)                                                                                                  \
    do {                                                                                                               \
        int htr_rc_ = (expr);                                                                                          \
        if (htr_rc_ < 0) return htr_rc_;                                                                               \
    } while (0)

// ---- weights --------------------------------------------------------------------------------------------------------

struct htr_weight {
    htr_device *dev = nullptr;
    size_t rows = 0, cols = 0;
    // q8_0 repacked: quants [rows][cols] int8, scales [rows][cols/32] f16
    int8_t *q = nullptr;
    _Float16 *d = nullptr;
    // dequantised f16 [rows][cols] (MFMA GEMM weights)
    _Float16 *h = nullptr;
};

// ---- kernel launchers (each returns 0 or -1 with the device latched) -------------------------------------------------

// the matvec family (q8_0.hip)
enum DmvMode { DMV_PLAIN = 0, DMV_NORM = 1, DMV_QKV = 2, DMV_FFN = 3 };
struct DmvMat {
    const int8_t *q;
    const _Float16 *d;
    int rows;
};
// rows per wave of the decoder-shaped matvec (one workgroup per CU), 0 when the shape is not one
int dmv_full_rw(htr_device *dev, int mode, const DmvMat *mats, int n_mats, int k);
int launch_dmv(htr_device *dev, hipStream_t st, int mode, const DmvMat *mats, int n_mats, int k, const float *x,
               const float *nw, float eps, float *y, int acc);
int launch_dmv_many(htr_device *dev, hipStream_t st, const DmvMat *mats, int n, int k, const float *x, float *y);
int launch_embed(htr_device *dev, hipStream_t st, const htr_weight *w, const uint32_t *tok, int n_tok, float *x);

// attention (attention.hip)
int launch_qkv_post(htr_device *dev, hipStream_t st, float *qkv, const float *qn, const float *kn, const float *rope,
                    int n_head, int n_kv, const int *pos_dev, int pos, int n_ctx, float eps, uint16_t *kc,
                    uint16_t *vc);
// split-K decode attention; n_keys = *n_keys_dev (+ add) when n_keys_dev != NULL, else n_keys. Scratch: part
// [n_head][max_chunk][130] f32 and counters [n_kv] u32 (zero, self-resetting)
struct AttnScratch {
    float *part;
    uint32_t *counters;
    int max_chunk, chunk;
};
int attn_chunk_for(int n_ctx);
// bytes of the split-K partials for n_head q heads and max_chunk chunks ([h][c][m, l, o[128]] f32)
size_t attn_part_bytes(int n_head, int max_chunk);
// bytes of the split-K ticket counters (one 128-byte line per KV head; zero, self-resetting)
size_t attn_counter_bytes(int n_kv);
// qkv_post's work done inside the attention (q then is the raw [q | k | v] row; the new key / value go to kc / vc)
struct AttnFuse {
    const float *qn, *kn, *rope;
    float eps;
    int n_head;
    _Float16 *kc, *vc;
};
// scale_after: the score is (q·k)·scale (the F32 path's attn_scores) instead of (q·scale)·k (not with fuse)
int launch_attn_decode(htr_device *dev, hipStream_t st, const float *q, const uint16_t *kc, const uint16_t *vc,
                       int n_head, int n_kv, int n_ctx, const int *pos_dev, int n_keys, float scale,
                       const AttnScratch &sc, float *out, const AttnFuse *fuse = nullptr, bool scale_after = false);
// prefill pieces: per-head norm + rope + KV store over n_tok rows
int launch_qk_norm_rope_rows(htr_device *dev, hipStream_t st, float *q, float *k, const float *v, const float *qn,
                             const float *kn, const float *rope, int n_tok, int n_head, int n_kv, int pos0, int n_ctx,
                             float eps, uint16_t *kc, uint16_t *vc);
// the causal prefill attention: q [n_q][n_head·128] f32 (normed, roped), the head-major f16 caches [n_kv][n_ctx][128]
// holding keys 0 … pos0 + n_q − 1; blocks: attn_causal_block_bytes(n_kv, pos0 + n_q) of device scratch (the key
// blocks' copy); out [n_q][n_head·128] f32, or f16 into out16 (the f16 path's o-projection input) when out is NULL
size_t attn_causal_block_bytes(int n_kv, int n_keys);
int launch_attn_causal(htr_device *dev, hipStream_t st, const float *q, const uint16_t *kc, const uint16_t *vc,
                       int n_q, int pos0, int n_head, int n_kv, int n_ctx, float scale, void *blocks, float *out,
                       _Float16 *out16 = nullptr);

// token choice (choose.hip)
struct ChooseArgs {
    float *logits;
    int n_vocab;
    uint32_t *hist;
    int hist_stride;
    const int *len_dev;  // NULL → len
    int len;
    int window;
    float rp;  // 1 → no penalty
    float fp;  // 0 → no frequency penalty
    uint32_t *counts;
    float *fpen;
    uint32_t *tok;
    int *advance;  // NULL, or { pos, len } incremented by the pick (the decode loop's device-resident counters)
    uint64_t *best;      // [rows] × 128 B, zero, self-resetting: the row's best key
    uint32_t *counters;  // [rows] × 128 B, zero, self-resetting: the row's ticket
    int rows;
};
// workgroups of the choice over n_vocab logits, span logits each
int choose_groups(int n_vocab, int span);
// bytes of the choice's per-row best keys and tickets (one 128-byte line per row; zero, self-resetting)
size_t choose_best_bytes(int rows);
size_t choose_ticket_bytes(int rows);
int launch_choose(htr_device *dev, hipStream_t st, const ChooseArgs &a);

// dense kernels (gemm.hip): Y[M,N] (+)= X[M,K]·Wᵀ with W q8_0 (exact dequant), f32; the same with X and W rounded to
// f16 at the tiles (the f16 compute path, any shape); rms_norm rows; swiglu; a weight's f16 plane made on the device
int launch_gemm_q8_0_f32(htr_device *dev, hipStream_t st, const float *x, const htr_weight *w, float *y, int m,
                         int acc);
int launch_gemm_q8_0_r16(htr_device *dev, hipStream_t st, const float *x, const htr_weight *w, float *y, int m,
                         int acc);
int weight_attach_f16(htr_device *dev, hipStream_t st, htr_weight *w);
int launch_rms_norm(htr_device *dev, hipStream_t st, const float *x, const float *w, float *y, int rows, int dim,
                    float eps);
int launch_swiglu(htr_device *dev, hipStream_t st, float *g, const float *u, size_t n);

// MFMA GEMM (mfma_gemm.hip): Y[M,N] (+)= X[M,K]·Wᵀ, X and W f16, f32 accumulation. GEMM_FFN: w = gate, w2 = up,
// y16 = f16(silu(X·Wgᵀ)·(X·Wuᵀ)·scale). W rows a multiple of 64 (the FFN: 128), K a multiple of 32.
enum { GEMM_F32 = 0, GEMM_ACC = 1, GEMM_FFN = 2 };
int launch_gemm_f16(htr_device *dev, hipStream_t st, int epi, const _Float16 *x, int m, const htr_weight *w,
                    const htr_weight *w2, float *y, _Float16 *y16, float scale);
// Q / K / V of one input as one GEMM over the three stacked weights (rows each a multiple of 64), three f32 outputs
// y += x·Wᵀ (the residual), then h16 = f16(rmsnorm(y)·norm_w) — in the K-split reduction when the GEMM splits K
int launch_gemm_f16_acc_norm(htr_device *dev, hipStream_t st, const _Float16 *x, int m, const htr_weight *w, float *y,
                             const float *norm_w, float eps, _Float16 *h16);
int launch_gemm_f16_qkv(htr_device *dev, hipStream_t st, const _Float16 *x, int m, const htr_weight *wq,
                        const htr_weight *wk, const htr_weight *wv, float *q, float *k, float *v);

// the vocabulary of a session's model (text_model.hip)
int session_n_vocab(const htr_session *s);

// GGUF (gguf.hip): tensor lookup, metadata, the streaming upload through two pinned buffers
typedef htr_gguf_tensor_info GgufTensor;
enum { GGUF_F32 = HTR_GGML_F32, GGUF_F16 = HTR_GGML_F16, GGUF_Q8_0 = HTR_GGML_Q8_0, GGUF_BF16 = HTR_GGML_BF16 };
struct GgufStager {
    htr_device *dev = nullptr;
    void *host[2] = {nullptr, nullptr};     // pinned
    void *dev_buf[2] = {nullptr, nullptr};  // device staging
    hipEvent_t ev[2] = {nullptr, nullptr};  // the last copy out of each
    int next = 0;
    int init(htr_device *d);
    ~GgufStager();
};
int gguf_find(htr_gguf *g, const char *name, const GgufTensor **out);
bool gguf_has(htr_gguf *g, const char *name);
bool gguf_has_key(htr_gguf *g, const char *key);
int gguf_meta_u32(htr_gguf *g, const char *key, uint32_t *out);
int gguf_meta_f32(htr_gguf *g, const char *key, float *out);
int gguf_meta_str(htr_gguf *g, const char *key, std::string *out);
// a q8_0 [rows][cols] weight (GGUF shape [cols, rows]) / an F32 [n] vector streamed onto the device (enqueued on the
// device's stream: synchronise before the staging goes away)
int gguf_upload_q8_0(GgufStager &sg, htr_gguf *g, const GgufTensor &t, size_t rows, size_t cols, htr_weight **out);
int gguf_upload_f32(GgufStager &sg, htr_gguf *g, const GgufTensor &t, size_t n, float **out);
// a vision weight [rows][cols] (BF16 or F32 in the file) streamed onto the device into dst16 (f16 of value × scale) or
// dst32 (a BF16 tensor's f16 values as f32, an F32 tensor's own); pairs of values beyond f16's range counted into
// d_over (device u32)
int gguf_upload_vision(GgufStager &sg, htr_gguf *g, const GgufTensor &t, size_t rows, size_t cols, float scale,
                       unsigned *d_over, _Float16 *dst16, float *dst32);
int gguf_meta_bool(htr_gguf *g, const char *key, bool *out);
int gguf_meta_f32_array(htr_gguf *g, const char *key, std::vector<float> *out);
const char *ggml_type_name(uint32_t ty);
std::string gguf_shape_str(const GgufTensor &t);  // "[a, b, …]"

// the vision encoder's other kernels (vision.hip)
int launch_patchify(htr_device *dev, hipStream_t st, const uint8_t *rgb, const float *lut, int w, int px, int n,
                    int side, float *P);
int launch_rms_norm_f16(htr_device *dev, hipStream_t st, const float *x, const float *w, _Float16 *y, int rows, int dim,
                        float eps);
// K / V of the vision attention as f16 key blocks of 8 KB per head (vision_kv_bytes in all)
int launch_heads_f16(htr_device *dev, hipStream_t st, const float *k, const float *v, _Float16 *kv, int n_tok,
                     int n_head, const float *cs, int px, int max_pos);
size_t vision_kv_bytes(int n_tok, int n_head);
int launch_attn_vision(htr_device *dev, hipStream_t st, const float *q, const _Float16 *kv, _Float16 *o, int n_tok,
                       int n_head, float scale, const float *cs, int px, int max_pos);
int launch_unfold2x2(htr_device *dev, hipStream_t st, const float *x, float *z, int px, int py, int dim);
int launch_gelu(htr_device *dev, hipStream_t st, float *x, size_t n);
// x f32 [m][k] → f16 rows of nseg segments of kp values: hi = f16(x), or lo = f16(x − hi) in the segments of lo_mask
int launch_split_f16(htr_device *dev, hipStream_t st, const float *x, int m, int k, int kp, int nseg, int lo_mask,
                     _Float16 *out);

// the decode step of the 1024 / 2048 / 3072 decoder as one launch per token (token_step.hip)
struct TokLayer {
    const int8_t *q[7];  // quant planes: q, k, v, o, gate, up, down
    const _Float16 *d[7];  // their scale planes
    const float *attn_norm, *q_norm, *k_norm, *ffn_norm;
    _Float16 *kc, *vc;  // the layer's f16 caches [n_kv][n_ctx][128]
};
struct TokArgs {
    const TokLayer *layers;  // device table, one entry a layer
    int n_layer, n_ctx, n_vocab;
    const int8_t *emb_q;  // token_embd: the embedding and the tied LM head
    const _Float16 *emb_d;
    uint32_t *tok;        // the token (device); the choice writes the next one here
    int *state;           // state[0]: its position, state[1]: the history's length (the choice advances both)
    const float *rope;    // [n_ctx][64] (cos, sin)
    float eps, scale;
    uint64_t *xw;         // exchange words (token_step_words of them)
    uint32_t *seq, *err;  // the session's token counter (tags); set when a wait ran past spin_ticks
    float *x_out;         // the residual after the last layer
    const float *out_norm;  // output_norm: the LM head's fused RMS norm
    float *logits;        // [n_vocab] (penalised in place when the choice runs)
    // the greedy choice on the logits (choose != 0): the arguments of k_choose for one row (ChooseArgs)
    int choose;
    uint32_t *hist;
    int window;
    float rp, fp;
    uint32_t *counts;
    float *fpen;
    unsigned long long *prof;  // optional: workgroup 0's wall-clock stamps, token_step_stamps(n_layer) of them
    long long spin_ticks;      // a wait's limit in wall-clock ticks
};
int token_step_stamps(int n_layer);
size_t token_step_words();
int token_step_ni(int n_ctx);  // keys a thread of the attention phase, 0 past 8192 rows
bool token_step_shape(const htr_text_config &c);
// 1 when the launch's 256 workgroups fit the device at once for this cache length, else 0 with the reason
int token_step_fits(htr_device *dev, int n_ctx, const char **why);
// 1 when a launch of the step's 256 workgroups puts the workgroups w ≡ x (mod 8) together on one XCD, for each x
// (the XCD-local hand-overs rest on it); 0 with *why when not; -1 on a HIP error. Looked at once a device.
int token_step_xcds(htr_device *dev, const char **why);
int launch_decode_token(htr_device *dev, hipStream_t st, int n_ctx, const TokArgs &a);
