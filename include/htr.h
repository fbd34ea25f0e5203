/*
 * htr.h — the C ABI of the MI355X (gfx950) LightOnOCR decode path.
 *
 * This boundary stands where the reference engine's wgpu device / buffer / dispatch layer stands for this path
 * (app/crates/ocr-wgpu/src/gpu.rs, the `Gpu` and `Batch` types) and under the decoder graph that drives it
 * (app/crates/ocr-wgpu/src/text.rs). Its callers are the ones the reference layer has: the decoder (TextModel /
 * Session / Choice), the vision encoder, and above them the engine's read loop (engine.rs read_text). Every entry point
 * names the reference function it replaces (paths relative to the reference repository root; `gpu.rs`, `text.rs`,
 * `vision.rs`, `engine.rs` are under app/crates/ocr-wgpu/src/).
 *
 * Conventions (gpu.rs:1391-1396, 884-897, text.rs:111-128):
 *   - every function returns int: 0 = ok, < 0 = error; htr_last_error() gives the calling thread's last message, with
 *     the numbers that failed (shape, limit, token id);
 *   - a device whose GPU failed is dead for good (sticky): every later call on it fails with the FIRST reason, and the
 *     fatal hook fires once;
 *   - handles are opaque and freed explicitly; a model must outlive its sessions, a session its choices;
 *   - device pointers (void* / float* named d_*) are device memory from htr_alloc; host pointers are named h_*;
 *   - one thread uses a device at a time (the reference's Gpu is !Sync); callbacks run on the calling thread;
 *   - all work is ordered on the device's one stream; the calls that return host data synchronise it.
 */
#ifndef HTR_H
#define HTR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct htr_device htr_device;
typedef struct htr_weight htr_weight;
typedef struct htr_text_model htr_text_model;
typedef struct htr_session htr_session;
typedef struct htr_choice htr_choice;

/* ---- errors ------------------------------------------------------------------------------------------------ */
/* the calling thread's last error message ("" if none) */
const char *htr_last_error(void);

/* ---- device (gpu.rs:1101-1345 Gpu::with_compute / drop, gpu.rs:1386-1396 alive, gpu.rs:884-897 FatalHook) ----- */
/* The environment at open: HTR_GRAPHS=0 launches the decode's kernels one by one instead of replaying graphs;
 * OCR_WGPU_COMPUTE picks the compute path (below); HTR_POISON=1 is the reference's OCR_WGPU_POISON=1 diagnostic
 * (gpu.rs:739-768, 821-823, 1307-1310): memory the device hands out is filled with 0xFF bytes (NaN as f32 and f16)
 * instead of zeros — except counters and tickets that must start at zero — and filled again when it is given back, so
 * a kernel reading what nothing wrote (or what was freed) reads NaN. The open also checks, with a few small launches,
 * how a launch places its workgroups on the device's 8 XCDs and whether a word stored at workgroup scope is seen by
 * the other workgroups of its XCD; the one-launch decode step, the decode attention's merge and the one-row choice
 * use their XCD-local forms only on a device where both hold. */
int htr_device_open(int ordinal, htr_device **out);
int htr_device_close(htr_device *dev);
/* 0 while the device is healthy; < 0 with the sticky reason once it is dead (gpu.rs:1386-1396 Gpu::alive) */
int htr_alive(htr_device *dev);
/* kind ∈ {"lost", "destroyed", "outOfMemory", "validation", "internal"} — called once, on the first failure */
typedef void (*htr_fatal_hook)(const char *kind, const char *message, void *user);
int htr_set_fatal_hook(htr_device *dev, htr_fatal_hook hook, void *user);
/* the reference tests' device.destroy() (gpu.rs:2421-2448): marks the device lost from the host, no GPU fault */
int htr_debug_mark_lost(htr_device *dev, const char *why);
/* wait for the device's queue (gpu.rs:1458-1485 Gpu::wait) */
int htr_sync(htr_device *dev);
/* the compute path (gpu.rs:1101-1137 Gpu::with_compute / Compute::choose, OCR_WGPU_COMPUTE): HTR_COMPUTE_F16 — the
 * default, and what the reference picks on a device with f16 and matrix units (F16Coop) — rounds the prefill GEMMs' X
 * and dequantised W to f16 and sums in f32 (matmul_coop_q8_0); HTR_COMPUTE_F32 computes them from the exact q8_0
 * values in f32 (matmul128_q8_0). OCR_WGPU_COMPUTE = f32 / f16 / coop at open sets it as the reference's env var does.
 * A text model keeps the path of its device at creation, for its prefill and its decode step: the F32 path's step is
 * the reference's (text.rs:555-576: rms_norm, one matvec per projection, qkv_post, the attention with each score
 * scaled after its dot product, swiglu), the f16 paths' the fused one (layers_fused, text.rs:630-647); both compute
 * in f32. The vision encoder runs its f16 path on either setting (its F32 path is not built). */
enum { HTR_COMPUTE_F32 = 0, HTR_COMPUTE_F16 = 1 };
int htr_device_set_compute(htr_device *dev, int compute);
int htr_device_compute(htr_device *dev, int *compute);
/* the device name and compute-unit count, for reports */
int htr_device_info(htr_device *dev, char *name, size_t name_len, int *n_cu);
/* HIP-event timing on the device's stream (measurement helpers, no reference counterpart — the reference's profiler
 * is gpu.rs:1004-1016 timestamp queries): begin records the start event; end records the stop event, waits for it
 * and returns the elapsed milliseconds */
int htr_timer_begin(htr_device *dev);
int htr_timer_end(htr_device *dev, float *ms);

/* the name of the last kernel this device launched, template arguments included (e.g. "k_dmv_full<4,1,qkv>"): for tests
 * that check which kernel instance an entry point dispatched (no reference counterpart) */
int htr_debug_last_kernel(htr_device *dev, char *name, size_t cap);
/* The hand-over the one-launch decode step rests on, measured on this device (csrc/handover.hip; no reference
 * counterpart). A launch of 256 workgroups passes tagged 64-bit words: kind 0, one word back and forth `iters` times
 * between workgroups a and b, stored at workgroup scope (it stays in the writer XCD's L2); kind 1, the same stored at
 * agent scope (written through); both read with agent-scope loads; kind 2, every workgroup passes words / 256 words
 * (256 … 3072, a multiple of 256) to all the others, `iters` times, its first poll `pause` × 64 clocks after its own
 * words (0, 4, 8, 12, 16, 20, 24 or 32). *us: µs a round trip (kinds 0, 1) or an exchange (kind 2). *seen: 1 when every wait saw its word, 0 when one
 * ran out after max_polls loads (a workgroup-scope word is not seen from another XCD). Not while capturing. */
int htr_debug_handover(htr_device *dev, int kind, int a, int b, int words, int pause, int iters, int max_polls,
                       double *us, int *seen);

/* ---- HIP graphs of the device's stream (no reference counterpart: the reference records a wgpu command buffer per
 *      submission, gpu.rs:1864-1960; here a caller records entry-point calls once and replays them) --------------- */
typedef struct htr_graph htr_graph;
/* begin recording the device's stream: the kernel entry points called until htr_capture_end are recorded, not run.
 * While recording, every call that allocates, frees, copies to or from the host or waits fails (an entry point whose
 * scratch would grow must have run once at that size before); so do htr_prefill, htr_step and htr_decode_gpu. */
int htr_capture_begin(htr_device *dev);
int htr_capture_end(htr_device *dev, htr_graph **out);
/* replay a recorded graph on the device's stream */
int htr_graph_launch(htr_graph *g);
int htr_graph_free(htr_graph *g);

/* ---- memory (gpu.rs:509-561 ledger per MemKind; gpu.rs:1489-1590 upload / scratch / readback / read_f32) ------- */
enum { HTR_MEM_WEIGHTS = 0, HTR_MEM_KV_CACHE = 1, HTR_MEM_WORK = 2, HTR_MEM_READBACK = 3 };
typedef struct {
    uint64_t weights, kv_cache, work, readback;
} htr_gpu_bytes;
int htr_mem_live(htr_device *dev, htr_gpu_bytes *out);
/* device memory of `bytes` bytes counted under `kind`; freed by htr_free. Zero-filled (0xFF bytes under HTR_POISON=1). */
int htr_alloc(htr_device *dev, size_t bytes, int kind, void **d_out);
int htr_free(htr_device *dev, void *d_ptr);
/* host ↔ device copies on the device's stream; htr_download waits for it */
int htr_upload(htr_device *dev, void *d_dst, const void *h_src, size_t bytes);
int htr_download(htr_device *dev, void *h_dst, const void *d_src, size_t bytes);
/* d_dst[0 … bytes) = d_src[0 … bytes) on the device's stream, both 16-byte aligned, not overlapping (gpu.rs:2102-2110
 * Batch::copy). Also the plain copy of known size that calibrates the HBM byte counters. */
int htr_copy(htr_device *dev, void *d_dst, const void *d_src, size_t bytes);
/* a read of d_src[0 … bytes) on the device's stream and nothing else (no reference counterpart: a measurement of this
 * device): every workgroup reads kb_per_workgroup KB (16, 32 or 64) through 16-byte loads, non-temporal when
 * `nontemporal`, all issued before the first use, and folds them into a word stored at d_sink only when it equals a
 * fixed value (so at most one u32 there is written). Timed with htr_timer_*, the read rate a streaming kernel such as
 * the q8_0 matvec can reach here. bytes a positive multiple of 16, d_src 16-byte aligned. */
int htr_debug_read(htr_device *dev, const void *d_src, size_t bytes, int nontemporal, int kb_per_workgroup,
                   uint32_t *d_sink);
/* the phase of the following work (gpu.rs:1349-1358 Gpu::phase: "vision", "prefill", "decode", "-" = none): a roctx
 * range on the calling thread that rocprofv3 --marker-trace records; the device's previous phase range ends */
int htr_phase(htr_device *dev, const char *name);

/* ---- weights (gpu.rs:1595-1677 upload_tensor with WeightType::Q8_0; text.rs:101-110 weight) -------------------- */
/* a [rows × cols] q8_0 tensor from its GGUF block bytes (rows × cols/32 blocks of 34 bytes: f16 d LE + 32 × i8 q;
 * ocr-gguf lib.rs:128-135). Repacked at load into an int8 plane [rows][cols] and an f16 scale plane [rows][cols/32]:
 * every matvec lane then issues 16-byte loads of contiguous quants. cols must be a multiple of 32. */
int htr_weight_q8_0(htr_device *dev, const void *h_blocks, size_t rows, size_t cols, htr_weight **out);
/* the same weight dequantised to f16 (q·d rounded to nearest even) for the MFMA GEMMs (vision.rs:122-142: the
 * reference converts its vision weights to f16 at load; scale multiplies every value first, as FFN_DOWN_SCALE) */
int htr_weight_q8_0_f16(htr_device *dev, const void *h_blocks, size_t rows, size_t cols, float scale,
                        htr_weight **out);
int htr_weight_free(htr_weight *w);
int htr_weight_shape(const htr_weight *w, size_t *rows, size_t *cols);

/* ---- kernels on device buffers (gpu.rs:1864 Batch::dispatch of the named kernels) ------------------------------ */
/* y[rows] (+)= W·x — dmv.wgsl (acc = 1 adds onto y); with d_norm_w != NULL the input is RMS-normed first
 * (dmv_norm: x · 1/sqrt(mean(x²)+eps) · norm_w). gpu.rs:2094 Batch::matvec, text.rs:551-552, 642, 644 */
int htr_matvec_q8_0(htr_device *dev, const htr_weight *w, const float *d_x, const float *d_norm_w, float eps,
                    float *d_y, int acc);
/* n matvecs y_i = W_i·x (one x, n weights of one shape, y [n][rows]) in ONE launch: the throughput of the matvec
 * kernel over a rotation of weight copies larger than the Infinity Cache (no reference counterpart: a measurement
 * entry) */
int htr_matvec_q8_0_many(htr_device *dev, const htr_weight *const *ws, size_t n, const float *d_x, float *d_y);
/* dmv_qkv.wgsl: attn_norm fused → [q | k | v] (text.rs:638) */
int htr_matvec_qkv(htr_device *dev, const htr_weight *wq, const htr_weight *wk, const htr_weight *wv,
                   const float *d_x, const float *d_norm_w, float eps, float *d_qkv);
/* dmv_ffn.wgsl: ffn_norm fused → g = silu(Wg·xn)·(Wu·xn) (text.rs:643) */
int htr_matvec_ffn(htr_device *dev, const htr_weight *wg, const htr_weight *wu, const float *d_x,
                   const float *d_norm_w, float eps, float *d_g);
/* qkv_post.wgsl (text.rs:639): per-head RMSNorm of q and k, RoPE NEOX at `pos` from the host table d_rope
 * [n_pos][64] × (cos, sin) (text.rs:132-142), q written back in place, k and v stored f16 (RNE) into the head-major
 * caches d_k / d_v [n_kv][n_ctx][128] at row pos. Head dim 128. */
int htr_qkv_post(htr_device *dev, float *d_qkv, const float *d_q_norm, const float *d_k_norm, const float *d_rope,
                 int n_head, int n_kv, int pos, int n_ctx, float eps, uint16_t *d_k, uint16_t *d_v);
/* split-K GQA decode attention (attn_decode.wgsl + attn_merge.wgsl, text.rs:640-641): q [n_head·128] f32, the
 * head-major f16 caches [n_kv][n_ctx][128], n_keys keys, scale → out [n_head·128] f32. GQA group 2. */
int htr_decode_attention(htr_device *dev, const float *d_q, const uint16_t *d_k, const uint16_t *d_v, int n_head,
                         int n_kv, int n_ctx, int n_keys, float scale, float *d_out);
/* htr_decode_attention without allocation: no counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid it): the same kernel and result,
 * bit for bit, with its split-K partials and tickets in a file-scope device array of 4 MiB per GPU (held until the
 * process ends) instead of library-allocated scratch. Shapes whose partials exceed it (n_head × chunks × 520 bytes
 * > 4 MiB − 8 KiB: 16 heads fit every cache size, 32 heads up to 64,256 rows) and more than 64 KV heads are
 * refused with an error. Calls that overlap on one GPU share the array and race; each call clears its tickets. */
int htr_decode_attention_static(htr_device *dev, const float *d_q, const uint16_t *d_k, const uint16_t *d_v,
                                int n_head, int n_kv, int n_ctx, int n_keys, float scale, float *d_out);
/* causal GQA prefill attention (attention_causal.wgsl, text.rs:484-499): q [n_q][n_head·128] f32 (normed and roped)
 * at positions pos0 …, the head-major f16 caches [n_kv][n_ctx][128] holding the keys 0 … pos0 + n_q − 1 → out
 * [n_q][n_head·128] f32 = softmax(q·scale·Kᵀ over the keys ≤ each query's position)·V. GQA group 2. */
int htr_causal_attention(htr_device *dev, const float *d_q, const uint16_t *d_k, const uint16_t *d_v, int n_q,
                         int pos0, int n_head, int n_kv, int n_ctx, float scale, float *d_out);
/* the GPU token choice of a greedy preset on n_vocab logits (choose_pen → choose_max → choose_pick,
 * text.rs:222-231; semantics of ocr-decode sampling.rs:38-62, bit-exact): the repetition penalty rp over the distinct
 * ids of d_hist[len − window … len) applied in place (< 0: × rp, else ÷ rp, IEEE round-to-nearest), the frequency
 * penalty (d_counts / d_fpen, both NULL when fp == 0) in the comparison, first maximum → d_tok[0] and d_hist[len].
 * rp must be 1 or a positive normal f32 (text.rs:154-163). */
int htr_choose(htr_device *dev, float *d_logits, int n_vocab, uint32_t *d_hist, int len, int window, float rp,
               float fp, uint32_t *d_counts, float *d_fpen, uint32_t *d_tok);
/* the same choice for n independent rows (logits [n][n_vocab], histories [n][hist_stride], tok[n]) in ONE launch:
 * the 10k-step measurement of the choice kernel (no reference counterpart) */
int htr_choose_many(htr_device *dev, float *d_logits, int n_vocab, int n, uint32_t *d_hist, int hist_stride, int len,
                    int window, float rp, uint32_t *d_tok);

/* Y[m][N] (+= with acc) X·Wᵀ, X f32 [m][K], W q8_0 [N][K] (gpu.rs:1963-2014 Batch::matmul with a q8_0 weight, the
 * prefill's GEMMs): on the device's compute path — F32: exact dequant, f32 fma (matmul128_q8_0 / matmul.wgsl);
 * F16: X and W rounded to f16 as they enter the tiles, f32 sums (matmul128h_q8_0 / matmul_coop_q8_0). Any shape
 * (K a multiple of 32). */
int htr_matmul_q8_0(htr_device *dev, const float *d_x, size_t m, const htr_weight *w, float *d_y, int acc);

/* ---- the vision encoder's GEMMs on the matrix cores (gpu.rs:2019-2042 Batch::matmul_f16x → matmul_coopd.wgsl,
 *      gpu.rs:2048-2086 Batch::ffn_f16 → ffn_coopd.wgsl) ------------------------------------------------------- */
/* d_y[m][N] (+= with acc) X·Wᵀ: d_x f16 [m][K] (IEEE binary16 bits), w an f16 weight (htr_weight_q8_0_f16) [N][K]
 * with N a multiple of 128 and K a multiple of 32; f32 accumulation */
int htr_gemm_f16(htr_device *dev, const uint16_t *d_x, size_t m, const htr_weight *w, float *d_y, int acc);
/* d_g[m][N] = f16(silu(X·Wgᵀ) · (X·Wuᵀ) · scale): the vision FFN's first half (the reference stores it × 1/64) */
int htr_gemm_ffn_f16(htr_device *dev, const uint16_t *d_x, size_t m, const htr_weight *w_gate, const htr_weight *w_up,
                     float scale, uint16_t *d_g);

/* ---- the vision encoder (vision.rs:37-263 VisionConfig / Vision, the f16 compute path run_f16 + project) -------- */
typedef struct htr_vision htr_vision;
/* VisionConfig (vision.rs:37-84): head dim 64, 2×2 merge, rope θ (10000 for LightOnOCR), the pixel mean / std */
typedef struct {
    int n_layer, dim, n_head, d_head, n_ff, patch, merge, image_size, proj_dim;
    float eps, rope_theta;
    float mean[3], std[3];
} htr_vision_config;
/* one encoder layer's tensors as host bytes: q8_0 GGUF blocks for the projections, f32 for the norms */
typedef struct {
    const float *ln1, *ln2;
    const void *q, *k, *v, *o, *gate, *up, *down;
} htr_vision_layer;
/* Vision::from_gguf (vision.rs:177-233): the projections and the projector converted to f16 at load (the down
 * projection × 64, vision.rs:31-35); patch_embd f32 [dim][3·patch²], norms f32 [dim], merger [dim][4·dim],
 * mm1 [proj_dim][dim], mm2 [proj_dim][proj_dim] as q8_0 blocks */
int htr_vision_create(htr_device *dev, const htr_vision_config *cfg, const float *patch_embd, const float *pre_ln,
                      const htr_vision_layer *layers, const float *input_norm, const void *merger, const void *mm1,
                      const void *mm2, htr_vision **out);
int htr_vision_free(htr_vision *v);
/* the configuration of an encoder (Vision::cfg, vision.rs:91) */
int htr_vision_get_config(htr_vision *v, htr_vision_config *out);
/* the output of an encode of a width × height page (Vision::grid, vision.rs:236-244: both sides on the patch·merge
 * grid, the longer ≤ image_size): n_layers < 0 → [n/4][proj_dim] embeddings; n_layers ≥ 0 → the residual after that
 * many layers [n][dim] (the reference's `layers` bisect hook, vision.rs:246-256) */
int htr_vision_out_shape(htr_vision *v, int width, int height, int n_layers, size_t *n_tokens, size_t *dim);
/* Vision::encode_gpu (vision.rs:258-263): RGB bytes [height][width][3] → d_out (device memory of the shape above) */
int htr_vision_encode(htr_vision *v, const uint8_t *h_rgb, int width, int height, int n_layers, float *d_out);

/* ---- GGUF files (ocr-gguf lib.rs:1-401: Gguf / TensorSource / TensorInfo) --------------------------------------- */
typedef struct htr_gguf htr_gguf;
/* ggml types the reader accepts (lib.rs:98-130); any other is an error */
enum { HTR_GGML_F32 = 0, HTR_GGML_F16 = 1, HTR_GGML_Q8_0 = 8, HTR_GGML_BF16 = 30 };
typedef struct {
    char name[128];
    uint32_t type;         /* HTR_GGML_* */
    uint32_t n_dims;       /* 1 … 4 */
    uint64_t shape[4];     /* ggml order: shape[0] is the contiguous (innermost) dimension */
    uint64_t n_elements, n_bytes;
    uint64_t offset;       /* from the start of the data section */
    uint64_t file_offset;  /* absolute */
} htr_gguf_tensor_info;
/* TensorSource::read_at: fill buf with the len bytes at off; 0, or nonzero on failure */
typedef int (*htr_read_fn)(void *user, uint64_t off, void *buf, size_t len);
/* Gguf::open / Gguf::from_source (lib.rs:316-346): the header (GGUF v2 / v3) parsed from a prefix of the source
 * (1 MiB, doubled while the header is longer); every tensor must end inside the source. The tensors' bytes are read
 * on demand. The file is read with pread (no mapping). */
int htr_gguf_open(const char *path, htr_gguf **out);
int htr_gguf_open_source(uint64_t len, htr_read_fn read, void *user, htr_gguf **out);
int htr_gguf_close(htr_gguf *g);
/* version, general.alignment (default 32), the data section's offset, the tensor count */
int htr_gguf_header(htr_gguf *g, uint32_t *version, uint64_t *alignment, uint64_t *data_offset, size_t *n_tensors);
/* TensorInfo by name (Gguf::info), or by file order when name is NULL */
int htr_gguf_tensor(htr_gguf *g, const char *name, size_t index, htr_gguf_tensor_info *out);
/* metadata (Gguf::u32 — a non-negative i32 reads too —, Gguf::f32, Gguf::str, Gguf::f32_array): the length of a
 * string / array is written to *len; a string is cut to cap − 1 bytes and terminated */
int htr_gguf_u32(htr_gguf *g, const char *key, uint32_t *out);
int htr_gguf_f32(htr_gguf *g, const char *key, float *out);
int htr_gguf_str(htr_gguf *g, const char *key, char *buf, size_t cap, size_t *len);
int htr_gguf_f32_array(htr_gguf *g, const char *key, float *out, size_t cap, size_t *len);
/* Gguf::read_small (lib.rs:484-493): a tensor of at most 1 MiB, raw bytes */
int htr_gguf_read_small(htr_gguf *g, const char *name, void *buf, size_t cap);

/* ---- the text decoder (text.rs:30-130 TextConfig / TextModel, text.rs:332-375 load) ------------------------------ */
typedef struct {
    int n_layer, dim, n_head, n_kv, d_head, n_ff, n_vocab, n_ctx_train;
    float eps, rope_base;
} htr_text_config;

/* one layer's tensors as host bytes: q8_0 GGUF blocks for the projections, f32 for the norms (text.rs:82-94) */
typedef struct {
    const void *q, *k, *v, *o, *gate, *up, *down;
    const float *attn_norm, *q_norm, *k_norm, *ffn_norm;
} htr_layer_tensors;

/* TextModel::load (text.rs:332-375): same shape checks (d_head 128, q8_0 rows of whole blocks, GQA group 2) */
int htr_text_model_create(htr_device *dev, const htr_text_config *cfg, const void *tok_embd, const float *output_norm,
                          const htr_layer_tensors *layers, htr_text_model **out);
int htr_text_model_free(htr_text_model *m);
/* TextModel::load from a GGUF (text.rs:43-76 TextConfig::from_gguf, text.rs:101-118 weight / vector, text.rs:332-375):
 * the qwen3.* metadata, the same shape / type / absent-tensor checks, the q8_0 projections streamed file → device
 * through two pinned 32 MiB buffers and repacked on the device (never a whole tensor in host memory) */
int htr_text_model_load_gguf(htr_device *dev, htr_gguf *g, htr_text_model **out);
/* the configuration a model was built with */
int htr_text_model_config(htr_text_model *m, htr_text_config *out);
/* Vision::load / Vision::from_gguf (vision.rs:177-233) from an mmproj GGUF: the configuration from the clip.* keys
 * (VisionConfig::from_gguf, vision.rs:55-84: projector "lightonocr", SwiGLU, head dim 64, rope θ 10000), the encoder
 * tensors v.blk.{i}.{ln1,ln2,attn_q,attn_k,attn_v,attn_out,ffn_gate,ffn_up,ffn_down}.weight, v.patch_embd.weight,
 * v.pre_ln.weight, mm.input_norm.weight, mm.patch_merger.weight, mm.1.weight, mm.2.weight streamed onto the device;
 * BF16 weights converted to f16 there (f16_from_bf16.wgsl; ffn_down × 64), F32 weights taken as they are (the
 * projections rounded to f16), F32 norms. Refused: another projector, a tensor the graph would read if present
 * (v.patch_embd.bias, v.post_ln.weight, mm.1.bias, mm.2.bias, v.token_embd.img_break, mm.input_norm.bias), a
 * weight of another type or shape, and values beyond f16's range (65504, after the scale) */
int htr_vision_load_gguf(htr_device *dev, htr_gguf *g, htr_vision **out);

/* TextModel::session (text.rs:378-434): n_ctx positions (prompt + new tokens); the KV cache is allocated here, once,
 * for all n_ctx rows (the reference's `session` grows it by 512 rows at a time instead — htr_session_create_grown) */
int htr_session_create(htr_text_model *m, size_t n_ctx, htr_session **out);
/* TextModel::session_grown (text.rs:389-434; `session` and `session_for` are it with kv_grow 512 and max(expect,
 * 512)): n_ctx positions, the KV cache allocated by the first prefill or step and grown with the read
 * (Session::reserve, text.rs:287-327) — whenever a prefill, a step or a GPU choice's run-ahead would write past its
 * end, to the rows asked + kv_grow (at most n_ctx). A growth waits for the launches in flight, copies the rows held
 * into the larger cache and frees the old one (both held meanwhile); the results are a presized cache's, bit for bit.
 * kv_grow = 0 is refused. */
int htr_session_create_grown(htr_text_model *m, size_t n_ctx, size_t kv_grow, htr_session **out);
/* the KV cache rows allocated now (Session::kv_rows, text.rs:282-285): n_ctx for htr_session_create */
int htr_session_kv_rows(htr_session *s, size_t *out);
int htr_session_free(htr_session *s);
/* positions recorded so far (Session::n_past) */
int htr_session_n_past(htr_session *s, size_t *out);
/* TextModel::prefill (text.rs:437-521): ids at positions n_past …; the last row's logits → h_logits (may be NULL) */
int htr_prefill(htr_session *s, const int32_t *ids, size_t n, float *h_logits);
/* TextModel::step (text.rs:524-537), the CPU-choice path: one token at n_past → its logits into h_logits */
int htr_step(htr_session *s, int32_t tok, float *h_logits);
/* the session's last logits (after prefill / step / a GPU choice: penalised in place) → h_logits */
int htr_session_logits(htr_session *s, float *h_logits);
/* the session's KV cache on the device (text.rs:242-260 Session::k / v, one buffer per layer there): f16 K and V,
 * each [n_layer][n_kv][n_ctx][d_head] (layer_stride halves per layer) — head-major, where the reference keeps
 * [pos][n_kv·d_head]; n_ctx here is the rows allocated (htr_session_kv_rows). For tests that read back or plant rows;
 * the pointers live until the cache grows or the session is freed. */
typedef struct {
    uint16_t *d_k, *d_v;
    int n_layer, n_kv, n_ctx, d_head;
    size_t layer_stride;
} htr_kv_view;
int htr_session_kv_cache(htr_session *s, htr_kv_view *out);
/* forget the positions ≥ n_past (≤ the current n_past): later steps rewrite their KV rows. No reference counterpart
 * (a read's session only grows, text.rs:242-328); it lets a bench replay one read's decode */
int htr_session_rewind(htr_session *s, size_t n_past);

/* the in-graph time of the decode step's kernel classes (a measurement entry, no reference counterpart: the
 * reference's profiler is the per-dispatch timestamps of gpu.rs:1004-1016): n_steps steps (1 … 256) recorded as one
 * HIP graph holding only the kernels of `classes` (HTR_STEP_* bits), all at the session's position (nothing advances
 * it; each step rewrites that KV row), replayed reps times after one untimed replay → milliseconds per step. A model of
 * the f16 paths; the session must be at a position 1 … n_ctx − 1. */
enum {
    HTR_STEP_EMBED = 1, HTR_STEP_QKV = 2, HTR_STEP_ATTENTION = 4, HTR_STEP_O = 8, HTR_STEP_FFN = 16,
    HTR_STEP_DOWN = 32, HTR_STEP_HEAD = 64, HTR_STEP_ALL = 127
};
int htr_session_profile_step(htr_session *s, unsigned classes, int n_steps, int reps, float *ms_per_step);

/* The decode step's form (text.rs:540-552 + layers_fused, text.rs:630-647: the same arithmetic either way, the
 * attention's softmax and split-K merge summing in another order). For the 1024 / 2048 / 3072 decoder (16 / 8 heads of 128, ≤ 42 layers,
 * ≤ 262144 vocabulary ids) on the f16 paths, with a cache of ≤ 8192 rows, a session steps by ONE launch per token:
 * the embedding, every layer, the LM head and — in htr_decode_gpu — the greedy choice (the semantics of htr_choose), as
 * 256 workgroups, all resident at once, that hand each phase's outputs to the next through tagged words in device
 * memory. That is the default when the device holds the 256 workgroups at once and spreads them round-robin over 8
 * XCDs (a KV head's attention phases run on one XCD and hand over through its L2; checked once a device; the
 * environment variable
 * HTR_FUSED_STEP=0 makes the per-kernel step the default instead); other models and the F32 path step kernel by
 * kernel. No reference counterpart (the reference records one dispatch per kernel).
 * set_fused_step(1) fails, with the reason, for a session that cannot take the one-launch form; fused_step reports the
 * session's form and, when the one-launch form is not available or the session went back from it, why (a static
 * string, or NULL). Every wait of the one-launch step is bounded (0.2 s of wall clock): a step whose wait ran out —
 * its 256 workgroups were not all resident at once, as when another process or stream holds CUs — is redone on the
 * per-kernel step, and the session keeps the per-kernel step from then on (htr_step redoes the step; htr_decode_gpu
 * redoes the chunk, see there); set_fused_step(1) takes the one-launch step up again.
 * profile_fused_step runs one one-launch step of `tok` at the session's position (not advanced; its KV row written
 * there; no choice) and returns workgroup 0's 1 + 12·n_layer + 3 wall-clock stamps in µs after the embed: per layer
 * the input of each phase taken and its output written, for qkv, attention, merge, o, gate/up, down; then the LM
 * head's input taken, its rows done, the end. */
int htr_session_set_fused_step(htr_session *s, int on);
int htr_session_fused_step(htr_session *s, int *on, const char **why_not);
int htr_session_profile_fused_step(htr_session *s, int32_t tok, double *us, int n);
/* the one-launch step's bound on each wait, in µs (≤ 0: the default 0.2 s), carried by the launches recorded from now
 * on. No reference counterpart: tests of the error path make every wait run out from the host (the kernels still end
 * through their bounded waits). The environment variable HTR_FUSED_SPIN_US sets it when the session is made. */
int htr_session_set_wait_limit(htr_session *s, double us);

/* ---- the GPU token choice and the run-ahead decode (text.rs:165-232 Choice, text.rs:587-625 decode_gpu) -------- */
/* the preset fields the choice reads (ocr-decode presets.rs:17-29) */
typedef struct {
    double temperature, top_p, repetition_penalty, frequency_penalty;
    size_t repetition_window, max_new_tokens;
} htr_preset;
/* Choice::new (text.rs:185-218): greedy presets only, rp 1 or a positive normal f32 (gpu_choice_capable,
 * text.rs:154-163), the history's last `window` ids seed the window (each inside the vocabulary), `chunk` choices per
 * graph launch (1…64), `depth` launches in flight (≥ 1) */
int htr_choice_create(htr_session *s, const htr_preset *p, const int32_t *history, size_t n, size_t chunk,
                      size_t depth, htr_choice **out);
int htr_choice_free(htr_choice *c);
/* 0 ⇒ stop the read; nonzero ⇒ go on */
typedef int (*htr_token_cb)(int32_t tok, void *user);
/* TextModel::decode_gpu (text.rs:587-625): up to max choices, the first from the session's logits, each later one
 * after a decode step that embeds the previous choice on the device. Steps are replayed as HIP graphs, `chunk` per
 * launch, `depth` launches in flight; 4 bytes per token come back. on_token returning 0 ends the read. A chunk's ids
 * reach on_token only once the chunk is known good (the reference's read_mapped_u32 fails before on_token sees a
 * submission, text.rs:616-623): a chunk in which a one-launch step's wait ran out passes none of its ids on, the
 * launches behind it are drained unseen, and the read goes on from the chunk's first step on the per-kernel step
 * (frequency counts, position and token rewound), which the session then keeps. */
int htr_decode_gpu(htr_session *s, htr_choice *c, size_t max, htr_token_cb on_token, void *user);

/* ---- the CPU-choice decode (ocr-decode sampling.rs:23-89, 252-278) ------------------------------------------------ */
/* choose (sampling.rs:38-89) on host logits, penalised in place: the repetition penalty over the distinct ids of the
 * history's last repetition_window (< 0: × rp, else ÷ rp), the frequency penalty fp · count over (count_ids, counts),
 * then the first maximum (temperature 0) or temperature + top-p sampling with the SplitMix64 state *rng (Rng,
 * sampling.rs:23-35; advanced once per sampled choice) → *out. The preset is checked as Preset::validate does
 * (presets.rs:35-55: temperature ≥ 0, 0 < top_p ≤ 1 and 1 when greedy, rp > 0, window ≥ 1, fp ≥ 0, max ≥ 1). */
int htr_choose_host(float *logits, size_t n_vocab, const htr_preset *p, const int32_t *history, size_t n_history,
                    const int32_t *count_ids, const uint32_t *counts, size_t n_counts, uint64_t *rng, int32_t *out);
/* generate (sampling.rs:252-278) over TextModel::step (text.rs:524-537): up to max_new_tokens choices on the CPU, the
 * first from the session's logits, each chosen token passed to on_token and then stepped on the device (htr_step).
 * history seeds the repetition window, seed the Rng; the frequency counts start empty. on_token returning 0 ends the
 * read before the token is stepped (the engine's end of generation or cancel). *n_out = the tokens passed to
 * on_token. */
int htr_generate(htr_session *s, const htr_preset *p, uint64_t seed, const int32_t *history, size_t n_history,
                 htr_token_cb on_token, void *user, size_t *n_out);

/* ---- seeded synthetic inputs (host-side data generation for tests and benches; not on the decode path) ------- */
/* q8_0 GGUF blocks: quants uniform in [−127, 127], d = f16(|N(0,1)|·0.002), from (seed, block index) */
int htr_synth_q8_0(uint64_t seed, size_t rows, size_t cols, void *h_blocks);
/* f32 values mean + std·N(0,1) from (seed, index) */
int htr_synth_normal(uint64_t seed, size_t n, float mean, float std, float *h_out);

#ifdef __cplusplus
}
#endif
#endif
