// The text decoder's host side: TextModel (text.rs:30-130, 332-375), Session (text.rs:242-434), the prefill
// (text.rs:437-521), the CPU-choice step (text.rs:524-537), the GPU token choice (text.rs:165-232) and the run-ahead
// decode (text.rs:587-625), on the kernels of q8_0.hip / attention.hip / choose.hip / gemm.hip.
//
// The decode step (record_step, text.rs:540-578 with layers_fused, text.rs:630-647) is 1 + 5·n_layer + 1 launches:
//   embed → per layer: qkv matvec (attn_norm fused) → split-K attention (q/k norm, RoPE and the f16 KV store fused)
//   (merge fused) → o matvec (+ residual) → gate/up matvec (ffn_norm + SwiGLU fused) → down matvec (+ residual)
//   → LM head (output_norm fused) [→ token choice].
// Position and history length live in device memory (state[0] = pos, state[1] = len), so one captured HIP graph of
// `chunk` steps is replayed for the whole read: the choice kernel advances both, the next step's embed reads the
// chosen token from device memory. Only the chosen ids (4 bytes a token) come back to the host.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <vector>

#include "htr_internal.h"

namespace {

constexpr int HEAD = 128;

struct Layer {
    htr_weight *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr, *gate = nullptr, *up = nullptr,
               *down = nullptr;
    float *attn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr, *ffn_norm = nullptr;
};

// text.rs:132-142: θ = f32(pos)·powf(base, −2i/d), cos / sin in f32
std::vector<float> rope_table(float base, int d_head, int n_pos) {
    const int half = d_head / 2;
    std::vector<float> out((size_t)n_pos * half * 2);
    for (int pos = 0; pos < n_pos; pos++)
        for (int i = 0; i < half; i++) {
            const float theta = (float)pos * powf(base, -((float)(2 * i)) / (float)d_head);
            out[2 * ((size_t)pos * half + i)] = cosf(theta);
            out[2 * ((size_t)pos * half + i) + 1] = sinf(theta);
        }
    return out;
}

}  // namespace

struct htr_text_model {
    htr_device *dev = nullptr;
    htr_text_config cfg{};
    int compute = HTR_COMPUTE_F16;  // the device's compute path at creation
    bool mfma16 = false;            // f16 path: the projections carry f16 planes for the MFMA GEMMs
    htr_weight *tok_embd = nullptr;
    float *output_norm = nullptr;
    std::vector<Layer> layers;
};

struct htr_session {
    htr_text_model *m = nullptr;
    htr_device *dev = nullptr;
    int n_ctx = 0, n_past = 0;
    // the KV cache: kv_rows rows allocated (≤ n_ctx; the row stride of its head-major layout), grown by reserve to
    // the rows asked + kv_grow; kv_gen counts the growths (a choice's graphs hold the layout they were captured with)
    int kv_rows = 0, kv_grow = 0;
    unsigned kv_gen = 0;
    size_t kv_layer = 0;  // halves per layer and cache (n_kv · kv_rows · 128)
    uint16_t *kc = nullptr, *vc = nullptr;
    float *rope = nullptr;
    float *x = nullptr, *qkv = nullptr, *attn = nullptr, *g = nullptr, *logits = nullptr;
    float *h = nullptr, *u = nullptr;  // the F32 path's step: the normed row and the up projection
    uint32_t *tok = nullptr;
    int *state = nullptr;  // [pos, len]
    AttnScratch asc{};
    hipGraphExec_t step_graph = nullptr;  // the CPU-choice step (no token choice)
    // the prefill's row buffers (ids, x, h, q, k, v, attention, g, u) for up to pre_cap rows, kept across calls
    void *pre = nullptr;
    // the causal attention's key blocks (a copy of the cache's keys 0 … pos0 + n − 1 in its LDS layout), grown on demand
    void *kvb = nullptr;
    size_t kvb_bytes = 0;
    size_t pre_cap = 0;
    // the one-launch step (token_step.hip) for the 1024 / 2048 / 3072 decoder: its layer table, exchange words and
    // [seq, err] words; `fused` selects it for the decode step (fused_why: why it cannot be, when it cannot)
    TokLayer *tl = nullptr;
    uint64_t *xw = nullptr;
    uint32_t *tseq = nullptr;
    bool fused = false;
    const char *fused_why = nullptr;
    long long spin_ticks = 0, spin_default = 0;
    // a one-launch step's wait ran past its limit and the session went back to the per-kernel step (the step or the
    // read was redone on it); htr_session_set_fused_step(1) takes the one-launch step up again
    bool fell_back = false;
    // bumped when what the captured graphs hold by value changes (the wait limit): a choice's graphs are re-captured
    unsigned cap_gen = 0;
};

struct htr_choice {
    htr_session *s = nullptr;
    int seed_len = 0, window = 1;
    float rp = 1.0f, fp = 0.0f;
    size_t max_new = 0, chunk = 1, depth = 1;
    int n_vocab = 0;
    uint32_t *hist = nullptr, *counts = nullptr, *counters = nullptr;
    uint64_t *best = nullptr;
    float *fpen = nullptr;
    uint32_t *h_ids = nullptr;  // pinned [depth][chunk], then [depth] one-launch error words
    std::vector<hipEvent_t> events;
    hipGraphExec_t g_first = nullptr, g_one = nullptr, g_chunk = nullptr;
    bool graphs_fused = false;  // the step form the graphs were captured with
    unsigned graphs_gen = 0;    // the session's cache layout (kv_gen) they were captured with
    unsigned graphs_cap = 0;    // and its cap_gen
};

namespace {

int check_model_cfg(const htr_text_config &c) {
    if (c.n_layer < 1 || c.dim < 32 || c.n_head < 1 || c.n_kv < 1 || c.n_ff < 32 || c.n_vocab < 1)
        return htr_fail("text config: %d layers, dim %d, %d / %d heads, ffn %d, vocab %d", c.n_layer, c.dim, c.n_head,
                        c.n_kv, c.n_ff, c.n_vocab);
    if (c.d_head != HEAD) return htr_fail("head dim %d: the attention kernels are written for 128", c.d_head);
    if (c.n_head % c.n_kv != 0) return htr_fail("%d q heads on %d kv heads", c.n_head, c.n_kv);
    const int qd = c.n_head * c.d_head;
    if (c.dim % 32 || c.n_ff % 32 || qd % 32)
        return htr_fail("dims %d / %d / %d: q8_0 rows must be whole blocks", c.dim, c.n_ff, qd);
    if (c.dim > 4096 || c.n_ff > 4096 || qd > 4096)
        return htr_fail("dims %d / %d / %d: the matvec kernels take K ≤ 4096", c.dim, c.n_ff, qd);
    return 0;
}

int upload_vec(htr_device *dev, const float *h, size_t n, float **out) {
    if (!h) return htr_fail("missing f32 tensor of %zu values", n);
    HTR_TRY(htr_dev_alloc(dev, n * 4, HTR_MEM_WEIGHTS, (void **)out));
    return htr_upload(dev, *out, h, n * 4);
}

int upload_w(htr_device *dev, const void *h, size_t rows, size_t cols, const char *what, htr_weight **out) {
    if (!h) return htr_fail("missing q8_0 tensor %s [%zu x %zu]", what, rows, cols);
    if (htr_weight_q8_0(dev, h, rows, cols, out) < 0) return htr_fail("%s: %s", what, htr_last_error());
    return 0;
}

// the F32 path's decode step (text.rs:555-576; its kernels stay the reference's on that path): rms_norm → q / k / v
// matvecs → qkv_post (per-head norms, RoPE, f16 KV store) → attention with the score scaled after its dot product
// (attn_scores.wgsl:38) → o matvec (+ residual) → rms_norm → gate and up matvecs → swiglu → down matvec (+ residual);
// the head as rms_norm + matvec (text.rs:655-658)
int record_step_f32(htr_session *s, hipStream_t st) {
    htr_text_model *m = s->m;
    htr_device *dev = s->dev;
    const htr_text_config &c = m->cfg;
    const int qd = c.n_head * HEAD, kvd = c.n_kv * HEAD;
    const float scale = 1.0f / sqrtf((float)HEAD);
    for (int li = 0; li < c.n_layer; li++) {
        const Layer &ly = m->layers[li];
        uint16_t *kc = s->kc + li * s->kv_layer, *vc = s->vc + li * s->kv_layer;
        HTR_TRY(launch_rms_norm(dev, st, s->x, ly.attn_norm, s->h, 1, c.dim, c.eps));
        const DmvMat q = {ly.q->q, ly.q->d, qd}, k = {ly.k->q, ly.k->d, kvd}, v = {ly.v->q, ly.v->d, kvd};
        HTR_TRY(launch_dmv(dev, st, DMV_PLAIN, &q, 1, c.dim, s->h, nullptr, 0.0f, s->qkv, 0));
        HTR_TRY(launch_dmv(dev, st, DMV_PLAIN, &k, 1, c.dim, s->h, nullptr, 0.0f, s->qkv + qd, 0));
        HTR_TRY(launch_dmv(dev, st, DMV_PLAIN, &v, 1, c.dim, s->h, nullptr, 0.0f, s->qkv + qd + kvd, 0));
        HTR_TRY(launch_qkv_post(dev, st, s->qkv, ly.q_norm, ly.k_norm, s->rope, c.n_head, c.n_kv, s->state, 0, s->kv_rows,
                                c.eps, kc, vc));
        HTR_TRY(launch_attn_decode(dev, st, s->qkv, kc, vc, c.n_head, c.n_kv, s->kv_rows, s->state, 0, scale, s->asc,
                                   s->attn, nullptr, true));
        const DmvMat o = {ly.o->q, ly.o->d, c.dim};
        HTR_TRY(launch_dmv(dev, st, DMV_PLAIN, &o, 1, qd, s->attn, nullptr, 0.0f, s->x, 1));
        HTR_TRY(launch_rms_norm(dev, st, s->x, ly.ffn_norm, s->h, 1, c.dim, c.eps));
        const DmvMat gm = {ly.gate->q, ly.gate->d, c.n_ff}, um = {ly.up->q, ly.up->d, c.n_ff};
        HTR_TRY(launch_dmv(dev, st, DMV_PLAIN, &gm, 1, c.dim, s->h, nullptr, 0.0f, s->g, 0));
        HTR_TRY(launch_dmv(dev, st, DMV_PLAIN, &um, 1, c.dim, s->h, nullptr, 0.0f, s->u, 0));
        HTR_TRY(launch_swiglu(dev, st, s->g, s->u, (size_t)c.n_ff));
        const DmvMat dn = {ly.down->q, ly.down->d, c.dim};
        HTR_TRY(launch_dmv(dev, st, DMV_PLAIN, &dn, 1, c.n_ff, s->g, nullptr, 0.0f, s->x, 1));
    }
    HTR_TRY(launch_rms_norm(dev, st, s->x, m->output_norm, s->h, 1, c.dim, c.eps));
    const DmvMat head = {m->tok_embd->q, m->tok_embd->d, c.n_vocab};
    return launch_dmv(dev, st, DMV_PLAIN, &head, 1, c.dim, s->h, nullptr, 0.0f, s->logits, 0);
}

// the one-launch step's arguments; with ca, the greedy choice of ca runs in the launch's tail
TokArgs token_args(htr_session *s, unsigned long long *prof, const ChooseArgs *ca) {
    const htr_text_config &c = s->m->cfg;
    TokArgs a{};
    a.layers = s->tl;
    a.n_layer = c.n_layer;
    a.n_ctx = s->kv_rows;
    a.n_vocab = c.n_vocab;
    a.emb_q = s->m->tok_embd->q;
    a.emb_d = s->m->tok_embd->d;
    a.tok = s->tok;
    a.state = s->state;
    a.rope = s->rope;
    a.eps = c.eps;
    a.scale = 1.0f / sqrtf((float)HEAD);
    a.xw = s->xw;
    a.seq = s->tseq;
    a.err = s->tseq + 1;
    a.x_out = s->x;
    a.out_norm = s->m->output_norm;
    a.logits = s->logits;
    if (ca) {
        a.choose = 1;
        a.hist = ca->hist;
        a.window = ca->window;
        a.rp = ca->rp;
        a.fp = ca->fp;
        a.counts = ca->counts;
        a.fpen = ca->fpen;
    }
    a.prof = prof;
    a.spin_ticks = s->spin_ticks;
    return a;
}

// the one-launch step's layer table: the model's planes and the session's caches (uploaded again when the cache
// grows; nothing reads it before the cache exists)
int token_step_table(htr_session *s) {
    if (!s->tl || !s->kc) return 0;
    htr_text_model *m = s->m;
    std::vector<TokLayer> tl(m->cfg.n_layer);
    for (int i = 0; i < m->cfg.n_layer; i++) {
        const Layer &l = m->layers[i];
        const htr_weight *w[7] = {l.q, l.k, l.v, l.o, l.gate, l.up, l.down};
        for (int k = 0; k < 7; k++) {
            tl[i].q[k] = w[k]->q;
            tl[i].d[k] = w[k]->d;
        }
        tl[i].attn_norm = l.attn_norm;
        tl[i].q_norm = l.q_norm;
        tl[i].k_norm = l.k_norm;
        tl[i].ffn_norm = l.ffn_norm;
        tl[i].kc = (_Float16 *)(s->kc + i * s->kv_layer);
        tl[i].vc = (_Float16 *)(s->vc + i * s->kv_layer);
    }
    return htr_upload(s->dev, s->tl, tl.data(), tl.size() * sizeof(TokLayer));
}

// the one-launch step's pieces for a session of the 1024 / 2048 / 3072 decoder on the f16 paths: the layer table, the
// exchange words (zero: no tag of a token), seq = 1, err = 0. Sets s->fused_why instead when the session cannot take
// it. The step's instance (keys a thread, chunk size) follows n_ctx, not the rows the cache holds.
int token_step_setup(htr_session *s) {
    htr_text_model *m = s->m;
    htr_device *dev = s->dev;
    const htr_text_config &c = m->cfg;
    if (m->compute != HTR_COMPUTE_F16) {
        s->fused_why = "the F32 path runs the reference's own kernel sequence";
        return 0;
    }
    if (!token_step_shape(c)) {
        s->fused_why = "the model is not the 1024 / 2048 / 3072 decoder (16 / 8 heads of 128, at most 42 layers, 256 "
                       "to 262144 ids)";
        return 0;
    }
    if (!token_step_fits(dev, s->n_ctx, &s->fused_why)) return 0;
    const int xr = token_step_xcds(dev, &s->fused_why);
    if (xr <= 0) return xr;
    HTR_TRY(htr_dev_alloc(dev, (size_t)c.n_layer * sizeof(TokLayer), HTR_MEM_WORK, (void **)&s->tl));
    HTR_TRY(token_step_table(s));
    const size_t xbytes = token_step_words() * 8;
    // zero, or 0xFF bytes under HTR_POISON=1: neither carries a token's tag (tags start at seq 1, and 0xFF…FF is no
    // exchange of any layer)
    HTR_TRY(htr_dev_alloc(dev, xbytes, HTR_MEM_WORK, (void **)&s->xw));
    HTR_TRY(htr_dev_alloc(dev, 64, HTR_MEM_WORK, (void **)&s->tseq));
    const uint32_t init[2] = {1, 0};
    HTR_TRY(htr_upload(dev, s->tseq, init, sizeof init));
    // a wait's limit: 0.2 s of the device's wall clock (a hand-over takes microseconds)
    int khz = 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev->ordinal) != hipSuccess || khz <= 0)
        khz = 100000;
    s->spin_default = s->spin_ticks = (long long)khz * 200;
    // HTR_FUSED_SPIN_US: another limit, in µs (tests of the error path set a tiny one: every wait then runs out)
    if (const char *e = getenv("HTR_FUSED_SPIN_US")) {
        const long long us = atoll(e);
        if (us > 0) s->spin_ticks = std::max(1LL, (long long)khz * us / 1000);
    }
    s->fused = true;
    return 0;
}

const char *const FELL_BACK_WHY = "a wait of the one-launch step ran past its limit (its 256 workgroups did not all run "
                                  "at once): the session went back to the per-kernel step";

// after one-launch steps ran (the stream synchronised): *failed = their err word was set. Then a workgroup that ran
// out of time may have started after workgroup 0 advanced seq and tagged its words with the next token's seq: seq
// skips that one as well, and err is cleared for the next launch
int token_step_err(htr_session *s, bool *failed) {
    *failed = false;
    if (!s->tl) return 0;
    uint32_t w[2];
    HTR_TRY(htr_download(s->dev, w, s->tseq, sizeof w));
    if (!w[1]) return 0;
    *failed = true;
    w[0] += 1;
    w[1] = 0;
    return htr_upload(s->dev, s->tseq, w, sizeof w);
}

// the session steps kernel by kernel from now on (its graphs of the one-launch step are dropped)
void fall_back(htr_session *s) {
    s->fused = false;
    s->fell_back = true;
    if (s->step_graph) {
        hipGraphExecDestroy(s->step_graph);
        s->step_graph = nullptr;
    }
}

// a measurement's one-launch step: its err word as an error
int token_step_check(htr_session *s) {
    bool failed = false;
    HTR_TRY(token_step_err(s, &failed));
    if (!failed) return 0;
    return htr_fail("decode step: a workgroup of the one-launch step waited past its limit (the 256 workgroups did not "
                    "all run at once); the step's logits and cache rows are invalid");
}

// one decode step on the session's stream: token s->tok at position state[0] → s->logits. The f16 paths' fused step
// (record_step, text.rs:540-552 + layers_fused), or the F32 path's (record_step_f32) for a model of that path.
// `only` (the in-graph timing of htr_session_profile_step) records just the kernels of the HTR_STEP_* classes it
// names; the decode records them all. ca: the choice that follows the step — the one-launch step runs it in its own
// tail (the caller then launches no choice kernel); the per-kernel step leaves it to the caller.
int record_step(htr_session *s, hipStream_t st, unsigned only = HTR_STEP_ALL, const ChooseArgs *ca = nullptr) {
    htr_text_model *m = s->m;
    htr_device *dev = s->dev;
    const htr_text_config &c = m->cfg;
    const int qd = c.n_head * HEAD, kvd = c.n_kv * HEAD;
    const float scale = 1.0f / sqrtf((float)HEAD);
    if (s->fused && only == HTR_STEP_ALL)  // embed, the layers, the LM head (and the choice of ca) in one launch
        return launch_decode_token(dev, st, s->n_ctx, token_args(s, nullptr, ca));
    if (only & HTR_STEP_EMBED) HTR_TRY(launch_embed(dev, st, m->tok_embd, s->tok, 1, s->x));
    if (m->compute == HTR_COMPUTE_F32) return record_step_f32(s, st);
    for (int li = 0; li < c.n_layer; li++) {
        const Layer &ly = m->layers[li];
        uint16_t *kc = s->kc + li * s->kv_layer, *vc = s->vc + li * s->kv_layer;
        DmvMat qkv[3] = {{ly.q->q, ly.q->d, qd}, {ly.k->q, ly.k->d, kvd}, {ly.v->q, ly.v->d, kvd}};
        if (only & HTR_STEP_QKV)
            HTR_TRY(launch_dmv(dev, st, DMV_QKV, qkv, 3, c.dim, s->x, ly.attn_norm, c.eps, s->qkv, 0));
        const AttnFuse fz{ly.q_norm, ly.k_norm, s->rope, c.eps, c.n_head, (_Float16 *)kc, (_Float16 *)vc};
        if (only & HTR_STEP_ATTENTION)
            HTR_TRY(launch_attn_decode(dev, st, s->qkv, kc, vc, c.n_head, c.n_kv, s->kv_rows, s->state, 0, scale,
                                       s->asc, s->attn, &fz));
        DmvMat o = {ly.o->q, ly.o->d, c.dim};
        if (only & HTR_STEP_O) HTR_TRY(launch_dmv(dev, st, DMV_PLAIN, &o, 1, qd, s->attn, nullptr, 0.0f, s->x, 1));
        DmvMat gu[2] = {{ly.gate->q, ly.gate->d, c.n_ff}, {ly.up->q, ly.up->d, c.n_ff}};
        if (only & HTR_STEP_FFN)
            HTR_TRY(launch_dmv(dev, st, DMV_FFN, gu, 2, c.dim, s->x, ly.ffn_norm, c.eps, s->g, 0));
        DmvMat dn = {ly.down->q, ly.down->d, c.dim};
        if (only & HTR_STEP_DOWN)
            HTR_TRY(launch_dmv(dev, st, DMV_PLAIN, &dn, 1, c.n_ff, s->g, nullptr, 0.0f, s->x, 1));
    }
    DmvMat head = {m->tok_embd->q, m->tok_embd->d, c.n_vocab};
    if (!(only & HTR_STEP_HEAD)) return 0;
    return launch_dmv(dev, st, DMV_NORM, &head, 1, c.dim, s->x, m->output_norm, c.eps, s->logits, 0);
}

ChooseArgs choice_args(htr_choice *ch, bool advance) {
    htr_session *s = ch->s;
    ChooseArgs a{};
    a.logits = s->logits;
    a.n_vocab = ch->n_vocab;
    a.hist = ch->hist;
    a.hist_stride = 0;
    a.len_dev = s->state + 1;
    a.window = ch->window;
    a.rp = ch->rp;
    a.fp = ch->fp;
    a.counts = ch->counts;
    a.fpen = ch->fpen;
    a.tok = s->tok;
    a.advance = advance ? s->state : nullptr;
    a.best = ch->best;
    a.counters = ch->counters;
    a.rows = 1;
    return a;
}

// [step?] then [choice?]: on the one-launch step the choice runs in the step's launch
int record_with_choice(htr_session *s, htr_choice *ch, bool with_step, hipStream_t st) {
    if (with_step && ch && s->fused) {
        const ChooseArgs ca = choice_args(ch, true);
        return record_step(s, st, HTR_STEP_ALL, &ca);
    }
    if (with_step) HTR_TRY(record_step(s, st));
    return ch ? launch_choose(s->dev, st, choice_args(ch, with_step)) : 0;
}

// capture `n` repetitions of [step? + choice] into an executable graph
int capture(htr_session *s, htr_choice *ch, int n, bool with_step, hipGraphExec_t *out) {
    htr_device *dev = s->dev;
    hipStream_t st = dev->stream;
    HTR_TRY(htr_hip(dev, hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture"));
    int rc = 0;
    for (int i = 0; i < n && rc == 0; i++) rc = record_with_choice(s, ch, with_step, st);
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(st, &graph);
    if (rc < 0) {
        if (graph) hipGraphDestroy(graph);
        return rc;
    }
    HTR_TRY(htr_hip(dev, e, "hipStreamEndCapture"));
    e = hipGraphInstantiate(out, graph, nullptr, nullptr, 0);
    hipGraphDestroy(graph);
    return htr_hip(dev, e, "hipGraphInstantiate");
}

// `n` repetitions of [step? + choice]: the captured graph `*g` (captured on first use) replayed, or — with graphs
// switched off on the device (HTR_GRAPHS=0: profilers that cannot follow stream capture) — the same kernels
// launched one by one on the stream
int run_steps(htr_session *s, htr_choice *ch, int n, bool with_step, hipGraphExec_t *g) {
    htr_device *dev = s->dev;
    hipStream_t st = dev->stream;
    if (!dev->use_graphs) {
        for (int i = 0; i < n; i++) HTR_TRY(record_with_choice(s, ch, with_step, st));
        return 0;
    }
    if (!*g) HTR_TRY(capture(s, ch, n, with_step, g));
    return htr_hip(dev, hipGraphLaunch(*g, st), "hipGraphLaunch");
}

int set_state(htr_session *s, int pos, int len) {
    int v[2] = {pos, len};
    // pinned staging: the copy reads it when the stream gets there, so wait for it before the staging is reused
    memcpy(s->dev->pinned, v, sizeof v);
    HTR_TRY(htr_hip(s->dev, hipMemcpyAsync(s->state, s->dev->pinned, sizeof v, hipMemcpyHostToDevice, s->dev->stream),
                    "state upload"));
    return htr_hip(s->dev, hipStreamSynchronize(s->dev->stream), "state upload sync");
}

// Session::reserve (text.rs:287-327): KV cache rows for positions 0 … rows − 1. When the cache holds fewer it grows to
// rows + kv_grow (at most n_ctx): the launches in flight end first (they read and write the old cache), the rows held
// so far move into the larger cache by one strided copy per cache (n_layer · n_kv runs of kv_rows rows each, the
// head-major layout's stride widening from the old row count to the new), the old cache is freed. What holds the
// layout follows: the one-launch step's layer table, the captured CPU-choice step (dropped here), a choice's graphs
// (dropped on their next use, by kv_gen). The attention's chunks and the one-launch step's instance follow n_ctx, not
// the rows held, so a grown cache computes what a presized one does, bit for bit. The growth's peak is the old cache
// and the new one together (the reference replaces 4 layers at a time, for a phone's memory).
int reserve(htr_session *s, size_t rows) {
    if (rows <= (size_t)s->kv_rows) return 0;
    if (rows > (size_t)s->n_ctx) return htr_fail("%zu KV cache rows asked, the session holds at most %d", rows, s->n_ctx);
    htr_device *dev = s->dev;
    const htr_text_config &c = s->m->cfg;
    const size_t new_rows = std::min(rows + (size_t)s->kv_grow, (size_t)s->n_ctx);
    const size_t runs = (size_t)c.n_layer * c.n_kv, row_bytes = (size_t)HEAD * 2;
    const size_t bytes = runs * new_rows * row_bytes;
    HTR_TRY(htr_sync(dev));
    uint16_t *nk = nullptr, *nv = nullptr;
    int rc = htr_dev_alloc(dev, bytes, HTR_MEM_KV_CACHE, (void **)&nk);
    if (rc == 0) rc = htr_dev_alloc(dev, bytes, HTR_MEM_KV_CACHE, (void **)&nv);
    if (rc == 0 && s->kv_rows > 0) {
        const size_t held = (size_t)s->kv_rows * row_bytes;  // a run's bytes in the old cache: its pitch and width
        rc = htr_hip(dev, hipMemcpy2DAsync(nk, new_rows * row_bytes, s->kc, held, held, runs, hipMemcpyDeviceToDevice,
                                           dev->stream), "KV cache growth (k)");
        if (rc == 0)
            rc = htr_hip(dev, hipMemcpy2DAsync(nv, new_rows * row_bytes, s->vc, held, held, runs,
                                               hipMemcpyDeviceToDevice, dev->stream), "KV cache growth (v)");
        if (rc == 0) rc = htr_sync(dev);
    }
    if (rc < 0) {
        for (void *p : {(void *)nk, (void *)nv})
            if (p) htr_dev_free(dev, p);
        return rc;
    }
    for (void *p : {(void *)s->kc, (void *)s->vc})
        if (p) htr_dev_free(dev, p);
    s->kc = nk;
    s->vc = nv;
    s->kv_rows = (int)new_rows;
    s->kv_layer = (size_t)c.n_kv * new_rows * HEAD;
    s->kv_gen += 1;
    if (s->step_graph) {
        hipGraphExecDestroy(s->step_graph);
        s->step_graph = nullptr;
    }
    return token_step_table(s);
}

// a choice's graphs hold the step form and the cache layout of their capture: dropped when either changed
void drop_stale_graphs(htr_choice *ch) {
    const htr_session *s = ch->s;
    if (ch->graphs_fused == s->fused && ch->graphs_gen == s->kv_gen && ch->graphs_cap == s->cap_gen) return;
    for (hipGraphExec_t *g : {&ch->g_first, &ch->g_one, &ch->g_chunk})
        if (*g) {
            hipGraphExecDestroy(*g);
            *g = nullptr;
        }
    ch->graphs_fused = s->fused;
    ch->graphs_gen = s->kv_gen;
    ch->graphs_cap = s->cap_gen;
}

}  // namespace

// ---- model ----------------------------------------------------------------------------------------------------------

extern "C" int htr_text_model_free(htr_text_model *m) {
    if (!m) return 0;
    htr_device *dev = m->dev;
    for (Layer &l : m->layers) {
        for (htr_weight *w : {l.q, l.k, l.v, l.o, l.gate, l.up, l.down}) htr_weight_free(w);
        for (float *p : {l.attn_norm, l.q_norm, l.k_norm, l.ffn_norm})
            if (p) htr_dev_free(dev, p);
    }
    htr_weight_free(m->tok_embd);
    if (m->output_norm) htr_dev_free(dev, m->output_norm);
    delete m;
    return 0;
}

namespace {

// where a model's tensors come from: host arrays (htr_text_model_create) or a GGUF file (htr_text_model_load_gguf).
// layer < 0: the model-level tensors (token_embd, output_norm)
struct TensorFeed {
    virtual int q8(int layer, const char *kind, size_t rows, size_t cols, htr_weight **out) = 0;
    virtual int vec(int layer, const char *kind, size_t n, float **out) = 0;
    virtual ~TensorFeed() = default;
};

struct ArrayFeed : TensorFeed {
    const htr_layer_tensors *layers;
    const void *tok_embd;
    const float *output_norm;
    ArrayFeed(const htr_layer_tensors *l, const void *te, const float *on) : layers(l), tok_embd(te), output_norm(on) {}
    int q8(int layer, const char *kind, size_t rows, size_t cols, htr_weight **out) override {
        const void *h = tok_embd;
        if (layer >= 0) {
            const htr_layer_tensors &t = layers[layer];
            const std::string k = kind;
            h = k == "attn_q" ? t.q : k == "attn_k" ? t.k : k == "attn_v" ? t.v : k == "attn_output" ? t.o
                : k == "ffn_gate" ? t.gate : k == "ffn_up" ? t.up : t.down;
        }
        return upload_w(dev_, h, rows, cols, kind, out);
    }
    int vec(int layer, const char *kind, size_t n, float **out) override {
        const float *h = output_norm;
        if (layer >= 0) {
            const htr_layer_tensors &t = layers[layer];
            const std::string k = kind;
            h = k == "attn_norm" ? t.attn_norm : k == "attn_q_norm" ? t.q_norm : k == "attn_k_norm" ? t.k_norm
                : t.ffn_norm;
        }
        return upload_vec(dev_, h, n, out);
    }
    htr_device *dev_ = nullptr;
};

struct GgufFeed : TensorFeed {
    htr_gguf *g;
    GgufStager sg;
    explicit GgufFeed(htr_gguf *gg) : g(gg) {}
    static std::string name(int layer, const char *kind) {
        return layer < 0 ? std::string(kind) + ".weight" : "blk." + std::to_string(layer) + "." + kind + ".weight";
    }
    int q8(int layer, const char *kind, size_t rows, size_t cols, htr_weight **out) override {
        const GgufTensor *t;
        HTR_TRY(gguf_find(g, name(layer, kind).c_str(), &t));
        return gguf_upload_q8_0(sg, g, *t, rows, cols, out);
    }
    int vec(int layer, const char *kind, size_t n, float **out) override {
        const GgufTensor *t;
        HTR_TRY(gguf_find(g, name(layer, kind).c_str(), &t));
        return gguf_upload_f32(sg, g, *t, n, out);
    }
};

// TextModel::load's body (text.rs:332-375) over either feed; the f16 planes of the f16 path made after the upload
int build_model(htr_device *dev, const htr_text_config &c, TensorFeed &feed, htr_text_model **out) {
    HTR_TRY(check_model_cfg(c));
    const size_t d = c.dim, f = c.n_ff, qd = (size_t)c.n_head * HEAD, kvd = (size_t)c.n_kv * HEAD;
    auto *m = new htr_text_model;
    m->dev = dev;
    m->cfg = c;
    m->layers.resize(c.n_layer);
    int rc = 0;
    for (int i = 0; i < c.n_layer && rc == 0; i++) {
        Layer &l = m->layers[i];
        rc = feed.vec(i, "attn_norm", d, &l.attn_norm);
        if (rc == 0) rc = feed.q8(i, "attn_q", qd, d, &l.q);
        if (rc == 0) rc = feed.q8(i, "attn_k", kvd, d, &l.k);
        if (rc == 0) rc = feed.q8(i, "attn_v", kvd, d, &l.v);
        if (rc == 0) rc = feed.q8(i, "attn_output", d, qd, &l.o);
        if (rc == 0) rc = feed.vec(i, "attn_q_norm", HEAD, &l.q_norm);
        if (rc == 0) rc = feed.vec(i, "attn_k_norm", HEAD, &l.k_norm);
        if (rc == 0) rc = feed.vec(i, "ffn_norm", d, &l.ffn_norm);
        if (rc == 0) rc = feed.q8(i, "ffn_gate", f, d, &l.gate);
        if (rc == 0) rc = feed.q8(i, "ffn_up", f, d, &l.up);
        if (rc == 0) rc = feed.q8(i, "ffn_down", d, f, &l.down);
        if (rc < 0) rc = htr_fail("blk.%d: %s", i, std::string(htr_last_error()).c_str());
    }
    if (rc == 0) rc = feed.q8(-1, "token_embd", c.n_vocab, d, &m->tok_embd);
    if (rc == 0) rc = feed.vec(-1, "output_norm", d, &m->output_norm);
    // the f16 compute path's prefill GEMMs read f16(q·d) planes (matmul_coop_q8_0 rounds the dequantised W to f16 as
    // it loads a tile); the MFMA kernels take rows in multiples of 64 (the FFN's 128), else the tiled kernel rounds
    m->compute = dev->compute;
    m->mfma16 = m->compute == HTR_COMPUTE_F16 && d % 64 == 0 && f % 128 == 0;
    for (int i = 0; i < c.n_layer && rc == 0 && m->mfma16; i++) {
        Layer &l = m->layers[i];
        for (htr_weight *w : {l.q, l.k, l.v, l.o, l.gate, l.up, l.down})
            if (rc == 0) rc = weight_attach_f16(dev, dev->stream, w);
    }
    if (rc == 0) rc = htr_sync(dev);
    if (rc < 0) {
        std::string keep = htr_last_error();
        htr_sync(dev);  // nothing in flight still reads the staging the caller frees next
        htr_text_model_free(m);
        return htr_fail("%s", keep.c_str());
    }
    *out = m;
    return 0;
}

// TextConfig::from_gguf (text.rs:43-76)
int config_from_gguf(htr_gguf *g, htr_text_config *c) {
    std::string arch;
    HTR_TRY(gguf_meta_str(g, "general.architecture", &arch));
    if (arch != "qwen3") return htr_fail("architecture \"%s\": this engine runs qwen3 only", arch.c_str());
    auto u = [&](const char *k, int *out) -> int {
        uint32_t v;
        HTR_TRY(gguf_meta_u32(g, (std::string("qwen3.") + k).c_str(), &v));
        if (v > (uint32_t)INT32_MAX) return htr_fail("qwen3.%s = %u", k, v);
        *out = (int)v;
        return 0;
    };
    int d_head, v_len;
    HTR_TRY(u("attention.key_length", &d_head));
    HTR_TRY(u("attention.value_length", &v_len));
    if (d_head != HEAD || v_len != HEAD) return htr_fail("head dim %d: the attention kernels are written for 128", d_head);
    c->d_head = d_head;
    HTR_TRY(u("attention.head_count", &c->n_head));
    HTR_TRY(u("attention.head_count_kv", &c->n_kv));
    if (c->n_kv == 0 || c->n_head % c->n_kv != 0) return htr_fail("%d q heads on %d kv heads", c->n_head, c->n_kv);
    if (gguf_has_key(g, "qwen3.rope.scaling.type") || gguf_has_key(g, "qwen3.rope.dimension_count"))
        return htr_fail("rope scaling / partial rope in the GGUF: not part of this engine's graph");
    const GgufTensor *tok;
    HTR_TRY(gguf_find(g, "token_embd.weight", &tok));
    HTR_TRY(u("block_count", &c->n_layer));
    HTR_TRY(u("embedding_length", &c->dim));
    HTR_TRY(u("feed_forward_length", &c->n_ff));
    HTR_TRY(gguf_meta_f32(g, "qwen3.attention.layer_norm_rms_epsilon", &c->eps));
    HTR_TRY(gguf_meta_f32(g, "qwen3.rope.freq_base", &c->rope_base));
    const uint64_t nv = tok->shape[tok->n_dims - 1];
    if (nv > (uint64_t)INT32_MAX) return htr_fail("token_embd: %llu rows", (unsigned long long)nv);
    c->n_vocab = (int)nv;
    HTR_TRY(u("context_length", &c->n_ctx_train));
    return 0;
}

}  // namespace

extern "C" int htr_text_model_create(htr_device *dev, const htr_text_config *cfg, const void *tok_embd,
                                     const float *output_norm, const htr_layer_tensors *layers, htr_text_model **out) {
    HTR_TRY(htr_check_alive(dev));
    if (!cfg || !layers || !out) return htr_fail("htr_text_model_create: null argument");
    ArrayFeed feed(layers, tok_embd, output_norm);
    feed.dev_ = dev;
    return build_model(dev, *cfg, feed, out);
}

// text.rs:332-375 TextModel::load
extern "C" int htr_text_model_load_gguf(htr_device *dev, htr_gguf *g, htr_text_model **out) {
    HTR_TRY(htr_check_alive(dev));
    if (!g || !out) return htr_fail("htr_text_model_load_gguf: null argument");
    htr_text_config c{};
    HTR_TRY(config_from_gguf(g, &c));
    for (int i = 0; i < c.n_layer; i++) {
        for (const char *absent : {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"}) {
            const std::string b = "blk." + std::to_string(i) + "." + absent + ".bias";
            if (gguf_has(g, b.c_str())) return htr_fail("%s is in the GGUF but not part of this engine's graph", b.c_str());
        }
        if (gguf_has(g, ("blk." + std::to_string(i) + ".attn_qkv.weight").c_str()))
            return htr_fail("blk.%d: a fused attn_qkv — this engine reads separate q / k / v", i);
    }
    if (gguf_has(g, "output.weight")) return htr_fail("output.weight is in the GGUF: this engine ties the output to token_embd");
    GgufFeed feed(g);
    HTR_TRY(feed.sg.init(dev));
    return build_model(dev, c, feed, out);
}

extern "C" int htr_text_model_config(htr_text_model *m, htr_text_config *out) {
    if (!m || !out) return htr_fail("htr_text_model_config: null argument");
    *out = m->cfg;
    return 0;
}

// ---- session --------------------------------------------------------------------------------------------------------

extern "C" int htr_session_free(htr_session *s) {
    if (!s) return 0;
    htr_device *dev = s->dev;
    if (s->step_graph) hipGraphExecDestroy(s->step_graph);
    for (void *p : {(void *)s->kc, (void *)s->vc, (void *)s->rope, (void *)s->x, (void *)s->qkv, (void *)s->attn,
                    (void *)s->g, (void *)s->logits, (void *)s->tok, (void *)s->state, (void *)s->asc.part,
                    (void *)s->asc.counters, s->pre, s->kvb, (void *)s->h, (void *)s->u, (void *)s->tl, (void *)s->xw,
                    (void *)s->tseq})
        if (p) htr_dev_free(dev, p);
    delete s;
    return 0;
}

namespace {

// TextModel::session_grown (text.rs:389-434): a session for n_ctx positions whose KV cache grows by kv_grow rows past
// the need (reserve); `presize`: the whole cache at once, here
int session_new(htr_text_model *m, size_t n_ctx, size_t kv_grow, bool presize, htr_session **out) {
    if (!m || !out) return htr_fail("htr_session_create: null argument");
    if (kv_grow == 0) return htr_fail("a KV cache growth of 0 rows");
    htr_device *dev = m->dev;
    HTR_TRY(htr_check_alive(dev));
    const htr_text_config &c = m->cfg;
    if (c.n_head != 2 * c.n_kv)
        return htr_fail("%d q heads on %d kv heads: the split decode attention is written for groups of 2", c.n_head,
                        c.n_kv);
    if (n_ctx < 1 || (c.n_ctx_train > 0 && n_ctx > (size_t)c.n_ctx_train))
        return htr_fail("%zu positions asked, the model was trained on %d", n_ctx, c.n_ctx_train);
    if (n_ctx > 65536) return htr_fail("%zu positions: the decode attention takes at most 65536", n_ctx);
    auto *s = new htr_session;
    s->m = m;
    s->dev = dev;
    s->n_ctx = (int)n_ctx;
    s->kv_grow = (int)std::min(kv_grow, n_ctx);
    const size_t qd = (size_t)c.n_head * HEAD, kvd = (size_t)c.n_kv * HEAD;
    s->asc.chunk = attn_chunk_for(s->n_ctx);
    s->asc.max_chunk = (s->n_ctx + s->asc.chunk - 1) / s->asc.chunk;
    std::vector<float> rope = rope_table(c.rope_base, HEAD, s->n_ctx);
    int rc = htr_dev_alloc(dev, rope.size() * 4, HTR_MEM_WORK, (void **)&s->rope);
    if (rc == 0) rc = htr_upload(dev, s->rope, rope.data(), rope.size() * 4);
    if (rc == 0) rc = htr_dev_alloc(dev, (size_t)c.dim * 4, HTR_MEM_WORK, (void **)&s->x);
    if (rc == 0) rc = htr_dev_alloc(dev, (qd + 2 * kvd) * 4, HTR_MEM_WORK, (void **)&s->qkv);
    if (rc == 0) rc = htr_dev_alloc(dev, qd * 4, HTR_MEM_WORK, (void **)&s->attn);
    if (rc == 0) rc = htr_dev_alloc(dev, (size_t)c.n_ff * 4, HTR_MEM_WORK, (void **)&s->g);
    if (rc == 0 && m->compute == HTR_COMPUTE_F32) rc = htr_dev_alloc(dev, (size_t)c.dim * 4, HTR_MEM_WORK, (void **)&s->h);
    if (rc == 0 && m->compute == HTR_COMPUTE_F32) rc = htr_dev_alloc(dev, (size_t)c.n_ff * 4, HTR_MEM_WORK, (void **)&s->u);
    if (rc == 0) rc = htr_dev_alloc(dev, (size_t)c.n_vocab * 4, HTR_MEM_WORK, (void **)&s->logits);
    if (rc == 0) rc = htr_dev_alloc(dev, 64, HTR_MEM_WORK, (void **)&s->tok);
    if (rc == 0) rc = htr_dev_alloc(dev, 64, HTR_MEM_WORK, (void **)&s->state);
    if (rc == 0)
        rc = htr_dev_alloc(dev, attn_part_bytes(c.n_head, s->asc.max_chunk), HTR_MEM_WORK, (void **)&s->asc.part);
    if (rc == 0) rc = htr_dev_alloc_zero(dev, attn_counter_bytes(c.n_kv), HTR_MEM_WORK, (void **)&s->asc.counters);
    if (rc == 0) rc = token_step_setup(s);
    if (rc == 0 && presize) rc = reserve(s, n_ctx);
    if (rc == 0 && s->fused) {
        // HTR_FUSED_STEP=0 keeps the per-kernel step (A/B timing); htr_session_set_fused_step switches per session
        const char *env = getenv("HTR_FUSED_STEP");
        if (env && env[0] == '0') s->fused = false;
    }
    if (rc == 0) rc = htr_sync(dev);
    if (rc < 0) {
        std::string keep = htr_last_error();
        htr_session_free(s);
        return htr_fail("%s", keep.c_str());
    }
    *out = s;
    return 0;
}

}  // namespace

extern "C" int htr_session_create(htr_text_model *m, size_t n_ctx, htr_session **out) {
    return session_new(m, n_ctx, n_ctx, true, out);
}

extern "C" int htr_session_create_grown(htr_text_model *m, size_t n_ctx, size_t kv_grow, htr_session **out) {
    return session_new(m, n_ctx, kv_grow, false, out);
}

extern "C" int htr_session_kv_rows(htr_session *s, size_t *out) {
    if (!s || !out) return htr_fail("htr_session_kv_rows: null argument");
    *out = (size_t)s->kv_rows;
    return 0;
}

extern "C" int htr_session_n_past(htr_session *s, size_t *out) {
    if (!s || !out) return htr_fail("htr_session_n_past: null argument");
    *out = (size_t)s->n_past;
    return 0;
}

extern "C" int htr_session_logits(htr_session *s, float *h_logits) {
    if (!s || !h_logits) return htr_fail("htr_session_logits: null argument");
    return htr_download(s->dev, h_logits, s->logits, (size_t)s->m->cfg.n_vocab * 4);
}

int session_n_vocab(const htr_session *s) { return s->m->cfg.n_vocab; }

extern "C" int htr_session_kv_cache(htr_session *s, htr_kv_view *out) {
    if (!s || !out) return htr_fail("htr_session_kv_cache: null argument");
    const htr_text_config &c = s->m->cfg;
    out->d_k = s->kc;
    out->d_v = s->vc;
    out->n_layer = c.n_layer;
    out->n_kv = c.n_kv;
    out->n_ctx = s->kv_rows;
    out->d_head = HEAD;
    out->layer_stride = s->kv_layer;
    return 0;
}

extern "C" int htr_session_rewind(htr_session *s, size_t n_past) {
    if (!s) return htr_fail("htr_session_rewind: null session");
    if (n_past > (size_t)s->n_past) return htr_fail("rewind to %zu: the session is at %d", n_past, s->n_past);
    s->n_past = (int)n_past;
    return 0;
}

extern "C" int htr_session_set_fused_step(htr_session *s, int on) {
    if (!s) return htr_fail("htr_session_set_fused_step: null session");
    if (on && !s->tl) return htr_fail("the one-launch decode step is not available: %s", s->fused_why);
    if (s->fused != (on != 0) && s->step_graph) {  // captured with the other step form
        hipGraphExecDestroy(s->step_graph);
        s->step_graph = nullptr;
    }
    s->fused = on != 0;
    if (on) s->fell_back = false;
    return 0;
}

extern "C" int htr_session_fused_step(htr_session *s, int *on, const char **why_not) {
    if (!s || !on) return htr_fail("htr_session_fused_step: null argument");
    *on = s->fused ? 1 : 0;
    if (why_not) *why_not = !s->tl ? s->fused_why : (!s->fused && s->fell_back) ? FELL_BACK_WHY : nullptr;
    return 0;
}

extern "C" int htr_session_set_wait_limit(htr_session *s, double us) {
    if (!s) return htr_fail("htr_session_set_wait_limit: null session");
    if (!s->tl) return htr_fail("the one-launch decode step is not available: %s", s->fused_why);
    int khz = 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, s->dev->ordinal) != hipSuccess || khz <= 0)
        khz = 100000;
    s->spin_ticks = us > 0.0 ? std::max(1LL, (long long)(us * khz / 1000.0)) : s->spin_default;
    s->cap_gen += 1;  // the launches recorded from now on carry the new limit
    if (s->step_graph) {
        hipGraphExecDestroy(s->step_graph);
        s->step_graph = nullptr;
    }
    return 0;
}

// one one-launch step at the session's position (not advanced; its KV row is written there), timed from inside:
// workgroup 0's wall-clock stamps, as microseconds after the first (after the embed): per layer 12 — the input of A
// (qkv) taken, A's output written, B's input (the KV head's q / k / v rows) taken, B's partials written, C's partials
// taken, C's output written, D's input taken, D's output written, E's, E's, F's, F's
extern "C" int htr_session_profile_fused_step(htr_session *s, int32_t token, double *us, int n) {
    if (!s || !us) return htr_fail("htr_session_profile_fused_step: null argument");
    htr_device *dev = s->dev;
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(htr_check_not_capturing(dev, "htr_session_profile_fused_step"));
    if (!s->tl) return htr_fail("the one-launch decode step is not available: %s", s->fused_why);
    const int n_stamp = token_step_stamps(s->m->cfg.n_layer);
    if (n != n_stamp) return htr_fail("htr_session_profile_fused_step: %d stamps asked, the step makes %d", n, n_stamp);
    if (s->n_past >= s->n_ctx) return htr_fail("position %d: the session holds %d", s->n_past, s->n_ctx);
    if (token < 0 || token >= s->m->cfg.n_vocab) return htr_fail("token %d is outside the vocabulary", token);
    HTR_TRY(reserve(s, (size_t)s->n_past + 1));
    uint32_t t = (uint32_t)token;
    HTR_TRY(htr_upload(dev, s->tok, &t, 4));
    HTR_TRY(set_state(s, s->n_past, 0));
    unsigned long long *prof = nullptr;
    HTR_TRY(htr_dev_alloc(dev, (size_t)n_stamp * 8, HTR_MEM_WORK, (void **)&prof));
    int rc = launch_decode_token(dev, dev->stream, s->n_ctx, token_args(s, prof, nullptr));
    if (rc == 0) rc = htr_sync(dev);
    if (rc == 0) rc = token_step_check(s);
    std::vector<unsigned long long> st(n_stamp);
    if (rc == 0) rc = htr_download(dev, st.data(), prof, (size_t)n_stamp * 8);
    htr_dev_free(dev, prof);
    if (rc < 0) return rc;
    int khz = 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev->ordinal) != hipSuccess || khz <= 0)
        khz = 100000;
    for (int i = 0; i < n_stamp; i++) us[i] = (double)(long long)(st[i] - st[0]) * 1000.0 / (double)khz;
    return 0;
}

// text.rs:437-521
extern "C" int htr_prefill(htr_session *s, const int32_t *ids, size_t n, float *h_logits) {
    if (!s || !ids) return htr_fail("htr_prefill: null argument");
    htr_device *dev = s->dev;
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(htr_check_not_capturing(dev, "htr_prefill"));
    htr_text_model *m = s->m;
    const htr_text_config &c = m->cfg;
    if (n == 0) return htr_fail("empty prompt");
    if ((size_t)s->n_past + n > (size_t)s->n_ctx)
        return htr_fail("%d + %zu positions overflow the session's %d", s->n_past, n, s->n_ctx);
    std::vector<uint32_t> tok(n);
    for (size_t i = 0; i < n; i++) {
        if (ids[i] < 0 || ids[i] >= c.n_vocab) return htr_fail("token %d is outside the vocabulary", ids[i]);
        tok[i] = (uint32_t)ids[i];
    }
    HTR_TRY(reserve(s, (size_t)s->n_past + n));
    const int l = (int)n, d = c.dim, f = c.n_ff, qd = c.n_head * HEAD, kvd = c.n_kv * HEAD;
    const int pos0 = s->n_past;
    hipStream_t st = dev->stream;
    // the row buffers, grown on demand and kept by the session (a prefill is often followed by more)
    const size_t per_row = 4 * ((size_t)2 * d + 2 * (size_t)qd + 2 * (size_t)kvd + 2 * (size_t)f) + 16;
    int rc = 0;
    if (n > s->pre_cap) {
        if (s->pre) htr_dev_free(dev, s->pre);
        s->pre = nullptr;
        s->pre_cap = 0;
        rc = htr_dev_alloc(dev, n * per_row, HTR_MEM_WORK, &s->pre);
        if (rc == 0) s->pre_cap = n;
    }
    const size_t kvb_need = attn_causal_block_bytes(c.n_kv, pos0 + l);
    if (rc == 0 && kvb_need > s->kvb_bytes) {
        if (s->kvb) htr_dev_free(dev, s->kvb);
        s->kvb = nullptr;
        s->kvb_bytes = 0;
        rc = htr_dev_alloc(dev, kvb_need, HTR_MEM_WORK, &s->kvb);
        if (rc == 0) s->kvb_bytes = kvb_need;
    }
    uint32_t *d_tok = nullptr;
    float *x = nullptr, *h = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *a = nullptr, *g = nullptr,
          *u = nullptr;
    if (rc == 0) {
        float *p = (float *)s->pre;
        const size_t cap = s->pre_cap;
        x = p, p += cap * d;
        h = p, p += cap * d;
        q = p, p += cap * qd;
        k = p, p += cap * kvd;
        v = p, p += cap * kvd;
        a = p, p += cap * qd;
        g = p, p += cap * f;
        u = p, p += cap * f;
        d_tok = (uint32_t *)p;
        rc = htr_upload(dev, d_tok, tok.data(), n * 4);
    }
    const float scale = 1.0f / sqrtf((float)HEAD);
    // the f16 path on the matrix cores: the GEMM inputs are written as f16 — the values matmul_coop_q8_0's tiles hold
    // (h, the attention output and g in the first halves of their f32 rows' space); the FFN's first GEMM fuses SwiGLU
    _Float16 *h16 = (_Float16 *)h, *a16 = (_Float16 *)a, *g16 = (_Float16 *)g;
    if (rc == 0) rc = launch_embed(dev, st, m->tok_embd, d_tok, l, x);
    // each residual GEMM also writes the next RMS norm's f16 rows (inside its K-split reduction where it splits)
    if (rc == 0 && m->mfma16) rc = launch_rms_norm_f16(dev, st, x, m->layers[0].attn_norm, h16, l, d, c.eps);
    for (int li = 0; li < c.n_layer && rc == 0 && m->mfma16; li++) {
        const Layer &ly = m->layers[li];
        uint16_t *kc = s->kc + li * s->kv_layer, *vc = s->vc + li * s->kv_layer;
        rc = launch_gemm_f16_qkv(dev, st, h16, l, ly.q, ly.k, ly.v, q, k, v);
        if (rc == 0)
            rc = launch_qk_norm_rope_rows(dev, st, q, k, v, ly.q_norm, ly.k_norm, s->rope, l, c.n_head, c.n_kv, pos0,
                                          s->kv_rows, c.eps, kc, vc);
        if (rc == 0)
            rc = launch_attn_causal(dev, st, q, kc, vc, l, pos0, c.n_head, c.n_kv, s->kv_rows, scale, s->kvb, nullptr,
                                    a16);
        if (rc == 0) rc = launch_gemm_f16_acc_norm(dev, st, a16, l, ly.o, x, ly.ffn_norm, c.eps, h16);
        if (rc == 0) rc = launch_gemm_f16(dev, st, GEMM_FFN, h16, l, ly.gate, ly.up, nullptr, g16, 1.0f);
        if (rc == 0 && li + 1 < c.n_layer)
            rc = launch_gemm_f16_acc_norm(dev, st, g16, l, ly.down, x, m->layers[li + 1].attn_norm, c.eps, h16);
        else if (rc == 0)
            rc = launch_gemm_f16(dev, st, GEMM_ACC, g16, l, ly.down, nullptr, x, nullptr, 1.0f);
    }
    // the F32 path (exact q8_0 values, f32 sums), or the f16 path's rounding on the tiled kernel for other shapes
    auto gemm = m->compute == HTR_COMPUTE_F32 ? launch_gemm_q8_0_f32 : launch_gemm_q8_0_r16;
    for (int li = 0; li < c.n_layer && rc == 0 && !m->mfma16; li++) {
        const Layer &ly = m->layers[li];
        uint16_t *kc = s->kc + li * s->kv_layer, *vc = s->vc + li * s->kv_layer;
        rc = launch_rms_norm(dev, st, x, ly.attn_norm, h, l, d, c.eps);
        if (rc == 0) rc = gemm(dev, st, h, ly.q, q, l, 0);
        if (rc == 0) rc = gemm(dev, st, h, ly.k, k, l, 0);
        if (rc == 0) rc = gemm(dev, st, h, ly.v, v, l, 0);
        if (rc == 0)
            rc = launch_qk_norm_rope_rows(dev, st, q, k, v, ly.q_norm, ly.k_norm, s->rope, l, c.n_head, c.n_kv, pos0,
                                          s->kv_rows, c.eps, kc, vc);
        if (rc == 0) rc = launch_attn_causal(dev, st, q, kc, vc, l, pos0, c.n_head, c.n_kv, s->kv_rows, scale, s->kvb, a);
        if (rc == 0) rc = gemm(dev, st, a, ly.o, x, l, 1);
        if (rc == 0) rc = launch_rms_norm(dev, st, x, ly.ffn_norm, h, l, d, c.eps);
        if (rc == 0) rc = gemm(dev, st, h, ly.gate, g, l, 0);
        if (rc == 0) rc = gemm(dev, st, h, ly.up, u, l, 0);
        if (rc == 0) rc = launch_swiglu(dev, st, g, u, (size_t)l * f);
        if (rc == 0) rc = gemm(dev, st, g, ly.down, x, l, 1);
    }
    // head (text.rs:655-658): output_norm + the tied LM head on the last row
    if (rc == 0) {
        DmvMat head = {m->tok_embd->q, m->tok_embd->d, c.n_vocab};
        rc = launch_dmv(dev, st, DMV_NORM, &head, 1, d, x + (size_t)(l - 1) * d, m->output_norm, c.eps, s->logits, 0);
    }
    if (rc == 0) rc = htr_sync(dev);
    if (rc == 0 && h_logits) rc = htr_download(dev, h_logits, s->logits, (size_t)c.n_vocab * 4);
    if (rc < 0) return rc;
    s->n_past += l;
    return 0;
}

// the in-graph time of a decode step's kernel classes: n_steps steps at the session's position (nothing advances it:
// every step re-runs at n_past, writing its KV row there) recorded as one graph with the kernels of `classes` only,
// replayed reps times after one untimed replay
extern "C" int htr_session_profile_step(htr_session *s, unsigned classes, int n_steps, int reps, float *ms_per_step) {
    if (!s || !ms_per_step) return htr_fail("htr_session_profile_step: null argument");
    htr_device *dev = s->dev;
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(htr_check_not_capturing(dev, "htr_session_profile_step"));
    if (n_steps < 1 || n_steps > 256 || reps < 1 || (classes & ~(unsigned)HTR_STEP_ALL) || !classes)
        return htr_fail("htr_session_profile_step: %d steps (1 … 256), %d replays, classes 0x%x", n_steps, reps, classes);
    if (s->n_past < 1 || s->n_past >= s->n_ctx)
        return htr_fail("htr_session_profile_step: the session is at %d of %d positions", s->n_past, s->n_ctx);
    if (s->m->compute != HTR_COMPUTE_F16) return htr_fail("htr_session_profile_step: the f16 paths' fused step only");
    HTR_TRY(reserve(s, (size_t)s->n_past + 1));
    HTR_TRY(set_state(s, s->n_past, 0));
    hipStream_t st = dev->stream;
    HTR_TRY(htr_hip(dev, hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture"));
    int rc = 0;
    for (int i = 0; i < n_steps && rc == 0; i++) rc = record_step(s, st, classes);
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(st, &graph);
    if (rc < 0) {
        if (graph) hipGraphDestroy(graph);
        return rc;
    }
    HTR_TRY(htr_hip(dev, e, "hipStreamEndCapture"));
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    hipGraphDestroy(graph);
    HTR_TRY(htr_hip(dev, e, "hipGraphInstantiate"));
    rc = htr_hip(dev, hipGraphLaunch(exec, st), "hipGraphLaunch");
    if (rc == 0) rc = htr_hip(dev, hipEventRecord(dev->t0, st), "hipEventRecord");
    for (int r = 0; r < reps && rc == 0; r++) rc = htr_hip(dev, hipGraphLaunch(exec, st), "hipGraphLaunch");
    float ms = 0.0f;
    if (rc == 0) rc = htr_hip(dev, hipEventRecord(dev->t1, st), "hipEventRecord");
    if (rc == 0) rc = htr_hip(dev, hipEventSynchronize(dev->t1), "hipEventSynchronize");
    if (rc == 0) rc = htr_hip(dev, hipEventElapsedTime(&ms, dev->t0, dev->t1), "hipEventElapsedTime");
    hipGraphExecDestroy(exec);
    if (rc < 0) return rc;
    *ms_per_step = ms / (float)(reps * n_steps);
    return 0;
}

// text.rs:524-537
extern "C" int htr_step(htr_session *s, int32_t token, float *h_logits) {
    if (!s) return htr_fail("htr_step: null session");
    htr_device *dev = s->dev;
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(htr_check_not_capturing(dev, "htr_step"));
    const htr_text_config &c = s->m->cfg;
    if (token < 0 || token >= c.n_vocab) return htr_fail("token %d is outside the vocabulary", token);
    if (s->n_past + 1 > s->n_ctx) return htr_fail("position %d: the session holds %d", s->n_past, s->n_ctx);
    HTR_TRY(reserve(s, (size_t)s->n_past + 1));
    uint32_t t = (uint32_t)token;
    HTR_TRY(htr_upload(dev, s->tok, &t, 4));
    HTR_TRY(set_state(s, s->n_past, 0));
    HTR_TRY(run_steps(s, nullptr, 1, true, &s->step_graph));
    HTR_TRY(htr_sync(dev));
    if (s->fused) {
        // a one-launch step whose wait ran out: the session steps kernel by kernel from now on, and this step is
        // redone that way (the state and the token are the host's; the KV row at the position is written again)
        bool failed = false;
        HTR_TRY(token_step_err(s, &failed));
        if (failed) {
            fall_back(s);
            HTR_TRY(set_state(s, s->n_past, 0));
            HTR_TRY(run_steps(s, nullptr, 1, true, &s->step_graph));
            HTR_TRY(htr_sync(dev));
        }
    }
    s->n_past += 1;
    if (h_logits) HTR_TRY(htr_download(dev, h_logits, s->logits, (size_t)c.n_vocab * 4));
    return 0;
}

// ---- the GPU token choice -------------------------------------------------------------------------------------------

extern "C" int htr_choice_free(htr_choice *ch) {
    if (!ch) return 0;
    htr_device *dev = ch->s->dev;
    for (hipGraphExec_t g : {ch->g_first, ch->g_one, ch->g_chunk})
        if (g) hipGraphExecDestroy(g);
    for (hipEvent_t e : ch->events) hipEventDestroy(e);
    for (void *p : {(void *)ch->hist, (void *)ch->counts, (void *)ch->fpen, (void *)ch->best, (void *)ch->counters})
        if (p) htr_dev_free(dev, p);
    if (ch->h_ids) hipHostFree(ch->h_ids);
    delete ch;
    return 0;
}

// text.rs:154-218
extern "C" int htr_choice_create(htr_session *s, const htr_preset *p, const int32_t *history, size_t n, size_t chunk,
                                 size_t depth, htr_choice **out) {
    if (!s || !p || !out || (n && !history)) return htr_fail("htr_choice_create: null argument");
    htr_device *dev = s->dev;
    HTR_TRY(htr_check_alive(dev));
    if (p->temperature != 0.0) return htr_fail("sampled (temperature > 0): the token is drawn on the CPU");
    const float rp = (float)p->repetition_penalty;
    if (p->repetition_penalty != 1.0 && !(std::isnormal(rp) && rp > 0.0f))
        return htr_fail("the repetition penalty is no positive normal f32");
    if (p->repetition_window < 1 || p->max_new_tokens < 1 || p->frequency_penalty < 0.0)
        return htr_fail("preset: window %zu, max new tokens %zu, fp %g", p->repetition_window, p->max_new_tokens,
                        p->frequency_penalty);
    if (chunk < 1 || chunk > 64 || depth < 1)
        return htr_fail("run-ahead %zu choices × %zu launches: 1…64 × ≥ 1", chunk, depth);
    const int n_vocab = s->m->cfg.n_vocab;
    const size_t seed_len = std::min(n, p->repetition_window);
    const int32_t *seed = history + (n - seed_len);
    std::vector<uint32_t> hist(seed_len + p->max_new_tokens, 0);
    for (size_t i = 0; i < seed_len; i++) {
        if (seed[i] < 0 || seed[i] >= n_vocab) return htr_fail("history token %d is outside the vocabulary", seed[i]);
        hist[i] = (uint32_t)seed[i];
    }
    auto *ch = new htr_choice;
    ch->s = s;
    ch->seed_len = (int)seed_len;
    ch->window = (int)std::min<size_t>(p->repetition_window, 1u << 30);
    ch->rp = p->repetition_penalty != 1.0 ? rp : 1.0f;
    ch->fp = p->frequency_penalty > 0.0 ? (float)p->frequency_penalty : 0.0f;
    ch->max_new = p->max_new_tokens;
    ch->chunk = chunk;
    ch->depth = depth;
    ch->n_vocab = n_vocab;
    const size_t words = ch->fp > 0.0f ? (size_t)n_vocab : 1;
    int rc = htr_dev_alloc(dev, hist.size() * 4, HTR_MEM_WORK, (void **)&ch->hist);
    if (rc == 0) rc = htr_upload(dev, ch->hist, hist.data(), hist.size() * 4);
    if (rc == 0) rc = htr_dev_alloc_zero(dev, words * 4, HTR_MEM_WORK, (void **)&ch->counts);
    if (rc == 0) rc = htr_dev_alloc(dev, words * 4, HTR_MEM_WORK, (void **)&ch->fpen);
    if (rc == 0) rc = htr_dev_alloc_zero(dev, choose_best_bytes(1), HTR_MEM_WORK, (void **)&ch->best);
    if (rc == 0) rc = htr_dev_alloc_zero(dev, choose_ticket_bytes(1), HTR_MEM_WORK, (void **)&ch->counters);
    if (rc == 0) rc = htr_hip(dev, hipHostMalloc((void **)&ch->h_ids, (depth * chunk + depth) * 4, hipHostMallocDefault), "hipHostMalloc");
    for (size_t i = 0; i < depth && rc == 0; i++) {
        hipEvent_t e;
        rc = htr_hip(dev, hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
        if (rc == 0) ch->events.push_back(e);
    }
    if (rc < 0) {
        std::string keep = htr_last_error();
        htr_choice_free(ch);
        return htr_fail("%s", keep.c_str());
    }
    *out = ch;
    return 0;
}

// a read's choices from `from` on were launched but are given up (a one-launch step's wait ran out in their chunk or
// before): the frequency counts they added are taken back (each choice i wrote its token at hist[seed_len + i] and
// added one to its count) — choices from … next − 1
int take_back_counts(htr_choice *ch, size_t from, size_t next) {
    if (ch->fp == 0.0f || from >= next) return 0;
    htr_device *dev = ch->s->dev;
    std::vector<uint32_t> ids(next - from), counts((size_t)ch->n_vocab);
    std::vector<float> fpen((size_t)ch->n_vocab);
    HTR_TRY(htr_download(dev, ids.data(), ch->hist + ch->seed_len + from, ids.size() * 4));
    HTR_TRY(htr_download(dev, counts.data(), ch->counts, counts.size() * 4));
    HTR_TRY(htr_download(dev, fpen.data(), ch->fpen, fpen.size() * 4));
    for (uint32_t t : ids) {
        if (t >= (uint32_t)ch->n_vocab || counts[t] == 0) return htr_fail("decode: a given-up choice's count is gone");
        counts[t] -= 1;
        fpen[t] = ch->fp * (float)counts[t];  // the value the step that counted last wrote: fp · count
    }
    HTR_TRY(htr_upload(dev, ch->counts, counts.data(), counts.size() * 4));
    return htr_upload(dev, ch->fpen, fpen.data(), fpen.size() * 4);
}

// text.rs:587-625. Each launch of `chunk` choices copies its ids back with the one-launch step's error word in the same
// stream order, and the ids reach on_token only after both have landed (the reference reads each submission's ids
// through read_mapped_u32, which fails on a dead device before on_token sees them, text.rs:616-623, gpu.rs:1391-1396).
// A set error word means a wait of some one-launch step of that chunk ran out (the 256 workgroups were not all resident
// at once): none of the chunk's ids is passed on, the launches after it are drained unseen, and the read goes on from
// the chunk's first step on the per-kernel step, which the session keeps — the counts, the position and the token
// rewound to what the chunk started from (its first choice, if it is the read's first, came from the prefill's logits
// by the choice kernel and is kept).
extern "C" int htr_decode_gpu(htr_session *s, htr_choice *ch, size_t max, htr_token_cb on_token, void *user) {
    if (!s || !ch || ch->s != s) return htr_fail("htr_decode_gpu: null argument or a choice of another session");
    htr_device *dev = s->dev;
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(htr_check_not_capturing(dev, "htr_decode_gpu"));
    const size_t cap = ch->max_new;
    if (max > cap) return htr_fail("%zu choices: the history holds %zu", max, cap);
    if (max == 0) return 0;
    if ((size_t)s->n_past + (max - 1) > (size_t)s->n_ctx)
        return htr_fail("%zu choices need %zu positions, the session holds %d", max, s->n_past + max - 1, s->n_ctx);
    hipStream_t st = dev->stream;
    HTR_TRY(set_state(s, s->n_past, ch->seed_len));
    uint32_t *h_err = ch->h_ids + ch->depth * ch->chunk;

    struct Pending {
        size_t slot, first, n;
    };
    std::deque<Pending> queue;
    std::vector<size_t> free_slots;
    for (size_t i = ch->depth; i-- > 0;) free_slots.push_back(i);
    size_t next = 0;          // choices launched
    int32_t last_tok = -1;    // the last choice passed to on_token
    int rc = 0;
    bool stop = false;
    while (rc == 0) {
        while (!stop && next < max && !free_slots.empty()) {
            // the slot's steps need their KV rows before its launches take the cache's layout: choices next …
            // next + n − 1, every one but the read's first a step at the position after the one before
            const size_t n_slot = std::min(ch->chunk, max - next);
            rc = reserve(s, (size_t)s->n_past + next + n_slot - 1);
            if (rc < 0) break;
            drop_stale_graphs(ch);
            const size_t slot = free_slots.back();
            free_slots.pop_back();
            size_t n_launched = 0;
            if (next == 0) {
                rc = run_steps(s, ch, 1, false, &ch->g_first);
                n_launched = 1;
            }
            // fill the slot up to `chunk` choices: whole chunk graphs, else single steps
            while (rc == 0 && n_launched < ch->chunk && next + n_launched < max) {
                const size_t left = std::min(ch->chunk - n_launched, max - next - n_launched);
                if (left == ch->chunk && ch->chunk > 1) {
                    rc = run_steps(s, ch, (int)ch->chunk, true, &ch->g_chunk);
                    n_launched += ch->chunk;
                } else {
                    rc = run_steps(s, ch, 1, true, &ch->g_one);
                    n_launched += 1;
                }
            }
            if (rc < 0) break;
            rc = htr_hip(dev,
                         hipMemcpyAsync(ch->h_ids + slot * ch->chunk, ch->hist + ch->seed_len + next, n_launched * 4,
                                        hipMemcpyDeviceToHost, st),
                         "token readback");
            h_err[slot] = 0;
            if (rc == 0 && s->tl)
                rc = htr_hip(dev, hipMemcpyAsync(h_err + slot, s->tseq + 1, 4, hipMemcpyDeviceToHost, st),
                             "error word readback");
            if (rc == 0) rc = htr_hip(dev, hipEventRecord(ch->events[slot], st), "hipEventRecord");
            queue.push_back({slot, next, n_launched});
            next += n_launched;
        }
        if (rc < 0 || queue.empty()) break;
        Pending pd = queue.front();
        queue.pop_front();
        rc = htr_hip(dev, hipEventSynchronize(ch->events[pd.slot]), "hipEventSynchronize");
        if (rc < 0) break;
        if (h_err[pd.slot]) {
            // drain what was launched after the chunk, clear the error word, step kernel by kernel from here
            rc = htr_sync(dev);
            bool failed = false;
            if (rc == 0) rc = token_step_err(s, &failed);
            if (rc < 0) break;
            fall_back(s);
            const size_t redo = std::max<size_t>(pd.first, 1);  // the first choice made after a step
            if (pd.first == 0) {  // the read's first choice: the choice kernel's, on the prefill's logits
                uint32_t t0 = 0;
                rc = htr_download(dev, &t0, ch->hist + ch->seed_len, 4);
                if (rc < 0) break;
                last_tok = (int32_t)t0;
                if (on_token && !on_token(last_tok, user)) stop = true;
            }
            rc = take_back_counts(ch, redo, next);
            if (rc < 0) break;
            queue.clear();
            free_slots.clear();
            for (size_t i = ch->depth; i-- > 0;) free_slots.push_back(i);
            next = redo;
            if (stop || next >= max) break;
            // the step of choice `redo` embeds choice redo − 1 at position n_past + redo − 1
            const uint32_t t = (uint32_t)last_tok;
            rc = htr_upload(dev, s->tok, &t, 4);
            if (rc == 0) rc = set_state(s, s->n_past + (int)redo - 1, ch->seed_len + (int)redo);
            continue;
        }
        for (size_t i = 0; i < pd.n && !stop; i++) {
            last_tok = (int32_t)ch->h_ids[pd.slot * ch->chunk + i];
            if (on_token && !on_token(last_tok, user)) stop = true;
        }
        free_slots.push_back(pd.slot);
        if (stop) {
            // the launches already queued finish on the device unseen
            while (!queue.empty()) queue.pop_front();
        }
    }
    if (rc == 0) rc = htr_sync(dev);
    if (rc == 0) {
        // launches past a stop ran unseen: a wait of theirs that ran out leaves the session on the per-kernel step
        bool failed = false;
        rc = token_step_err(s, &failed);
        if (rc == 0 && failed) fall_back(s);
    }
    if (rc < 0) return rc;
    // the steps launched: every choice but the first of the read advanced the position by one
    s->n_past += (int)(next - 1);
    return 0;
}
