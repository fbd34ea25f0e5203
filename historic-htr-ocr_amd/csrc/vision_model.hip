// The vision encoder's host side: Vision (vision.rs:87-263) — weights at load (q8_0 → f16 for the matrix-core GEMMs,
// the down projection × 64), the patch grid checks, and the f16 compute path's graph (vision.rs:328-423 run_f16 +
// project) on the kernels of mfma_gemm.hip / vision.hip / gemm.hip.
#include <cmath>
#include <cstring>
#include <vector>

#include "htr_internal.h"

namespace {

constexpr float FFN_DOWN_SCALE = 64.0f;  // vision.rs:31-35: the SwiGLU product stored ÷ 64, the down weights × 64

struct VLayer {
    float *ln1 = nullptr, *ln2 = nullptr;
    htr_weight *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr, *gate = nullptr, *up = nullptr, *down = nullptr;
};

// vision.rs:159-175: [half][pos][k] × (cos, sin), the angle multiplied up step by step in f32
std::vector<float> rope2d_table(float theta, int d_head, int max_pos) {
    const int n_dims = d_head / 2;
    const float theta_scale = powf(theta, -2.0f / (float)n_dims);
    std::vector<float> out;
    out.reserve((size_t)2 * max_pos * (n_dims / 2) * 2);
    for (int half = 0; half < 2; half++) {
        const float freq_scale = half == 0 ? 1.0f : powf(theta, -2.0f / (float)d_head);
        for (int pos = 0; pos < max_pos; pos++) {
            float t = (float)pos;
            for (int k = 0; k < n_dims / 2; k++) {
                const float a = freq_scale * t;
                out.push_back(cosf(a));
                out.push_back(sinf(a));
                t *= theta_scale;
            }
        }
    }
    return out;
}

}  // namespace

struct htr_vision {
    htr_device *dev = nullptr;
    htr_vision_config cfg{};
    float *lut = nullptr, *patch_embd = nullptr, *pre_ln = nullptr, *input_norm = nullptr;
    std::vector<VLayer> layers;
    htr_weight *merger = nullptr, *mm1 = nullptr, *mm2 = nullptr;
    // the encode's buffers, sized for the largest page seen (rows n_cap)
    int n_cap = 0, pos_cap = 0;
    uint8_t *rgb = nullptr;
    size_t rgb_cap = 0;
    float *P = nullptr, *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *tmp = nullptr, *cs = nullptr;
    _Float16 *h16 = nullptr, *a16 = nullptr, *g16 = nullptr, *kv = nullptr;
    // the f32 operands of the patch embedding and the projector as f16 pieces (k_split_f16): the patch embedding
    // weight [dim][hi | lo | hi] in segments of pe_kp (the patch's 3·p² values padded to a multiple of 32); the
    // projector weights are stored [w | w]; xs holds an activation's pieces
    htr_weight *pe = nullptr;
    int pe_kp = 0;
    _Float16 *xs = nullptr;
};

namespace {

int up_vec(htr_device *dev, const float *h, size_t n, const char *what, float **out) {
    if (!h) return htr_fail("missing f32 tensor %s [%zu]", what, n);
    HTR_TRY(htr_dev_alloc(dev, n * 4, HTR_MEM_WEIGHTS, (void **)out));
    return htr_upload(dev, *out, h, n * 4);
}

int up_w16(htr_device *dev, const void *h, size_t rows, size_t cols, float scale, const char *what, htr_weight **out) {
    if (!h) return htr_fail("missing q8_0 tensor %s [%zu x %zu]", what, rows, cols);
    if (htr_weight_q8_0_f16(dev, h, rows, cols, scale, out) < 0) return htr_fail("%s: %s", what, htr_last_error());
    return 0;
}

// W [N][K] f16 → [N][2K] = [w | w]: the projector's f32 activations go in as [hi | lo] (k_split_f16)
int widen_w16(htr_device *dev, htr_weight *w) {
    _Float16 *h2 = nullptr;
    const size_t n = w->rows, k = w->cols;
    HTR_TRY(htr_dev_alloc(dev, n * 2 * k * 2, HTR_MEM_WEIGHTS, (void **)&h2));
    int rc = 0;
    for (int s = 0; s < 2 && rc == 0; s++)
        rc = htr_hip(dev, hipMemcpy2DAsync(h2 + s * k, 2 * k * 2, w->h, k * 2, k * 2, n, hipMemcpyDeviceToDevice,
                                           dev->stream), "widen a projector weight");
    if (rc == 0) rc = htr_sync(dev);
    if (rc < 0) {
        htr_dev_free(dev, h2);
        return -1;
    }
    htr_dev_free(dev, w->h);
    w->h = h2;
    w->cols = 2 * k;
    return 0;
}

// the f32 patch embedding [dim][3·p²] → the f16 weight [dim][hi | lo | hi] (segments of pe_kp); the f32 copy is freed
int split_patch_embd(htr_vision *v, size_t pp) {
    htr_device *dev = v->dev;
    const int d = v->cfg.dim, kp = (int)((pp + 31) / 32 * 32);
    auto *w = new htr_weight;
    w->dev = dev;
    w->rows = d;
    w->cols = (size_t)3 * kp;
    v->pe = w;
    v->pe_kp = kp;
    HTR_TRY(htr_dev_alloc(dev, w->rows * w->cols * 2, HTR_MEM_WEIGHTS, (void **)&w->h));
    HTR_TRY(launch_split_f16(dev, dev->stream, v->patch_embd, d, (int)pp, kp, 3, 0b010, w->h));
    HTR_TRY(htr_sync(dev));
    htr_dev_free(dev, v->patch_embd);
    v->patch_embd = nullptr;
    return 0;
}

void free_bufs(htr_vision *v) {
    for (void *p : {(void *)v->rgb, (void *)v->P, (void *)v->x, (void *)v->q, (void *)v->k, (void *)v->v, (void *)v->tmp,
                    (void *)v->cs, (void *)v->h16, (void *)v->a16, (void *)v->g16, (void *)v->kv, (void *)v->xs})
        if (p) htr_dev_free(v->dev, p);
    v->rgb = nullptr;
    v->P = v->x = v->q = v->k = v->v = v->tmp = v->cs = nullptr;
    v->h16 = v->a16 = v->g16 = v->kv = v->xs = nullptr;
    v->n_cap = v->pos_cap = 0;
    v->rgb_cap = 0;
}

// buffers for n patches (and the projector: unfold n·dim, merged n/4·dim, mm.1 n/4·proj_dim fit in q / k / v)
int ensure_bufs(htr_vision *v, int n, int max_pos, size_t rgb_bytes) {
    const htr_vision_config &c = v->cfg;
    htr_device *dev = v->dev;
    if (n > v->n_cap || max_pos > v->pos_cap || rgb_bytes > v->rgb_cap) {
        free_bufs(v);
        const size_t d = c.dim, f = c.n_ff, pp = 3 * (size_t)c.patch * c.patch;
        const size_t qkv = (size_t)n * std::max<size_t>(d, (size_t)c.proj_dim);
        int rc = htr_dev_alloc(dev, rgb_bytes, HTR_MEM_WORK, (void **)&v->rgb);
        if (rc == 0) rc = htr_dev_alloc(dev, (size_t)n * pp * 4, HTR_MEM_WORK, (void **)&v->P);
        if (rc == 0) rc = htr_dev_alloc(dev, (size_t)n * d * 4, HTR_MEM_WORK, (void **)&v->x);
        if (rc == 0) rc = htr_dev_alloc(dev, qkv * 4, HTR_MEM_WORK, (void **)&v->q);
        if (rc == 0) rc = htr_dev_alloc(dev, qkv * 4, HTR_MEM_WORK, (void **)&v->k);
        if (rc == 0) rc = htr_dev_alloc(dev, qkv * 4, HTR_MEM_WORK, (void **)&v->v);
        if (rc == 0) rc = htr_dev_alloc(dev, (size_t)n * d * 4, HTR_MEM_WORK, (void **)&v->tmp);
        if (rc == 0) rc = htr_dev_alloc(dev, (size_t)2 * max_pos * (c.d_head / 4) * 2 * 4, HTR_MEM_WORK, (void **)&v->cs);
        if (rc == 0) rc = htr_dev_alloc(dev, (size_t)n * d * 2, HTR_MEM_WORK, (void **)&v->h16);
        if (rc == 0) rc = htr_dev_alloc(dev, (size_t)n * d * 2, HTR_MEM_WORK, (void **)&v->a16);
        if (rc == 0) rc = htr_dev_alloc(dev, (size_t)n * f * 2, HTR_MEM_WORK, (void **)&v->g16);
        if (rc == 0) rc = htr_dev_alloc(dev, vision_kv_bytes((int)n, c.n_head), HTR_MEM_WORK, (void **)&v->kv);
        // the split activations: patches [n][3·pe_kp], the merger's input [n/4][2·4d], mm.1 / mm.2's [n/4][2·width]
        const size_t xs = std::max({(size_t)n * 3 * v->pe_kp, (size_t)(n / 4) * 2 * 4 * d,
                                    (size_t)(n / 4) * 2 * std::max<size_t>(d, (size_t)c.proj_dim)});
        if (rc == 0) rc = htr_dev_alloc(dev, xs * 2, HTR_MEM_WORK, (void **)&v->xs);
        if (rc < 0) {
            std::string keep = htr_last_error();
            free_bufs(v);
            return htr_fail("%s", keep.c_str());
        }
        v->n_cap = n;
        v->pos_cap = max_pos;
        v->rgb_cap = rgb_bytes;
    }
    return 0;
}

}  // namespace

extern "C" int htr_vision_free(htr_vision *v) {
    if (!v) return 0;
    htr_device *dev = v->dev;
    free_bufs(v);
    for (VLayer &l : v->layers) {
        for (htr_weight *w : {l.q, l.k, l.v, l.o, l.gate, l.up, l.down}) htr_weight_free(w);
        for (float *p : {l.ln1, l.ln2})
            if (p) htr_dev_free(dev, p);
    }
    for (htr_weight *w : {v->merger, v->mm1, v->mm2, v->pe}) htr_weight_free(w);
    for (float *p : {v->lut, v->patch_embd, v->pre_ln, v->input_norm})
        if (p) htr_dev_free(dev, p);
    delete v;
    return 0;
}

namespace {

// where the encoder's tensors come from: host arrays (htr_vision_create) or an mmproj GGUF (htr_vision_load_gguf).
// Names are the GGUF's (v.blk.{i}.attn_q.weight …); w16 fills an f16 [rows][cols] plane (× scale), patch an f32 one
struct VisionFeed {
    virtual int w16(int layer, const char *kind, size_t rows, size_t cols, float scale, htr_weight **out) = 0;
    virtual int vec(int layer, const char *kind, size_t n, float **out) = 0;
    virtual int patch(size_t rows, size_t cols, float **out) = 0;
    virtual ~VisionFeed() = default;
    static std::string name(int layer, const char *kind) {
        return layer < 0 ? std::string(kind) + ".weight" : "v.blk." + std::to_string(layer) + "." + kind + ".weight";
    }
};

struct ArrayVisionFeed : VisionFeed {
    htr_device *dev;
    const htr_vision_layer *layers;
    const float *patch_embd, *pre_ln, *input_norm;
    const void *merger, *mm1, *mm2;
    int w16(int layer, const char *kind, size_t rows, size_t cols, float scale, htr_weight **out) override {
        const std::string k = kind;
        const void *h = k == "mm.patch_merger" ? merger : k == "mm.1" ? mm1 : mm2;
        if (layer >= 0) {
            const htr_vision_layer &t = layers[layer];
            h = k == "attn_q" ? t.q : k == "attn_k" ? t.k : k == "attn_v" ? t.v : k == "attn_out" ? t.o
                : k == "ffn_gate" ? t.gate : k == "ffn_up" ? t.up : t.down;
        }
        return up_w16(dev, h, rows, cols, scale, name(layer, kind).c_str(), out);
    }
    int vec(int layer, const char *kind, size_t n, float **out) override {
        const std::string k = kind;
        const float *h = k == "v.pre_ln" ? pre_ln : input_norm;
        if (layer >= 0) h = k == "ln1" ? layers[layer].ln1 : layers[layer].ln2;
        return up_vec(dev, h, n, name(layer, kind).c_str(), out);
    }
    int patch(size_t rows, size_t cols, float **out) override {
        return up_vec(dev, patch_embd, rows * cols, "v.patch_embd.weight", out);
    }
};

struct GgufVisionFeed : VisionFeed {
    htr_gguf *g;
    GgufStager sg;
    unsigned *over = nullptr;  // device u32: pairs of values beyond f16's range
    explicit GgufVisionFeed(htr_gguf *gg) : g(gg) {}
    ~GgufVisionFeed() override {
        if (over) htr_dev_free(sg.dev, over);
    }
    int w16(int layer, const char *kind, size_t rows, size_t cols, float scale, htr_weight **out) override {
        const GgufTensor *t;
        HTR_TRY(gguf_find(g, name(layer, kind).c_str(), &t));
        auto *w = new htr_weight;
        w->dev = sg.dev;
        w->rows = rows;
        w->cols = cols;
        int rc = htr_dev_alloc(sg.dev, rows * cols * 2, HTR_MEM_WEIGHTS, (void **)&w->h);
        if (rc == 0) rc = gguf_upload_vision(sg, g, *t, rows, cols, scale, over, w->h, nullptr);
        if (rc < 0) {
            std::string keep = htr_last_error();
            htr_weight_free(w);
            return htr_fail("%s", keep.c_str());
        }
        *out = w;
        return 0;
    }
    int vec(int layer, const char *kind, size_t n, float **out) override {
        const GgufTensor *t;
        HTR_TRY(gguf_find(g, name(layer, kind).c_str(), &t));
        if (t->type != GGUF_F32 || t->n_dims != 1 || t->shape[0] != n)  // vision.rs:144-150
            return htr_fail("%s: %s %s, expected F32 [%zu]", t->name, ggml_type_name(t->type), gguf_shape_str(*t).c_str(),
                            n);
        return gguf_upload_f32(sg, g, *t, n, out);
    }
    int patch(size_t rows, size_t cols, float **out) override {
        const GgufTensor *t;
        HTR_TRY(gguf_find(g, "v.patch_embd.weight", &t));
        HTR_TRY(htr_dev_alloc(sg.dev, rows * cols * 4, HTR_MEM_WEIGHTS, (void **)out));
        return gguf_upload_vision(sg, g, *t, rows, cols, 1.0f, over, nullptr, *out);
    }
};

int check_vision_cfg(const htr_vision_config &c) {
    if (c.n_layer < 1 || c.dim < 64 || c.n_head < 1 || c.patch < 1 || c.proj_dim < 1 || c.n_ff < 1)
        return htr_fail("vision config: %d layers, dim %d, %d heads, patch %d, projection %d, ffn %d", c.n_layer, c.dim,
                        c.n_head, c.patch, c.proj_dim, c.n_ff);
    if (c.d_head != 64 || c.dim != c.n_head * 64)
        return htr_fail("head dim %d (dim %d / %d heads): the attention kernel is written for 64", c.d_head, c.dim,
                        c.n_head);
    if (c.merge != 2 || c.n_ff < 4 * c.dim) return htr_fail("merge %d / n_ff %d: the unfold kernel is 2×2", c.merge, c.n_ff);
    if (c.dim % 128 || c.n_ff % 128 || c.proj_dim % 64)
        return htr_fail("dims %d / %d / projection %d: the matrix-core GEMMs take widths that are multiples of 128 (the "
                        "projection: of 64)", c.dim, c.n_ff, c.proj_dim);
    return 0;
}

// Vision::from_gguf's body (vision.rs:196-227) over either feed, in its order: the layers, then the patch embedding,
// pre_ln, the projector. Then the device forms of the f32-activation products (projector [w | w], patch [hi | lo | hi])
int build_vision(htr_device *dev, const htr_vision_config &c, VisionFeed &feed, htr_vision *v) {
    v->dev = dev;
    v->cfg = c;
    v->layers.resize(c.n_layer);
    const size_t d = c.dim, f = c.n_ff, pp = 3 * (size_t)c.patch * c.patch;
    for (int i = 0; i < c.n_layer; i++) {
        VLayer &l = v->layers[i];
        HTR_TRY(feed.vec(i, "ln1", d, &l.ln1));
        HTR_TRY(feed.vec(i, "ln2", d, &l.ln2));
        HTR_TRY(feed.w16(i, "attn_q", d, d, 1.0f, &l.q));
        HTR_TRY(feed.w16(i, "attn_k", d, d, 1.0f, &l.k));
        HTR_TRY(feed.w16(i, "attn_v", d, d, 1.0f, &l.v));
        HTR_TRY(feed.w16(i, "attn_out", d, d, 1.0f, &l.o));
        HTR_TRY(feed.w16(i, "ffn_gate", f, d, 1.0f, &l.gate));
        HTR_TRY(feed.w16(i, "ffn_up", f, d, 1.0f, &l.up));
        HTR_TRY(feed.w16(i, "ffn_down", d, f, FFN_DOWN_SCALE, &l.down));
    }
    // vision.rs:143-146 pixel_lut
    std::vector<float> lut(768);
    for (int ch = 0; ch < 3; ch++)
        for (int i = 0; i < 256; i++) lut[ch * 256 + i] = ((float)i / 255.0f - c.mean[ch]) / c.std[ch];
    HTR_TRY(up_vec(dev, lut.data(), 768, "pixel lut", &v->lut));
    HTR_TRY(feed.patch(d, pp, &v->patch_embd));
    HTR_TRY(feed.vec(-1, "v.pre_ln", d, &v->pre_ln));
    HTR_TRY(feed.vec(-1, "mm.input_norm", d, &v->input_norm));
    HTR_TRY(feed.w16(-1, "mm.patch_merger", d, 4 * d, 1.0f, &v->merger));
    HTR_TRY(feed.w16(-1, "mm.1", c.proj_dim, d, 1.0f, &v->mm1));
    HTR_TRY(feed.w16(-1, "mm.2", c.proj_dim, c.proj_dim, 1.0f, &v->mm2));
    for (htr_weight *w : {v->merger, v->mm1, v->mm2}) HTR_TRY(widen_w16(dev, w));
    return split_patch_embd(v, pp);
}

int finish(htr_vision *v, int rc, htr_vision **out) {
    if (rc < 0) {
        std::string keep = htr_last_error();
        htr_vision_free(v);
        return htr_fail("%s", keep.c_str());
    }
    *out = v;
    return 0;
}

// VisionConfig::from_gguf (vision.rs:55-84)
int vision_config_from_gguf(htr_gguf *g, htr_vision_config *out) {
    htr_vision_config c{};
    std::string proj;
    HTR_TRY(gguf_meta_str(g, "clip.projector_type", &proj));
    if (proj != "lightonocr") return htr_fail("projector \"%s\": this engine runs lightonocr only", proj.c_str());
    bool silu = false;
    HTR_TRY(gguf_meta_bool(g, "clip.use_silu", &silu));
    if (!silu) return htr_fail("clip.use_silu is false: the encoder's FFN would not be SwiGLU");
    uint32_t u[8];
    const char *keys[8] = {"clip.vision.embedding_length", "clip.vision.attention.head_count",
                           "clip.vision.block_count",      "clip.vision.feed_forward_length",
                           "clip.vision.patch_size",       "clip.vision.spatial_merge_size",
                           "clip.vision.image_size",       "clip.vision.projection_dim"};
    for (int k = 0; k < 2; k++) HTR_TRY(gguf_meta_u32(g, keys[k], &u[k]));
    if (u[1] == 0 || u[0] % u[1] != 0 || u[0] / u[1] != 64)
        return htr_fail("head dim %u/%u: the attention kernel is written for 64", u[0], u[1]);
    for (int k = 2; k < 8; k++) HTR_TRY(gguf_meta_u32(g, keys[k], &u[k]));
    for (int k = 0; k < 8; k++)
        if (u[k] > (1u << 24)) return htr_fail("%s = %u is not a vision encoder's size", keys[k], u[k]);
    c.dim = (int)u[0];
    c.n_head = (int)u[1];
    c.d_head = c.dim / c.n_head;
    c.n_layer = (int)u[2];
    c.n_ff = (int)u[3];
    c.patch = (int)u[4];
    c.merge = (int)u[5];
    c.image_size = (int)u[6];
    c.proj_dim = (int)u[7];
    HTR_TRY(gguf_meta_f32(g, "clip.vision.attention.layer_norm_epsilon", &c.eps));
    c.rope_theta = 10000.0f;  // vision.rs:28-29: clip.cpp's LIGHTONOCR constant; the GGUF has no key for it
    std::vector<float> three;
    for (int k = 0; k < 2; k++) {
        const char *key = k ? "clip.vision.image_std" : "clip.vision.image_mean";
        HTR_TRY(gguf_meta_f32_array(g, key, &three));
        if (three.size() != 3) return htr_fail("%s has %zu values", key, three.size());
        for (int ch = 0; ch < 3; ch++) (k ? c.std : c.mean)[ch] = three[ch];
    }
    *out = c;
    return 0;
}

}  // namespace

// Vision::from_gguf (vision.rs:177-233) from host tensors
extern "C" int htr_vision_create(htr_device *dev, const htr_vision_config *cfg, const float *patch_embd,
                                 const float *pre_ln, const htr_vision_layer *layers, const float *input_norm,
                                 const void *merger, const void *mm1, const void *mm2, htr_vision **out) {
    HTR_TRY(htr_check_alive(dev));
    if (!cfg || !layers || !out) return htr_fail("htr_vision_create: null argument");
    HTR_TRY(check_vision_cfg(*cfg));
    ArrayVisionFeed feed;
    feed.dev = dev;
    feed.layers = layers;
    feed.patch_embd = patch_embd;
    feed.pre_ln = pre_ln;
    feed.input_norm = input_norm;
    feed.merger = merger;
    feed.mm1 = mm1;
    feed.mm2 = mm2;
    auto *v = new htr_vision;
    return finish(v, build_vision(dev, *cfg, feed, v), out);
}

// Vision::from_gguf (vision.rs:177-233) from an mmproj GGUF: BF16 weights converted to f16 on the device as they
// arrive (the down projection × 64), a load refused when any value lies beyond f16's range (vision.rs:224-232)
extern "C" int htr_vision_load_gguf(htr_device *dev, htr_gguf *g, htr_vision **out) {
    HTR_TRY(htr_check_alive(dev));
    if (!g || !out) return htr_fail("htr_vision_load_gguf: null argument");
    htr_vision_config c{};
    HTR_TRY(vision_config_from_gguf(g, &c));
    HTR_TRY(check_vision_cfg(c));
    // vision.rs:209-214: tensors the graph would use if present (checked before any weight is streamed)
    for (const char *absent : {"v.patch_embd.bias", "v.post_ln.weight", "mm.1.bias", "mm.2.bias",
                               "v.token_embd.img_break", "mm.input_norm.bias"})
        if (gguf_has(g, absent)) return htr_fail("%s is in the GGUF but not part of this engine's graph", absent);
    GgufVisionFeed feed(g);
    HTR_TRY(feed.sg.init(dev));
    HTR_TRY(htr_dev_alloc_zero(dev, 4, HTR_MEM_WORK, (void **)&feed.over));
    auto *v = new htr_vision;
    int rc = build_vision(dev, c, feed, v);
    unsigned n_over = 0;
    if (rc == 0) rc = htr_hip(dev, hipMemcpyAsync(&n_over, feed.over, 4, hipMemcpyDeviceToHost, dev->stream),
                              "read the f16 range count");
    if (rc == 0) rc = htr_sync(dev);
    if (rc == 0 && n_over > 0)
        rc = htr_fail("%u words of vision weights hold values beyond f16's range (65504): this model cannot run on the "
                      "f16 compute path", n_over);
    return finish(v, rc, out);
}

extern "C" int htr_vision_get_config(htr_vision *v, htr_vision_config *out) {
    if (!v || !out) return htr_fail("htr_vision_get_config: null argument");
    *out = v->cfg;
    return 0;
}

// vision.rs:236-244 grid + the output shape of an encode
extern "C" int htr_vision_out_shape(htr_vision *v, int width, int height, int n_layers, size_t *n_tokens, size_t *dim) {
    if (!v) return htr_fail("htr_vision_out_shape: null vision");
    const htr_vision_config &c = v->cfg;
    const int grid = c.patch * c.merge;
    if (width <= 0 || height <= 0 || width % grid || height % grid || std::max(width, height) > c.image_size)
        return htr_fail("image %dx%d is not baked (both sides on the %d px grid, longest ≤ %d)", width, height, grid,
                        c.image_size);
    if (n_layers > c.n_layer) return htr_fail("%d layers asked, the encoder has %d", n_layers, c.n_layer);
    const size_t n = (size_t)(width / c.patch) * (height / c.patch);
    if (n_tokens) *n_tokens = n_layers < 0 ? n / 4 : n;
    if (dim) *dim = n_layers < 0 ? (size_t)c.proj_dim : (size_t)c.dim;
    return 0;
}

// Vision::encode_gpu / encode (vision.rs:248-263, 328-423)
extern "C" int htr_vision_encode(htr_vision *v, const uint8_t *h_rgb, int width, int height, int n_layers,
                                 float *d_out) {
    if (!v || !h_rgb || !d_out) return htr_fail("htr_vision_encode: null argument");
    htr_device *dev = v->dev;
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(htr_vision_out_shape(v, width, height, n_layers, nullptr, nullptr));
    const htr_vision_config &c = v->cfg;
    const int px = width / c.patch, py = height / c.patch, n = px * py, d = c.dim, pp = 3 * c.patch * c.patch;
    const int max_pos = std::max(px, py);
    const size_t rgb_bytes = (size_t)width * height * 3;
    HTR_TRY(ensure_bufs(v, n, max_pos, rgb_bytes));
    hipStream_t st = dev->stream;
    HTR_TRY(htr_upload(dev, v->rgb, h_rgb, rgb_bytes));
    const std::vector<float> cs = rope2d_table(c.rope_theta, c.d_head, max_pos);
    HTR_TRY(htr_upload(dev, v->cs, cs.data(), cs.size() * 4));
    const float scale = 1.0f / sqrtf((float)c.d_head);
    const int nl = n_layers < 0 ? c.n_layer : n_layers;
    HTR_TRY(launch_patchify(dev, st, v->rgb, v->lut, width, px, n, c.patch, v->P));
    // the patch embedding in f32 grade: [xh | xh | xl]·[wh | wl | wh]ᵀ
    HTR_TRY(launch_split_f16(dev, st, v->P, n, pp, v->pe_kp, 3, 0b100, v->xs));
    HTR_TRY(launch_gemm_f16(dev, st, GEMM_F32, v->xs, n, v->pe, nullptr, v->tmp, nullptr, 1.0f));
    HTR_TRY(launch_rms_norm(dev, st, v->tmp, v->pre_ln, v->x, n, d, c.eps));
    for (int li = 0; li < nl; li++) {
        const VLayer &l = v->layers[li];
        HTR_TRY(launch_rms_norm_f16(dev, st, v->x, l.ln1, v->h16, n, d, c.eps));
        if (c.dim % 256 == 0) {
            HTR_TRY(launch_gemm_f16_qkv(dev, st, v->h16, n, l.q, l.k, l.v, v->q, v->k, v->v));
        } else {
            HTR_TRY(launch_gemm_f16(dev, st, GEMM_F32, v->h16, n, l.q, nullptr, v->q, nullptr, 1.0f));
            HTR_TRY(launch_gemm_f16(dev, st, GEMM_F32, v->h16, n, l.k, nullptr, v->k, nullptr, 1.0f));
            HTR_TRY(launch_gemm_f16(dev, st, GEMM_F32, v->h16, n, l.v, nullptr, v->v, nullptr, 1.0f));
        }
        // rope2d is applied as K is rounded into its blocks and as the attention reads q
        HTR_TRY(launch_heads_f16(dev, st, v->k, v->v, v->kv, n, c.n_head, v->cs, px, max_pos));
        HTR_TRY(launch_attn_vision(dev, st, v->q, v->kv, v->a16, n, c.n_head, scale, v->cs, px, max_pos));
        HTR_TRY(launch_gemm_f16(dev, st, GEMM_ACC, v->a16, n, l.o, nullptr, v->x, nullptr, 1.0f));
        HTR_TRY(launch_rms_norm_f16(dev, st, v->x, l.ln2, v->h16, n, d, c.eps));
        HTR_TRY(launch_gemm_f16(dev, st, GEMM_FFN, v->h16, n, l.gate, l.up, nullptr, v->g16, 1.0f / FFN_DOWN_SCALE));
        HTR_TRY(launch_gemm_f16(dev, st, GEMM_ACC, v->g16, n, l.down, nullptr, v->x, nullptr, 1.0f));
    }
    if (n_layers >= 0) {
        HTR_TRY(htr_hip(dev, hipMemcpyAsync(d_out, v->x, (size_t)n * d * 4, hipMemcpyDeviceToDevice, st), "copy"));
        return htr_sync(dev);
    }
    // project (vision.rs:405-423): input_norm → unfold 2×2 → merger → mm.1 → gelu → mm.2
    const int n_out = n / 4;
    HTR_TRY(launch_rms_norm(dev, st, v->x, v->input_norm, v->tmp, n, d, c.eps));
    HTR_TRY(launch_unfold2x2(dev, st, v->tmp, v->q, px, py, d));
    // the projector's f32 activations as [hi | lo] against its weights [w | w]
    HTR_TRY(launch_split_f16(dev, st, v->q, n_out, 4 * d, 4 * d, 2, 0b10, v->xs));
    HTR_TRY(launch_gemm_f16(dev, st, GEMM_F32, v->xs, n_out, v->merger, nullptr, v->k, nullptr, 1.0f));
    HTR_TRY(launch_split_f16(dev, st, v->k, n_out, d, d, 2, 0b10, v->xs));
    HTR_TRY(launch_gemm_f16(dev, st, GEMM_F32, v->xs, n_out, v->mm1, nullptr, v->v, nullptr, 1.0f));
    HTR_TRY(launch_gelu(dev, st, v->v, (size_t)n_out * c.proj_dim));
    HTR_TRY(launch_split_f16(dev, st, v->v, n_out, c.proj_dim, c.proj_dim, 2, 0b10, v->xs));
    HTR_TRY(launch_gemm_f16(dev, st, GEMM_F32, v->xs, n_out, v->mm2, nullptr, d_out, nullptr, 1.0f));
    return htr_sync(dev);
}
