// GGUF reader and the streaming weight upload (ocr-gguf lib.rs:1-401, gpu.rs:1595-1677 Gpu::upload_tensor).
//
// The file layout is ggml's gguf.cpp (v2 / v3): magic "GGUF", version, tensor count, metadata count (u64s, little
// endian); metadata KVs (key string, value type, value; strings are u64 length + bytes, arrays element type + u64
// count + elements, not nested); tensor infos (name, n_dims ≤ 4, dims, ggml type, offset into the data section); the
// data section at the header's end rounded up to general.alignment (u32, a power of two, default 32). The reader
// parses the header from a prefix of the file (1 MiB, doubled while the header runs past it) and keeps a tensor as
// (offset, bytes, type, shape): the bytes stay in the file. Readable types: F32, F16, BF16, Q8_0 (lib.rs:98-130);
// any other is an error.
//
// Upload of a q8_0 tensor: the file range goes through two pinned 32 MiB host buffers (the next range is read while
// the last one is copied), a device staging buffer per host buffer, and k_repack_q8_0, which splits the 34-byte
// blocks into the weight's int8 plane and f16 scale plane on the device. GGUF rows are whole blocks and row-major,
// so block b lands at quants 32·b and scale b whatever the rows. The host never holds a whole tensor.
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <exception>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "htr_internal.h"

namespace {

constexpr uint64_t DEFAULT_ALIGNMENT = 32;
constexpr size_t FIRST_PREFIX = 1 << 20;
constexpr size_t STAGE_BYTES = (32u << 20) / 34 * 34;  // whole q8_0 blocks

struct Value {
    uint32_t type = 0;  // the GGUF value type (0 u8 … 12 f64, 8 string, 9 array)
    uint64_t u = 0;     // unsigned / bool
    int64_t i = 0;      // signed
    double f = 0;       // f32 / f64
    std::string s;
    uint32_t elem = 0;  // array element type
    std::vector<Value> arr;
};

// "the header ran past the prefix": read more
struct NeedMore {};

struct Cursor {
    const uint8_t *b;
    size_t n, pos = 0;
    const uint8_t *take(size_t k) {
        if (k > n - pos) throw NeedMore{};
        const uint8_t *p = b + pos;
        pos += k;
        return p;
    }
    template <typename T> T le() {
        T v;
        memcpy(&v, take(sizeof(T)), sizeof(T));
        return v;
    }
    std::string str() {
        const uint64_t k = le<uint64_t>();
        if (k > n) throw NeedMore{};
        const uint8_t *p = take((size_t)k);
        return std::string((const char *)p, (size_t)k);
    }
};

}  // namespace

struct htr_gguf {
    // the source: a file (fd ≥ 0) or the caller's reads
    int fd = -1;
    htr_read_fn read = nullptr;
    void *user = nullptr;
    uint64_t len = 0;
    uint32_t version = 0;
    uint64_t alignment = DEFAULT_ALIGNMENT, data_offset = 0;
    std::map<std::string, Value> meta;
    std::vector<GgufTensor> tensors;  // file order
    std::map<std::string, size_t> by_name;
};

namespace {

int src_read(htr_gguf *g, uint64_t off, void *buf, size_t n) {
    if (off > g->len || n > g->len - off) return htr_fail("read of %zu bytes at %llu: the source has %llu", n,
                                                          (unsigned long long)off, (unsigned long long)g->len);
    if (g->fd >= 0) {
        uint8_t *p = (uint8_t *)buf;
        while (n) {
            const ssize_t r = pread(g->fd, p, n, (off_t)off);
            if (r <= 0) return htr_fail("read of %zu bytes at %llu failed", n, (unsigned long long)off);
            p += r, off += (uint64_t)r, n -= (size_t)r;
        }
        return 0;
    }
    if (g->read(g->user, off, buf, n) != 0) return htr_fail("the source's read of %zu bytes at %llu failed", n,
                                                           (unsigned long long)off);
    return 0;
}

// a value of type ty (depth 0: arrays allowed); returns "" or the error
std::string parse_value(Cursor &c, uint32_t ty, int depth, Value &v) {
    v.type = ty;
    switch (ty) {
    case 0: v.u = c.le<uint8_t>(); break;
    case 1: v.i = c.le<int8_t>(); break;
    case 2: v.u = c.le<uint16_t>(); break;
    case 3: v.i = c.le<int16_t>(); break;
    case 4: v.u = c.le<uint32_t>(); break;
    case 5: v.i = c.le<int32_t>(); break;
    case 6: v.f = c.le<float>(); break;
    case 7: {
        const uint8_t b = c.le<uint8_t>();
        if (b > 1) return "GGUF bool value " + std::to_string(b);
        v.u = b;
        break;
    }
    case 8: v.s = c.str(); break;
    case 9: {
        if (depth > 0) return "GGUF nested arrays are not part of the format";
        v.elem = c.le<uint32_t>();
        const uint64_t n = c.le<uint64_t>();
        if (n > c.n - c.pos) throw NeedMore{};  // every element takes at least a byte of what is left
        v.arr.resize((size_t)n);
        for (uint64_t k = 0; k < n; k++) {
            std::string e = parse_value(c, v.elem, depth + 1, v.arr[(size_t)k]);
            if (!e.empty()) return e;
        }
        break;
    }
    case 10: v.u = c.le<uint64_t>(); break;
    case 11: v.i = c.le<int64_t>(); break;
    case 12: v.f = c.le<double>(); break;
    default: return "GGUF value type " + std::to_string(ty) + " unknown";
    }
    return "";
}

// (elements per block, bytes per block) of the readable ggml types (lib.rs:98-130), or {0, 0}
std::pair<uint64_t, uint64_t> type_block(uint32_t t) {
    switch (t) {
    case GGUF_F32: return {1, 4};
    case GGUF_F16:
    case GGUF_BF16: return {1, 2};
    case GGUF_Q8_0: return {32, 34};
    }
    return {0, 0};
}

// the header from a prefix of b bytes; returns "" (parsed), "more" (the prefix is too short) or the error
std::string parse_header(const uint8_t *b, size_t n, htr_gguf &g) {
    Cursor c{b, n};
    try {
        if (memcmp(c.take(4), "GGUF", 4) != 0) return "no GGUF magic";
        g.version = c.le<uint32_t>();
        if (g.version < 2 || g.version > 3) return "GGUF version " + std::to_string(g.version) + " (2 or 3 expected)";
        const uint64_t n_tensors = c.le<uint64_t>(), n_kv = c.le<uint64_t>();
        g.meta.clear();
        for (uint64_t k = 0; k < n_kv; k++) {
            std::string key = c.str();
            const uint32_t ty = c.le<uint32_t>();
            Value v;
            std::string e = parse_value(c, ty, 0, v);
            if (!e.empty()) return "metadata key " + key + ": " + e;
            if (!g.meta.emplace(key, std::move(v)).second) return "duplicate metadata key " + key;
        }
        g.alignment = DEFAULT_ALIGNMENT;
        auto al = g.meta.find("general.alignment");
        if (al != g.meta.end()) {
            if (al->second.type != 4) return "general.alignment has the wrong type";
            g.alignment = al->second.u;
        }
        if (g.alignment == 0 || (g.alignment & (g.alignment - 1)))
            return "general.alignment " + std::to_string(g.alignment) + " is not a power of two";
        g.tensors.clear();
        g.by_name.clear();
        for (uint64_t k = 0; k < n_tensors; k++) {
            GgufTensor t{};
            std::string name = c.str();
            const uint32_t n_dims = c.le<uint32_t>();
            if (n_dims == 0 || n_dims > 4) return "tensor " + name + ": " + std::to_string(n_dims) + " dimensions";
            t.n_dims = n_dims;
            for (uint32_t d = 0; d < n_dims; d++) t.shape[d] = c.le<uint64_t>();
            t.type = c.le<uint32_t>();
            const auto blk = type_block(t.type);
            if (blk.first == 0)
                return "tensor " + name + ": ggml type " + std::to_string(t.type) +
                       " is not supported (F32, F16, BF16, Q8_0 only)";
            t.offset = c.le<uint64_t>();
            if (t.offset % g.alignment)
                return "tensor " + name + ": offset " + std::to_string(t.offset) + " not aligned to " +
                       std::to_string(g.alignment);
            if (t.shape[0] % blk.first)
                return "tensor " + name + ": row of " + std::to_string(t.shape[0]) +
                       " elements is not a whole number of blocks";
            uint64_t elems = 1;
            for (uint32_t d = 0; d < n_dims; d++) {
                if (t.shape[d] && elems > UINT64_MAX / t.shape[d]) return "tensor " + name + ": shape overflows";
                elems *= t.shape[d];
            }
            t.n_elements = elems;
            if (elems / blk.first > UINT64_MAX / blk.second) return "tensor " + name + ": size overflows";
            t.n_bytes = elems / blk.first * blk.second;
            snprintf(t.name, sizeof t.name, "%s", name.c_str());
            if (name.size() >= sizeof t.name) return "tensor name " + name + " is too long";
            if (!g.by_name.emplace(name, g.tensors.size()).second) return "duplicate tensor " + name;
            g.tensors.push_back(t);
        }
        g.data_offset = (c.pos + g.alignment - 1) / g.alignment * g.alignment;
        for (GgufTensor &t : g.tensors) t.file_offset = g.data_offset + t.offset;
    } catch (NeedMore &) {
        return "more";
    }
    return "";
}

int open_parsed(htr_gguf *g, htr_gguf **out) {
    size_t want = FIRST_PREFIX;
    // a hostile header (counts, lengths) must end in an error, not in an exception through the C ABI
    try {
        for (;;) {
            const size_t n = (size_t)std::min<uint64_t>(want, g->len);
            std::vector<uint8_t> prefix(n);
            if (src_read(g, 0, prefix.data(), n) < 0) return -1;
            const std::string e = parse_header(prefix.data(), n, *g);
            if (e.empty()) break;
            if (e != "more") return htr_fail("%s", e.c_str());
            if (n >= g->len) return htr_fail("GGUF truncated: the header runs past the end of the file");
            want *= 2;
        }
    } catch (const std::exception &x) {
        return htr_fail("GGUF header: %s", x.what());
    }
    // every tensor inside the file (lib.rs:328-334), its end computed without overflowing
    const uint64_t len = g->len;
    for (const GgufTensor &t : g->tensors) {
        if (g->data_offset > len || t.offset > len - g->data_offset || t.n_bytes > len - g->data_offset - t.offset) {
            const uint64_t a = g->data_offset, b = t.offset, c = t.n_bytes;
            if (b > UINT64_MAX - a || c > UINT64_MAX - a - b)
                return htr_fail("tensor %s ends past byte 2^64 (%llu + %llu + %llu), the file has %llu", t.name,
                                (unsigned long long)a, (unsigned long long)b, (unsigned long long)c,
                                (unsigned long long)len);
            return htr_fail("tensor %s ends at byte %llu, the file has %llu", t.name, (unsigned long long)(a + b + c),
                            (unsigned long long)len);
        }
    }
    *out = g;
    return 0;
}

const Value *meta(htr_gguf *g, const char *key) {
    auto it = g->meta.find(key);
    if (it == g->meta.end()) {
        htr_fail("GGUF has no metadata key %s", key);
        return nullptr;
    }
    return &it->second;
}

// 34-byte q8_0 blocks (2-byte aligned: f16 d little endian, 32 × i8) → quants q[32·b …] and scales d[b]
__global__ __launch_bounds__(256) void k_repack_q8_0(const uint8_t *blk, size_t n_blocks, int8_t *q, uint16_t *d) {
    for (size_t b = blockIdx.x * (size_t)256 + threadIdx.x; b < n_blocks; b += (size_t)gridDim.x * 256) {
        const uint16_t *p = reinterpret_cast<const uint16_t *>(blk + 34 * b);
        d[b] = p[0];
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; i++) w[i] = (uint32_t)p[1 + 2 * i] | ((uint32_t)p[2 + 2 * i] << 16);
        int4 *o = reinterpret_cast<int4 *>(q + 32 * b);
        o[0] = make_int4((int)w[0], (int)w[1], (int)w[2], (int)w[3]);
        o[1] = make_int4((int)w[4], (int)w[5], (int)w[6], (int)w[7]);
    }
}

// a vision weight's values (BF16 or F32, n of them, starting on an even element of the tensor) × scale → f16 (OUT_F32:
// the f16 values widened to f32 for a BF16 source, an F32 source's own values). f16_from_bf16.wgsl: each pair of
// values (one 32-bit word of a BF16 tensor) holding a magnitude above 65504 counts once into *over
template <bool BF16, bool OUT_F32>
__global__ __launch_bounds__(256) void k_vision_weight(const void *src, size_t n, float scale, void *dst,
                                                       unsigned *over) {
    const size_t pairs = (n + 1) / 2;
    for (size_t p = blockIdx.x * (size_t)256 + threadIdx.x; p < pairs; p += (size_t)gridDim.x * 256) {
        const size_t i = 2 * p;
        const bool two = i + 1 < n;
        float v0, v1 = 0.0f;
        if constexpr (BF16) {
            const uint16_t *s = static_cast<const uint16_t *>(src);
            v0 = __uint_as_float((uint32_t)s[i] << 16);
            if (two) v1 = __uint_as_float((uint32_t)s[i + 1] << 16);
        } else {
            const float *s = static_cast<const float *>(src);
            v0 = s[i];
            if (two) v1 = s[i + 1];
        }
        v0 *= scale;
        v1 *= scale;
        const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
        if constexpr (OUT_F32) {
            float *d = static_cast<float *>(dst);
            d[i] = BF16 ? (float)h0 : v0;
            if (two) d[i + 1] = BF16 ? (float)h1 : v1;
        } else {
            _Float16 *d = static_cast<_Float16 *>(dst);
            d[i] = h0;
            if (two) d[i + 1] = h1;
        }
        if constexpr (BF16 || !OUT_F32) {
            // one atomic a wave: lane 0 is active whenever any lane of its wave is (p rises with the lane)
            const unsigned long long m = __ballot(fabsf(v0) > 65504.0f || fabsf(v1) > 65504.0f);
            if ((threadIdx.x & 63) == 0 && m) atomicAdd(over, (unsigned)__popcll(m));
        }
    }
}

}  // namespace

std::string gguf_shape_str(const GgufTensor &t) {
    std::string s = "[";
    for (uint32_t k = 0; k < t.n_dims; k++) s += (k ? ", " : "") + std::to_string(t.shape[k]);
    return s + "]";
}

const char *ggml_type_name(uint32_t ty) {
    switch (ty) {
    case GGUF_F32: return "F32";
    case GGUF_F16: return "F16";
    case GGUF_Q8_0: return "Q8_0";
    case GGUF_BF16: return "BF16";
    default: return "an unknown ggml type";
    }
}

// ---- the streaming upload ---------------------------------------------------------------------------------------------

GgufStager::~GgufStager() {
    for (int i = 0; i < 2; i++) {
        if (ev[i]) {
            hipEventSynchronize(ev[i]);
            hipEventDestroy(ev[i]);
        }
        if (host[i]) hipHostFree(host[i]);
        if (dev_buf[i]) htr_dev_free(dev, dev_buf[i]);
    }
}

int GgufStager::init(htr_device *d) {
    dev = d;
    for (int i = 0; i < 2; i++) {
        hipError_t e = hipHostMalloc(&host[i], STAGE_BYTES, hipHostMallocDefault);
        if (e != hipSuccess) return htr_fail("hipHostMalloc of the upload staging: %s", hipGetErrorString(e));
        HTR_TRY(htr_dev_alloc(dev, STAGE_BYTES, HTR_MEM_WORK, &dev_buf[i]));
        if ((e = hipEventCreateWithFlags(&ev[i], hipEventDisableTiming)) != hipSuccess)
            return htr_fail("hipEventCreate: %s", hipGetErrorString(e));
    }
    return 0;
}

int gguf_find(htr_gguf *g, const char *name, const GgufTensor **out) {
    auto it = g->by_name.find(name);
    if (it == g->by_name.end()) return htr_fail("GGUF has no tensor %s", name);
    *out = &g->tensors[it->second];
    return 0;
}

bool gguf_has(htr_gguf *g, const char *name) { return g->by_name.count(name) != 0; }

int gguf_upload_q8_0(GgufStager &sg, htr_gguf *g, const GgufTensor &t, size_t rows, size_t cols, htr_weight **out) {
    htr_device *dev = sg.dev;
    if (t.type != GGUF_Q8_0) return htr_fail("%s: ggml type %u — the text decoder's kernels read q8_0 weights", t.name, t.type);
    if (t.n_dims != 2 || t.shape[0] != cols || t.shape[1] != rows)
        return htr_fail("%s: shape [%llu, %llu], expected [%zu, %zu]", t.name, (unsigned long long)t.shape[0],
                        (unsigned long long)(t.n_dims > 1 ? t.shape[1] : 1), cols, rows);
    auto *w = new htr_weight;
    w->dev = dev;
    w->rows = rows;
    w->cols = cols;
    const size_t n_blocks = rows * cols / 32;
    int rc = htr_dev_alloc(dev, rows * cols, HTR_MEM_WEIGHTS, (void **)&w->q);
    // the scale plane has 16 bytes of slack: the matvec's scale staging reads whole 16-byte units
    if (rc == 0) rc = htr_dev_alloc(dev, n_blocks * 2 + 16, HTR_MEM_WEIGHTS, (void **)&w->d);
    const size_t per = STAGE_BYTES / 34;
    for (size_t b0 = 0; b0 < n_blocks && rc == 0; b0 += per) {
        const size_t nb = std::min(per, n_blocks - b0);
        const int i = sg.next;
        sg.next ^= 1;
        hipError_t e = hipEventSynchronize(sg.ev[i]);  // the copy out of this buffer two ranges ago is done
        if (e != hipSuccess) rc = htr_fail("hipEventSynchronize: %s", hipGetErrorString(e));
        if (rc == 0) rc = src_read(g, t.file_offset + 34 * (uint64_t)b0, sg.host[i], nb * 34);
        if (rc == 0 && (e = hipMemcpyAsync(sg.dev_buf[i], sg.host[i], nb * 34, hipMemcpyHostToDevice, dev->stream)) !=
                           hipSuccess)
            rc = htr_fail("hipMemcpyAsync: %s", hipGetErrorString(e));
        if (rc == 0) {
            const int grid = (int)std::min<size_t>((nb + 255) / 256, (size_t)dev->n_cu * 8);
            hipLaunchKernelGGL(k_repack_q8_0, dim3(grid), dim3(256), 0, dev->stream, (const uint8_t *)sg.dev_buf[i],
                               nb, w->q + 32 * b0, (uint16_t *)w->d + b0);
            rc = htr_launched(dev, "k_repack_q8_0");
        }
        if (rc == 0 && (e = hipEventRecord(sg.ev[i], dev->stream)) != hipSuccess)
            rc = htr_fail("hipEventRecord: %s", hipGetErrorString(e));
    }
    if (rc < 0) {
        std::string keep = htr_last_error();
        htr_weight_free(w);
        return htr_fail("%s", keep.c_str());
    }
    *out = w;
    return 0;
}

int gguf_upload_f32(GgufStager &sg, htr_gguf *g, const GgufTensor &t, size_t n, float **out) {
    if (t.type != GGUF_F32 || t.n_dims != 1 || t.shape[0] != n)
        return htr_fail("%s: ggml type %u, %u dims [%llu …], expected F32 [%zu]", t.name, t.type, t.n_dims,
                        (unsigned long long)t.shape[0], n);
    if (n * 4 > STAGE_BYTES) return htr_fail("%s: %zu values is not a vector", t.name, n);
    const int i = sg.next;
    sg.next ^= 1;
    hipError_t e = hipEventSynchronize(sg.ev[i]);
    if (e != hipSuccess) return htr_fail("hipEventSynchronize: %s", hipGetErrorString(e));
    HTR_TRY(src_read(g, t.file_offset, sg.host[i], n * 4));
    HTR_TRY(htr_dev_alloc(sg.dev, n * 4, HTR_MEM_WEIGHTS, (void **)out));
    if ((e = hipMemcpyAsync(*out, sg.host[i], n * 4, hipMemcpyHostToDevice, sg.dev->stream)) != hipSuccess)
        return htr_fail("hipMemcpyAsync: %s", hipGetErrorString(e));
    if ((e = hipEventRecord(sg.ev[i], sg.dev->stream)) != hipSuccess)
        return htr_fail("hipEventRecord: %s", hipGetErrorString(e));
    return 0;
}

// vision.rs:117-142 weight(): the shape check ([cols…, rows]: the last dimension is the output row), BF16 or F32,
// then the device conversion of each staged range into dst16 (f16) or dst32 (f32)
int gguf_upload_vision(GgufStager &sg, htr_gguf *g, const GgufTensor &t, size_t rows, size_t cols, float scale,
                       unsigned *d_over, _Float16 *dst16, float *dst32) {
    htr_device *dev = sg.dev;
    uint64_t inner = 1;
    for (uint32_t k = 0; k + 1 < t.n_dims; k++) inner *= t.shape[k];
    if (t.n_dims < 1 || t.shape[t.n_dims - 1] != rows || inner != cols)
        return htr_fail("%s: shape %s, expected %zu values × %zu rows", t.name, gguf_shape_str(t).c_str(), cols, rows);
    if (t.type != GGUF_BF16 && t.type != GGUF_F32)
        return htr_fail("%s: %s weights are not supported in the vision encoder", t.name, ggml_type_name(t.type));
    const bool bf16 = t.type == GGUF_BF16;
    const size_t es = bf16 ? 2 : 4, n = rows * cols;
    const size_t per = STAGE_BYTES / 4 / 256 * 256;  // values a staged range: even, whole for either width
    for (size_t e0 = 0; e0 < n; e0 += per) {
        const size_t ne = std::min(per, n - e0);
        const int i = sg.next;
        sg.next ^= 1;
        hipError_t e = hipEventSynchronize(sg.ev[i]);
        if (e != hipSuccess) return htr_fail("hipEventSynchronize: %s", hipGetErrorString(e));
        HTR_TRY(src_read(g, t.file_offset + es * (uint64_t)e0, sg.host[i], ne * es));
        if ((e = hipMemcpyAsync(sg.dev_buf[i], sg.host[i], ne * es, hipMemcpyHostToDevice, dev->stream)) != hipSuccess)
            return htr_fail("hipMemcpyAsync: %s", hipGetErrorString(e));
        const int grid = (int)std::min<size_t>((ne / 2 + 256) / 256, (size_t)dev->n_cu * 8);
        void *dst = dst32 ? (void *)(dst32 + e0) : (void *)(dst16 + e0);
        if (bf16 && dst32)
            hipLaunchKernelGGL((k_vision_weight<true, true>), dim3(grid), dim3(256), 0, dev->stream, sg.dev_buf[i], ne,
                               scale, dst, d_over);
        else if (bf16)
            hipLaunchKernelGGL((k_vision_weight<true, false>), dim3(grid), dim3(256), 0, dev->stream, sg.dev_buf[i], ne,
                               scale, dst, d_over);
        else if (dst32)
            hipLaunchKernelGGL((k_vision_weight<false, true>), dim3(grid), dim3(256), 0, dev->stream, sg.dev_buf[i], ne,
                               scale, dst, d_over);
        else
            hipLaunchKernelGGL((k_vision_weight<false, false>), dim3(grid), dim3(256), 0, dev->stream, sg.dev_buf[i],
                               ne, scale, dst, d_over);
        HTR_TRY(htr_launched(dev, "k_vision_weight"));
        if ((e = hipEventRecord(sg.ev[i], dev->stream)) != hipSuccess)
            return htr_fail("hipEventRecord: %s", hipGetErrorString(e));
    }
    return 0;
}

int gguf_meta_bool(htr_gguf *g, const char *key, bool *out) {
    const Value *v = meta(g, key);
    if (!v) return -1;
    if (v->type != 7) return htr_fail("%s is of GGUF type %u, not bool", key, v->type);
    *out = v->u != 0;
    return 0;
}

int gguf_meta_f32_array(htr_gguf *g, const char *key, std::vector<float> *out) {
    const Value *v = meta(g, key);
    if (!v) return -1;
    if (v->type != 9) return htr_fail("%s is of GGUF type %u, not an array", key, v->type);
    if (v->elem != 6) return htr_fail("%s holds GGUF type %u, not f32", key, v->elem);
    out->clear();
    for (const Value &x : v->arr) out->push_back((float)x.f);
    return 0;
}

int gguf_meta_u32(htr_gguf *g, const char *key, uint32_t *out) {
    const Value *v = meta(g, key);
    if (!v) return -1;
    if (v->type == 4) *out = (uint32_t)v->u;
    else if (v->type == 5 && v->i >= 0) *out = (uint32_t)v->i;  // lib.rs:404-410: a non-negative i32 reads as u32
    else return htr_fail("%s is of GGUF type %u, not u32", key, v->type);
    return 0;
}

int gguf_meta_f32(htr_gguf *g, const char *key, float *out) {
    const Value *v = meta(g, key);
    if (!v) return -1;
    if (v->type != 6) return htr_fail("%s is of GGUF type %u, not f32", key, v->type);
    *out = (float)v->f;
    return 0;
}

int gguf_meta_str(htr_gguf *g, const char *key, std::string *out) {
    const Value *v = meta(g, key);
    if (!v) return -1;
    if (v->type != 8) return htr_fail("%s is of GGUF type %u, not a string", key, v->type);
    *out = v->s;
    return 0;
}

bool gguf_has_key(htr_gguf *g, const char *key) { return g->meta.count(key) != 0; }

// ---- ABI ------------------------------------------------------------------------------------------------------------

extern "C" int htr_gguf_open(const char *path, htr_gguf **out) {
    if (!path || !out) return htr_fail("htr_gguf_open: null argument");
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return htr_fail("cannot open %s", path);
    auto *g = new htr_gguf;
    g->fd = fd;
    const off_t end = lseek(fd, 0, SEEK_END);
    if (end < 0) {
        htr_gguf_close(g);
        return htr_fail("cannot size %s", path);
    }
    g->len = (uint64_t)end;
    if (open_parsed(g, out) < 0) {
        const std::string keep = htr_last_error();
        htr_gguf_close(g);
        return htr_fail("%s is not a readable GGUF: %s", path, keep.c_str());
    }
    return 0;
}

extern "C" int htr_gguf_open_source(uint64_t len, htr_read_fn read, void *user, htr_gguf **out) {
    if (!read || !out) return htr_fail("htr_gguf_open_source: null argument");
    auto *g = new htr_gguf;
    g->read = read;
    g->user = user;
    g->len = len;
    if (open_parsed(g, out) < 0) {
        const std::string keep = htr_last_error();
        htr_gguf_close(g);
        return htr_fail("%s", keep.c_str());
    }
    return 0;
}

extern "C" int htr_gguf_close(htr_gguf *g) {
    if (!g) return 0;
    if (g->fd >= 0) close(g->fd);
    delete g;
    return 0;
}

extern "C" int htr_gguf_header(htr_gguf *g, uint32_t *version, uint64_t *alignment, uint64_t *data_offset,
                               size_t *n_tensors) {
    if (!g) return htr_fail("htr_gguf_header: null file");
    if (version) *version = g->version;
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_offset;
    if (n_tensors) *n_tensors = g->tensors.size();
    return 0;
}

extern "C" int htr_gguf_tensor(htr_gguf *g, const char *name, size_t index, htr_gguf_tensor_info *out) {
    if (!g || !out) return htr_fail("htr_gguf_tensor: null argument");
    const GgufTensor *t;
    if (name) {
        HTR_TRY(gguf_find(g, name, &t));
    } else {
        if (index >= g->tensors.size()) return htr_fail("tensor %zu: the GGUF has %zu", index, g->tensors.size());
        t = &g->tensors[index];
    }
    *out = *t;
    return 0;
}

extern "C" int htr_gguf_u32(htr_gguf *g, const char *key, uint32_t *out) {
    if (!g || !key || !out) return htr_fail("htr_gguf_u32: null argument");
    return gguf_meta_u32(g, key, out);
}

extern "C" int htr_gguf_f32(htr_gguf *g, const char *key, float *out) {
    if (!g || !key || !out) return htr_fail("htr_gguf_f32: null argument");
    return gguf_meta_f32(g, key, out);
}

extern "C" int htr_gguf_str(htr_gguf *g, const char *key, char *buf, size_t cap, size_t *len) {
    if (!g || !key) return htr_fail("htr_gguf_str: null argument");
    std::string s;
    HTR_TRY(gguf_meta_str(g, key, &s));
    if (len) *len = s.size();
    if (buf && cap) {
        const size_t n = std::min(cap - 1, s.size());
        memcpy(buf, s.data(), n);
        buf[n] = 0;
    }
    return 0;
}

extern "C" int htr_gguf_f32_array(htr_gguf *g, const char *key, float *out, size_t cap, size_t *len) {
    if (!g || !key) return htr_fail("htr_gguf_f32_array: null argument");
    const Value *v = meta(g, key);
    if (!v) return -1;
    if (v->type != 9) return htr_fail("%s is of GGUF type %u, not an array", key, v->type);
    if (v->elem != 6) return htr_fail("%s holds GGUF type %u, not f32", key, v->elem);
    if (len) *len = v->arr.size();
    for (size_t k = 0; out && k < v->arr.size() && k < cap; k++) out[k] = (float)v->arr[k].f;
    return 0;
}

extern "C" int htr_gguf_read_small(htr_gguf *g, const char *name, void *buf, size_t cap) {
    if (!g || !name || !buf) return htr_fail("htr_gguf_read_small: null argument");
    const GgufTensor *t;
    HTR_TRY(gguf_find(g, name, &t));
    if (t->n_bytes > (1u << 20))
        return htr_fail("%s: %llu bytes is not small — stream it (htr_text_model_load_gguf)", name,
                        (unsigned long long)t->n_bytes);
    if (cap < t->n_bytes) return htr_fail("%s: %llu bytes into %zu", name, (unsigned long long)t->n_bytes, cap);
    return src_read(g, t->file_offset, buf, (size_t)t->n_bytes);
}
