// The device runtime of libhtr: device open / close, the sticky health latch and fatal hook (the reference's Health,
// gpu.rs:900-970, and FatalHook, gpu.rs:884-897), device memory with a ledger per kind (gpu.rs:509-561), host ↔ device
// copies (gpu.rs:1489-1590), q8_0 weight repacking (gpu.rs:1595-1677 upload_tensor), and the seeded synthetic inputs.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include <rocprofiler-sdk-roctx/roctx.h>

#include "htr_internal.h"

// ---- errors ---------------------------------------------------------------------------------------------------------

static thread_local std::string g_err;

int htr_fail(const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return -1;
}

extern "C" const char *htr_last_error(void) { return g_err.c_str(); }

int htr_latch(htr_device *dev, const char *kind, const char *msg) {
    if (dev->dead_msg.empty()) {
        dev->dead_kind = kind;
        dev->dead_msg = msg;
        if (dev->hook) dev->hook(kind, msg, dev->hook_user);
    }
    return htr_fail("device %d is dead (%s): %s", dev->ordinal, dev->dead_kind.c_str(), dev->dead_msg.c_str());
}

int htr_check_alive(htr_device *dev) {
    if (!dev) return htr_fail("null device");
    if (!dev->dead_msg.empty())
        return htr_fail("device %d is dead (%s): %s", dev->ordinal, dev->dead_kind.c_str(), dev->dead_msg.c_str());
    return 0;
}

int htr_hip(htr_device *dev, hipError_t e, const char *what) {
    if (e == hipSuccess) return 0;
    (void)hipGetLastError();  // the runtime's per-thread error is this one: clear it for later launch checks
    char msg[512];
    snprintf(msg, sizeof msg, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
    const char *kind = e == hipErrorOutOfMemory ? "outOfMemory" : (e == hipErrorInvalidValue ? "validation" : "internal");
    return htr_latch(dev, kind, msg);
}

int htr_launched(htr_device *dev, const char *kernel) {
    dev->last_kernel = kernel;
    return htr_hip(dev, hipGetLastError(), kernel);
}

int htr_check_not_capturing(htr_device *dev, const char *what) {
    if (dev->capturing) return htr_fail("%s: the device's stream is being captured (htr_capture_begin)", what);
    return 0;
}

extern "C" int htr_debug_last_kernel(htr_device *dev, char *name, size_t cap) {
    if (!dev || !name || !cap) return htr_fail("htr_debug_last_kernel: null argument");
    snprintf(name, cap, "%s", dev->last_kernel.c_str());
    return 0;
}

// ---- device ---------------------------------------------------------------------------------------------------------

extern "C" int htr_device_open(int ordinal, htr_device **out) {
    if (!out) return htr_fail("htr_device_open: null out");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return htr_fail("no HIP device (%s)", hipGetErrorString(e));
    if (ordinal < 0 || ordinal >= n) return htr_fail("device %d: %d devices present", ordinal, n);
    if ((e = hipSetDevice(ordinal)) != hipSuccess) return htr_fail("hipSetDevice(%d): %s", ordinal, hipGetErrorString(e));
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, ordinal)) != hipSuccess)
        return htr_fail("hipGetDeviceProperties: %s", hipGetErrorString(e));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return htr_fail("device %d is %s: this library is built for gfx950 (MI355X) only", ordinal, prop.gcnArchName);
    auto *dev = new htr_device;
    dev->ordinal = ordinal;
    const char *graphs = getenv("HTR_GRAPHS");
    dev->use_graphs = !(graphs && strcmp(graphs, "0") == 0);
    // gpu.rs:739-768, 821-823, 1307-1310 (OCR_WGPU_POISON=1): a diagnostic fill of fresh and given-back memory
    const char *poison = getenv("HTR_POISON");
    dev->poison = poison && strcmp(poison, "1") == 0;
    // gpu.rs:1107-1115: OCR_WGPU_COMPUTE forces a compute path (coop and f16 are one path here: f16 operands into the
    // matrix cores, f32 sums); unset, the best one — f16 on matrix units, as Compute::choose picks on such a device
    if (const char *want = getenv("OCR_WGPU_COMPUTE")) {
        if (strcmp(want, "f32") == 0) {
            dev->compute = HTR_COMPUTE_F32;
        } else if (strcmp(want, "f16") == 0 || strcmp(want, "coop") == 0) {
            dev->compute = HTR_COMPUTE_F16;
        } else {
            delete dev;
            return htr_fail("OCR_WGPU_COMPUTE=%s: f32, f16 or coop", want);
        }
    }
    snprintf(dev->name, sizeof dev->name, "%s (%s)", prop.name, prop.gcnArchName);
    dev->n_cu = prop.multiProcessorCount;
    // default priority: one stream for every launch of this device
    if ((e = hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking)) != hipSuccess) {
        delete dev;
        return htr_fail("hipStreamCreate: %s", hipGetErrorString(e));
    }
    dev->pinned_bytes = 1 << 20;
    if ((e = hipHostMalloc(&dev->pinned, dev->pinned_bytes, hipHostMallocDefault)) != hipSuccess) {
        hipStreamDestroy(dev->stream);
        delete dev;
        return htr_fail("hipHostMalloc: %s", hipGetErrorString(e));
    }
    if ((e = hipEventCreate(&dev->t0)) != hipSuccess || (e = hipEventCreate(&dev->t1)) != hipSuccess) {
        hipHostFree(dev->pinned);
        hipStreamDestroy(dev->stream);
        delete dev;
        return htr_fail("hipEventCreate: %s", hipGetErrorString(e));
    }
    // with the device current: its address of the allocation-free attention's scratch array
    if (attn_static_scratch_init(dev) < 0) {
        std::string keep = htr_last_error();
        hipEventDestroy(dev->t0);
        hipEventDestroy(dev->t1);
        hipHostFree(dev->pinned);
        hipStreamDestroy(dev->stream);
        delete dev;
        return htr_fail("%s", keep.c_str());
    }
    // how a launch places its workgroups on the 8 XCDs, and whether a word stored at workgroup scope is seen across an
    // XCD's workgroups (token_step_xcds), checked once here: the one-launch decode step and the decode attention's
    // XCD-local merge rest on both
    const char *why = nullptr;
    if (token_step_xcds(dev, &why) < 0) {
        std::string keep = htr_last_error();
        htr_device_close(dev);
        return htr_fail("%s", keep.c_str());
    }
    *out = dev;
    return 0;
}

extern "C" int htr_device_set_compute(htr_device *dev, int compute) {
    if (!dev) return htr_fail("htr_device_set_compute: null device");
    if (compute != HTR_COMPUTE_F32 && compute != HTR_COMPUTE_F16)
        return htr_fail("compute path %d: HTR_COMPUTE_F32 (%d) or HTR_COMPUTE_F16 (%d)", compute, HTR_COMPUTE_F32,
                        HTR_COMPUTE_F16);
    dev->compute = compute;
    return 0;
}

extern "C" int htr_device_compute(htr_device *dev, int *compute) {
    if (!dev || !compute) return htr_fail("htr_device_compute: null argument");
    *compute = dev->compute;
    return 0;
}

extern "C" int htr_timer_begin(htr_device *dev) {
    HTR_TRY(htr_check_alive(dev));
    return htr_hip(dev, hipEventRecord(dev->t0, dev->stream), "hipEventRecord");
}

extern "C" int htr_timer_end(htr_device *dev, float *ms) {
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(htr_check_not_capturing(dev, "htr_timer_end"));
    if (!ms) return htr_fail("htr_timer_end: null out");
    HTR_TRY(htr_hip(dev, hipEventRecord(dev->t1, dev->stream), "hipEventRecord"));
    HTR_TRY(htr_hip(dev, hipEventSynchronize(dev->t1), "hipEventSynchronize"));
    return htr_hip(dev, hipEventElapsedTime(ms, dev->t0, dev->t1), "hipEventElapsedTime");
}

extern "C" int htr_device_close(htr_device *dev) {
    if (!dev) return 0;
    if (dev->phase_open) roctxRangePop();
    hipSetDevice(dev->ordinal);
    if (dev->capturing) {  // a capture left open: end it and drop what it recorded
        hipGraph_t g = nullptr;
        if (hipStreamEndCapture(dev->stream, &g) == hipSuccess && g) hipGraphDestroy(g);
        dev->capturing = false;
    }
    if (dev->dead_msg.empty()) hipStreamSynchronize(dev->stream);
    for (auto &a : dev->allocs) hipFree(a.first);
    dev->allocs.clear();
    if (dev->pinned) hipHostFree(dev->pinned);
    if (dev->t0) hipEventDestroy(dev->t0);
    if (dev->t1) hipEventDestroy(dev->t1);
    hipStreamDestroy(dev->stream);
    delete dev;
    return 0;
}

extern "C" int htr_alive(htr_device *dev) { return htr_check_alive(dev); }

extern "C" int htr_set_fatal_hook(htr_device *dev, htr_fatal_hook hook, void *user) {
    if (!dev) return htr_fail("null device");
    dev->hook = hook;
    dev->hook_user = user;
    return 0;
}

extern "C" int htr_debug_mark_lost(htr_device *dev, const char *why) {
    if (!dev) return htr_fail("null device");
    htr_latch(dev, "destroyed", why && *why ? why : "marked lost by htr_debug_mark_lost");
    return 0;
}

extern "C" int htr_sync(htr_device *dev) {
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(htr_check_not_capturing(dev, "htr_sync"));
    return htr_hip(dev, hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
}

// ---- stream capture into HIP graphs -----------------------------------------------------------------------------------

struct htr_graph {
    htr_device *dev = nullptr;
    hipGraphExec_t exec = nullptr;
};

extern "C" int htr_capture_begin(htr_device *dev) {
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(htr_check_not_capturing(dev, "htr_capture_begin"));
    HTR_TRY(htr_hip(dev, hipStreamBeginCapture(dev->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture"));
    dev->capturing = true;
    return 0;
}

extern "C" int htr_capture_end(htr_device *dev, htr_graph **out) {
    if (!dev || !out) return htr_fail("htr_capture_end: null argument");
    if (!dev->capturing) return htr_fail("htr_capture_end: no capture in progress");
    dev->capturing = false;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(dev->stream, &graph);
    HTR_TRY(htr_hip(dev, e, "hipStreamEndCapture"));
    auto *g = new htr_graph;
    g->dev = dev;
    e = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
    hipGraphDestroy(graph);
    if (e != hipSuccess) {
        delete g;
        return htr_hip(dev, e, "hipGraphInstantiate");
    }
    *out = g;
    return 0;
}

extern "C" int htr_graph_launch(htr_graph *g) {
    if (!g) return htr_fail("htr_graph_launch: null graph");
    HTR_TRY(htr_check_alive(g->dev));
    HTR_TRY(htr_check_not_capturing(g->dev, "htr_graph_launch"));
    return htr_hip(g->dev, hipGraphLaunch(g->exec, g->dev->stream), "hipGraphLaunch");
}

extern "C" int htr_graph_free(htr_graph *g) {
    if (!g) return 0;
    if (g->exec) hipGraphExecDestroy(g->exec);
    delete g;
    return 0;
}

extern "C" int htr_device_info(htr_device *dev, char *name, size_t name_len, int *n_cu) {
    if (!dev) return htr_fail("null device");
    if (name && name_len) snprintf(name, name_len, "%s", dev->name);
    if (n_cu) *n_cu = dev->n_cu;
    return 0;
}

// gpu.rs:1349-1358 Gpu::phase: the label of the following work. Here a roctx range on the calling thread (what
// rocprofv3 --marker-trace records): the device's open range, if any, ends; a name other than NULL, "" or "-" opens
// the next one
extern "C" int htr_phase(htr_device *dev, const char *name) {
    HTR_TRY(htr_check_alive(dev));
    if (dev->phase_open) {
        roctxRangePop();
        dev->phase_open = false;
    }
    if (name && *name && strcmp(name, "-") != 0) {
        roctxRangePushA(name);
        dev->phase_open = true;
    }
    return 0;
}

// ---- memory ---------------------------------------------------------------------------------------------------------

static uint64_t *ledger(htr_device *dev, int kind) {
    switch (kind) {
    case HTR_MEM_WEIGHTS: return &dev->live.weights;
    case HTR_MEM_KV_CACHE: return &dev->live.kv_cache;
    case HTR_MEM_READBACK: return &dev->live.readback;
    default: return &dev->live.work;
    }
}

// HTR_POISON=1 (the reference's OCR_WGPU_POISON=1, gpu.rs:739-768, 821-823): memory is 0xFF bytes — NaN as f32 and
// f16 — when it is handed out (htr_dev_alloc_zero's excepted) and again when it is given back, so a kernel that reads
// what nothing wrote reads NaN, and one that reads memory after it was freed (a launch outliving its buffer) too
static int fill_new(htr_device *dev, void *p, size_t b, bool zero) {
    return htr_hip(dev, hipMemsetAsync(p, zero || !dev->poison ? 0 : 0xFF, b, dev->stream), "hipMemsetAsync");
}

static int alloc_filled(htr_device *dev, size_t bytes, int kind, bool zero, void **out) {
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(htr_check_not_capturing(dev, "device allocation"));
    if (kind < HTR_MEM_WEIGHTS || kind > HTR_MEM_READBACK) return htr_fail("memory kind %d: 0…3", kind);
    size_t b = std::max<size_t>(bytes, 4);
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, b);
    if (e != hipSuccess) {
        char what[128];
        snprintf(what, sizeof what, "hipMalloc(%zu bytes)", b);
        return htr_hip(dev, e, what);
    }
    HTR_TRY(fill_new(dev, p, b, zero));
    dev->allocs[p] = {b, kind};
    *ledger(dev, kind) += b;
    *out = p;
    return 0;
}

int htr_dev_alloc(htr_device *dev, size_t bytes, int kind, void **out) { return alloc_filled(dev, bytes, kind, false, out); }

int htr_dev_alloc_zero(htr_device *dev, size_t bytes, int kind, void **out) {
    return alloc_filled(dev, bytes, kind, true, out);
}

int htr_dev_free(htr_device *dev, void *p) {
    if (!p) return 0;
    auto it = dev->allocs.find(p);
    if (it == dev->allocs.end()) return htr_fail("htr_free: %p is not an allocation of device %d", p, dev->ordinal);
    HTR_TRY(htr_check_not_capturing(dev, "htr_free"));
    // the stream's work that may still read it finishes first (a Buf outlives every submission that binds it)
    if (dev->dead_msg.empty()) {
        if (dev->poison) hipMemsetAsync(p, 0xFF, it->second.first, dev->stream);
        hipStreamSynchronize(dev->stream);
    }
    *ledger(dev, it->second.second) -= it->second.first;
    dev->allocs.erase(it);
    hipFree(p);
    return 0;
}

int htr_scratch(htr_device *dev, int slot, size_t bytes, void **out) {
    if (dev->scratch_bytes[slot] < bytes) {
        if (dev->scratch[slot]) HTR_TRY(htr_dev_free(dev, dev->scratch[slot]));
        dev->scratch[slot] = nullptr;
        dev->scratch_bytes[slot] = 0;
        // the self-resetting words (best keys, tickets) start at zero; the rest is written before it is read
        const bool zero = slot == SCR_CHOOSE_PART || slot == SCR_CHOOSE_CNT || slot == SCR_ATTN_CNT;
        HTR_TRY(alloc_filled(dev, bytes, HTR_MEM_WORK, zero, &dev->scratch[slot]));
        dev->scratch_bytes[slot] = bytes;
    }
    *out = dev->scratch[slot];
    return 0;
}

extern "C" int htr_mem_live(htr_device *dev, htr_gpu_bytes *out) {
    if (!dev || !out) return htr_fail("htr_mem_live: null argument");
    *out = dev->live;
    return 0;
}

extern "C" int htr_alloc(htr_device *dev, size_t bytes, int kind, void **d_out) {
    if (!d_out) return htr_fail("htr_alloc: null out");
    return htr_dev_alloc(dev, bytes, kind, d_out);
}

extern "C" int htr_free(htr_device *dev, void *d_ptr) {
    if (!dev) return htr_fail("null device");
    return htr_dev_free(dev, d_ptr);
}

extern "C" int htr_upload(htr_device *dev, void *d_dst, const void *h_src, size_t bytes) {
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(htr_check_not_capturing(dev, "htr_upload"));
    if (!bytes) return 0;
    HTR_TRY(htr_hip(dev, hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, dev->stream), "upload"));
    // pageable source: the copy is complete once the stream reaches it; waiting keeps the caller's buffer free to reuse
    return htr_hip(dev, hipStreamSynchronize(dev->stream), "upload sync");
}

extern "C" int htr_download(htr_device *dev, void *h_dst, const void *d_src, size_t bytes) {
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(htr_check_not_capturing(dev, "htr_download"));
    if (!bytes) return 0;
    HTR_TRY(htr_hip(dev, hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, dev->stream), "download"));
    return htr_hip(dev, hipStreamSynchronize(dev->stream), "download sync");
}

// ---- device copy (gpu.rs:2102-2110 Batch::copy → copy_words.wgsl) ---------------------------------------------------

// dst[i] = src[i] over n 16-byte units (grid-stride, non-temporal: a copy touches each byte once), then the tail of
// < 16 bytes
typedef int gint4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void k_copy16(const int4 *src, int4 *dst, size_t n16, const uint8_t *src_tail,
                                                uint8_t *dst_tail, int tail) {
    const auto *s = (const __attribute__((address_space(1))) gint4 *)(uintptr_t)src;
    auto *d = (__attribute__((address_space(1))) gint4 *)(uintptr_t)dst;
    for (size_t i = blockIdx.x * (size_t)256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
        __builtin_nontemporal_store(__builtin_nontemporal_load(s + i), d + i);
    if (blockIdx.x == 0 && (int)threadIdx.x < tail) dst_tail[threadIdx.x] = src_tail[threadIdx.x];
}

extern "C" int htr_copy(htr_device *dev, void *d_dst, const void *d_src, size_t bytes) {
    HTR_TRY(htr_check_alive(dev));
    if (!bytes) return 0;
    if (!d_dst || !d_src) return htr_fail("htr_copy: null pointer");
    if (((uintptr_t)d_dst | (uintptr_t)d_src) & 15) return htr_fail("htr_copy: pointers must be 16-byte aligned");
    const char *s = (const char *)d_src;
    char *d = (char *)d_dst;
    if ((s < d + bytes) && (d < s + bytes)) return htr_fail("htr_copy: %zu bytes from %p to %p overlap", bytes, d_src, d_dst);
    const size_t n16 = bytes / 16;
    const int tail = (int)(bytes % 16);
    const int grid = (int)std::max<size_t>(1, std::min<size_t>((n16 + 255) / 256, (size_t)dev->n_cu * 8));
    hipLaunchKernelGGL(k_copy16, dim3(grid), dim3(256), 0, dev->stream, (const int4 *)d_src, (int4 *)d_dst, n16,
                       (const uint8_t *)(s + 16 * n16), (uint8_t *)(d + 16 * n16), tail);
    return htr_launched(dev, "k_copy16");
}

// ---- a read of known size: the read rate a streaming kernel can reach on this device --------------------------------

// every workgroup reads PER consecutive 4 KB blocks (256 threads × 16 bytes), all its loads issued before the first
// use, and folds them into one word that is stored only if it equals a value no fold of a zero buffer gives (the
// loads stay; the store is one word at sink, whatever the buffer holds)
template <bool NT, int PER> __global__ __launch_bounds__(256) void k_read16(const int4 *src, size_t n16, uint32_t *sink) {
    const auto *s = (const __attribute__((address_space(1))) gint4 *)(uintptr_t)src;
    const size_t base = (size_t)blockIdx.x * PER * 256 + threadIdx.x;
    gint4 v[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const size_t at = base + (size_t)i * 256;
        v[i] = at < n16 ? (NT ? __builtin_nontemporal_load(s + at) : s[at]) : gint4{0, 0, 0, 0};
    }
    int f = 0;
#pragma unroll
    for (int i = 0; i < PER; i++) f ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (f == 0x7fffffff) sink[0] = (uint32_t)f;
}

extern "C" int htr_debug_read(htr_device *dev, const void *d_src, size_t bytes, int nontemporal, int kb_per_workgroup,
                              uint32_t *d_sink) {
    HTR_TRY(htr_check_alive(dev));
    if (!d_src || !d_sink) return htr_fail("htr_debug_read: null pointer");
    if (((uintptr_t)d_src & 15) || bytes % 16 || !bytes)
        return htr_fail("htr_debug_read: %zu bytes at %p (a positive multiple of 16, 16-byte aligned)", bytes, d_src);
    const int per = kb_per_workgroup / 4;
    if (per != 4 && per != 8 && per != 16) return htr_fail("htr_debug_read: %d KB a workgroup (16, 32 or 64)", kb_per_workgroup);
    const size_t n16 = bytes / 16, grid = (n16 + (size_t)per * 256 - 1) / ((size_t)per * 256);
    if (grid > (size_t)INT32_MAX) return htr_fail("htr_debug_read: %zu bytes", bytes);
    const auto *p = (const int4 *)d_src;
#define HTR_READ(NT, PER)                                                                                              \
    hipLaunchKernelGGL((k_read16<NT, PER>), dim3((unsigned)grid), dim3(256), 0, dev->stream, p, n16, d_sink)
    if (nontemporal) {
        if (per == 4) HTR_READ(true, 4);
        else if (per == 8) HTR_READ(true, 8);
        else HTR_READ(true, 16);
    } else {
        if (per == 4) HTR_READ(false, 4);
        else if (per == 8) HTR_READ(false, 8);
        else HTR_READ(false, 16);
    }
#undef HTR_READ
    return htr_launched(dev, "k_read16");
}

// ---- weights --------------------------------------------------------------------------------------------------------

static inline uint16_t f16_bits_rne(float v);  // below

// GGUF q8_0 blocks → quant plane + scale plane (host side, threads over rows)
static void repack_rows(const uint8_t *blocks, size_t rows, size_t cols, int8_t *q, uint16_t *d) {
    size_t nb = cols / 32;
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; t++) {
        th.emplace_back([=] {
            for (size_t r = t; r < rows; r += nt) {
                for (size_t b = 0; b < nb; b++) {
                    const uint8_t *blk = blocks + 34 * (r * nb + b);
                    d[r * nb + b] = (uint16_t)(blk[0] | (blk[1] << 8));
                    memcpy(q + r * cols + 32 * b, blk + 2, 32);
                }
            }
        });
    }
    for (auto &x : th) x.join();
}

extern "C" int htr_weight_q8_0(htr_device *dev, const void *h_blocks, size_t rows, size_t cols, htr_weight **out) {
    HTR_TRY(htr_check_alive(dev));
    if (!h_blocks || !out) return htr_fail("htr_weight_q8_0: null argument");
    if (rows == 0 || cols == 0 || cols % 32 != 0)
        return htr_fail("q8_0 weight [%zu x %zu]: cols must be a positive multiple of 32 (whole blocks)", rows, cols);
    std::vector<int8_t> q(rows * cols);
    std::vector<uint16_t> d(rows * cols / 32);
    repack_rows((const uint8_t *)h_blocks, rows, cols, q.data(), d.data());
    auto *w = new htr_weight;
    w->dev = dev;
    w->rows = rows;
    w->cols = cols;
    int rc = htr_dev_alloc(dev, q.size(), HTR_MEM_WEIGHTS, (void **)&w->q);
    // the scale plane has 16 bytes of slack: the matvec's scale staging reads whole 16-byte units
    if (rc == 0) rc = htr_dev_alloc(dev, d.size() * 2 + 16, HTR_MEM_WEIGHTS, (void **)&w->d);
    if (rc == 0) rc = htr_upload(dev, w->q, q.data(), q.size());
    if (rc == 0) rc = htr_upload(dev, w->d, d.data(), d.size() * 2);
    if (rc < 0) {
        std::string keep = g_err;
        htr_weight_free(w);
        g_err = keep;
        return -1;
    }
    *out = w;
    return 0;
}

extern "C" int htr_weight_q8_0_f16(htr_device *dev, const void *h_blocks, size_t rows, size_t cols, float scale,
                                   htr_weight **out) {
    HTR_TRY(htr_check_alive(dev));
    if (!h_blocks || !out) return htr_fail("htr_weight_q8_0_f16: null argument");
    if (rows == 0 || cols == 0 || cols % 32 != 0)
        return htr_fail("q8_0 weight [%zu x %zu]: cols must be a positive multiple of 32 (whole blocks)", rows, cols);
    std::vector<uint16_t> h(rows * cols);
    const uint8_t *blocks = (const uint8_t *)h_blocks;
    size_t nb = cols / 32;
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; t++) {
        th.emplace_back([&, t] {
            for (size_t r = t; r < rows; r += nt) {
                for (size_t b = 0; b < nb; b++) {
                    const uint8_t *blk = blocks + 34 * (r * nb + b);
                    _Float16 dh;
                    uint16_t bits = (uint16_t)(blk[0] | (blk[1] << 8));
                    memcpy(&dh, &bits, 2);
                    float df = (float)dh;
                    for (int i = 0; i < 32; i++)
                        h[r * cols + 32 * b + i] = f16_bits_rne((float)(int8_t)blk[2 + i] * df * scale);
                }
            }
        });
    }
    for (auto &x : th) x.join();
    auto *w = new htr_weight;
    w->dev = dev;
    w->rows = rows;
    w->cols = cols;
    int rc = htr_dev_alloc(dev, h.size() * 2, HTR_MEM_WEIGHTS, (void **)&w->h);
    if (rc == 0) rc = htr_upload(dev, w->h, h.data(), h.size() * 2);
    if (rc < 0) {
        std::string keep = g_err;
        htr_weight_free(w);
        g_err = keep;
        return -1;
    }
    *out = w;
    return 0;
}

extern "C" int htr_weight_free(htr_weight *w) {
    if (!w) return 0;
    if (w->q) htr_dev_free(w->dev, w->q);
    if (w->d) htr_dev_free(w->dev, w->d);
    if (w->h) htr_dev_free(w->dev, w->h);
    delete w;
    return 0;
}

extern "C" int htr_weight_shape(const htr_weight *w, size_t *rows, size_t *cols) {
    if (!w) return htr_fail("null weight");
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    return 0;
}

// ---- seeded synthetic inputs ----------------------------------------------------------------------------------------

static inline uint64_t mix64(uint64_t z) {  // SplitMix64 finaliser
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static inline uint64_t draw(uint64_t seed, uint64_t i) { return mix64(mix64(seed) ^ (i * 0xD1B54A32D192ED03ull)); }
// (0, 1]
static inline double unit_open(uint64_t r) { return ((double)(r >> 11) + 1.0) * (1.0 / 9007199254740992.0); }
static inline double normal_at(uint64_t seed, uint64_t i) {
    uint64_t a = draw(seed, 2 * i), b = draw(seed, 2 * i + 1);
    return std::sqrt(-2.0 * std::log(unit_open(a))) * std::cos(6.283185307179586 * (unit_open(b) - 0.5));
}

static inline uint16_t f16_bits_rne(float v) {
    _Float16 h = (_Float16)v;  // IEEE round to nearest even (host conversion)
    uint16_t b;
    memcpy(&b, &h, 2);
    return b;
}

template <typename F> static void parallel_for(size_t n, F f) {
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<std::thread> th;
    size_t per = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; t++) {
        size_t a = t * per, b = std::min(n, a + per);
        if (a >= b) break;
        th.emplace_back([=] { f(a, b); });
    }
    for (auto &x : th) x.join();
}

extern "C" int htr_synth_q8_0(uint64_t seed, size_t rows, size_t cols, void *h_blocks) {
    if (!h_blocks || cols % 32 != 0) return htr_fail("htr_synth_q8_0: null buffer or cols %% 32 != 0");
    uint8_t *o = (uint8_t *)h_blocks;
    size_t nblk = rows * cols / 32;
    parallel_for(nblk, [=](size_t a, size_t b) {
        for (size_t k = a; k < b; k++) {
            uint8_t *blk = o + 34 * k;
            float d = (float)(std::fabs(normal_at(seed, k)) * 0.002);
            uint16_t dh = f16_bits_rne(d);
            blk[0] = (uint8_t)(dh & 0xff);
            blk[1] = (uint8_t)(dh >> 8);
            for (int j = 0; j < 8; j++) {
                uint64_t r = draw(seed ^ 0x5bd1e9955bd1e995ull, k * 8 + j);
                for (int t = 0; t < 4; t++) {
                    uint32_t u16 = (uint32_t)((r >> (16 * t)) & 0xffff);
                    int q = (int)((u16 * 255u) >> 16) - 127;  // uniform over −127 … 127
                    blk[2 + 4 * j + t] = (uint8_t)(int8_t)q;
                }
            }
        }
    });
    return 0;
}

extern "C" int htr_synth_normal(uint64_t seed, size_t n, float mean, float std, float *h_out) {
    if (!h_out) return htr_fail("htr_synth_normal: null buffer");
    parallel_for(n, [=](size_t a, size_t b) {
        for (size_t i = a; i < b; i++) h_out[i] = (float)(mean + std * normal_at(seed, i));
    });
    return 0;
}
