// The GPU token choice of greedy presets for gfx950: the windowed repetition penalty fused with a two-pass argmax.
//
// Semantics: ocr-decode sampling.rs:38-62 (`choose`, greedy), bit for bit — the reference GPU kernels
// choose_pen.wgsl:85-106, choose_max.wgsl:28-61 and choose_pick.wgsl:32-69 restate the same (text.rs:222-231):
//   - each DISTINCT id among hist[len − window … len) (its first occurrence) → logit < 0: logit·rp, else logit / rp,
//     both one IEEE-754 f32 operation rounded to nearest even (hipcc's f32 division is correctly rounded), written
//     back in place;
//   - frequency penalty: a token with counts > 0 compares as logit − fpen (fpen = fp·count, stored by the pick);
//   - first maximum wins (ties → lowest index); NaN never wins; a NaN at index 0 (after the penalty) → token 0, as the
//     CPU loop `if l > logits[best]` starting at best = 0 decides; every logit NaN → 0.
//
// Schedule: grid (groups, rows); a workgroup owns SP consecutive logits of one row (2048 for a single row: 75
// workgroups over 151,936; 4096 for many), stages them in LDS, marks the logits whose id is in the window (a mark per
// logit in LDS: an id repeated in the window marks the same logit, so each distinct id is penalised once with no
// search for its first occurrence), applies the penalty as it reduces (value, index) to its best. The row's best of all
// workgroups is one 64-bit atomic max on an order-preserving key (value bits mapped to unsigned order, −0 as +0, then
// the complemented index, so ties go to the lowest index); the last workgroup of the row (atomic ticket) reads it,
// writes the token, appends it to the history and updates the counts. One launch per choice; the key and the ticket
// reset themselves.
//
// Cross-workgroup traffic is device-scope atomics only: on this multi-XCD GPU a release fence in every workgroup
// would write back the L2 each time, which costs more than the whole scan. Many rows in one launch (no frequency
// penalty) take k_choose_rows instead: a workgroup a row, so nothing crosses between workgroups at all.
#include <cmath>

#include "choose_key.h"
#include "htr_internal.h"
#include "wave.h"

namespace {

constexpr int CW = 256;
constexpr int LINE = 16;            // u64 words between rows' best keys / u32 between tickets: one 128-byte line each

// block-wide best of (v, i) → returned to every thread
__device__ __forceinline__ void block_best(float &v, uint32_t &i) {
    __shared__ float s_v[CW / 64];
    __shared__ uint32_t s_i[CW / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    wave_best(v, i, lane);
    __syncthreads();
    if (lane == 0) {
        s_v[wave] = v;
        s_i[wave] = i;
    }
    __syncthreads();
    v = s_v[0];
    i = s_i[0];
#pragma unroll
    for (int w = 1; w < CW / 64; w++)
        if (better(s_v[w], s_i[w], v, i)) {
            v = s_v[w];
            i = s_i[w];
        }
}

// XL (one row): the launch holds 8 workgroups a span and only those of XCD 0 (blockIdx.x ≡ 0 mod 8 on a device whose
// launches spread workgroups round-robin over its 8 XCDs, checked at open) work, so the row's best key and ticket are
// atomics in that XCD's L2 (workgroup scope) instead of at the coherence point
template <int SP, bool XL = false> __global__ __launch_bounds__(CW) void k_choose(const ChooseArgs a) {
    if (XL && (blockIdx.x & 7)) return;
    constexpr int PER_ = SP / CW;  // logits a thread
    __shared__ float s_l[SP];
    __shared__ __attribute__((aligned(16))) uint8_t s_pen[SP];  // the span's logits whose id is in the window
    __shared__ int s_last;
    const int g = XL ? blockIdx.x >> 3 : blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int lo = g * SP, hi = min(a.n_vocab, lo + SP);
    float *logits = a.logits + (size_t)row * a.n_vocab;
    uint32_t *hist = a.hist + (size_t)row * a.hist_stride;
    const int len = a.len_dev ? *a.len_dev : a.len;
    const int start = len - min(len, a.window);
    const int n_win = a.rp != 1.0f ? len - start : 0;
    // the window's first ids (one load a thread), issued with the logits' loads
    const uint32_t w0 = tid < n_win ? hist[start + tid] : 0xffffffffu;
    // the span's logits → LDS: every load issued before the first store (16-byte loads when the row is aligned)
    if ((((uintptr_t)(logits + lo)) & 15) == 0) {
        float4 lv[PER_ / 4];
#pragma unroll
        for (int i = 0; i < PER_ / 4; i++) {
            const int e = 4 * tid + 4 * CW * i;
            lv[i] = lo + e + 3 < hi ? *reinterpret_cast<const float4 *>(logits + lo + e) : make_float4(0, 0, 0, 0);
            if (lo + e + 3 >= hi) {  // the row's ragged end
                float t[4] = {0, 0, 0, 0};
                for (int u = 0; u < 4; u++)
                    if (lo + e + u < hi) t[u] = logits[lo + e + u];
                lv[i] = make_float4(t[0], t[1], t[2], t[3]);
            }
        }
#pragma unroll
        for (int i = 0; i < PER_ / 4; i++) *reinterpret_cast<float4 *>(s_l + 4 * tid + 4 * CW * i) = lv[i];
    } else {
        float lv[PER_];
#pragma unroll
        for (int i = 0; i < PER_; i++) lv[i] = lo + tid + CW * i < hi ? logits[lo + tid + CW * i] : 0.0f;
#pragma unroll
        for (int i = 0; i < PER_; i++) s_l[tid + CW * i] = lv[i];
    }
    // the penalty marks: cleared, then every window id in [lo, hi) sets its logit's mark. An id that occurs several
    // times in the window sets the same mark: each DISTINCT id is penalised once, as its first occurrence is in
    // sampling.rs:39-48 (the order of the window does not matter)
    if (n_win > 0) {
        for (int u = tid; u < SP / 16; u += CW) reinterpret_cast<uint4 *>(s_pen)[u] = make_uint4(0, 0, 0, 0);
        __syncthreads();
        if (w0 >= (uint32_t)lo && w0 < (uint32_t)hi) s_pen[w0 - lo] = 1;
        for (int j = tid + CW; j < n_win; j += CW) {
            const uint32_t t = hist[start + j];
            if (t >= (uint32_t)lo && t < (uint32_t)hi) s_pen[t - lo] = 1;
        }
    }
    __syncthreads();
    // pass 1: the penalties (rp on the marked logits, written back in place; then fp) and this workgroup's best
    // (NaN never wins: `better` is false for it); a fixed count of LDS reads, all issued before the first compare
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    float xs[PER_];
    bool pen[PER_];
#pragma unroll
    for (int i = 0; i < PER_; i++) {
        xs[i] = s_l[tid + CW * i];
        pen[i] = n_win > 0 && s_pen[tid + CW * i];
    }
#pragma unroll
    for (int i = 0; i < PER_; i++) {
        const int e = tid + CW * i;
        if (lo + e < hi) {
            float x = xs[i];
            const uint32_t k = (uint32_t)(lo + e);
            if (pen[i]) {
                x = x < 0.0f ? x * a.rp : x / a.rp;
                logits[k] = x;
                if (e == 0) s_l[0] = x;  // the NaN-at-index-0 rule below reads the penalised value
            }
            if (a.fp != 0.0f && a.counts[k] != 0u) x = x - a.fpen[k];
            if (better(x, k, bv, bi)) {
                bv = x;
                bi = k;
            }
        }
    }
    block_best(bv, bi);
    uint64_t *best = a.best + (size_t)row * LINE;
    uint32_t *ticket = a.counters + (size_t)row * LINE;
    if (tid == 0) {
        // a NaN at index 0 after the penalty decides token 0 (the CPU loop never finds a greater value): top key
        const bool nan0 = lo == 0 && s_l[0] != s_l[0];
        const uint64_t key = nan0 ? ~0ull : choose_key(bv, bi);
        if (XL) __hip_atomic_fetch_max(best, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        else __hip_atomic_fetch_max(best, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // the max is performed before the ticket: wait for its return
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        s_last = (XL ? __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                     : __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) ==
                 (XL ? gridDim.x >> 3 : gridDim.x) - 1;
    }
    __syncthreads();
    if (!s_last || tid != 0) return;
    // pass 2 (the row's last workgroup): the final key → token
    const uint64_t key = __hip_atomic_load(best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t t = ~(uint32_t)key;
    const uint32_t tk = t < (uint32_t)a.n_vocab ? t : 0u;  // 0xffffffff (every logit NaN) → 0; the NaN-at-0 key → 0
    a.tok[row] = tk;
    hist[len] = tk;
    if (a.fp != 0.0f) {
        const uint32_t c = a.counts[tk] + 1u;
        a.counts[tk] = c;
        a.fpen[tk] = a.fp * (float)c;
    }
    if (a.len_dev) *(int *)a.len_dev = len + 1;
    if (a.advance) a.advance[0] += 1;
    // ready for the next launch (seen by it: a kernel boundary)
    if (XL) {
        __hip_atomic_store(best, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    } else {
        __hip_atomic_store(best, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Many rows (no frequency penalty): one workgroup a row, nothing handed between workgroups. The window's ids set one bit
// each in an LDS bitmap of the row (a repeated id sets the same bit: each distinct id is penalised once); the row
// streams through in 16-byte loads, RU of them in flight a thread, each group of 4 logits tested against its 4 bits
// (one LDS word holds the bits of 32 logits), penalised and written back where marked, and folded into the thread's
// best by `better`; the workgroup's best is the token. The NaN-at-index-0 rule as in k_choose. Rows of another
// alignment or a vocabulary not a multiple of 4 take one logit a step.
constexpr int RW_T = 512, RU = 8;
typedef float gfloat4 __attribute__((ext_vector_type(4)));

template <bool VEC> __global__ __launch_bounds__(RW_T) void k_choose_rows(const ChooseArgs a) {
    extern __shared__ uint32_t s_bits[];  // ⌈n_vocab / 32⌉ words
    __shared__ float s_v[RW_T / 64];
    __shared__ uint32_t s_i[RW_T / 64];
    __shared__ int s_nan0;
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nv = a.n_vocab, words = (nv + 31) >> 5;
    float *logits = a.logits + (size_t)row * nv;
    uint32_t *hist = a.hist + (size_t)row * a.hist_stride;
    const int len = a.len;
    const int start = len - min(len, a.window);
    const int n_win = a.rp != 1.0f ? len - start : 0;
    if (n_win > 0) {
        for (int w = tid; w < words; w += RW_T) s_bits[w] = 0u;
        __syncthreads();
        for (int j = tid; j < n_win; j += RW_T) {
            const uint32_t t = hist[start + j];
            if (t < (uint32_t)nv) atomicOr(&s_bits[t >> 5], 1u << (t & 31));
        }
        __syncthreads();
    }
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    bool nan0 = false;
    auto take = [&](float x, uint32_t k, bool pen) {
        if (pen) {
            x = x < 0.0f ? x * a.rp : x / a.rp;
            logits[k] = x;
        }
        if (k == 0) nan0 = x != x;  // the NaN-at-index-0 rule reads the penalised value
        if (better(x, k, bv, bi)) {
            bv = x;
            bi = k;
        }
    };
    if constexpr (VEC) {
        const auto *l4 = (const __attribute__((address_space(1))) gfloat4 *)(uintptr_t)logits;
        const int n4 = nv >> 2;
        for (int u0 = tid; u0 < n4; u0 += RU * RW_T) {
            gfloat4 v[RU];
#pragma unroll
            for (int k = 0; k < RU; k++) {
                const int u = u0 + k * RW_T;
                v[k] = u < n4 ? __builtin_nontemporal_load(l4 + u) : gfloat4{0.0f, 0.0f, 0.0f, 0.0f};
            }
#pragma unroll
            for (int k = 0; k < RU; k++) {
                const int u = u0 + k * RW_T;
                if (u < n4) {
                    const uint32_t b = n_win > 0 ? (s_bits[u >> 3] >> (4 * (u & 7))) & 15u : 0u;
                    const uint32_t k0 = 4u * (uint32_t)u;
                    take(v[k].x, k0, b & 1u);
                    take(v[k].y, k0 + 1, b & 2u);
                    take(v[k].z, k0 + 2, b & 4u);
                    take(v[k].w, k0 + 3, b & 8u);
                }
            }
        }
    } else {
        for (int k = tid; k < nv; k += RW_T)
            take(logits[k], (uint32_t)k, n_win > 0 && ((s_bits[k >> 5] >> (k & 31)) & 1u));
    }
    wave_best(bv, bi, lane);
    if (tid == 0) s_nan0 = nan0;  // thread 0 holds index 0
    if (lane == 0) {
        s_v[wave] = bv;
        s_i[wave] = bi;
    }
    __syncthreads();
    if (tid != 0) return;
    float v = s_v[0];
    uint32_t i = s_i[0];
#pragma unroll
    for (int w = 1; w < RW_T / 64; w++)
        if (better(s_v[w], s_i[w], v, i)) {
            v = s_v[w];
            i = s_i[w];
        }
    // a NaN at index 0 → token 0; every logit NaN (no best) → 0
    const uint32_t tk = s_nan0 || i >= (uint32_t)nv ? 0u : i;
    a.tok[row] = tk;
    hist[len] = tk;
}

}  // namespace

int choose_groups(int n_vocab, int span) { return (n_vocab + span - 1) / span; }

size_t choose_best_bytes(int rows) { return (size_t)rows * LINE * 8; }
size_t choose_ticket_bytes(int rows) { return (size_t)rows * LINE * 4; }

int launch_choose(htr_device *dev, hipStream_t st, const ChooseArgs &a) {
    if (a.n_vocab <= 0 || a.rows <= 0) return htr_fail("choose: %d logits, %d rows", a.n_vocab, a.rows);
    // one row: 2048 logits a workgroup (75 over 151,936), a step 10.8 µs launched alone against 11.6 µs with 4096 and
    // 12.8 µs with 8192
    if (a.rows == 1) {
        // on XCD 0 alone where the placement holds: 5.55 → 5.38 µs a step as a graph node (A/B twice on one box,
        // tokens and penalised logits identical) — the L2's atomics gain a little more than one XCD's share of the
        // read costs
        if (dev->xcd_round_robin == 1)
            hipLaunchKernelGGL((k_choose<2048, true>), dim3(8 * choose_groups(a.n_vocab, 2048), 1), dim3(CW), 0, st,
                               a);
        else
            hipLaunchKernelGGL(k_choose<2048>, dim3(choose_groups(a.n_vocab, 2048), 1), dim3(CW), 0, st, a);
        return htr_launched(dev, "k_choose");
    }
    // many rows without the frequency penalty or the device-resident counters: a workgroup a row, the window's bitmap
    // in LDS (up to 64 KB)
    const size_t bitmap = (size_t)(a.n_vocab + 31) / 32 * 4;
    if (a.fp == 0.0f && !a.len_dev && !a.advance && bitmap <= 65536) {
        const bool vec = a.n_vocab % 4 == 0 && ((uintptr_t)a.logits & 15) == 0;
        if (vec) hipLaunchKernelGGL(k_choose_rows<true>, dim3(a.rows), dim3(RW_T), bitmap, st, a);
        else hipLaunchKernelGGL(k_choose_rows<false>, dim3(a.rows), dim3(RW_T), bitmap, st, a);
        return htr_launched(dev, "k_choose_rows");
    }
    // otherwise 4096 logits a workgroup of each row (4.3 TB/s over the bench's 512 rows; k_choose_rows 5.2–5.5)
    hipLaunchKernelGGL(k_choose<4096>, dim3(choose_groups(a.n_vocab, 4096), a.rows), dim3(CW), 0, st, a);
    return htr_launched(dev, "k_choose");
}

// the penalty must be 1 or a positive normal f32 (gpu_choice_capable, text.rs:154-163)
static int check_rp(float rp) {
    if (rp == 1.0f) return 0;
    if (!(rp > 0.0f) || !std::isnormal(rp)) return htr_fail("repetition penalty %g: 1 or a positive normal f32", rp);
    return 0;
}

static int choose_scratch(htr_device *dev, int rows, uint64_t **best, uint32_t **counters) {
    HTR_TRY(htr_scratch(dev, SCR_CHOOSE_PART, choose_best_bytes(rows), (void **)best));
    return htr_scratch(dev, SCR_CHOOSE_CNT, choose_ticket_bytes(rows), (void **)counters);
}

extern "C" int htr_choose(htr_device *dev, float *d_logits, int n_vocab, uint32_t *d_hist, int len, int window, float rp,
                          float fp, uint32_t *d_counts, float *d_fpen, uint32_t *d_tok) {
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(check_rp(rp));
    if (!d_logits || !d_hist || !d_tok) return htr_fail("htr_choose: null argument");
    if (len < 0 || window < 1 || n_vocab < 1) return htr_fail("htr_choose: len %d, window %d, %d logits", len, window, n_vocab);
    if (fp < 0.0f || (fp > 0.0f && (!d_counts || !d_fpen))) return htr_fail("htr_choose: fp %g needs counts and fpen", fp);
    ChooseArgs a{};
    a.logits = d_logits;
    a.n_vocab = n_vocab;
    a.hist = d_hist;
    a.hist_stride = 0;
    a.len = len;
    a.window = window;
    a.rp = rp;
    a.fp = fp;
    a.counts = d_counts;
    a.fpen = d_fpen;
    a.tok = d_tok;
    a.rows = 1;
    HTR_TRY(choose_scratch(dev, 1, &a.best, &a.counters));
    return launch_choose(dev, dev->stream, a);
}

extern "C" int htr_choose_many(htr_device *dev, float *d_logits, int n_vocab, int n, uint32_t *d_hist, int hist_stride,
                               int len, int window, float rp, uint32_t *d_tok) {
    HTR_TRY(htr_check_alive(dev));
    HTR_TRY(check_rp(rp));
    if (!d_logits || !d_hist || !d_tok || n < 1) return htr_fail("htr_choose_many: null argument or n < 1");
    if (len < 0 || len >= hist_stride || window < 1)
        return htr_fail("htr_choose_many: len %d, history stride %d, window %d", len, hist_stride, window);
    if (n > 65535) return htr_fail("htr_choose_many: %d rows (at most 65535 per launch)", n);
    ChooseArgs a{};
    a.logits = d_logits;
    a.n_vocab = n_vocab;
    a.hist = d_hist;
    a.hist_stride = hist_stride;
    a.len = len;
    a.window = window;
    a.rp = rp;
    a.tok = d_tok;
    a.rows = n;
    HTR_TRY(choose_scratch(dev, n, &a.best, &a.counters));
    return launch_choose(dev, dev->stream, a);
}
