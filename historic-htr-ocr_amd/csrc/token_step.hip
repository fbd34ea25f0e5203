// The decode step of the 1024-dim decoder (LightOnOCR's text model: dim 1024, 16 q / 8 KV heads of 128, SwiGLU 3072)
// as ONE launch per token: embed → 28 × (qkv, attention, merge, o, gate/up, down) → the residual for the LM head.
//
// Reference semantics: the f16 paths' fused step, text.rs:540-552 + layers_fused (text.rs:630-647): dmv_qkv.wgsl
// (attn_norm fused), qkv_post.wgsl (per-head norms, RoPE NEOX, f16 KV store), attn_decode.wgsl + attn_merge.wgsl
// (q·scale, f32 softmax), dmv.wgsl (o, down: + residual), dmv_ffn.wgsl (ffn_norm, SwiGLU), embed_q8_0.wgsl. The same
// arithmetic as the per-kernel step of q8_0.hip / attention.hip (dot16 group sums times the block scale, wave sums,
// the fused attention's butterfly); the attention's softmax runs per wave over its 16 keys (the waves' sums weighted
// by e^(m_w − M) in the chunk's partial) and the split-K merge sums its chunks in another order.
//
// Why one launch: at batch 1 every projection is a few MB spread over 256 CUs, so a kernel of the per-kernel step
// spends most of its time in the launch itself and in the first load's latency; a layer is 5 such launches. Here
// 256 workgroups (one a CU, all resident together) run every phase of the token, and each phase hands its outputs
// to the next through an exchange area instead of a kernel boundary:
//
//   words     every value handed over is one 64-bit word, the f32 value in the low half and a tag in the high half,
//             stored and loaded as one agent-scope 64-bit atomic (single-copy atomic: a reader sees the old word or the
//             new one, never half of each). A reader polls its words until each carries the tag it expects, so the
//             value arrives with its own proof of being current: no flag, no fence, no counter. Tags are
//             seq·256 + (6·layer + exchange): seq counts the session's tokens (read by every workgroup at start,
//             advanced by workgroup 0 at the end, after every workgroup has read it), so no tag repeats within 2^24
//             tokens, and every word a phase reads is rewritten every token (idle attention workgroups write empty
//             partials), so a stale word is at most one token old;
//   phases   A qkv (16 rows a workgroup, attn_norm fused) → B attention (workgroup = KV head × chunk of C keys,
//            32 a KV head; the q / k norms, RoPE and the new KV row made from the exchanged raw rows) → C merge (each
//            workgroup 8 dims of one q head over the head's chunks) → D o (4 rows, + residual) → E gate / up
//            (12 + 12 rows, ffn_norm, SwiGLU) → F down (4 rows, + residual) → A of the next layer;
//   XCDs     the 256 workgroups spread round-robin over the 8 XCDs (w ≡ x mod 8 on XCD x; checked on the host once a
//            device, token_step_xcds). A, B and C of KV head h run on XCD h: its 32 workgroups make the head's q / k /
//            v rows, attend over its chunks and merge them, so the A → B and B → C words never leave the XCD. They
//            are stored at workgroup scope and stay in the XCD's L2, where the readers' agent-scope loads hit them:
//            a one-way hand-over of about 0.2 µs against 0.6 µs through the fabric (one word back and forth between
//            two workgroups, htr_debug_handover in handover.hip; the step: 2194 → 2378 tokens/s). A word never seen (a workgroup on another XCD) is
//            a wait that runs out, never a stale value: the tag proves the word current;
//   overlap  a phase issues its loads first (a norm's weights, cache hits, ahead of the rows), then, after a pause
//            tuned for each hand-over, polls for its input: the HBM latency of the weights runs under the
//            hand-over's. B's K rows go out in A right after A's wait, its V rows right after B's. A wave's loads
//            complete in order, so nothing else is loaded ahead of the polls: the layer table, read once a phase
//            for its pointers, is read by scalar loads;
//   reuse    one word area per exchange, rewritten every layer. A workgroup writes exchange e of layer l + 1 only after
//            it has read inputs that every workgroup produced after reading exchange e of layer l (checked per
//            exchange in the comment of k_decode_token), so no word is overwritten before all its readers are done;
//   waits    every wait is bounded by the wall clock: past `spin_ticks` the thread sets *err, stops waiting for the
//            rest of the launch and the launch runs out (wrong values, no hang). The host refuses the path unless the
//            256 workgroups fit the device at once and spread over its XCDs as above, and reports *err after the step.
#include <utility>

#include "choose_key.h"
#include "htr_internal.h"
#include "wave.h"

namespace {

constexpr int NWG = 256;  // workgroups, all resident together
constexpr int TPB = 256;  // threads a workgroup
constexpr int D = 128;    // head dim
constexpr int DIM = 1024, QD = 2048, KVD = 1024, NFF = 3072, NQKV = QD + 2 * KVD;
constexpr int NKV = KVD / D;       // 8
constexpr int WPK = NWG / NKV;     // 32 workgroups a KV head
constexpr int XPL = 6;             // exchanges a layer
constexpr int PART_W = 2 * (D + 2);  // a chunk's partials: two heads × (m, l, o[128])
// word offsets of the exchanges
constexpr int OFF_QKV = 0;
constexpr int OFF_PART = OFF_QKV + NQKV;
constexpr int OFF_ATT = OFF_PART + NWG * PART_W;
constexpr int OFF_H1 = OFF_ATT + QD;
constexpr int OFF_FF = OFF_H1 + DIM;
constexpr int OFF_H2 = OFF_FF + NFF;
constexpr int OFF_BEST = OFF_H2 + DIM;  // the choice: each workgroup's best key as two words (high, low half)
constexpr int XWORDS = OFF_BEST + 2 * NWG;
static_assert(NQKV / NWG == 16 && DIM / NWG == 4 && NFF / NWG == 12, "rows a workgroup");

typedef int gint4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 ld16_stream(const void *p) {
    const gint4 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) gint4 *)(uintptr_t)p);
    return make_int4(v.x, v.y, v.z, v.w);
}
typedef float gfloat4 __attribute__((ext_vector_type(4)));
// global loads (pointers read from the layer table have lost their address space: these are not flat loads)
__device__ __forceinline__ float4 ld16f(const float *p) {
    const gfloat4 v = *(const __attribute__((address_space(1))) gfloat4 *)(uintptr_t)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float ld_half(const _Float16 *p) {
    return (float)*(const __attribute__((address_space(1))) _Float16 *)(uintptr_t)p;
}
__device__ __forceinline__ uint64_t ld_word(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void put_word(uint64_t *p, float v, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// a word whose readers run on the writer's own XCD: stored at workgroup scope it stays in that XCD's L2 (no write
// through to the fabric), where the readers' agent-scope loads find it
__device__ __forceinline__ void put_word_xcd(uint64_t *p, float v, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// the XCD this workgroup runs on (hardware register XCC_ID, bits 3:0)
__device__ __forceinline__ int xcd_id() { return __builtin_amdgcn_s_getreg(20 | (0 << 6) | ((4 - 1) << 11)) & 7; }

__device__ __forceinline__ float dot16(const int4 q, const float *x) {
    const int w[4] = {q.x, q.y, q.z, q.w};
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int b = 0; b < 4; b++) s = fmaf((float)(int8_t)(w[i] >> (8 * b)), x[4 * i + b], s);
    return s;
}

__device__ __forceinline__ void unpack8(const int4 w, float (&f)[8]) {
    const uint32_t u[4] = {(uint32_t)w.x, (uint32_t)w.y, (uint32_t)w.z, (uint32_t)w.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        _Float16 lo, hi;
        const uint16_t a = (uint16_t)(u[i] & 0xffff), b = (uint16_t)(u[i] >> 16);
        __builtin_memcpy(&lo, &a, 2);
        __builtin_memcpy(&hi, &b, 2);
        f[2 * i] = (float)lo;
        f[2 * i + 1] = (float)hi;
    }
}
__device__ __forceinline__ int4 pack8(const float (&f)[8]) {
    uint32_t u[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const _Float16 lo = (_Float16)f[2 * i], hi = (_Float16)f[2 * i + 1];
        uint16_t a, b;
        __builtin_memcpy(&a, &lo, 2);
        __builtin_memcpy(&b, &hi, 2);
        u[i] = (uint32_t)a | ((uint32_t)b << 16);
    }
    return make_int4((int)u[0], (int)u[1], (int)u[2], (int)u[3]);
}

// A wait's first loads go out this long after the workgroup's own outputs (s_sleep units of 64 clocks, ≈ 30 ns):
// the producers' words take about that long to become visible, and a first poll that comes back with old words
// costs a whole round trip more. Measured on one MI355X at the 28-layer read (µs a token): no pause 482 … 488,
// 8 → 465, 12 → 461, 16 → 460 … 469, 24 → 466, 32 → 479; two polls in flight instead (more traffic) 523. With the
// attention's hand-overs kept on their XCD (tokens/s): 8 → 2308, 12 → 2350 … 2375, 16 → 2380 … 2389. With the layer
// table read by scalar loads, one pause for the four cross-XCD waits (tokens/s, twice each on one box): 12 → 2354,
// 14 → 2439, 16 → 2531, 18 → 2571, 20 → 2577, 22 → 2573, 24 → 2562, 28 → 2552, 32 → 2520; the phases' own optima
// differ (qkv's wait is shortest at 16 … 18, o's at 16 … 20, gate/up's at 24 … 28, down's at 20 … 24), and with one
// a phase — qkv 18, o 18, gate/up 26, down 22, the attention's raw rows 10, the merge 4 — 2618 against 2577 for 20
// everywhere (A/B on two boxes). The LM head's wait at 16 or 22: the same.
constexpr int POLL_SLEEP = 16;      // the LM head's input and the choice's keys
constexpr int POLL_SLEEP_QKV = 18;  // A: the residual of the layer before (1024 words)
constexpr int POLL_SLEEP_O = 18;    // D: the attention output (2048 words)
constexpr int POLL_SLEEP_GU = 26;   // E: the residual after o (1024 words)
constexpr int POLL_SLEEP_DOWN = 22; // F: the SwiGLU output (3072 words)
// Words from the workgroup's own XCD are there sooner: the attention's raw rows (B) 10, the chunks' partials (C) 4
// (with the cross-XCD pause at 16: 12 → 2350 tokens/s, 8 → 2371, 4 → 2378, 0 → 2378 for both)
constexpr int POLL_SLEEP_RAW = 10;
constexpr int POLL_SLEEP_PART = 4;

template <bool B> struct BoolC {
    static constexpr bool value = B;
};

struct Waiter {
    long long limit;  // wall-clock ticks a wait may take
    uint32_t *err;
    bool broken;  // this thread ran out of time once: it waits no more in this launch
    int polls;    // of the current wait
    // true when the wait that began at t0 (0: not yet) has run out — past the limit on the wall clock, or past 2^22
    // polls (seconds: each is a memory round trip) should the clock not advance; then err is set and the thread waits
    // no more
    __device__ __forceinline__ bool expired(long long &t0) {
        const long long now = wall_clock64();
        if (t0 == 0) {
            t0 = now;
            polls = 0;
            return false;
        }
        if (now - t0 <= limit && ++polls < (1 << 22)) return false;
        broken = true;
        __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return true;
    }
};

// The NP words idx = tid + 256·k (k < NP, idx < n) of src, each once it carries `tag`, → dst[idx] (LDS); then a
// workgroup barrier. The first loads of every word go out together; a word that is not there yet is loaded again
// until it is, or until the wall clock passes the limit. No barrier ahead of the stores into dst: every dst is read
// last at least two barriers before (each exchange has its own LDS array, the residual one a copy for A and D and
// one for E and F)
template <int NP, int SLEEP = POLL_SLEEP>
__device__ __forceinline__ void take(Waiter &wt, const uint64_t *src, int n, uint32_t tag, float *dst) {
    const int tid = threadIdx.x;
    uint64_t v[NP];
    __builtin_amdgcn_s_sleep(SLEEP);
#pragma unroll
    for (int k = 0; k < NP; k++) {
        const int idx = tid + TPB * k;
        v[k] = idx < n ? ld_word(src + idx) : (uint64_t)tag << 32;
    }
    long long t0 = 0;
    for (;;) {
        bool all = true;
#pragma unroll
        for (int k = 0; k < NP; k++) all = all && (uint32_t)(v[k] >> 32) == tag;
        if (all || wt.broken) break;
#pragma unroll
        for (int k = 0; k < NP; k++) {
            const int idx = tid + TPB * k;
            if ((uint32_t)(v[k] >> 32) != tag) v[k] = ld_word(src + idx);
        }
        if (wt.expired(t0)) break;  // the clock is read while the loads travel
    }
#pragma unroll
    for (int k = 0; k < NP; k++) {
        const int idx = tid + TPB * k;
        if (idx < n) dst[idx] = __uint_as_float((uint32_t)v[k]);
    }
    __syncthreads();
}

// the layer table through the constant address space: the host writes it before the launch and nothing in the kernel
// does, so its loads are scalar. As vector loads (the table is in device memory) a phase's first pointer load sat in
// the wave's vector-memory order behind the previous phase's output stores, and its weights went out only once those
// stores had been acknowledged
typedef const __attribute__((address_space(4))) TokLayer const_layer;
__device__ __forceinline__ const_layer &layer_at(const TokArgs &a, int l) { return ((const_layer *)a.layers)[l]; }

// workgroup 0's wall-clock stamps, kept in LDS (a store to memory here would wait for the phase's own stores) and
// written out at the end of the launch
constexpr int MAX_LAYERS = 42;
constexpr int N_STAMPS = 1 + 12 * MAX_LAYERS + 3;
constexpr int MAX_HEAD_ROWS = 1024;  // LM-head rows a workgroup: n_vocab ≤ 256 · 1024
__device__ __forceinline__ void stamp(unsigned long long *s_stamp, bool on, int at) {
    if (on && threadIdx.x == 0) s_stamp[at] = (unsigned long long)wall_clock64();
}

// wave_max / wave_sum of two values at once, their steps interleaved (the same partners and order as wave.h's, so
// each result is the single reduction's)
__device__ __forceinline__ void wave_max2(float &a, float &b, int lane) {
    a = fmaxf(a, lane_swap<32>(a, lane)), b = fmaxf(b, lane_swap<32>(b, lane));
    a = fmaxf(a, lane_swap<16>(a, lane)), b = fmaxf(b, lane_swap<16>(b, lane));
    a = fmaxf(a, lane_swap<8>(a, lane)), b = fmaxf(b, lane_swap<8>(b, lane));
    a = fmaxf(a, lane_swap<4>(a, lane)), b = fmaxf(b, lane_swap<4>(b, lane));
    a = fmaxf(a, lane_swap<2>(a, lane)), b = fmaxf(b, lane_swap<2>(b, lane));
    a = fmaxf(a, lane_swap<1>(a, lane)), b = fmaxf(b, lane_swap<1>(b, lane));
}
__device__ __forceinline__ void wave_sum2(float &a, float &b, int lane) {
    a += lane_swap<32>(a, lane), b += lane_swap<32>(b, lane);
    a += lane_swap<16>(a, lane), b += lane_swap<16>(b, lane);
    a += lane_swap<8>(a, lane), b += lane_swap<8>(b, lane);
    a += lane_swap<4>(a, lane), b += lane_swap<4>(b, lane);
    a += lane_swap<2>(a, lane), b += lane_swap<2>(b, lane);
    a += lane_swap<1>(a, lane), b += lane_swap<1>(b, lane);
}

// the value of lane n of the lane's row of 16 (DPP row_newbcast)
template <int n> __device__ __forceinline__ float row_bcast(float v) {
    static_assert(n >= 0 && n < 16, "lane of a row");
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + n, 0xF, 0xF, false));
}
// pw[idx] for idx < N: the value idx of the lane's row, held as pr[idx % NR] by lane idx / NR (NR > 1: 16 or more
// values a row) or as pr[0] by lane idx << (4 − S) (fewer: one a group of 16 >> S lanes)
template <int N, int NR, int S, int... I>
__device__ __forceinline__ void row_gather(const float (&pr)[NR], float (&pw)[N], std::integer_sequence<int, I...>) {
    ((pw[I] = row_bcast<(N >= 16 ? I / NR : I << (4 - S))>(pr[N >= 16 ? I % NR : 0])), ...);
}

// the fused RMS norm of a lane's 16·NG inputs (the wave holds all K of them): x·1/sqrt(Σx²/K + eps)·w
template <int NG>
__device__ __forceinline__ void norm16(float (&xv)[NG][16], const float (&wv)[NG][16], float eps, int k, int lane) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NG; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) s = fmaf(xv[i][e], xv[i][e], s);
    const float scale = 1.0f / sqrtf(wave_sum(s, lane) / (float)k + eps);
#pragma unroll
    for (int i = 0; i < NG; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) xv[i][e] = (xv[i][e] * scale) * wv[i][e];
}

// lane's inputs x[16g … 16g + 15], g = lane + 64·i, from LDS
template <int NG> __device__ __forceinline__ void lds_x(float (&xv)[NG][16], const float *s, int lane) {
#pragma unroll
    for (int i = 0; i < NG; i++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 v = *reinterpret_cast<const float4 *>(s + 16 * (lane + 64 * i) + 4 * q);
            xv[i][4 * q] = v.x, xv[i][4 * q + 1] = v.y, xv[i][4 * q + 2] = v.z, xv[i][4 * q + 3] = v.w;
        }
}
template <int NG> __device__ __forceinline__ void glob_x(float (&xv)[NG][16], const float *s, int lane) {
#pragma unroll
    for (int i = 0; i < NG; i++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 v = ld16f(s + 16 * (lane + 64 * i) + 4 * q);
            xv[i][4 * q] = v.x, xv[i][4 * q + 1] = v.y, xv[i][4 * q + 2] = v.z, xv[i][4 * q + 3] = v.w;
        }
}

// a row's quants and scales for the lane's groups g = lane + 64·i of a K = 1024·NG matrix (repacked planes). The
// layers' quants go out as non-temporal loads, the LM head's (KEEP) as plain ones: with the layers' 470 MB and the
// KV rows streaming past without displacing it, more of the head's 165 MB is still cached at the next token's head
// (2172 → 2192 tokens/s in the decode read of 1024 + 512 tokens; every load plain: 2130)
template <int NG> struct RowW {
    int4 q[NG];
    float d[NG];
};
__device__ __forceinline__ int4 ld16_keep(const void *p) {
    const gint4 v = *(const __attribute__((address_space(1))) gint4 *)(uintptr_t)p;
    return make_int4(v.x, v.y, v.z, v.w);
}
template <int NG, bool KEEP = false>
__device__ __forceinline__ void row_issue(RowW<NG> &r, const int8_t *q, const _Float16 *d, int row, int lane) {
    constexpr int K = 1024 * NG;
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const int g = lane + 64 * i;
        r.q[i] = KEEP ? ld16_keep(q + (size_t)row * K + 16 * g) : ld16_stream(q + (size_t)row * K + 16 * g);
        r.d[i] = ld_half(d + (size_t)row * (K / 32) + (g >> 1));
    }
}
template <int NG> __device__ __forceinline__ float row_dot(const RowW<NG> &r, const float (&xv)[NG][16]) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NG; i++) s = fmaf(dot16(r.q[i], xv[i]), r.d[i], s);
    return s;
}

// the q / k norm and RoPE NEOX of one head's raw row (LDS) for the 8 dims 8j … 8j + 7 (partners in slice j ^ 8; the
// 16 lanes j of a lane row hold the head: Σx² over them), rope pairs cs of indices 8(j % 8) … + 7
// nw: the norm weights of those dims and of the partner dims (NormW, loaded before the wait)
struct NormW {
    float4 a[2], b[2];
    __device__ __forceinline__ void issue(const float *w, int j) {
        a[0] = ld16f(w + 8 * j), a[1] = ld16f(w + 8 * j + 4);
        b[0] = ld16f(w + 8 * (j ^ 8)), b[1] = ld16f(w + 8 * (j ^ 8) + 4);
    }
};
__device__ __forceinline__ void head_post(const float *raw, const NormW &nw, const float (&cs)[16], int j, int lane,
                                          float eps, float (&out)[8]) {
    const int jp = j ^ 8;
    float a8[8], b8[8];
    const float wa[8] = {nw.a[0].x, nw.a[0].y, nw.a[0].z, nw.a[0].w, nw.a[1].x, nw.a[1].y, nw.a[1].z, nw.a[1].w};
    const float wb[8] = {nw.b[0].x, nw.b[0].y, nw.b[0].z, nw.b[0].w, nw.b[1].x, nw.b[1].y, nw.b[1].z, nw.b[1].w};
#pragma unroll
    for (int e = 0; e < 8; e++) {
        a8[e] = raw[8 * j + e];
        b8[e] = raw[8 * jp + e];
    }
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) ss = fmaf(a8[e], a8[e], ss);
    ss = group_sum<8>(ss, lane);
    const float scale = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float ya = (a8[e] * scale) * wa[e], yb = (b8[e] * scale) * wb[e];
        const float c = cs[2 * e], s = cs[2 * e + 1];
        out[e] = j < 8 ? ya * c - yb * s : yb * s + ya * c;
    }
}

// k_decode_token: grid 256 × 256 threads; NI: keys a thread in the attention (chunks of C = 16·NI keys, 32 a KV
// head: n_ctx ≤ 512·NI).
//
// Reuse of the exchange words, layer l → l + 1 (each arrow: "waited for the words of"):
//   QKV  written in A(l+1), read in B(l): A(l+1) waits for H2(l) from every workgroup, written after its D(l), which
//        waited for every workgroup's C(l), which came after its B(l);
//   PART written in B(l+1), read in C(l): B(l+1) follows A(l+1) → H2(l) of all → D(l) of all → C(l) of all;
//   ATT  written in C(l+1), read in D(l): C(l+1) follows A(l+1) → H2(l) of all, each written after its D(l);
//   H1   written in D(l+1), read in E(l): D(l+1) follows ATT of all → C(l+1) … A(l+1) of all → H2(l) of all, each
//        written after its E(l);
//   FF   written in E(l+1), read in F(l): E(l+1) follows H1(l+1) of all → D(l+1) → ATT of all → … → A(l+1) of all,
//        each after its F(l) read;
//   H2   written in F(l+1), read in A(l+1): F(l+1) follows FF(l+1) of all, each written after its A(l+1).
template <int NI> __global__ __launch_bounds__(TPB) void k_decode_token(const TokArgs a) {
    constexpr int C = 16 * NI;
    constexpr int N = NI <= 1 ? 2 : NI <= 2 ? 4 : NI <= 4 ? 8 : NI <= 8 ? 16 : 32;  // 2·NI scores, padded
    // the exchanged inputs: the residual entering the layer (A, D) and after o (E, F), the attention output (D), the
    // SwiGLU output (F)
    __shared__ __attribute__((aligned(16))) float s_x[DIM], s_h[DIM], s_att[QD], s_ff[NFF];
    __shared__ __attribute__((aligned(16))) float s_raw[4][D];  // B: raw q (two heads), k, v rows of the KV head
    __shared__ __attribute__((aligned(16))) float s_post[3][D];  // B: q (× scale, two heads) and k, normed and roped
    __shared__ float s_ws[4][4];  // B: each wave's max and sum of p, per head
    __shared__ float s_o[4][2][D];
    __shared__ float s_ml[2][WPK];
    __shared__ __attribute__((aligned(16))) float s_mo[WPK][8];
    __shared__ unsigned long long s_stamp[N_STAMPS];
    __shared__ __attribute__((aligned(16))) uint8_t s_pen[MAX_HEAD_ROWS];  // T: the rows whose id is in the window
    __shared__ float s_bv[4];
    __shared__ uint32_t s_bi[4];
    __shared__ int s_nan0;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int w = blockIdx.x;
    const bool prof_on = a.prof && w == 0;
    Waiter wt{a.spin_ticks, a.err, false, 0};
    const int pos = *a.state;
    if (pos < 0 || pos >= a.n_ctx) return;  // every workgroup alike (the host checks positions first)
    const uint32_t seq = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(a.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    uint64_t *xw = a.xw;

    // embed (every workgroup the whole row): x = dequant(token_embd[tok]); an id out of range leaves x as it was
    {
        const uint32_t id = *a.tok;
        const int c = 4 * tid;
        if (id < (uint32_t)a.n_vocab) {
            const char4 q4 = *reinterpret_cast<const char4 *>(a.emb_q + (size_t)id * DIM + c);
            const float d = (float)a.emb_d[((size_t)id * DIM + c) >> 5];
            s_x[c] = (float)q4.x * d, s_x[c + 1] = (float)q4.y * d, s_x[c + 2] = (float)q4.z * d,
            s_x[c + 3] = (float)q4.w * d;
        } else {
            const float4 v = ld16f(a.x_out + c);
            s_x[c] = v.x, s_x[c + 1] = v.y, s_x[c + 2] = v.z, s_x[c + 3] = v.w;
        }
        __syncthreads();
    }
    stamp(s_stamp, prof_on, 0);

    // KV head kvh's q / k / v rows, attention chunks and merge run on XCD kvh (its 32 workgroups w ≡ kvh mod 8)
    const int kvh = xcd_id(), cw = w >> 3, h0 = 2 * kvh;
    const int n_keys = pos + 1, n_chunk = (n_keys + C - 1) / C;
    const int j = tid & 15, kk = tid >> 4;

    for (int l = 0; l < a.n_layer; l++) {
        const_layer &L = layer_at(a, l);
        const uint32_t tbase = seq * 256u + (uint32_t)(XPL * l);

        int4 kr[NI];  // B's K rows (issued in A)
        // ---- A: q | k | v rows 16w … 16w + 15 (one matrix: the boundaries 2048, 3072 are multiples of 16), attn_norm
        {
            const int mat = cw < 16 ? 0 : cw < 24 ? 1 : 2;
            const int lr0 = mat == 0 ? 2 * D * kvh + 16 * cw : D * kvh + 16 * (cw - (mat == 1 ? 16 : 24));
            const int f0 = lr0 + (mat == 0 ? 0 : mat == 1 ? QD : QD + KVD);  // the first row's word
            const int8_t *q = mat == 0 ? L.q[0] : mat == 1 ? L.q[1] : L.q[2];
            const _Float16 *d = mat == 0 ? L.d[0] : mat == 1 ? L.d[1] : L.d[2];
            // the norm weights first (cache hits): issued behind the rows, they came back only with them (A and E:
            // 2670 → 2693 and 2684 tokens/s)
            float wv[1][16];
            glob_x<1>(wv, L.attn_norm, lane);
            RowW<1> rw[4];
#pragma unroll
            for (int r = 0; r < 4; r++) row_issue<1>(rw[r], q, d, lr0 + 4 * wave + r, lane);
            if (l > 0) take<4, POLL_SLEEP_QKV>(wt, xw + OFF_H2, DIM, tbase - 1, s_x);  // F of the layer before
            // B's K rows now, behind A's own wait (before it, A's polls would queue behind them) and ahead of B's:
            // every chunk loads them, an idle one the row at pos (in bounds, not used). Against issuing them in B:
            // 2456 → 2466 tokens/s at the 1536-row cache, 2366 → 2388 at 2560 rows (twice on one box)
#pragma unroll
            for (int i = 0; i < NI; i++)
                kr[i] = ld16_stream(L.kc + ((size_t)kvh * a.n_ctx + min(cw * C + kk + 16 * i, pos)) * D + 8 * j);
            stamp(s_stamp, prof_on, 1 + 12 * l);
            float xv[1][16];
            lds_x<1>(xv, s_x, lane);
            norm16<1>(xv, wv, a.eps, DIM, lane);
            float acc[4];
#pragma unroll
            for (int r = 0; r < 4; r++) acc[r] = row_dot<1>(rw[r], xv);
            const float v = wave_sum_rows<4>(acc, lane);
            if ((lane & 15) == 0) put_word_xcd(xw + OFF_QKV + f0 + 4 * wave + (lane >> 4), v, tbase + 0);
        }
        stamp(s_stamp, prof_on, 2 + 12 * l);

        // ---- B: attention of KV head kvh over keys cw·C … cw·C + C − 1
        {
            const bool busy = cw < n_chunk;  // uniform
            const int k0 = cw * C;
            const _Float16 *vb = L.vc + (size_t)kvh * a.n_ctx * D;
            int4 vr[NI];
            float4 rope4[4];
            NormW hnw;  // the norm weights of this wave's head (waves 0, 1: q; 2: k)
            if (busy) {
                const float *rr = a.rope + (size_t)pos * D + 16 * (j & 7);
#pragma unroll
                for (int i = 0; i < 4; i++) rope4[i] = ld16f(rr + 4 * i);
                hnw.issue(wave == 2 ? L.k_norm : L.q_norm, j);
                // the KV head's raw rows: q heads h0, h0 + 1, then k, v → s_raw (512 words, 2 a thread)
                const uint64_t *src0 = xw + OFF_QKV;
                uint64_t vv[2];
                int at[2];
                __builtin_amdgcn_s_sleep(POLL_SLEEP_RAW);
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const int idx = tid + TPB * k, part = idx >> 7, dd = idx & 127;
                    at[k] = part < 2 ? (h0 + part) * D + dd : part == 2 ? QD + kvh * D + dd : QD + KVD + kvh * D + dd;
                    vv[k] = ld_word(src0 + at[k]);
                }
                long long t0 = 0;
                for (;;) {
                    const bool all = (uint32_t)(vv[0] >> 32) == tbase && (uint32_t)(vv[1] >> 32) == tbase;
                    if (all || wt.broken) break;
#pragma unroll
                    for (int k = 0; k < 2; k++)
                        if ((uint32_t)(vv[k] >> 32) != tbase) vv[k] = ld_word(src0 + at[k]);
                    if (wt.expired(t0)) break;
                }
                // the V rows now: issued before the wait, the raw rows' loads would queue behind them (the K rows,
                // needed first, are in by here): 2434 → 2455 tokens/s, the attention's wait 1.25 → 1.17 µs a layer
#pragma unroll
                for (int i = 0; i < NI; i++) vr[i] = ld16_stream(vb + (size_t)min(k0 + kk + 16 * i, pos) * D + 8 * j);
                // (s_raw was read last in the layer before's B: no barrier needed ahead of these stores)
#pragma unroll
                for (int k = 0; k < 2; k++) (&s_raw[0][0])[tid + TPB * k] = __uint_as_float((uint32_t)vv[k]);
                __syncthreads();
            }
            stamp(s_stamp, prof_on, 3 + 12 * l);
            if (busy) {
                // the per-head norms and RoPE, one head a wave (waves 0, 1: the q heads, times the softmax scale;
                // wave 2: k; the four 16-lane rows of a wave compute the same values, the first writes them)
                if (wave < 3) {
                    float cs[16];
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        cs[4 * i] = rope4[i].x, cs[4 * i + 1] = rope4[i].y, cs[4 * i + 2] = rope4[i].z,
                        cs[4 * i + 3] = rope4[i].w;
                    float t8[8];
                    head_post(s_raw[wave], hnw, cs, j, lane, a.eps, t8);
                    if (lane < 16) {
#pragma unroll
                        for (int e = 0; e < 8; e++) s_post[wave][8 * j + e] = wave < 2 ? t8[e] * a.scale : t8[e];
                    }
                }
                __syncthreads();
                float qa[8], qb[8], kn8[8], v8[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    qa[e] = s_post[0][8 * j + e];
                    qb[e] = s_post[1][8 * j + e];
                    kn8[e] = s_post[2][8 * j + e];
                    v8[e] = s_raw[3][8 * j + e];
                }
                const int4 knew = pack8(kn8), vnew = pack8(v8);
                // the chunk that holds pos: its keys at or past pos take the new row (past pos they are masked), and
                // it stores the row into the cache (no workgroup of this launch reads it); the other chunks' keys are
                // all cache rows below pos
                auto attend = [&](auto last_c) {
                    constexpr bool LAST = decltype(last_c)::value;
                    if constexpr (LAST) {
                        // every thread stores (the 16 threads of a slice j the same 16 bytes): with the store under a
                        // runtime branch the compiler could not count it, and p·v's wait for the V rows became a wait
                        // for these stores too — the chunk holding pos then finished 0.5 µs after the others (2478 →
                        // 2501 tokens/s)
                        *reinterpret_cast<int4 *>(L.kc + ((size_t)kvh * a.n_ctx + pos) * D + 8 * j) = knew;
                        *reinterpret_cast<int4 *>(L.vc + ((size_t)kvh * a.n_ctx + pos) * D + 8 * j) = vnew;
                    }
                    float v[N];
#pragma unroll
                    for (int i = 0; i < NI; i++) {
                        float kf[8];
                        unpack8(LAST && k0 + kk + 16 * i >= pos ? knew : kr[i], kf);
                        float da = 0.0f, db = 0.0f;
#pragma unroll
                        for (int e = 0; e < 8; e++) {
                            da = fmaf(qa[e], kf[e], da);
                            db = fmaf(qb[e], kf[e], db);
                        }
                        v[2 * i] = da;
                        v[2 * i + 1] = db;
                    }
#pragma unroll
                    for (int i = 2 * NI; i < N; i++) v[i] = 0.0f;  // the padding: no key
                    // the lane's scores, summed over the 16 lanes j of its row: NR values, idx = NR·j + r (16 or more
                    // a thread), else one, idx = j >> (4 − S), whole in every lane of its group of 16 >> S; idx → key
                    // kk + 16·(idx >> 1), head idx & 1
                    constexpr int S = N >= 16 ? 4 : N == 2 ? 1 : N == 4 ? 2 : 3;
                    constexpr int NR = N >= 16 ? N / 16 : 1;
                    float sc[NR];
                    if constexpr (N >= 16) {
                        halve<N, 8, 4>(v, lane);
#pragma unroll
                        for (int r = 0; r < NR; r++) sc[r] = v[r];
                    } else {
                        halve<N, 8, S>(v, lane);
                        sc[0] = group_sum<(8 >> S)>(v[0], lane);
                    }
                    const bool rep = N >= 16 || (j & ((16 >> S) - 1)) == 0;  // counts its values in the sums
                    // the wave's own softmax over its keys (rows kk = 4·wave … 4·wave + 3), both heads as two
                    // interleaved chains; the four waves' statistics meet in the sum of their partials below
                    float mx[2] = {-INFINITY, -INFINITY};
                    int hr[NR];
#pragma unroll
                    for (int r = 0; r < NR; r++) {
                        const int idx = N >= 16 ? NR * j + r : j >> (4 - S);
                        hr[r] = idx & 1;
                        if ((2 * NI < N && (idx >> 1) >= NI) || (LAST && k0 + kk + 16 * (idx >> 1) >= n_keys))
                            sc[r] = -INFINITY;
                        mx[0] = hr[r] ? mx[0] : fmaxf(mx[0], sc[r]);
                        mx[1] = hr[r] ? fmaxf(mx[1], sc[r]) : mx[1];
                    }
                    wave_max2(mx[0], mx[1], lane);
                    float pr[NR], l_h[2] = {0.0f, 0.0f};
#pragma unroll
                    for (int r = 0; r < NR; r++) {
                        // masked keys, and every key of a head whose keys in this wave are all masked (max −inf): 0
                        pr[r] = sc[r] == -INFINITY ? 0.0f : expf(sc[r] - (hr[r] ? mx[1] : mx[0]));
                        const float c = rep ? pr[r] : 0.0f;
                        l_h[0] += hr[r] ? 0.0f : c;
                        l_h[1] += hr[r] ? c : 0.0f;
                    }
                    wave_sum2(l_h[0], l_h[1], lane);
                    // p of the thread's keys kk + 16·i, both heads, from the lanes of its row that hold them
                    float pw[N];
                    row_gather<N, NR, S>(pr, pw, std::make_integer_sequence<int, N>{});
                    float o[16];
#pragma unroll
                    for (int e = 0; e < 16; e++) o[e] = 0.0f;
#pragma unroll
                    for (int i = 0; i < NI; i++) {
                        float vf[8];
                        unpack8(LAST && k0 + kk + 16 * i >= pos ? vnew : vr[i], vf);
                        const float pa = pw[2 * i], pb = pw[2 * i + 1];
#pragma unroll
                        for (int e = 0; e < 8; e++) {
                            o[e] = fmaf(pa, vf[e], o[e]);
                            o[8 + e] = fmaf(pb, vf[e], o[8 + e]);
                        }
                    }
                    halve<16, 32, 2>(o, lane);
                    {
                        const int base = 8 * ((lane >> 5) & 1) + 4 * ((lane >> 4) & 1);
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const int idx = base + r, h = idx >> 3, e = idx & 7;
                            s_o[wave][h][8 * j + e] = o[r];
                        }
                    }
                    if (lane == 0) s_ws[wave][0] = mx[0], s_ws[wave][1] = mx[1], s_ws[wave][2] = l_h[0],
                                   s_ws[wave][3] = l_h[1];
                    __syncthreads();
                    // the chunk's partial: M = max of the waves' maxima (finite: key k0 is valid), each wave's sums
                    // weighted by e^(m_w − M) (0 for a wave with no valid key of the head)
                    const int hh = tid >> 7, dd = tid & 127;
                    float mw[4], wt[4];
#pragma unroll
                    for (int q = 0; q < 4; q++) mw[q] = s_ws[q][hh];
                    const float M = fmaxf(fmaxf(mw[0], mw[1]), fmaxf(mw[2], mw[3]));
#pragma unroll
                    for (int q = 0; q < 4; q++) wt[q] = mw[q] == -INFINITY ? 0.0f : expf(mw[q] - M);
                    const float oc = (s_o[0][hh][dd] * wt[0] + s_o[1][hh][dd] * wt[1]) +
                                     (s_o[2][hh][dd] * wt[2] + s_o[3][hh][dd] * wt[3]);
                    uint64_t *pc = xw + OFF_PART + (size_t)(kvh * WPK + cw) * PART_W + hh * (D + 2);
                    put_word_xcd(pc + 2 + dd, oc, tbase + 1);
                    if (dd == 0) put_word_xcd(pc, M, tbase + 1);
                    if (dd == 1) {
                        const float lsum = (s_ws[0][2 + hh] * wt[0] + s_ws[1][2 + hh] * wt[1]) +
                                           (s_ws[2][2 + hh] * wt[2] + s_ws[3][2 + hh] * wt[3]);
                        put_word_xcd(pc + 1, lsum, tbase + 1);
                    }
                };
                if (cw == n_chunk - 1)
                    attend(BoolC<true>{});
                else
                    attend(BoolC<false>{});
            } else {
                // an idle chunk: empty partials (no reader merges them; written so every word stays current)
                const int hh = tid >> 7, dd = tid & 127;
                uint64_t *pc = xw + OFF_PART + (size_t)(kvh * WPK + cw) * PART_W + hh * (D + 2);
                put_word_xcd(pc + 2 + dd, 0.0f, tbase + 1);
                if (dd == 0) put_word_xcd(pc, -INFINITY, tbase + 1);
                if (dd == 1) put_word_xcd(pc + 1, 0.0f, tbase + 1);
            }
        }
        stamp(s_stamp, prof_on, 4 + 12 * l);

        // ---- C: merge — workgroup (kvh, cw) → head h0 + cw / 16, dims 8·(cw % 16) … + 7, over the head's n_chunk
        // chunks: M = max m_c, w_c = e^(m_c − M), out = Σ o_c·w_c / Σ l_c·w_c
        {
            const int hh = cw >> 4, d0 = 8 * (cw & 15);
            const uint64_t *pk = xw + OFF_PART + (size_t)(kvh * WPK) * PART_W + hh * (D + 2);
            const int cc = tid >> 3, e = tid & 7;  // o word of chunk cc, dim d0 + e
            const bool has_o = cc < n_chunk;
            const int cm = tid >> 1;  // threads < 2·n_chunk: m (even) / l (odd) of chunk tid / 2
            const bool has_m = tid < 2 * n_chunk;
            __builtin_amdgcn_s_sleep(POLL_SLEEP_PART);
            uint64_t vo = has_o ? ld_word(pk + (size_t)cc * PART_W + 2 + d0 + e) : (uint64_t)(tbase + 1) << 32;
            uint64_t vm = has_m ? ld_word(pk + (size_t)cm * PART_W + (tid & 1)) : (uint64_t)(tbase + 1) << 32;
            long long t0 = 0;
            for (;;) {
                const bool all = (uint32_t)(vo >> 32) == tbase + 1 && (uint32_t)(vm >> 32) == tbase + 1;
                if (all || wt.broken) break;
                if ((uint32_t)(vo >> 32) != tbase + 1) vo = ld_word(pk + (size_t)cc * PART_W + 2 + d0 + e);
                if ((uint32_t)(vm >> 32) != tbase + 1) vm = ld_word(pk + (size_t)cm * PART_W + (tid & 1));
                if (wt.expired(t0)) break;
            }
            if (has_o) s_mo[cc][e] = __uint_as_float((uint32_t)vo);
            if (has_m) s_ml[tid & 1][cm] = __uint_as_float((uint32_t)vm);
            __syncthreads();
            stamp(s_stamp, prof_on, 5 + 12 * l);
            if (wave == 0) {
                // lane ℓ: chunk ℓ % 32 (past n_chunk: weight 0), dims 4·(ℓ / 32) … + 3 of the eight. Every LDS read
                // is unconditional (in bounds for any chunk index) and issued at once; the sums run over the 32 lanes
                // of each half (lane bits 4 … 0), so both halves hold M and L
                const int cl = lane & 31, half = lane >> 5;
                const bool valid = cl < n_chunk;
                const float mr = s_ml[0][cl], lr = s_ml[1][cl];
                const float4 o4 = *reinterpret_cast<const float4 *>(&s_mo[cl][4 * half]);
                const float m = valid ? mr : -INFINITY;
                const float M = group_max<16>(m, lane);
                const float wc = valid ? expf(m - M) : 0.0f;
                // (chunks past n_chunk: whatever the LDS holds there, selected away — 0·inf would be NaN)
                const float Lsum = group_sum<16>(valid ? lr * wc : 0.0f, lane);
                const float o0 = valid ? o4.x * wc : 0.0f, o1 = valid ? o4.y * wc : 0.0f;
                const float o2 = valid ? o4.z * wc : 0.0f, o3 = valid ? o4.w * wc : 0.0f;
                // exchange-and-halve across lane bits 4 and 3 (as wave.h's halve, written out on scalars: an array
                // here would be indexed per lane), then a plain sum over bits 2 … 0: lane keeps dim 2·b4 + b3
                const bool b4 = (lane & 16) != 0, b3 = (lane & 8) != 0;
                const float p0 = (b4 ? o2 : o0) + lane_swap<16>(b4 ? o0 : o2, lane);
                const float p1 = (b4 ? o3 : o1) + lane_swap<16>(b4 ? o1 : o3, lane);
                const float q = (b3 ? p1 : p0) + lane_swap<8>(b3 ? p0 : p1, lane);
                const float O = group_sum<4>(q, lane);
                if ((lane & 7) == 0)
                    put_word(xw + OFF_ATT + (h0 + hh) * D + d0 + 4 * half + ((lane >> 3) & 3), O / Lsum, tbase + 2);
            }
        }
        stamp(s_stamp, prof_on, 6 + 12 * l);

        // ---- D: o rows 4w + wave (K = 2048), + residual
        {
            const int row = 4 * w + wave;
            RowW<2> rw;
            row_issue<2>(rw, L.q[3], L.d[3], row, lane);
            take<8, POLL_SLEEP_O>(wt, xw + OFF_ATT, QD, tbase + 2, s_att);
            stamp(s_stamp, prof_on, 7 + 12 * l);
            float xv[2][16];
            lds_x<2>(xv, s_att, lane);
            const float v = wave_sum(row_dot<2>(rw, xv), lane);
            if (lane == 0) put_word(xw + OFF_H1 + row, s_x[row] + v, tbase + 3);
        }
        stamp(s_stamp, prof_on, 8 + 12 * l);

        // ---- E: gate / up rows 12w + 3·wave + r (K = 1024), ffn_norm, SwiGLU
        {
            float wv[1][16];
            glob_x<1>(wv, L.ffn_norm, lane);  // the norm weights first, as in A
            RowW<1> rg[3], ru[3];
#pragma unroll
            for (int r = 0; r < 3; r++) {
                const int row = 12 * w + 3 * wave + r;
                row_issue<1>(rg[r], L.q[4], L.d[4], row, lane);
                row_issue<1>(ru[r], L.q[5], L.d[5], row, lane);
            }
            take<4, POLL_SLEEP_GU>(wt, xw + OFF_H1, DIM, tbase + 3, s_h);
            stamp(s_stamp, prof_on, 9 + 12 * l);
            float xv[1][16];
            lds_x<1>(xv, s_h, lane);
            norm16<1>(xv, wv, a.eps, DIM, lane);
            float ag[4], au[4];
#pragma unroll
            for (int r = 0; r < 3; r++) {
                ag[r] = row_dot<1>(rg[r], xv);
                au[r] = row_dot<1>(ru[r], xv);
            }
            ag[3] = 0.0f, au[3] = 0.0f;
            const float g = wave_sum_rows<4>(ag, lane), u = wave_sum_rows<4>(au, lane);
            if ((lane & 15) == 0 && (lane >> 4) < 3)
                put_word(xw + OFF_FF + 12 * w + 3 * wave + (lane >> 4), (g / (1.0f + expf(-g))) * u, tbase + 4);
        }
        stamp(s_stamp, prof_on, 10 + 12 * l);

        // ---- F: down rows 4w + wave (K = 3072), + residual
        {
            const int row = 4 * w + wave;
            RowW<3> rw;
            row_issue<3>(rw, L.q[6], L.d[6], row, lane);
            take<12, POLL_SLEEP_DOWN>(wt, xw + OFF_FF, NFF, tbase + 4, s_ff);
            stamp(s_stamp, prof_on, 11 + 12 * l);
            float xv[3][16];
            lds_x<3>(xv, s_ff, lane);
            const float v = wave_sum(row_dot<3>(rw, xv), lane);
            const float xn = s_h[row] + v;
            if (lane == 0) {
                put_word(xw + OFF_H2 + row, xn, tbase + 5);  // the next layer's, or the LM head's, input
                if (l + 1 == a.n_layer) a.x_out[row] = xn;  // the residual (an out-of-range id's embedding)
            }
        }
        stamp(s_stamp, prof_on, 12 + 12 * l);
    }
    // ---- T: the LM head (output_norm fused, dmv_norm over token_embd: the tied head, text.rs:655-658) on workgroup
    // w's rows [r0, r1) (a 256th of the vocabulary), and with `choose` the greedy choice of k_choose on them
    // (sampling.rs:38-62: each distinct window id penalised once, in place; fp compared; first maximum; NaN never wins,
    // NaN at index 0 → token 0): each workgroup's best key (choose_key) goes to workgroup 0 as two tagged words (no
    // atomics: 256 on one address would queue), which keeps the largest, writes the token, appends it to the history
    // and advances position and length.
    {
        const uint32_t ttag = seq * 256u + (uint32_t)(XPL * a.n_layer - 1);  // F's words of the last layer
        const uint64_t *xlast = xw;
        const int nv = a.n_vocab;
        const int r0 = (int)(((long long)w * nv) / NWG), r1 = (int)(((long long)(w + 1) * nv) / NWG);
        const int cnt = r1 - r0;
        const int nb = (cnt + 31) / 32;  // batches of 8 rows a wave: rows r0 + wave + 4·(8b + i)
        auto issue = [&](RowW<1>(&bt)[8], int b) {
#pragma unroll
            for (int i = 0; i < 8; i++)
                row_issue<1, true>(bt[i], a.emb_q, a.emb_d, min(r0 + wave + 4 * (8 * b + i), r1 - 1), lane);
        };
        RowW<1> cur[8];
        float wv[1][16];
        glob_x<1>(wv, a.out_norm, lane);
        // the choice's window: ids hist[len − min(len, window) … len) (penalised when rp ≠ 1) that fall in [r0, r1)
        // mark their rows (a repeated id marks the same row: each distinct id is penalised once)
        const int len = a.choose ? a.state[1] : 0;
        const int n_win = a.choose && a.rp != 1.0f ? min(len, a.window) : 0;
        const uint32_t w_id = tid < n_win ? a.hist[len - n_win + tid] : 0xffffffffu;
        for (int u = tid; u < MAX_HEAD_ROWS / 16; u += TPB) reinterpret_cast<uint4 *>(s_pen)[u] = make_uint4(0, 0, 0, 0);
        if (tid == 0) s_nan0 = 0;
        take<4>(wt, xlast + OFF_H2, DIM, ttag, s_x);  // its barrier also orders the clearing before the marks
        // the first batch's loads after the wait, not ahead of its polls (the head's rows, unlike a layer's, take
        // many batches, the later ones hidden under the arithmetic): 2661 → 2671 tokens/s
        issue(cur, 0);
        stamp(s_stamp, prof_on, 1 + 12 * a.n_layer);
        if (w_id >= (uint32_t)r0 && w_id < (uint32_t)r1) s_pen[w_id - r0] = 1;
        for (int j = tid + TPB; j < n_win; j += TPB) {
            const uint32_t t = a.hist[len - n_win + j];
            if (t >= (uint32_t)r0 && t < (uint32_t)r1) s_pen[t - r0] = 1;
        }
        float xv[1][16];
        lds_x<1>(xv, s_x, lane);
        norm16<1>(xv, wv, a.eps, DIM, lane);
        __syncthreads();  // the marks
        float bv = -INFINITY;
        uint32_t bi = 0xffffffffu;
        for (int b = 0; b < nb; b++) {
            RowW<1> nxt[8];
            issue(nxt, min(b + 1, nb - 1));  // the next batch's loads go out before this one's arithmetic
            float acc[8];
#pragma unroll
            for (int i = 0; i < 8; i++) acc[i] = row_dot<1>(cur[i], xv);
            const float v = wave_sum_rows<8>(acc, lane);  // lane 8i holds row i of the batch
            const int row = r0 + wave + 4 * (8 * b + (lane >> 3));
            if ((lane & 7) == 0 && row < r1) {
                float x = v;
                if (a.choose) {
                    if (s_pen[row - r0]) x = x < 0.0f ? x * a.rp : x / a.rp;
                    if (row == 0 && x != x) s_nan0 = 1;
                }
                a.logits[row] = x;
                if (a.choose && a.fp != 0.0f && a.counts[row] != 0u) x = x - a.fpen[row];
                if (better(x, (uint32_t)row, bv, bi)) {
                    bv = x;
                    bi = (uint32_t)row;
                }
            }
#pragma unroll
            for (int i = 0; i < 8; i++) cur[i] = nxt[i];
        }
        stamp(s_stamp, prof_on, 2 + 12 * a.n_layer);
        if (a.choose) {
            // the workgroup's best → its key (NaN at index 0 after the penalty: the top key, token 0) → two words
            wave_best(bv, bi, lane);
            if (lane == 0) {
                s_bv[wave] = bv;
                s_bi[wave] = bi;
            }
            __syncthreads();
            const uint32_t ctag = seq * 256u + (uint32_t)(XPL * a.n_layer);
            if (tid == 0) {
#pragma unroll
                for (int q = 1; q < 4; q++)
                    if (better(s_bv[q], s_bi[q], bv, bi)) {
                        bv = s_bv[q];
                        bi = s_bi[q];
                    }
                const uint64_t key = s_nan0 ? ~0ull : choose_key(bv, bi);
                put_word(xw + OFF_BEST + 2 * w, __uint_as_float((uint32_t)(key >> 32)), ctag);
                put_word(xw + OFF_BEST + 2 * w + 1, __uint_as_float((uint32_t)key), ctag);
            }
            // workgroup 0 takes the 256 keys, keeps the largest (the first maximum of the whole vocabulary), writes
            // the token, appends it to the history and advances position and length
            if (w == 0) {
                take<2>(wt, xw + OFF_BEST, 2 * NWG, ctag, s_att);
                if (wave == 0) {
                    uint64_t k = 0;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int g = lane + 64 * q;
                        const uint64_t kq =
                            ((uint64_t)__float_as_uint(s_att[2 * g]) << 32) | __float_as_uint(s_att[2 * g + 1]);
                        k = kq > k ? kq : k;
                    }
#pragma unroll
                    for (int m = 32; m >= 1; m >>= 1) {
                        uint32_t ohi, olo;
                        const uint32_t hi = (uint32_t)(k >> 32), lo = (uint32_t)k;
                        switch (m) {
                        case 32: ohi = lane_swap_u32<32>(hi, lane), olo = lane_swap_u32<32>(lo, lane); break;
                        case 16: ohi = lane_swap_u32<16>(hi, lane), olo = lane_swap_u32<16>(lo, lane); break;
                        case 8: ohi = lane_swap_u32<8>(hi, lane), olo = lane_swap_u32<8>(lo, lane); break;
                        case 4: ohi = lane_swap_u32<4>(hi, lane), olo = lane_swap_u32<4>(lo, lane); break;
                        case 2: ohi = lane_swap_u32<2>(hi, lane), olo = lane_swap_u32<2>(lo, lane); break;
                        default: ohi = lane_swap_u32<1>(hi, lane), olo = lane_swap_u32<1>(lo, lane); break;
                        }
                        const uint64_t o = ((uint64_t)ohi << 32) | olo;
                        k = o > k ? o : k;
                    }
                    if (lane == 0) {
                        const uint32_t t = ~(uint32_t)k;
                        const uint32_t tk = t < (uint32_t)nv ? t : 0u;  // every logit NaN, or NaN at 0 → 0
                        a.tok[0] = tk;
                        a.hist[len] = tk;
                        if (a.fp != 0.0f) {
                            const uint32_t c = a.counts[tk] + 1u;
                            a.counts[tk] = c;
                            a.fpen[tk] = a.fp * (float)c;
                        }
                        a.state[1] = len + 1;
                        a.state[0] = pos + 1;  // every workgroup read pos at its start, before its key
                    }
                }
            }
        }
        stamp(s_stamp, prof_on, 3 + 12 * a.n_layer);
    }
    // every workgroup has read seq: workgroup 0 has waited for the last layer's words of all of them
    if (w == 0 && tid == 0) __hip_atomic_store(a.seq, seq + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prof_on) {
        __syncthreads();
        for (int i = tid; i < 1 + 12 * a.n_layer + 3; i += TPB) a.prof[i] = s_stamp[i];
    }
}

}  // namespace

size_t token_step_words() { return XWORDS; }

int token_step_stamps(int n_layer) { return 1 + 12 * n_layer + 3; }

// the smallest chunk of 16·NI keys whose 32 chunks a KV head cover the cache: at the bench's 1536-row cache, chunks
// of 48 keys (every workgroup busy at the read's last keys) against 64: the attention's wait 1.42 → 1.25 µs a layer,
// its work 1.76 → 1.67, 2395 → 2434 tokens/s (A/B twice on one box)
int token_step_ni(int n_ctx) {
    static const int nis[] = {2, 3, 4, 6, 8, 12, 16};
    for (int ni : nis)
        if (n_ctx <= 16 * ni * WPK) return ni;
    return 0;
}

// the LM-head tail gives every workgroup at least one row (its first batch's loads are clamped into its share), so
// the vocabulary holds at least one row a workgroup
bool token_step_shape(const htr_text_config &c) {
    return c.dim == DIM && c.n_head * c.d_head == QD && c.n_kv * c.d_head == KVD && c.n_ff == NFF && c.d_head == D &&
           c.n_head == 2 * c.n_kv && c.n_layer <= MAX_LAYERS && c.n_vocab >= NWG && c.n_vocab <= NWG * MAX_HEAD_ROWS;
}

int token_step_fits(htr_device *dev, int n_ctx, const char **why) {
    const int ni = token_step_ni(n_ctx);
    if (!ni) {
        *why = "the cache is longer than 8192 rows";
        return 0;
    }
    int per_cu = 0;
    hipError_t e = hipSuccess;
    switch (ni) {
    case 2: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_token<2>, TPB, 0); break;
    case 3: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_token<3>, TPB, 0); break;
    case 4: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_token<4>, TPB, 0); break;
    case 6: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_token<6>, TPB, 0); break;
    case 8: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_token<8>, TPB, 0); break;
    case 12: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_token<12>, TPB, 0); break;
    default: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_token<16>, TPB, 0); break;
    }
    if (e != hipSuccess) {
        *why = "the occupancy query failed";
        return 0;
    }
    if (per_cu * dev->n_cu < NWG) {
        *why = "its 256 workgroups do not fit the device at once";
        return 0;
    }
    return 1;
}

// each workgroup's XCD in a launch of the step's shape
__global__ __launch_bounds__(TPB) void k_xcd_map(int *out) {
    if (threadIdx.x == 0) out[blockIdx.x] = xcd_id();
}

int token_step_xcds(htr_device *dev, const char **why) {
    if (dev->xcd_round_robin < 0) {
        int *d = nullptr;
        HTR_TRY(htr_dev_alloc(dev, NWG * sizeof(int), HTR_MEM_WORK, (void **)&d));
        hipLaunchKernelGGL(k_xcd_map, dim3(NWG), dim3(TPB), 0, dev->stream, d);
        int rc = htr_launched(dev, "k_xcd_map");
        int x[NWG];
        if (rc == 0) rc = htr_download(dev, x, d, sizeof x);
        htr_dev_free(dev, d);
        if (rc) return rc;
        // every XCD holds the workgroups of one residue mod 8 (x[0 … 7] distinct), so its slots w >> 3 are 0 … 31
        bool ok = true;
        unsigned seen = 0;
        for (int w = 0; w < NWG; w++) ok = ok && x[w] == x[w & 7];
        for (int w = 0; w < 8; w++) seen |= 1u << (x[w] & 7);
        dev->xcd_round_robin = ok && seen == 0xffu ? 1 : 0;
        // the premise of the two XCD-local hand-overs: a word stored at workgroup scope is seen by the agent-scope
        // loads of another workgroup on the same XCD (it stays in that XCD's L2). A cache behaviour of this part, not
        // a guarantee of the memory model: probed once a device, on every XCD, with bounded waits (a word never seen
        // ends its wait after 2^16 polls and the probe reports it)
        for (int x = 0; x < 8 && dev->xcd_round_robin == 1; x++) {
            double us = 0.0;
            int vis = 0;
            HTR_TRY(htr_debug_handover(dev, 0, x, x + 8, 1024, 16, 32, 1 << 16, &us, &vis));
            if (!vis) dev->xcd_round_robin = 2;
        }
    }
    if (dev->xcd_round_robin == 0) *why = "its workgroups do not spread round-robin over 8 XCDs";
    if (dev->xcd_round_robin == 2)
        *why = "a word stored at workgroup scope was not seen by another workgroup of its XCD (the XCD-local "
               "hand-overs' premise)";
    return dev->xcd_round_robin == 1;
}

int launch_decode_token(htr_device *dev, hipStream_t st, int n_ctx, const TokArgs &a) {
    const int ni = token_step_ni(n_ctx);
    switch (ni) {
    case 2: hipLaunchKernelGGL(k_decode_token<2>, dim3(NWG), dim3(TPB), 0, st, a); break;
    case 3: hipLaunchKernelGGL(k_decode_token<3>, dim3(NWG), dim3(TPB), 0, st, a); break;
    case 4: hipLaunchKernelGGL(k_decode_token<4>, dim3(NWG), dim3(TPB), 0, st, a); break;
    case 6: hipLaunchKernelGGL(k_decode_token<6>, dim3(NWG), dim3(TPB), 0, st, a); break;
    case 8: hipLaunchKernelGGL(k_decode_token<8>, dim3(NWG), dim3(TPB), 0, st, a); break;
    case 12: hipLaunchKernelGGL(k_decode_token<12>, dim3(NWG), dim3(TPB), 0, st, a); break;
    case 16: hipLaunchKernelGGL(k_decode_token<16>, dim3(NWG), dim3(TPB), 0, st, a); break;
    default: return htr_fail("decode token: a %d-row cache (at most 8192)", n_ctx);
    }
    char name[32];
    snprintf(name, sizeof name, "k_decode_token<%d>", ni);
    return htr_launched(dev, name);
}
