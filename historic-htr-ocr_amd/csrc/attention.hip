// Attention for gfx950: the decode step's q/k post-processing and split-K GQA decode attention, and the prefill's
// per-head norm + RoPE + KV store and causal flash attention.
//
// Reference semantics: qkv_post.wgsl:31-83, attn_decode.wgsl:34-100 + attn_merge.wgsl:22-39 (text.rs:639-641),
// rms_norm.wgsl / rope_neox.wgsl / kv_store.wgsl / attention_causal.wgsl (text.rs:484-499). Head dim 128.
//
// KV cache layout (this library's): f16, head-major per layer, [n_kv][n_ctx][128] — one KV head's keys are
// contiguous, so a workgroup working on (kv head, key chunk) reads one contiguous range (256 bytes per key).
#include "htr_internal.h"
#include "wave.h"

namespace {

constexpr int D = 128;

// one head's 128 values held as (lane, lane + 64) by a 64-lane wave: RMS norm with w, then RoPE NEOX with (c, s)
__device__ __forceinline__ void norm_rope(float &x0, float &x1, const float *w, const float *rope_row, int lane,
                                          float eps) {
    const float ss = wave_sum(x0 * x0 + x1 * x1, lane);
    const float scale = 1.0f / sqrtf(ss / (float)D + eps);
    const float y0 = (x0 * scale) * w[lane], y1 = (x1 * scale) * w[lane + 64];
    const float c = rope_row[2 * lane], s = rope_row[2 * lane + 1];
    x0 = y0 * c - y1 * s;
    x1 = y0 * s + y1 * c;
}

// qkv_post: block h < n_head: q head (norm, rope, in place); < n_head + n_kv: k head (norm, rope, f16 cache);
// else v head (f16 cache). One wave per head.
__global__ __launch_bounds__(64) void k_qkv_post(float *qkv, const float *qn, const float *kn, const float *rope,
                                                 int n_head, int n_kv, const int *pos_dev, int pos_arg, int n_ctx,
                                                 float eps, _Float16 *kc, _Float16 *vc) {
    const int h = blockIdx.x, lane = threadIdx.x;
    const int pos = pos_dev ? *pos_dev : pos_arg;
    if (pos < 0 || pos >= n_ctx) return;  // the cache has no such row (the host checks positions first)
    float *x = qkv + (size_t)h * D;
    float x0 = x[lane], x1 = x[lane + 64];
    if (h >= n_head + n_kv) {
        _Float16 *o = vc + ((size_t)(h - n_head - n_kv) * n_ctx + pos) * D;
        o[lane] = (_Float16)x0;
        o[lane + 64] = (_Float16)x1;
        return;
    }
    norm_rope(x0, x1, h < n_head ? qn : kn, rope + (size_t)pos * D, lane, eps);
    if (h < n_head) {
        x[lane] = x0;
        x[lane + 64] = x1;
    } else {
        _Float16 *o = kc + ((size_t)(h - n_head) * n_ctx + pos) * D;
        o[lane] = (_Float16)x0;
        o[lane + 64] = (_Float16)x1;
    }
}

// prefill rows: block (t, h): q heads, k heads (→ f16 cache rows pos0 + t), v heads (→ f16 cache)
__global__ __launch_bounds__(64) void k_qk_rows(float *q, float *k, const float *v, const float *qn, const float *kn,
                                                const float *rope, int n_head, int n_kv, int pos0, int n_ctx,
                                                float eps, _Float16 *kc, _Float16 *vc) {
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int pos = pos0 + t;
    if (h < n_head) {
        float *x = q + ((size_t)t * n_head + h) * D;
        float x0 = x[lane], x1 = x[lane + 64];
        norm_rope(x0, x1, qn, rope + (size_t)pos * D, lane, eps);
        x[lane] = x0;
        x[lane + 64] = x1;
    } else if (h < n_head + n_kv) {
        const int j = h - n_head;
        float *x = k + ((size_t)t * n_kv + j) * D;
        float x0 = x[lane], x1 = x[lane + 64];
        norm_rope(x0, x1, kn, rope + (size_t)pos * D, lane, eps);
        _Float16 *o = kc + ((size_t)j * n_ctx + pos) * D;
        o[lane] = (_Float16)x0;
        o[lane + 64] = (_Float16)x1;
    } else {
        const int j = h - n_head - n_kv;
        const float *x = v + ((size_t)t * n_kv + j) * D;
        _Float16 *o = vc + ((size_t)j * n_ctx + pos) * D;
        o[lane] = (_Float16)x[lane];
        o[lane + 64] = (_Float16)x[lane + 64];
    }
}

// ---- split-K decode attention -----------------------------------------------------------------------------------------
//
// grid chunks · n_kv, 256 threads. A workgroup takes C = 16·NI keys of one KV head and both of its q heads (GQA
// group 2), so every K / V byte is read once. Thread t owns the 16-byte slice j = t & 15 (dims 8j … 8j+7) of the keys
// kk + 16·i (kk = t >> 4, i < NI): one wave-wide load reads 4 keys (1 KiB), and every K and V load of the chunk is
// issued before the first use.
//   1. scores s[h][key] = (q_h·scale)·k: 8 products per slice, summed over the 16 slices of a key by an
//      exchange-and-halve butterfly over all 2·NI (key, head) values at once → LDS (barrier)
//   2. every wave: m = max s, p = exp(s − m), l = Σ p for both heads → its own LDS copy of p (no barrier)
//   3. o[h][·] = Σ p·v from the V registers, summed over the 16 key positions (lane bits 5, 4, then the 4 waves in
//      LDS: barrier)
//   4. the chunk's (m, l, o) → partials [h][c][130]; the last workgroup of the KV head (atomic ticket) merges:
//      M = max m_c, w_c = e^(m_c − M), O = Σ o_c·w_c / Σ l_c·w_c — each wave one (head, 64 dims), its loads of all
//      chunks issued at once, no workgroup barrier. A single-chunk call writes O = o / l directly.
// Cross-lane moves are DPP / permlane VALU moves (wave.h). Cross-workgroup traffic is the partials' stores and loads
// plus the ticket atomic (one 128-byte line per KV head), with no release fence (one per workgroup would write back
// the L2 each time): with 8 KV heads, on a device whose launches put workgroup b on XCD b mod 8 and whose L2 shows a
// workgroup-scope store to the other workgroups of its XCD (both checked at open), every workgroup of a KV head shares
// one XCD, and the stores and the ticket stay in its L2 (workgroup scope); otherwise they go through the coherence
// point (agent scope, sc1).
constexpr int AW = 256;
constexpr int MAX_CHUNK_KEYS = 256;  // C ≤ 256 (NI ≤ 16)
constexpr int MAX_CHUNKS = 256;      // chunks per KV head: n_ctx ≤ 65536
constexpr int MERGE_FAST = 32;       // chunks merged by the branch-free path (each merging thread holds their o
                                     // partials in registers; n_ctx ≤ 8192 stays within it)
static_assert(MAX_CHUNKS % MERGE_FAST == 0, "the merge's weight groups fit s_w");
constexpr int CNT_STRIDE = 32;       // ticket counters 128 bytes apart: the KV heads' atomics do not share a line

// the KV cache stream: non-temporal loads (each key / value is read once a step)
typedef int gint4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 aload16(const void *p) {
    const gint4 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) gint4 *)(uintptr_t)p);
    return make_int4(v.x, v.y, v.z, v.w);
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

__device__ __forceinline__ float ld_dev(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// XL: every workgroup of a KV head runs on one XCD — the partials and the ticket are handed over in that XCD's L2
// (workgroup-scope stores and atomic, read by agent-scope loads that find the L2's lines); else through the coherence
// point (agent scope)
__device__ __forceinline__ void st_part(float *p, float v, bool xl) {
    if (xl) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// qkv_post.wgsl's per-head RMS norm and RoPE NEOX (pairs (i, i + 64)) at one position, for the 8 dims 8j … 8j + 7
// of one head's raw row: the 16 lanes j = 0 … 15 of a lane row hold the head together (Σx² over them); the lane also
// holds the partner dims (slice j ^ 8). Loads first (post_load), the arithmetic later (post_apply), so that the
// loads go out before the K / V loads and the arithmetic waits for these alone.
struct PostIn {
    float4 a[2], b[2], wa[2], wb[2];
};
__device__ __forceinline__ void post_load(PostIn &p, const float *x, const float *w, int j) {
    const int jp = j ^ 8;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        p.a[h] = *reinterpret_cast<const float4 *>(x + 8 * j + 4 * h);
        p.b[h] = *reinterpret_cast<const float4 *>(x + 8 * jp + 4 * h);
        p.wa[h] = *reinterpret_cast<const float4 *>(w + 8 * j + 4 * h);
        p.wb[h] = *reinterpret_cast<const float4 *>(w + 8 * jp + 4 * h);
    }
}
__device__ __forceinline__ void unpack4x2(const float4 (&v)[2], float (&f)[8]) {
    f[0] = v[0].x, f[1] = v[0].y, f[2] = v[0].z, f[3] = v[0].w, f[4] = v[1].x, f[5] = v[1].y, f[6] = v[1].z, f[7] = v[1].w;
}
// cs: the (c, s) pairs of rope indices 8(j % 8) … + 7
__device__ __forceinline__ void post_apply(const PostIn &p, const float (&cs)[16], int j, int lane, float eps,
                                           float (&out)[8]) {
    float a[8], b[8], wa[8], wb[8];
    unpack4x2(p.a, a);
    unpack4x2(p.b, b);
    unpack4x2(p.wa, wa);
    unpack4x2(p.wb, wb);
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) ss = fmaf(a[e], a[e], ss);
    ss = group_sum<8>(ss, lane);
    const float scale = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float ya = (a[e] * scale) * wa[e], yb = (b[e] * scale) * wb[e];
        const float c = cs[2 * e], s = cs[2 * e + 1];
        out[e] = j < 8 ? ya * c - yb * s : yb * s + ya * c;
    }
}

// FUSED: q is the raw [q | k | v] row of the qkv matvec and the kernel does qkv_post's work itself: each workgroup
// norms and ropes its two q heads; the new key / value (position n_keys − 1) are made from the raw row, rounded to
// f16 as the cache holds them, used in place of the cache row by the workgroup whose chunk holds them, and stored
// into the cache by that workgroup (no other workgroup reads that row)
template <int NI, bool FUSED>
__global__ __launch_bounds__(AW) void k_attn_decode(const float *q, const _Float16 *kc, const _Float16 *vc, int n_kv,
                                                    int n_ctx, const int *pos_dev, int n_keys_arg, int max_chunk,
                                                    float scale, float post, float *part, uint32_t *counters,
                                                    float *out, AttnFuse fz, int xl) {
    constexpr int C = 16 * NI;
    constexpr int N = 2 * NI;              // (key, head) values per thread
    constexpr int KL = C >= 64 ? C / 64 : 1;  // keys per lane in the softmax
    __shared__ float s_sc[2][C];
    __shared__ float s_pw[4][2][C];  // each wave's copy of p
    __shared__ float s_lw[2];
    __shared__ float s_o[4][2][D];
    __shared__ float s_w[4][MAX_CHUNKS];
    __shared__ int s_last;
    // a 1D grid of the KV heads' chunks; with 8 KV heads workgroup b runs on XCD b mod 8 (a launch spreads its
    // workgroups round-robin), so a KV head's chunks and its merge's loads of their partials share one XCD's L2: at
    // 512 keys 5.52 → 5.25 µs a graph node (the same at 2048 and 8192 keys)
    const int nb = gridDim.x / n_kv;
    const int c = n_kv == 8 ? (int)blockIdx.x >> 3 : (int)blockIdx.x % nb;
    const int kvh = n_kv == 8 ? (int)blockIdx.x & 7 : (int)blockIdx.x / nb;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = tid & 15, kk = tid >> 4;
    // keys beyond the cache are never read (the host checks positions first; a bad one yields no output)
    const int n_keys = min(pos_dev ? *pos_dev + 1 : n_keys_arg, n_ctx);
    if (FUSED && pos_dev && *pos_dev >= n_ctx) return;  // the cache has no such row (the host checks positions first)
    const int n_chunk = (n_keys + C - 1) / C;
    if (c >= n_chunk || n_chunk > max_chunk) return;  // uniform per workgroup
    const int k0 = c * C;
    const int h0 = 2 * kvh;

    // FUSED: the raw q / k / v slices, norm weights and rope row go out first (they come from L2, the keys from HBM)
    const int pos = n_keys - 1;
    PostIn pin[3];
    float4 vraw[2], rope4[4];
    if constexpr (FUSED) {
        post_load(pin[0], q + (size_t)h0 * D, fz.qn, j);
        post_load(pin[1], q + (size_t)(h0 + 1) * D, fz.qn, j);
        post_load(pin[2], q + (size_t)(fz.n_head + kvh) * D, fz.kn, j);
        const float *vr0 = q + (size_t)(fz.n_head + n_kv + kvh) * D + 8 * j;
        vraw[0] = *reinterpret_cast<const float4 *>(vr0);
        vraw[1] = *reinterpret_cast<const float4 *>(vr0 + 4);
        const float *rr = fz.rope + (size_t)pos * D + 16 * (j & 7);
#pragma unroll
        for (int i = 0; i < 4; i++) rope4[i] = *reinterpret_cast<const float4 *>(rr + 4 * i);
        __builtin_amdgcn_sched_barrier(0);
    }

    // 0. every K and V load of the chunk (keys past n_keys read the last key and are masked)
    const _Float16 *kb = kc + (size_t)kvh * n_ctx * D, *vb = vc + (size_t)kvh * n_ctx * D;
    int4 kr[NI], vr[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int key = min(k0 + kk + 16 * i, n_keys - 1);
        kr[i] = aload16(kb + (size_t)key * D + 8 * j);
    }
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int key = min(k0 + kk + 16 * i, n_keys - 1);
        vr[i] = aload16(vb + (size_t)key * D + 8 * j);
    }
    if constexpr (FUSED) __builtin_amdgcn_sched_barrier(0);  // the K / V loads are out before the arithmetic
    float qa[8], qb[8];
    int4 knew = make_int4(0, 0, 0, 0), vnew = make_int4(0, 0, 0, 0);
    if constexpr (FUSED) {
        float cs[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            cs[4 * i] = rope4[i].x, cs[4 * i + 1] = rope4[i].y, cs[4 * i + 2] = rope4[i].z, cs[4 * i + 3] = rope4[i].w;
        }
        float ta[8], tb[8], kn8[8], v8[8];
        post_apply(pin[0], cs, j, lane, fz.eps, ta);
        post_apply(pin[1], cs, j, lane, fz.eps, tb);
        post_apply(pin[2], cs, j, lane, fz.eps, kn8);
        unpack4x2(vraw, v8);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            qa[e] = ta[e] * scale;
            qb[e] = tb[e] * scale;
        }
        knew = pack8(kn8);
        vnew = pack8(v8);
        if (c == n_chunk - 1 && kk == 0) {
            *reinterpret_cast<int4 *>(fz.kc + ((size_t)kvh * n_ctx + pos) * D + 8 * j) = knew;
            *reinterpret_cast<int4 *>(fz.vc + ((size_t)kvh * n_ctx + pos) * D + 8 * j) = vnew;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            qa[e] = q[h0 * D + 8 * j + e] * scale;
            qb[e] = q[(h0 + 1) * D + 8 * j + e] * scale;
        }
    }

    // 1. scores. FUSED: every key at or past pos takes the new row (keys past pos were clamped onto row pos, whose
    // cache contents are stale — a rewound session's old row — and being rewritten by this workgroup): masked keys
    // then multiply finite values by 0 below, whatever the cache held
    float v[N];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        float kf[8];
        unpack8(FUSED && k0 + kk + 16 * i >= pos ? knew : kr[i], kf);
        float da = 0.0f, db = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            da = fmaf(qa[e], kf[e], da);
            db = fmaf(qb[e], kf[e], db);
        }
        v[2 * i] = da;
        v[2 * i + 1] = db;
    }
    if constexpr (N >= 16) {
        halve<N, 8, 4>(v, lane);  // lane j keeps values (N/16)·j + r
#pragma unroll
        for (int r = 0; r < N / 16; r++) {
            const int idx = (N / 16) * j + r, i = idx >> 1, h = idx & 1;
            const int key = kk + 16 * i;
            s_sc[h][key] = k0 + key < n_keys ? v[r] * post : -INFINITY;
        }
    } else {
        constexpr int S = N == 2 ? 1 : N == 4 ? 2 : 3;  // log2 N
        halve<N, 8, S>(v, lane);                         // lane j keeps value j >> (4 − S)
        const float t = group_sum<(8 >> S)>(v[0], lane);
        if ((j & ((16 >> S) - 1)) == 0) {
            const int idx = j >> (4 - S), i = idx >> 1, h = idx & 1;
            const int key = kk + 16 * i;
            s_sc[h][key] = k0 + key < n_keys ? t * post : -INFINITY;
        }
    }
    __syncthreads();

    // 2. softmax statistics, every wave for both heads into its own copy of p
    float l_h[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        float sv[KL], mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < KL; i++) {
            const int key = lane + 64 * i;
            sv[i] = key < C ? s_sc[h][key] : -INFINITY;
            mx = fmaxf(mx, sv[i]);
        }
        mx = wave_max(mx, lane);
        float l = 0.0f;
#pragma unroll
        for (int i = 0; i < KL; i++) {
            const int key = lane + 64 * i;
            const float p = expf(sv[i] - mx);  // masked keys: exp(−inf) = 0
            if (key < C) s_pw[wave][h][key] = p;
            l += p;
        }
        l_h[h] = wave_sum(l, lane);
        if (h == 0 && wave == 0 && lane == 0) s_lw[0] = mx;
        if (h == 1 && wave == 0 && lane == 0) s_lw[1] = mx;
    }
    __builtin_amdgcn_wave_barrier();

    // 3. values
    float o[16];  // [h][e]
#pragma unroll
    for (int e = 0; e < 16; e++) o[e] = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        float vf[8];
        unpack8(FUSED && k0 + kk + 16 * i >= pos ? vnew : vr[i], vf);
        const float pa = s_pw[wave][0][kk + 16 * i], pb = s_pw[wave][1][kk + 16 * i];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            o[e] = fmaf(pa, vf[e], o[e]);
            o[8 + e] = fmaf(pb, vf[e], o[8 + e]);
        }
    }
    halve<16, 32, 2>(o, lane);  // over lane bits 5, 4: lane keeps values 8·b5 + 4·b4 + r
    {
        const int base = 8 * ((lane >> 5) & 1) + 4 * ((lane >> 4) & 1);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int idx = base + r, h = idx >> 3, e = idx & 7;
            s_o[wave][h][8 * j + e] = o[r];
        }
    }
    __syncthreads();
    const int hh = tid >> 7, d = tid & 127;  // 256 threads = 2 heads × 128 dims
    const float oc = (s_o[0][hh][d] + s_o[1][hh][d]) + (s_o[2][hh][d] + s_o[3][hh][d]);
    const float lc = l_h[hh];  // every wave holds both heads' sums
    const int h = h0 + hh;
    if (n_chunk == 1) {
        out[h * D + d] = oc / lc;
        return;
    }

    // 4. partials, then the last workgroup of the KV head merges
    float *pc = part + ((size_t)h * max_chunk + c) * (D + 2);  // [h][c][m, l, o[128]]
    st_part(pc + 2 + d, oc, xl);
    if (d == 0) st_part(pc, s_lw[hh], xl);
    if (d == 1) st_part(pc + 1, lc, xl);
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's stores are performed
    __syncthreads();
    uint32_t *ticket = counters + (size_t)kvh * CNT_STRIDE;
    if (tid == 0)
        s_last = (xl ? __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                     : __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) ==
                 (uint32_t)(n_chunk - 1);
    __syncthreads();
    if (!s_last) return;
    // the merge: wave w → head h0 + (w >> 1), dims (w & 1)·64 + lane
    const int mh = h0 + (wave >> 1), md = (wave & 1) * 64 + lane;
    const float *ph = part + (size_t)mh * max_chunk * (D + 2);
    float O = 0.0f, L;
    if (n_chunk <= MERGE_FAST) {
        // every load at once, branch-free (chunk indexes clamped; what lies past n_chunk gets weight 0): lane ℓ's
        // chunk statistics (m, l of chunk ℓ) and this thread's dim of every chunk's o; the weights are worked out
        // while the o loads are in flight
        const int cl = min(lane, n_chunk - 1);
        float mv = ld_dev(ph + (size_t)cl * (D + 2)), lv = ld_dev(ph + (size_t)cl * (D + 2) + 1);
        float ov[MERGE_FAST];
#pragma unroll
        for (int i = 0; i < MERGE_FAST; i++) ov[i] = ld_dev(ph + (size_t)min(i, n_chunk - 1) * (D + 2) + 2 + md);
        if (lane >= n_chunk) mv = -INFINITY, lv = 0.0f;
        const float mx = wave_max(mv, lane);
        const float w = expf(mv - mx);  // lanes past n_chunk: e^(−inf) = 0
        L = wave_sum(lv * w, lane);
        // the weights straight from the lanes that hold them (a scalar operand of the fma)
#pragma unroll
        for (int i = 0; i < MERGE_FAST; i++)
            O = fmaf(ov[i], __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), i)), O);
    } else {
        // long contexts: the weights through LDS (zero past n_chunk up to a whole group), the o partials in groups of
        // MERGE_FAST chunks, each group's loads at once
        float mx = -INFINITY;
        for (int cc = lane; cc < n_chunk; cc += 64) mx = fmaxf(mx, ld_dev(ph + (size_t)cc * (D + 2)));
        mx = wave_max(mx, lane);
        const int n_up = (n_chunk + MERGE_FAST - 1) / MERGE_FAST * MERGE_FAST;
        float l = 0.0f;
        for (int cc = lane; cc < n_up; cc += 64) {
            const int cl = min(cc, n_chunk - 1);
            const float mc = ld_dev(ph + (size_t)cl * (D + 2)), lc = ld_dev(ph + (size_t)cl * (D + 2) + 1);
            const float w = cc < n_chunk ? expf(mc - mx) : 0.0f;
            s_w[wave][cc] = w;
            l = fmaf(lc, w, l);
        }
        L = wave_sum(l, lane);
        __builtin_amdgcn_wave_barrier();
        for (int c0 = 0; c0 < n_chunk; c0 += MERGE_FAST) {
            float ov[MERGE_FAST];
#pragma unroll
            for (int i = 0; i < MERGE_FAST; i++)
                ov[i] = ld_dev(ph + (size_t)min(c0 + i, n_chunk - 1) * (D + 2) + 2 + md);
#pragma unroll
            for (int i = 0; i < MERGE_FAST; i++) O = fmaf(ov[i], s_w[wave][c0 + i], O);
        }
    }
    out[mh * D + md] = O / L;
    if (tid == 0) {  // for the next launch
        if (xl) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        else __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---- prefill causal attention ----------------------------------------------------------------------------------------
//
// attention_causal.wgsl's arithmetic (text.rs:484-499; the same on every compute path): q·scale in f32, scores as
// f32 dot products with the f16 keys, an online softmax in f32 from a running max of −3e38 over the keys each query
// sees (0 … its position), out = acc · (1 / l). Here on the f16 matrix cores (v_mfma_f32_16x16x32_f16) with f32-grade
// operands: q·scale = qh + ql and p·2^14 = ph + pl, each half rounded to f16 (the pair holds 22 bits; K and V are f16
// already), so every product is exact and every sum f32; the 2^14 (exact) keeps small p out of f16's subnormals and
// comes off with 1/l at the end.
//
//   blocks   a pre-pass (k_kv_blocks) copies the keys 0 … n_keys − 1 of each KV head into blocks of 32 keys, 16 KB each,
//            laid out as LDS holds them: K [32 keys][128 dims] with row r's 16-byte chunk c at 16r + (c ^ r%16), then
//            Vᵀ [128 dims][32 keys] with row d's chunk g at 512 + 4d + (g ^ (d/4)%4), the keys of chunk g in the order
//            the P·V MFMA consumes them: 4g … 4g+3, 16 + 4g … 16 + 4g + 3 (the keys lane group g holds in its two
//            score tiles) — so 16 lanes' fragment reads fall on 16 bank groups and a stage is a plain copy;
//   work     a workgroup takes 16 queries (one query block) of both q heads of a KV head: 4 waves = 2 heads × 2 halves
//            of the key blocks (even / odd), the two halves merged through LDS at the end. Stages of 2 blocks go
//            global → LDS by direct loads, the next stage in flight while one is used. Workgroup j takes query block
//            n_qb − 1 − j/n_kv for the first half of the grid and j/n_kv − half for the second, so the two workgroups
//            a CU holds have complementary lengths;
//   scores   Sᵀ (16 keys × 16 queries) = K·(qh + ql)ᵀ: lane ℓ = 16g + c holds query c's scores of keys 4g … 4g + 3 of
//            each 16-key tile; the max and the sum over a query's keys are one swap across lane bits 4 and 5 each;
//   values   Oᵀ (128 dims × 16 queries) += Vᵀ·(ph + pl)ᵀ, the P operand straight from the lane's score registers,
//            lane ℓ accumulating dims 16t + 4g … of query c, so the rescale by the query's correction stays in the lane.
constexpr int CQ = 16, CK = 32, CB_CHUNKS = 1024;  // queries a block, keys a block, 16-byte chunks a key block
constexpr float P_SCALE = 16384.0f, P_UNSCALE = 1.0f / 16384.0f;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int kb_kslot(int r, int c) { return 16 * r + (c ^ (r & 15)); }
__device__ __forceinline__ int kb_vslot(int d, int g) { return 512 + 4 * d + (g ^ ((d >> 2) & 3)); }
// the key of chunk slot j (0 … 7) of Vᵀ chunk g
__device__ __forceinline__ int kb_vkey(int g, int j) { return j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4); }

// grid (n_blk, n_kv), 256 threads, 4 chunks a thread; keys ≥ n_keys are zeros (masked wherever they are read)
__global__ __launch_bounds__(256) void k_kv_blocks(const _Float16 *kc, const _Float16 *vc, int n_ctx, int n_keys,
                                                   int4 *out) {
    const int kb = blockIdx.x, kvh = blockIdx.y, n_blk = gridDim.x;
    const _Float16 *kh = kc + (size_t)kvh * n_ctx * D, *vh = vc + (size_t)kvh * n_ctx * D;
    int4 *ob = out + ((size_t)kvh * n_blk + kb) * CB_CHUNKS;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int u = threadIdx.x + 256 * i;
        int4 v = make_int4(0, 0, 0, 0);
        if (u < 512) {
            const int r = u >> 4, c = (u & 15) ^ (r & 15), key = CK * kb + r;
            if (key < n_keys) v = *reinterpret_cast<const int4 *>(kh + (size_t)key * D + 8 * c);
        } else {
            const int w = u - 512, d = w >> 2, g = (w & 3) ^ ((d >> 2) & 3);
            _Float16 e[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int key = CK * kb + kb_vkey(g, j);
                e[j] = key < n_keys ? vh[(size_t)key * D + d] : (_Float16)0.0f;
            }
            __builtin_memcpy(&v, e, 16);
        }
        ob[u] = v;
    }
}

// OT: the output's type — f32, or f16 (rounded to nearest even: the value the f16 path's o-projection tile holds)
template <typename OT>
__global__ __launch_bounds__(256) void k_attn_causal(const float *q, const int4 *kvb, int n_blk, int n_q, int pos0,
                                                     int n_head, int n_kv, float scale, OT *out) {
    __shared__ __attribute__((aligned(16))) int4 s_kv[2][2][CB_CHUNKS];  // [buffer][half][chunk]
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, c = lane & 15;
    const int n_qb = (n_q + CQ - 1) / CQ, half_grid = (n_qb + 1) / 2;
    const int kvh = blockIdx.x % n_kv, rank = blockIdx.x / n_kv;
    const int qb = rank < half_grid ? n_qb - 1 - rank : rank - half_grid;
    const int hh = wave & 1, kh = wave >> 1, h = 2 * kvh + hh;
    const int q_first = CQ * qb, q_last = min(q_first + CQ - 1, n_q - 1);
    const int qi = min(q_first + c, n_q - 1), qpos = pos0 + qi;
    const int nkb = (pos0 + q_last + 1 + CK - 1) / CK;  // key blocks the last query of the block sees
    const int n_stage = (nkb + 1) / 2;
    const int4 *src = kvb + (size_t)kvh * n_blk * CB_CHUNKS;

    // stage st → buffer: blocks 2st, 2st + 1 (clamped to the last: loaded, not used), 8 direct loads a wave
    auto issue = [&](int st, int buf) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int u = 64 * (wave + 4 * i);  // the wave's 64 chunks of the stage's 2048
            const int blk = min(2 * st + (u >> 10), nkb - 1);
            __builtin_amdgcn_global_load_lds((const void *)(src + (size_t)blk * CB_CHUNKS + (u & 1023) + lane),
                                             (void __attribute__((address_space(3))) *)&s_kv[buf][u >> 10][u & 1023],
                                             16, 0, 0);
        }
    };
    issue(0, 0);

    // q·scale as f16 pairs: B operand of step ks = dims 32ks + 8g … + 7 of query c
    half8 qh[4], ql[4];
    {
        const float *qrow = q + ((size_t)qi * n_head + h) * D;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const float4 a0 = *reinterpret_cast<const float4 *>(qrow + 32 * ks + 8 * g);
            const float4 a1 = *reinterpret_cast<const float4 *>(qrow + 32 * ks + 8 * g + 4);
            const float x[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float qs = x[e] * scale;
                const _Float16 hi = (_Float16)qs;
                qh[ks][e] = hi;
                ql[ks][e] = (_Float16)(qs - (float)hi);
            }
        }
    }
    f32x4 o[8];
#pragma unroll
    for (int t = 0; t < 8; t++) o[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -3.0e38f, l = 0.0f;

    for (int st = 0; st < n_stage; st++) {
        const int buf = st & 1;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's loads of stage st
        __builtin_amdgcn_s_barrier();                       // everyone's; and stage st − 1 is read by all
        asm volatile("" ::: "memory");
        if (st + 1 < n_stage) issue(st + 1, buf ^ 1);
        const int kb = 2 * st + kh;
        if (kb >= nkb) continue;
        const int4 *blk = s_kv[buf][kh];
        f32x4 s[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            s[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const half8 a = *reinterpret_cast<const half8 *>(blk + kb_kslot(16 * t + c, 4 * ks + g));
                s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qh[ks], s[t], 0, 0, 0);
                s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[ks], s[t], 0, 0, 0);
            }
        }
        // keys after the query (only in the block that holds the query block's positions) take no part
        const bool diag = CK * kb + CK - 1 > pos0 + q_first;
        float mx = m;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                if (diag && CK * kb + 16 * t + 4 * g + r > qpos) s[t][r] = -INFINITY;
                mx = fmaxf(mx, s[t][r]);
            }
        mx = pair_max<32>(pair_max<16>(mx));
        const float corr = expf(m - mx);
        float p[2][4], ps = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                p[t][r] = expf(s[t][r] - mx);  // masked: e^(−inf) = 0
                ps += p[t][r];
            }
        l = l * corr + pair_sum<32>(pair_sum<16>(ps));
        m = mx;
        if (__builtin_amdgcn_ballot_w64(corr != 1.0f)) {
#pragma unroll
            for (int t = 0; t < 8; t++) o[t] *= corr;
        }
        half8 ph, pl;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float ps2 = p[t][r] * P_SCALE;
                const _Float16 hi = (_Float16)ps2;
                ph[4 * t + r] = hi;
                pl[4 * t + r] = (_Float16)(ps2 - (float)hi);
            }
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const half8 a = *reinterpret_cast<const half8 *>(blk + kb_vslot(16 * t + c, g));
            o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ph, o[t], 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pl, o[t], 0, 0, 0);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no LDS load in flight past this point
    // merge the two key halves of each head through LDS (the stage buffers are free after this barrier)
    __syncthreads();
    float *s_o = reinterpret_cast<float *>(&s_kv[0][0][0]);  // [head][128 dims][16 queries] + [head][2][16]
    float *s_ml = s_o + 2 * D * CQ;
    if (kh == 1) {
#pragma unroll
        for (int t = 0; t < 8; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) s_o[(hh * D + 16 * t + 4 * g + r) * CQ + c] = o[t][r];
        if (g == 0) {
            s_ml[(hh * 2) * CQ + c] = m;
            s_ml[(hh * 2 + 1) * CQ + c] = l;
        }
    }
    __syncthreads();
    if (kh == 1 || q_first + c >= n_q) return;
    const float m1 = s_ml[(hh * 2) * CQ + c], l1 = s_ml[(hh * 2 + 1) * CQ + c];
    const float mm = fmaxf(m, m1), a0 = expf(m - mm), a1 = expf(m1 - mm);
    const float inv = (1.0f / (l * a0 + l1 * a1)) * P_UNSCALE;
    OT *orow = out + ((size_t)(q_first + c) * n_head + h) * D + 4 * g;
#pragma unroll
    for (int t = 0; t < 8; t++) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; r++) v[r] = (o[t][r] * a0 + s_o[(hh * D + 16 * t + 4 * g + r) * CQ + c] * a1) * inv;
        if constexpr (sizeof(OT) == 4) {
            *reinterpret_cast<float4 *>(orow + 16 * t) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
            const half4 hv = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
            *reinterpret_cast<half4 *>(orow + 16 * t) = hv;
        }
    }
}

}  // namespace

int attn_chunk_for(int n_ctx) {
    // 16 keys per workgroup, doubled while a KV head would need more than 32 chunks (at most 32 partials per head are
    // merged for n_ctx ≤ 8192), up to 256 keys. Measured on one MI355X at 1536 keys: 24 chunks of 64 keys 6.95 µs a
    // launch, 48 of 32 8.2 µs, 96 of 16 12.3 µs, 12 of 128 7.15 µs (the merge and the ticket grow with the chunk
    // count, the workgroup's own load phase with its keys). At most 16 or 8 chunks a KV head instead (graph nodes,
    // µs at 512 / 2048 / 8192 keys): 5.26 / 6.19 / 10.19 with 32, 5.25 / 6.48 / 10.15 with 16, 5.22 / 8.24 / 10.19
    // with 8 — 512 keys sit at the launch's floor whatever the split
    int chunk = 16;
    while ((n_ctx + chunk - 1) / chunk > 32 && chunk < MAX_CHUNK_KEYS) chunk *= 2;
    return chunk;
}

size_t attn_part_bytes(int n_head, int max_chunk) { return (size_t)n_head * max_chunk * (D + 2) * 4; }

size_t attn_counter_bytes(int n_kv) { return (size_t)n_kv * CNT_STRIDE * 4; }

int launch_qkv_post(htr_device *dev, hipStream_t st, float *qkv, const float *qn, const float *kn, const float *rope,
                    int n_head, int n_kv, const int *pos_dev, int pos, int n_ctx, float eps, uint16_t *kc,
                    uint16_t *vc) {
    hipLaunchKernelGGL(k_qkv_post, dim3(n_head + 2 * n_kv), dim3(64), 0, st, qkv, qn, kn, rope, n_head, n_kv, pos_dev,
                       pos, n_ctx, eps, (_Float16 *)kc, (_Float16 *)vc);
    return htr_launched(dev, "k_qkv_post");
}

int launch_attn_decode(htr_device *dev, hipStream_t st, const float *q, const uint16_t *kc, const uint16_t *vc,
                       int n_head, int n_kv, int n_ctx, const int *pos_dev, int n_keys, float scale,
                       const AttnScratch &sc, float *out, const AttnFuse *fuse, bool scale_after) {
    if (n_head != 2 * n_kv) return htr_fail("decode attention: %d q heads on %d kv heads (groups of 2)", n_head, n_kv);
    if (sc.chunk < 16 || sc.chunk > MAX_CHUNK_KEYS || (sc.chunk & (sc.chunk - 1)))
        return htr_fail("decode attention: chunk %d (a power of two, 16 … %d)", sc.chunk, MAX_CHUNK_KEYS);
    if (!pos_dev && (n_keys < 1 || n_keys > n_ctx)) return htr_fail("decode attention: %d keys, cache %d", n_keys, n_ctx);
    if ((size_t)sc.max_chunk * sc.chunk < (size_t)n_ctx || sc.max_chunk > MAX_CHUNKS)
        return htr_fail("decode attention: %d chunks of %d keys for a %d-row cache (at most %d chunks)", sc.max_chunk,
                        sc.chunk, n_ctx, MAX_CHUNKS);
    const int grid_x = pos_dev ? sc.max_chunk : (n_keys + sc.chunk - 1) / sc.chunk;
    const dim3 grid(grid_x * n_kv);
    const AttnFuse fz = fuse ? *fuse : AttnFuse{};
    if (fuse && (fz.n_head != n_head || !fz.qn || !fz.kn || !fz.rope || !fz.kc || !fz.vc))
        return htr_fail("decode attention: incomplete qkv_post arguments");
    // the F32 path scales each score after its dot product (attn_scores.wgsl:38); the f16 paths scale q first
    // (attn_decode.wgsl:40). A scale of exactly 1 on the other side leaves the values as they are.
    if (scale_after && fuse) return htr_fail("decode attention: the fused step pre-scales q");
    const float pre = scale_after ? 1.0f : scale, post = scale_after ? scale : 1.0f;
    // 8 KV heads: workgroup b takes KV head b mod 8 and runs on XCD b mod 8, so a head's chunks share one XCD's L2
    // where the device's placement and XCD-local visibility were checked at open (token_step_xcds): 512 / 2048 / 8192
    // keys 5.25 → 4.93, 6.17 → 5.82, 10.2 → 9.83 µs a graph node (A/B twice on one box, outputs bit-identical)
    const int xl = n_kv == 8 && dev->xcd_round_robin == 1;
#define HTR_ATTN(NI)                                                                                                   \
    if (fuse)                                                                                                          \
        hipLaunchKernelGGL((k_attn_decode<NI, true>), grid, dim3(AW), 0, st, q, (const _Float16 *)kc,                  \
                           (const _Float16 *)vc, n_kv, n_ctx, pos_dev, n_keys, sc.max_chunk, pre, post, sc.part,       \
                           sc.counters, out, fz, xl);                                                                  \
    else                                                                                                               \
        hipLaunchKernelGGL((k_attn_decode<NI, false>), grid, dim3(AW), 0, st, q, (const _Float16 *)kc,                 \
                           (const _Float16 *)vc, n_kv, n_ctx, pos_dev, n_keys, sc.max_chunk, pre, post, sc.part,       \
                           sc.counters, out, fz, xl)
    switch (sc.chunk / 16) {
    case 1: HTR_ATTN(1); break;
    case 2: HTR_ATTN(2); break;
    case 4: HTR_ATTN(4); break;
    case 8: HTR_ATTN(8); break;
    default: HTR_ATTN(16); break;
    }
#undef HTR_ATTN
    return htr_launched(dev, "k_attn_decode");
}

int launch_qk_norm_rope_rows(htr_device *dev, hipStream_t st, float *q, float *k, const float *v, const float *qn,
                             const float *kn, const float *rope, int n_tok, int n_head, int n_kv, int pos0, int n_ctx,
                             float eps, uint16_t *kc, uint16_t *vc) {
    hipLaunchKernelGGL(k_qk_rows, dim3(n_tok, n_head + 2 * n_kv), dim3(64), 0, st, q, k, v, qn, kn, rope, n_head, n_kv,
                       pos0, n_ctx, eps, (_Float16 *)kc, (_Float16 *)vc);
    return htr_launched(dev, "k_qk_rows");
}

size_t attn_causal_block_bytes(int n_kv, int n_keys) {
    return (size_t)n_kv * ((n_keys + CK - 1) / CK) * CB_CHUNKS * 16;
}

int launch_attn_causal(htr_device *dev, hipStream_t st, const float *q, const uint16_t *kc, const uint16_t *vc,
                       int n_q, int pos0, int n_head, int n_kv, int n_ctx, float scale, void *blocks, float *out,
                       _Float16 *out16) {
    if (n_head != 2 * n_kv) return htr_fail("causal attention: %d q heads on %d kv heads (groups of 2)", n_head, n_kv);
    if (n_q < 1 || pos0 < 0 || pos0 + n_q > n_ctx)
        return htr_fail("causal attention: %d queries from position %d in a %d-row cache", n_q, pos0, n_ctx);
    if (!out == !out16) return htr_fail("causal attention: one output, f32 or f16");
    if (!blocks) return htr_fail("causal attention: no key-block buffer");
    const int n_keys = pos0 + n_q, n_blk = (n_keys + CK - 1) / CK;
    hipLaunchKernelGGL(k_kv_blocks, dim3(n_blk, n_kv), dim3(256), 0, st, (const _Float16 *)kc, (const _Float16 *)vc,
                       n_ctx, n_keys, (int4 *)blocks);
    HTR_TRY(htr_launched(dev, "k_kv_blocks"));
    const dim3 grid(((n_q + CQ - 1) / CQ) * n_kv);
    if (out) {
        hipLaunchKernelGGL(k_attn_causal<float>, grid, dim3(256), 0, st, q, (const int4 *)blocks, n_blk, n_q, pos0,
                           n_head, n_kv, scale, out);
        return htr_launched(dev, "k_attn_causal");
    }
    hipLaunchKernelGGL(k_attn_causal<_Float16>, grid, dim3(256), 0, st, q, (const int4 *)blocks, n_blk, n_q, pos0,
                       n_head, n_kv, scale, out16);
    return htr_launched(dev, "k_attn_causal<f16>");
}

// ---- the allocation-free decode attention ----------------------------------------------------------------------------
//
// htr_decode_attention_static keeps its split-K partials and ticket counters in one file-scope device array instead
// of device memory the library allocates. Every GPU the library runs on holds its own copy (STATIC_SCRATCH_BYTES,
// until the process ends); its address on a device is looked up once, when the device is opened
// (attn_static_scratch_init), and kept in the device object — host code passes that address, never the array's name
// (which on the host is a stand-in, not a device address). Layout: the tickets of up to STATIC_MAX_KV KV heads (one
// 128-byte line each), then the partials [n_head][max_chunk][130] f32. Every call clears the tickets it uses with a
// fill kernel first; calls that overlap on one GPU share the array and race.
namespace {

constexpr size_t STATIC_SCRATCH_BYTES = 4u << 20;
constexpr int STATIC_MAX_KV = 64;
constexpr size_t STATIC_CNT_BYTES = (size_t)STATIC_MAX_KV * CNT_STRIDE * 4;
static __device__ __align__(256) unsigned char scratch[STATIC_SCRATCH_BYTES];

__global__ __launch_bounds__(256) void k_zero_u32(uint32_t *p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0u;
}

}  // namespace

int attn_static_scratch_init(htr_device *dev) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return htr_fail("hipGetSymbolAddress of the static attention scratch on device %d: %s", dev->ordinal,
                        hipGetErrorString(e));
    dev->static_scratch = p;
    return 0;
}

// ---- ABI ------------------------------------------------------------------------------------------------------------

extern "C" int htr_qkv_post(htr_device *dev, float *d_qkv, const float *d_q_norm, const float *d_k_norm,
                            const float *d_rope, int n_head, int n_kv, int pos, int n_ctx, float eps, uint16_t *d_k,
                            uint16_t *d_v) {
    HTR_TRY(htr_check_alive(dev));
    if (!d_qkv || !d_q_norm || !d_k_norm || !d_rope || !d_k || !d_v) return htr_fail("htr_qkv_post: null argument");
    if (pos < 0 || pos >= n_ctx || n_head <= 0 || n_kv <= 0)
        return htr_fail("htr_qkv_post: position %d of a %d-row cache, %d / %d heads", pos, n_ctx, n_head, n_kv);
    return launch_qkv_post(dev, dev->stream, d_qkv, d_q_norm, d_k_norm, d_rope, n_head, n_kv, nullptr, pos, n_ctx, eps,
                           d_k, d_v);
}

extern "C" int htr_causal_attention(htr_device *dev, const float *d_q, const uint16_t *d_k, const uint16_t *d_v,
                                    int n_q, int pos0, int n_head, int n_kv, int n_ctx, float scale, float *d_out) {
    HTR_TRY(htr_check_alive(dev));
    if (!d_q || !d_k || !d_v || !d_out) return htr_fail("htr_causal_attention: null argument");
    if (n_q < 1 || pos0 < 0 || n_ctx < 1 || pos0 > n_ctx - n_q)
        return htr_fail("htr_causal_attention: %d queries from position %d in a %d-row cache", n_q, pos0, n_ctx);
    void *blocks;
    HTR_TRY(htr_scratch(dev, SCR_CAUSAL_BLOCKS, attn_causal_block_bytes(n_kv, pos0 + n_q), &blocks));
    return launch_attn_causal(dev, dev->stream, d_q, d_k, d_v, n_q, pos0, n_head, n_kv, n_ctx, scale, blocks, d_out);
}

extern "C" int htr_decode_attention(htr_device *dev, const float *d_q, const uint16_t *d_k, const uint16_t *d_v,
                                    int n_head, int n_kv, int n_ctx, int n_keys, float scale, float *d_out) {
    HTR_TRY(htr_check_alive(dev));
    if (!d_q || !d_k || !d_v || !d_out) return htr_fail("htr_decode_attention: null argument");
    if (n_keys < 1 || n_keys > n_ctx) return htr_fail("htr_decode_attention: %d keys in a %d-row cache", n_keys, n_ctx);
    if (n_ctx > MAX_CHUNKS * MAX_CHUNK_KEYS)
        return htr_fail("htr_decode_attention: a %d-row cache (at most %d)", n_ctx, MAX_CHUNKS * MAX_CHUNK_KEYS);
    AttnScratch sc{};
    sc.chunk = attn_chunk_for(n_ctx);
    sc.max_chunk = (n_ctx + sc.chunk - 1) / sc.chunk;
    HTR_TRY(htr_scratch(dev, SCR_ATTN_PART, attn_part_bytes(n_head, sc.max_chunk), (void **)&sc.part));
    HTR_TRY(htr_scratch(dev, SCR_ATTN_CNT, attn_counter_bytes(n_kv), (void **)&sc.counters));
    return launch_attn_decode(dev, dev->stream, d_q, d_k, d_v, n_head, n_kv, n_ctx, nullptr, n_keys, scale, sc, d_out);
}

extern "C" int htr_decode_attention_static(htr_device *dev, const float *d_q, const uint16_t *d_k, const uint16_t *d_v,
                                           int n_head, int n_kv, int n_ctx, int n_keys, float scale, float *d_out) {
    HTR_TRY(htr_check_alive(dev));
    if (!d_q || !d_k || !d_v || !d_out) return htr_fail("htr_decode_attention_static: null argument");
    if (n_keys < 1 || n_keys > n_ctx)
        return htr_fail("htr_decode_attention_static: %d keys in a %d-row cache", n_keys, n_ctx);
    if (n_ctx > MAX_CHUNKS * MAX_CHUNK_KEYS)
        return htr_fail("htr_decode_attention_static: a %d-row cache (at most %d)", n_ctx, MAX_CHUNKS * MAX_CHUNK_KEYS);
    if (n_kv < 1 || n_kv > STATIC_MAX_KV)
        return htr_fail("htr_decode_attention_static: %d KV heads (the static scratch has tickets for %d)", n_kv,
                        STATIC_MAX_KV);
    if (!dev->static_scratch) return htr_fail("htr_decode_attention_static: the device has no static scratch address");
    AttnScratch sc{};
    sc.chunk = attn_chunk_for(n_ctx);
    sc.max_chunk = (n_ctx + sc.chunk - 1) / sc.chunk;
    const size_t part = attn_part_bytes(n_head, sc.max_chunk);
    if (part > STATIC_SCRATCH_BYTES - STATIC_CNT_BYTES)
        return htr_fail("htr_decode_attention_static: %d heads x %d chunks need %zu bytes of partials, the static scratch "
                        "holds %zu",
                        n_head, sc.max_chunk, part, STATIC_SCRATCH_BYTES - STATIC_CNT_BYTES);
    unsigned char *base = (unsigned char *)dev->static_scratch;
    sc.counters = (uint32_t *)base;
    sc.part = (float *)(base + STATIC_CNT_BYTES);
    const int n_cnt = n_kv * CNT_STRIDE;
    hipLaunchKernelGGL(k_zero_u32, dim3((n_cnt + 255) / 256), dim3(256), 0, dev->stream, sc.counters, n_cnt);
    HTR_TRY(htr_launched(dev, "k_zero_u32"));
    return launch_attn_decode(dev, dev->stream, d_q, d_k, d_v, n_head, n_kv, n_ctx, nullptr, n_keys, scale, sc, d_out);
}
