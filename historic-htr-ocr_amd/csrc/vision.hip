// The vision encoder's non-GEMM kernels for gfx950, and the f16 pieces of the f32 operands that its patch embedding
// and projector multiply on the matrix cores.
//
// Reference semantics (the f16 compute path, vision.rs:328-423): patchify.wgsl (normalise + im2col), rms_norm.wgsl /
// rms_norm_h (gpu.rs:268-275), rope2d.wgsl (+ vision.rs:159-175; applied as K and q are read), heads_f16.wgsl,
// attention_coop.wgsl (flash attention with q·scale, K, V and P rounded to f16, f32 sums, the output rounded to f16),
// unfold2x2.wgsl, gelu.wgsl; the f32 matmuls of the patch embedding (K = 588) and the projector (f32 activations,
// f16-valued weights) run as f16 GEMMs over split operands (k_split_f16).
#include <cmath>
#include <type_traits>

#include "htr_internal.h"
#include "wave.h"

namespace {

constexpr int VW = 256;

__device__ __forceinline__ size_t gsize() { return (size_t)gridDim.x * VW; }
__device__ __forceinline__ size_t gid() { return blockIdx.x * (size_t)VW + threadIdx.x; }

// patchify.wgsl: P[t][c·p·p + ky·p + kx] = lut[c·256 + rgb[((ty·p + ky)·w + tx·p + kx)·3 + c]]
__global__ __launch_bounds__(VW) void k_patchify(const uint8_t *rgb, const float *lut, int w, int px, int n, int side,
                                                 float *P) {
    const int pp = side * side;
    const size_t total = (size_t)n * 3 * pp;
    for (size_t i = gid(); i < total; i += gsize()) {
        const int t = (int)(i / (3 * pp)), r = (int)(i % (3 * pp));
        const int c = r / pp, ky = (r % pp) / side, kx = r % side;
        const int x = (t % px) * side + kx, y = (t / px) * side + ky;
        P[i] = lut[c * 256 + rgb[((size_t)y * w + x) * 3 + c]];
    }
}

// one workgroup per row: y = x·1/sqrt(mean(x²) + eps)·w, as f32 or rounded to f16
template <typename T>
__global__ __launch_bounds__(VW) void k_rms_norm_rows(const float *x, const float *w, T *y, int dim, float eps) {
    __shared__ float red[VW / 64];
    const size_t base = (size_t)blockIdx.x * dim;
    const int tid = threadIdx.x, lane = tid & 63;
    float s = 0.0f;
    for (int i = tid; i < dim; i += VW) s = fmaf(x[base + i], x[base + i], s);
    s = wave_sum(s, lane);
    if (lane == 0) red[tid >> 6] = s;
    __syncthreads();
    const float scale = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)dim + eps);
    for (int i = tid; i < dim; i += VW) y[base + i] = (T)((x[base + i] * scale) * w[i]);
}

// the same for dim = 1024·NV: a thread holds NV float4 of the row, so x is read once, in 16-byte loads
template <typename T, int NV>
__global__ __launch_bounds__(VW) void k_rms_norm_rows4(const float *x, const float *w, T *y, int dim, float eps) {
    __shared__ float red[VW / 64];
    const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)blockIdx.x * dim);
    const int tid = threadIdx.x, lane = tid & 63;
    float4 v[NV];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        v[j] = xr[tid + VW * j];
        s = fmaf(v[j].x, v[j].x, s);
        s = fmaf(v[j].y, v[j].y, s);
        s = fmaf(v[j].z, v[j].z, s);
        s = fmaf(v[j].w, v[j].w, s);
    }
    s = wave_sum(s, lane);
    if (lane == 0) red[tid >> 6] = s;
    __syncthreads();
    const float scale = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)dim + eps);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    typedef T t4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const float4 ww = w4[tid + VW * j];
        const t4 o = {(T)((v[j].x * scale) * ww.x), (T)((v[j].y * scale) * ww.y), (T)((v[j].z * scale) * ww.z),
                      (T)((v[j].w * scale) * ww.w)};
        *reinterpret_cast<t4 *>(y + (size_t)blockIdx.x * dim + 4 * (tid + VW * j)) = o;
    }
}

// rope2d.wgsl on 8 consecutive dims d0 … d0 + 7 of a head (d0 a multiple of 8, head dim 64), in registers: the
// pairs (2k, 2k + 1) of each 32-dim half, half 0 turned by the row t / px, half 1 by the column t % px;
// cs = [half][pos][k] × (cos, sin), 16 pairs a half
__device__ __forceinline__ void rope8(float (&x)[8], const float *cs, int t, int px, int max_pos, int d0) {
    const int half = d0 >> 5, k0 = (d0 & 31) >> 1, pos = half == 0 ? t / px : t % px;
    const float4 *c4 = reinterpret_cast<const float4 *>(cs + 2 * (((size_t)half * max_pos + pos) * 16 + k0));
    const float4 a = c4[0], b = c4[1];
    const float c[4] = {a.x, a.z, b.x, b.z}, sn[4] = {a.y, a.w, b.y, b.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float x0 = x[2 * e], x1 = x[2 * e + 1];
        x[2 * e] = x0 * c[e] - x1 * sn[e];
        x[2 * e + 1] = x0 * sn[e] + x1 * c[e];
    }
}

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

// Key order of the transposed values inside a block of 32 keys: stored slot 16s + 8h + j (s, h < 2, j < 8) holds key
// 16s + 8(j / 4) + 4h + j % 4. These are the keys whose scores lane half h holds in registers 8s … 8s + 7 after the
// 32x32 score MFMAs below, so P·V step s takes its P operand straight from those registers.
__device__ __forceinline__ int vt_key(int slot) {
    const int st = slot >> 4, hf = (slot >> 3) & 1, j = slot & 7;
    return 16 * st + 8 * (j >> 2) + 4 * hf + (j & 3);
}

// K / V of one head in blocks of 32 keys, 8 KB a block: K [32 keys][64 dims] then Vᵀ [64 dims][32 slots], f16, in
// 16-byte chunks placed so that the attention's fragment reads from LDS hit 16 different 16-byte bank groups in every
// 16 lanes (gfx950's LDS serves 16 lanes of a 16-byte read a cycle across 256 bytes): K row r, chunk j (dims 8j …) at
// chunk r·8 + (j ^ (r/2 % 8)); Vᵀ row d, chunk q (slots 8q …) at 256 + d·4 + (q ^ (d/4 % 4))
constexpr int KVB = 8192;
__device__ __forceinline__ int kv_kchunk(int r, int j) { return r * 8 + (j ^ ((r >> 1) & 7)); }
__device__ __forceinline__ int kv_vchunk(int d, int q) { return 256 + d * 4 + (q ^ ((d >> 2) & 3)); }

// rope2d.wgsl on K, then heads_f16.wgsl's rounding: K, V f32 [n][H·64] → f16 blocks as above, keys n … ⌈n/32⌉·32 − 1
// zero. grid (blocks, H), one block of one head per workgroup; V goes through LDS for the transposition.
__global__ __launch_bounds__(VW) void k_heads_f16(const float *K, const float *V, _Float16 *KV, int n_tok, int n_head,
                                                  int n_blk, const float *cs, int px, int max_pos) {
    __shared__ _Float16 s_v[32][64 + 2];
    const int b = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int r = tid >> 3, j8 = tid & 7, t = 32 * b + r;
    float kv[8] = {}, vv[8] = {};
    if (t < n_tok) {
        const float4 *ks = reinterpret_cast<const float4 *>(K + (size_t)t * n_head * 64 + h * 64 + 8 * j8);
        const float4 *vs = reinterpret_cast<const float4 *>(V + (size_t)t * n_head * 64 + h * 64 + 8 * j8);
        const float4 k0 = ks[0], k1 = ks[1], v0 = vs[0], v1 = vs[1];
        kv[0] = k0.x, kv[1] = k0.y, kv[2] = k0.z, kv[3] = k0.w, kv[4] = k1.x, kv[5] = k1.y, kv[6] = k1.z, kv[7] = k1.w;
        vv[0] = v0.x, vv[1] = v0.y, vv[2] = v0.z, vv[3] = v0.w, vv[4] = v1.x, vv[5] = v1.y, vv[6] = v1.z, vv[7] = v1.w;
        rope8(kv, cs, t, px, max_pos, 8 * j8);
    }
    half8 kh;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        kh[j] = (_Float16)kv[j];
        s_v[r][8 * j8 + j] = (_Float16)vv[j];
    }
    half8 *blk = reinterpret_cast<half8 *>(KV + ((size_t)h * n_blk + b) * (KVB / 2));
    blk[kv_kchunk(r, j8)] = kh;
    __syncthreads();
    const int d = tid >> 2, q = tid & 3;
    half8 vt;
#pragma unroll
    for (int j = 0; j < 8; j++) vt[j] = s_v[vt_key(8 * q + j)][d];
    blk[kv_vchunk(d, q)] = vt;
}

// attention_coop.wgsl's arithmetic on the f16 MFMAs: O[t][h] = softmax(q16·K16ᵀ)·V16 with q16 = f16(q·scale), keys in
// blocks of 32 with the running max (start −3e38), P = f16(e^(S − max)), l = l·corr + Σ P, O = O·corr + P·V (f32
// accumulation in the matrix unit, as the reference's cooperative matrices accumulate); O / l → f16.
// A wave takes QG groups of 32 queries of one head. Per key block and group, Sᵀ (32 keys × 32 queries) = K·q16ᵀ is 4
// MFMAs 32x32x16: lane ℓ = 32h + c then holds query c's scores of keys 8(i / 4) + 4h + i % 4 (i < 16), the other 16
// in lane ℓ ^ 32. Oᵀ (64 dims × 32 queries) += Vᵀ·Pᵀ is 4 more, lane ℓ accumulating dims 32t + 8(i / 4) + 4h + i % 4
// of query c, so the rescale by the query's corr stays in the lane.
// The 4 waves of a workgroup (128·QG queries) share the key blocks: stages of AST blocks are copied from memory to LDS
// (coalesced 16-byte loads, the next stage's in flight while the current one is in use) and each wave reads its
// fragments from there. grid: ⌈n / (128·QG)⌉ · H workgroups, numbered so that the workgroups of one head run on one
// XCD.
constexpr int FQ = 32, FB = 32, FWAVES = VW / 64, AST = 2;

// QG groups of 32 queries a wave: the groups share every K / V fragment read from LDS and give the wave QG
// independent chains (Sᵀ MFMAs → max → exp → P·V) to interleave
template <int QG>
__global__ __launch_bounds__(VW) void k_attn_vision(const float *Q, const _Float16 *KV, _Float16 *O, int n_tok,
                                                    int n_head, int n_blk, int n_qt, float scale, const float *cs,
                                                    int px, int max_pos) {
    __shared__ __attribute__((aligned(16))) half8 s_kv[2][AST * KVB / 16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hf = lane >> 5, c = lane & 31;
    // workgroup b runs on XCD b % 8: with H a multiple of 8, XCD x takes heads x·H/8 … (x + 1)·H/8 − 1
    int h, qt;
    if (n_head % 8 == 0) {
        const int i = blockIdx.x / 8;
        h = (blockIdx.x % 8) * (n_head / 8) + i / n_qt;
        qt = i % n_qt;
    } else {
        h = blockIdx.x / n_qt;
        qt = blockIdx.x % n_qt;
    }
    const int row = n_head * 64, q0 = (qt * FWAVES + wave) * FQ * QG;
    half8 qf[QG][4];  // B operand of step ks: q16[query c][dims 16ks + 8h … + 7], q turned by rope2d first
#pragma unroll
    for (int g = 0; g < QG; g++) {
        const int qi = min(q0 + FQ * g + c, n_tok - 1);
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const float4 *src = reinterpret_cast<const float4 *>(Q + (size_t)qi * row + h * 64 + 16 * ks + 8 * hf);
            const float4 x0 = src[0], x1 = src[1];
            float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            rope8(x, cs, qi, px, max_pos, 16 * ks + 8 * hf);
#pragma unroll
            for (int e = 0; e < 8; e++) qf[g][ks][e] = (_Float16)(x[e] * scale);
        }
    }
    // the lane's fragment chunks within a block: K step ks (key c, dims 16ks + 8h …), Vᵀ tile t step st (dim 32t + c,
    // slots 16st + 8h …)
    int kc[4], vc[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) kc[ks] = kv_kchunk(c, 2 * ks + hf);
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int st = 0; st < 2; st++) vc[2 * t + st] = kv_vchunk(32 * t + c, 2 * st + hf);
    // stage copies: AST blocks of 512 chunks, 2·AST chunks a thread (blocks past the last repeat it: in bounds)
    const half8 *gkv = reinterpret_cast<const half8 *>(KV) + (size_t)h * n_blk * (KVB / 16);
    half8 stg[2 * AST];
    auto gload = [&](int stage) {
#pragma unroll
        for (int i = 0; i < 2 * AST; i++) {
            const int blk = min(stage * AST + i / 2, n_blk - 1);
            stg[i] = gkv[(size_t)blk * (KVB / 16) + (i % 2) * VW + tid];
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 2 * AST; i++) s_kv[buf][(i / 2) * (KVB / 16) + (i % 2) * VW + tid] = stg[i];
    };
    f32x16 o[QG][2];
    float m[QG], l[QG];
#pragma unroll
    for (int g = 0; g < QG; g++) {
        m[g] = -3.0e38f;
        l[g] = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) o[g][t][i] = 0.0f;
    }
    // one key block at k0 from LDS; MASK: the block holds keys ≥ n_tok (the last one only), which take no part in
    // the max and get p = 0. A rescale by corr = 1 is skipped (x·1 = x).
    auto block = [&](const half8 *sb, int k0, auto mask) {
        constexpr bool MASK = decltype(mask)::value;
        half8 fk[4], fv[4];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) fk[ks] = sb[kc[ks]];
#pragma unroll
        for (int i = 0; i < 4; i++) fv[i] = sb[vc[i]];
        f32x16 s[QG];
#pragma unroll
        for (int g = 0; g < QG; g++) {
#pragma unroll
            for (int i = 0; i < 16; i++) s[g][i] = 0.0f;
#pragma unroll
            for (int ks = 0; ks < 4; ks++) s[g] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fk[ks], qf[g][ks], s[g], 0, 0, 0);
        }
        half8 pb[QG][2];
#pragma unroll
        for (int g = 0; g < QG; g++) {
            float mx = m[g];
#pragma unroll
            for (int i = 0; i < 16; i++)
                if (!MASK || k0 + 8 * (i >> 2) + 4 * hf + (i & 3) < n_tok) mx = fmaxf(mx, s[g][i]);
            mx = pair_max<32>(mx);
            // e^(s − mx) = 2^(s·log2 e − mx·log2 e): one fma and v_exp_f32 a score; P rounded to f16 in pairs
            // (v_cvt_pk_f16_f32, round to nearest even) and summed as f32 by v_dot2 against (1, 1)
            constexpr float LOG2E = 1.4426950408889634f;
            const float corr = __builtin_amdgcn_exp2f((m[g] - mx) * LOG2E), nml = -mx * LOG2E;
            if (__builtin_amdgcn_ballot_w64(corr != 1.0f)) {
#pragma unroll
                for (int t = 0; t < 2; t++) o[g][t] *= corr;
            }
            float ps = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                float2_t e = {__builtin_amdgcn_exp2f(fmaf(s[g][i], LOG2E, nml)),
                              __builtin_amdgcn_exp2f(fmaf(s[g][i + 1], LOG2E, nml))};
                if (MASK) {
                    if (k0 + 8 * (i >> 2) + 4 * hf + (i & 3) >= n_tok) e[0] = 0.0f;
                    if (k0 + 8 * (i >> 2) + 4 * hf + (i & 3) + 1 >= n_tok) e[1] = 0.0f;
                }
                const half2_t p2 = __builtin_convertvector(e, half2_t);
                pb[g][i >> 3][i & 7] = p2[0];
                pb[g][i >> 3][(i & 7) + 1] = p2[1];
                ps = __builtin_amdgcn_fdot2(p2, half2_t{(_Float16)1.0f, (_Float16)1.0f}, ps, false);
            }
            l[g] = l[g] * corr + pair_sum<32>(ps);
            m[g] = mx;
        }
#pragma unroll
        for (int g = 0; g < QG; g++)
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int st = 0; st < 2; st++)
                    o[g][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fv[2 * t + st], pb[g][st], o[g][t], 0, 0, 0);
    };
    // stages 0 … n_full − 1 hold full blocks only: the loop body has one path, so O stays in the same registers
    // through every iteration (a masked path inside the loop makes the compiler copy it each block)
    const int n_stage = (n_blk + AST - 1) / AST, n_full = n_tok / (AST * FB);
    gload(0);
    lstore(0);
    __syncthreads();
    for (int sg = 0; sg < n_full; sg++) {
        const int buf = sg & 1;
        if (sg + 1 < n_stage) gload(sg + 1);
#pragma unroll
        for (int j = 0; j < AST; j++) block(s_kv[buf] + j * (KVB / 16), (sg * AST + j) * FB, std::false_type{});
        // the other buffer was last read in the previous stage, before the barrier that ended it
        if (sg + 1 < n_stage) lstore(buf ^ 1);
        __syncthreads();
    }
    // the last stage, when it holds keys ≥ n_tok (copied to buffer n_full % 2 by the loop's last iteration, or
    // before the loop when n_full is 0)
    if (n_full < n_stage) {
        const int buf = n_full & 1;
        for (int j = 0; j < AST; j++) {
            const int k0 = (n_full * AST + j) * FB;
            if (k0 + FB <= n_tok)
                block(s_kv[buf] + j * (KVB / 16), k0, std::false_type{});
            else if (k0 < n_tok)
                block(s_kv[buf] + j * (KVB / 16), k0, std::true_type{});
        }
    }
#pragma unroll
    for (int g = 0; g < QG; g++) {
        if (q0 + FQ * g + c < n_tok) {
            typedef _Float16 half4 __attribute__((ext_vector_type(4)));
            const float inv = 1.0f / l[g];
            _Float16 *dst = O + (size_t)(q0 + FQ * g + c) * row + h * 64 + 4 * hf;
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    *reinterpret_cast<half4 *>(dst + 32 * t + 8 * r) =
                        half4{(_Float16)(o[g][t][4 * r] * inv), (_Float16)(o[g][t][4 * r + 1] * inv),
                              (_Float16)(o[g][t][4 * r + 2] * inv), (_Float16)(o[g][t][4 * r + 3] * inv)};
        }
    }
}

// unfold2x2.wgsl: Z[o][c·4 + ky·2 + kx] = X[(2·oy + ky)·px + 2·ox + kx][c]
__global__ __launch_bounds__(VW) void k_unfold2x2(const float *X, float *Z, int px, int py, int dim) {
    const int ox_n = px / 2;
    const size_t total = (size_t)(px / 2) * (py / 2) * dim * 4;
    for (size_t i = gid(); i < total; i += gsize()) {
        const int kx = (int)(i % 2), ky = (int)((i / 2) % 2), c = (int)((i / 4) % dim);
        const int o = (int)(i / (4 * (size_t)dim));
        const int ox = o % ox_n, oy = o / ox_n;
        Z[i] = X[((size_t)(2 * oy + ky) * px + 2 * ox + kx) * dim + c];
    }
}

// gelu.wgsl in place (tanh form, argument clamped to ±15)
__global__ __launch_bounds__(VW) void k_gelu(float *X, size_t n) {
    for (size_t i = gid(); i < n; i += gsize()) {
        const float x = X[i];
        const float t = fminf(fmaxf(0.7978845608028654f * x * (1.0f + 0.044715f * x * x), -15.0f), 15.0f);
        X[i] = 0.5f * x * (1.0f + tanhf(t));
    }
}

// f32 values as f16 pieces for f32-grade products on the f16 matrix cores: x [m][k] → rows of nseg segments of kp
// values (kp ≥ k, a multiple of 32, the values past k zero); segment s holds hi = f16(x), or lo = f16(x − hi) where bit
// s of lo_mask is set. x − hi is exact in f32 and hi + lo is x within 2^-22·|x| (|x| < 65504). With X as [hi, hi, lo]
// and W as [hi, lo, hi] one f16 GEMM over 3·kp sums xh·wh + xh·wl + xl·wh in f32; f16-valued W: X [hi, lo], W [w, w].
__global__ __launch_bounds__(VW) void k_split_f16(const float *x, int m, int k, int kp, int nseg, int lo_mask,
                                                  _Float16 *out) {
    const size_t total = (size_t)m * kp;
    for (size_t i = gid(); i < total; i += gsize()) {
        const int c = (int)(i % kp);
        const size_t r = i / kp;
        const float v = c < k ? x[r * k + c] : 0.0f;
        const _Float16 hi = (_Float16)v, lo = (_Float16)(v - (float)hi);
        for (int s = 0; s < nseg; s++) out[(r * nseg + s) * kp + c] = (lo_mask >> s) & 1 ? lo : hi;
    }
}

int grid_for(size_t total) { return (int)std::max<size_t>(1, std::min<size_t>((total + VW - 1) / VW, 65536)); }

}  // namespace

int launch_patchify(htr_device *dev, hipStream_t st, const uint8_t *rgb, const float *lut, int w, int px, int n,
                    int side, float *P) {
    hipLaunchKernelGGL(k_patchify, dim3(grid_for((size_t)n * 3 * side * side)), dim3(VW), 0, st, rgb, lut, w, px, n,
                       side, P);
    return htr_launched(dev, "k_patchify");
}

int launch_rms_norm_f16(htr_device *dev, hipStream_t st, const float *x, const float *w, _Float16 *y, int rows, int dim,
                        float eps) {
    switch (dim % (4 * VW) ? 0 : dim / (4 * VW)) {
    case 1: hipLaunchKernelGGL((k_rms_norm_rows4<_Float16, 1>), dim3(rows), dim3(VW), 0, st, x, w, y, dim, eps); break;
    case 2: hipLaunchKernelGGL((k_rms_norm_rows4<_Float16, 2>), dim3(rows), dim3(VW), 0, st, x, w, y, dim, eps); break;
    case 4: hipLaunchKernelGGL((k_rms_norm_rows4<_Float16, 4>), dim3(rows), dim3(VW), 0, st, x, w, y, dim, eps); break;
    default: hipLaunchKernelGGL(k_rms_norm_rows<_Float16>, dim3(rows), dim3(VW), 0, st, x, w, y, dim, eps); break;
    }
    return htr_launched(dev, "k_rms_norm_rows<f16>");
}

int launch_heads_f16(htr_device *dev, hipStream_t st, const float *k, const float *v, _Float16 *kv, int n_tok,
                     int n_head, const float *cs, int px, int max_pos) {
    if (px < 1 || (n_tok + px - 1) / px > max_pos || px > max_pos)
        return htr_fail("vision heads: %d tokens on %d columns, rope table of %d positions", n_tok, px, max_pos);
    const int n_blk = (n_tok + FB - 1) / FB;
    hipLaunchKernelGGL(k_heads_f16, dim3(n_blk, n_head), dim3(VW), 0, st, k, v, kv, n_tok, n_head, n_blk, cs, px,
                       max_pos);
    return htr_launched(dev, "k_heads_f16");
}

size_t vision_kv_bytes(int n_tok, int n_head) { return (size_t)n_head * ((n_tok + FB - 1) / FB) * KVB; }

int launch_attn_vision(htr_device *dev, hipStream_t st, const float *q, const _Float16 *kv, _Float16 *o, int n_tok,
                       int n_head, float scale, const float *cs, int px, int max_pos) {
    if (n_tok < 1) return htr_fail("vision attention: %d tokens", n_tok);
    if (px < 1 || (n_tok + px - 1) / px > max_pos || px > max_pos)
        return htr_fail("vision attention: %d tokens on %d columns, rope table of %d positions", n_tok, px, max_pos);
    // two query groups a wave: 0.69 ms a layer at 12100 patches against 0.79 ms with one (223 VGPRs, 2 waves a SIMD;
    // forcing 3 spills 111 of them)
    constexpr int QG = 2;
    const int n_qt = (n_tok + QG * FQ * FWAVES - 1) / (QG * FQ * FWAVES), n_blk = (n_tok + FB - 1) / FB;
    hipLaunchKernelGGL(k_attn_vision<QG>, dim3(n_qt * n_head), dim3(VW), 0, st, q, kv, o, n_tok, n_head, n_blk, n_qt,
                       scale, cs, px, max_pos);
    return htr_launched(dev, "k_attn_vision");
}

int launch_unfold2x2(htr_device *dev, hipStream_t st, const float *x, float *z, int px, int py, int dim) {
    hipLaunchKernelGGL(k_unfold2x2, dim3(grid_for((size_t)px * py * dim)), dim3(VW), 0, st, x, z, px, py, dim);
    return htr_launched(dev, "k_unfold2x2");
}

int launch_gelu(htr_device *dev, hipStream_t st, float *x, size_t n) {
    hipLaunchKernelGGL(k_gelu, dim3(grid_for(n)), dim3(VW), 0, st, x, n);
    return htr_launched(dev, "k_gelu");
}

int launch_split_f16(htr_device *dev, hipStream_t st, const float *x, int m, int k, int kp, int nseg, int lo_mask,
                     _Float16 *out) {
    if (m < 1 || k < 1 || kp < k || kp % 32 || nseg < 1 || nseg > 3)
        return htr_fail("split_f16: [%d x %d] into %d segments of %d", m, k, nseg, kp);
    hipLaunchKernelGGL(k_split_f16, dim3(grid_for((size_t)m * kp)), dim3(VW), 0, st, x, m, k, kp, nseg, lo_mask, out);
    return htr_launched(dev, "k_split_f16");
}
