// GEMMs on gfx950's matrix cores: Y[M,N] (+)= X[M,K] · W[N,K]ᵀ with X and W f16 in memory and f32 accumulation,
// the fused FFN first half G = silu(X·Wgᵀ) · (X·Wuᵀ) · scale → f16, and Q / K / V as one GEMM over the three
// stacked weights. The vision encoder's GEMMs and, on the f16 compute path, the text prefill's.
//
// Reference semantics: matmul_coopd.wgsl (Batch::matmul_f16x, gpu.rs:2019-2042), ffn_coopd.wgsl (Batch::ffn_f16,
// gpu.rs:2048-2086; out_scale = 1/64, vision.rs:31-35) and matmul_coop.wgsl (Batch::matmul on F16Coop,
// gpu.rs:1976-1984: X and the dequantised W rounded to f16, f32 accumulation). The schedule is this library's own:
//
//   tile      a workgroup owns a BM × BN tile of X rows × W rows, split over a WM × WN grid of waves, each wave
//             TM × TN v_mfma_f32_32x32x16_f16 tiles (lane layouts checked on the GPU: A lane ℓ holds
//             A[ℓ%32][8(ℓ/32) …+7], B lane ℓ holds B[8(ℓ/32) …+7][ℓ%32], D lane ℓ register r is row 8(r/4) + 4(ℓ/32)
//             + r%4, column ℓ%32). Tile shapes: 256 × 256 and 192 × 256 (8 waves of 128 × 64 / 96 × 64), 128 × 128
//             and 64 × 64 (4 waves of 64 × 64 / 32 × 32); the launch takes the largest that still gives half a
//             workgroup per CU, 192 rows where that takes fewer rows × rounds, and splits K for prompt-sized M.
//             The FFN's W tile is BN/2 gate rows and the same BN/2 up rows in alternating blocks of 32, so a wave's
//             two column tiles are one gate and one up tile of the same outputs;
//   K         through a ring of LDS stages filled by direct-to-LDS loads (global_load_lds_dwordx4): the 256-wide
//             tiles in stages of 64 (a row's 128 bytes of the stage, whole cache lines) in a ring of 2, the stage
//             after next loading while one is computed; the smaller tiles in stages of 32 in a ring of 4, the stage
//             3 ahead loading. Inside a stage a row's 16-byte chunks sit XOR-placed (chunk ^ (row/4 % 4) for 4 a
//             row, chunk ^ (row/2 % 8) for 8): 16 consecutive rows of one chunk fall on 16 different 16-byte bank
//             groups (gfx950's LDS serves 16 lanes of a 16-byte read a cycle across 256 bytes);
//   pipeline  each k-step of 16 reads the next one's fragments from LDS under its MFMAs. Stages of 32: stage kt
//             runs its first half of MFMAs, then waits for stage kt + 1 and the workgroup barrier while they drain,
//             issues the loads of stage kt + 3 and the fragment reads of stage kt + 1, then its second half. Stages
//             of 64: before the last k-step every wave has its reads of the stage done and its loads of the next
//             stage in; after the barrier the loads of stage kt + 2 go out into the freed buffer. Waits are explicit
//             s_waitcnt vmcnt / lgkmcnt and a bare s_barrier (no fence that would wait for the stages in flight);
//   order     tiles are dealt to the 8 XCDs in contiguous bands (workgroup b runs on XCD b mod 8); inside a band
//             groups of 4 tile rows are walked column by column, so the workgroups resident on an XCD share both
//             their X rows and their W rows in its L2;
//   edges     rows past M read row M − 1 and are not stored; W rows past a weight's end (a last tile that runs over)
//             are read clamped and not stored. Stacked weights start on tile boundaries. K/32 may be odd.
// Measured at M = 12100 on one MI355X (a vision layer's four GEMMs, one box): stages of 64 against 32 — Q/K/V 98 →
// 93 µs, o 46 → 44, down 138–144 → 131–135, gate/up 227–228 → 215–238 (the noisiest); 820–840 TFLOP/s for the
// layer. Timing-only copies without the direct loads or without the fragment reads run 15–20 % and 10 % faster;
// without both (MFMAs, barriers and epilogues alone) about 1.3 PFLOP/s. gfx950's LDS serves about 240 bytes a clock
// to ds_read_b128 (a probe of reads alone), so its bandwidth is not what bounds the loop.
#include <algorithm>

#include "htr_internal.h"
#include "wave.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// AM: X rows a stage loads (≥ BM; the rows past BM are the next tile's, loaded so that every wave issues the same
// direct loads, and not used); KS: K a stage (32 or 64), NST: stages in the LDS ring
template <int BM_, int BN_, int WM_, int WN_, int AM_ = BM_, int KS_ = 32, int NST_ = 4> struct Tile {
    static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, AM = AM_;  // tile: X rows × W rows; wave grid
    static constexpr int KS = KS_, NST = NST_, CPR = KS / 8;        // K and ring stages; 16-byte chunks a row
    static constexpr int NW = WM * WN, GW = 64 * NW;                // waves, threads
    static constexpr int TM = BM / WM / 32, TN = BN / WN / 32;      // MFMA tiles a wave
    static constexpr int ACH = AM * CPR, BCH = BN * CPR, SCH = ACH + BCH;  // 16-byte chunks: A, B, a stage
    static constexpr int AI = ACH / GW, BI = BCH / GW;              // direct-to-LDS loads a wave a stage
    static_assert(TM >= 1 && TN >= 1 && AI * GW == ACH && BI * GW == BCH && AM >= BM, "tile shape");
    static_assert((KS == 32 && NST >= 3) || (KS == 64 && NST == 2), "K stages");
};
using T256 = Tile<256, 256, 2, 4, 256, 64, 2>;
using T192 = Tile<192, 256, 2, 4, 256, 64, 2>;
using T128 = Tile<128, 128, 2, 2>;
using T64 = Tile<64, 64, 2, 2>;

constexpr int GROUP = 4;   // tile rows walked together
constexpr int XCDS = 8;
constexpr int MAX_W = 3;

struct GemmK {
    const _Float16 *x;          // [M][K]
    const _Float16 *w[MAX_W];   // F32 / ACC: the stacked weights; FFN: gate, up
    int n_w;                    // weights
    int rows[MAX_W];            // rows of each (FFN: both the gate's)
    int start[MAX_W];           // F32 / ACC: the first stacked row of each (a multiple of BN)
    float *y[MAX_W];            // F32 / ACC: [M][rows[i]] each (the output columns of weight i)
    _Float16 *y16;              // FFN: [M][rows[0]] f16
    int m, k;
    float scale;                // FFN output scale
    int tiles_m, tiles_n;
    // K split over `split` workgroups a tile (F32 / ACC, one weight): each takes k_per of K and stores its product
    // into part [split][M][N]; k_split_reduce then adds the slices in split order (onto y with ACC)
    int split, k_per;
    float *part;
    // ACC with K split: the reduction also writes h16 = f16(rmsnorm(y)·norm_w) when norm_w is set (rows of 1024·NV)
    const float *norm_w;
    float eps;
    _Float16 *norm_out;
};

// y += ((p_0 + p_1) + p_2) + …, then h = f16(y·1/sqrt(mean(y²) + eps)·w): one row of 1024·NV a workgroup, the sums
// in k_split_reduce's order and the norm in k_rms_norm_rows4's (a thread's 4·NV values, then the wave and the 4
// waves), so the result is the two kernels' one after the other
template <int NV>
__global__ __launch_bounds__(256) void k_split_reduce_norm(const float *part, int split, size_t stride, float *y,
                                                           const float *w, float eps, _Float16 *h) {
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63, n = 1024 * NV;
    const size_t row = blockIdx.x * (size_t)n;
    float4 v[NV];
    float s2 = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const size_t off = row + 4 * (size_t)(tid + 256 * j);
        float4 s = *reinterpret_cast<const float4 *>(part + off);
        for (int q = 1; q < split; q++) {
            const float4 p = *reinterpret_cast<const float4 *>(part + q * stride + off);
            s.x += p.x, s.y += p.y, s.z += p.z, s.w += p.w;
        }
        const float4 b = *reinterpret_cast<const float4 *>(y + off);
        s = make_float4(b.x + s.x, b.y + s.y, b.z + s.z, b.w + s.w);
        *reinterpret_cast<float4 *>(y + off) = s;
        v[j] = s;
        s2 = fmaf(s.x, s.x, s2);
        s2 = fmaf(s.y, s.y, s2);
        s2 = fmaf(s.z, s.z, s2);
        s2 = fmaf(s.w, s.w, s2);
    }
    s2 = wave_sum(s2, lane);
    if (lane == 0) red[tid >> 6] = s2;
    __syncthreads();
    const float scale = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)n + eps);
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const float4 ww = reinterpret_cast<const float4 *>(w)[tid + 256 * j];
        const h4 o = {(_Float16)((v[j].x * scale) * ww.x), (_Float16)((v[j].y * scale) * ww.y),
                      (_Float16)((v[j].z * scale) * ww.z), (_Float16)((v[j].w * scale) * ww.w)};
        *reinterpret_cast<h4 *>(h + row + 4 * (tid + 256 * j)) = o;
    }
}

// y (+)= ((p_0 + p_1) + p_2) + …: the split slices of a GEMM in split order, 4 values a thread
__global__ __launch_bounds__(256) void k_split_reduce(const float *part, int split, size_t n4, float *y, int acc) {
    const size_t stride = n4 * 4;
    for (size_t i = blockIdx.x * (size_t)256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        float4 s = *reinterpret_cast<const float4 *>(part + 4 * i);
        for (int q = 1; q < split; q++) {
            const float4 v = *reinterpret_cast<const float4 *>(part + q * stride + 4 * i);
            s.x += v.x, s.y += v.y, s.z += v.z, s.w += v.w;
        }
        float4 *o = reinterpret_cast<float4 *>(y + 4 * i);
        if (acc) {
            const float4 b = *o;
            s = make_float4(b.x + s.x, b.y + s.y, b.z + s.z, b.w + s.w);
        }
        *o = s;
    }
}

// silu(g) = g / (1 + e^−g) on the hardware's 2^x and reciprocal (v_exp_f32, v_rcp_f32: about 1 ulp each, as the
// reference's WGSL exp and division are not correctly rounded either): ffn_coopd's epilogue evaluates it for every
// one of the tile's 32K outputs, where an exact expf and an IEEE division cost about 40 VALU instructions each value.
// Large −g: 2^x → inf, 1 / inf = 0, g·0 = −0; large g: 1 / 1 → g; NaN stays NaN
__device__ __forceinline__ float silu(float g) {
    const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
    return g * __builtin_amdgcn_rcpf(1.0f + e);
}

// the 16-byte chunk slot of (row r, chunk c) in a stage region of rows of CPR chunks: the chunk index XORed with a
// function of the row, so that the 16 lanes of a fragment read (16 consecutive rows, one chunk) fall on 16 different
// 16-byte bank groups of the 256 bytes the LDS serves a cycle — rows of 4 chunks: chunk ^ (row/4 % 4); rows of 8
// (128 bytes, two rows a bank window): chunk ^ (row/2 % 8). The same XOR maps a slot's chunk back to the row's chunk.
template <int CPR> __device__ __forceinline__ int chunk_swz(int r) {
    return CPR == 4 ? (r >> 2) & 3 : (r >> 1) & 7;
}
template <int CPR> __device__ __forceinline__ int chunk_slot(int r, int c) { return CPR * r + (c ^ chunk_swz<CPR>(r)); }

template <int EPI, class T, bool SPLIT> __global__ __launch_bounds__(T::GW) void k_gemm_f16(const GemmK a) {
    constexpr int BM = T::BM, BN = T::BN, WN = T::WN, NW = T::NW, TM = T::TM, TN = T::TN;
    constexpr int ACH = T::ACH, SCH = T::SCH, AI = T::AI, BI = T::BI;
    constexpr int KS = T::KS, ST = T::NST, CPR = T::CPR, H = KS / 16;  // H: MFMA k-steps a stage
    static_assert(EPI != GEMM_FFN || TN == 2, "the FFN pairs one gate and one up tile a wave");
    __shared__ __attribute__((aligned(16))) int4 s_t[ST * SCH];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    // tile: XCD band, then groups of GROUP tile rows walked column by column
    int tm, tn;
    const int sp = SPLIT ? (int)blockIdx.x % a.split : 0;  // this workgroup's part of K
    const int tile = SPLIT ? (int)blockIdx.x / a.split : (int)blockIdx.x;
    {
        const int total = a.tiles_m * a.tiles_n, b = tile, xcd = b % XCDS, i = b / XCDS;
        const int per = total / XCDS, extra = total % XCDS;
        const int t = xcd * per + min(xcd, extra) + i;
        const int gsz = GROUP * a.tiles_n, g = t / gsz, gr = t % gsz, gm = min(GROUP, a.tiles_m - g * GROUP);
        tm = g * GROUP + gr % gm;
        tn = gr / gm;
    }
    const int row0 = tm * BM, k = a.k, m = a.m;
    const int nk = (SPLIT ? a.k_per : k) / KS, kbeg = SPLIT ? sp * a.k_per : 0;
    // the W rows of tile row r (0 … BN−1): F32 / ACC the tile's rows of the stacked weights (one weight a tile, rows
    // past its end clamped); FFN blocks of 32 alternating gate / up rows of the tile's BN/2 outputs
    int wsel = 0;
    if (EPI != GEMM_FFN)
        for (int i = 1; i < a.n_w; i++) wsel += tn * BN >= a.start[i];
    const _Float16 *wbase = a.w[wsel];
    const int wrows = a.rows[wsel];
    const int wrow0 = EPI == GEMM_FFN ? tn * (BN / 2) : tn * BN - a.start[wsel];
    auto w_row = [&](int r, const _Float16 *&base) -> int {
        if (EPI == GEMM_FFN) {
            base = (r >> 5) & 1 ? a.w[1] : a.w[0];
            return wrow0 + (r >> 6) * 32 + (r & 31);
        }
        base = wbase;
        return min(wrow0 + r, wrows - 1);
    };
    auto issue = [&](int ks, int buf) {
        const size_t kk = (size_t)kbeg + (size_t)min(ks, nk - 1) * KS;
#pragma unroll
        for (int i = 0; i < AI; i++) {
            const int s = 64 * (wave + NW * i) + lane, r = s / CPR, c = (s % CPR) ^ chunk_swz<CPR>(r);
            __builtin_amdgcn_global_load_lds((const void *)(a.x + (size_t)min(row0 + r, m - 1) * k + kk + 8 * c),
                                             (void __attribute__((address_space(3))) *)&s_t[buf * SCH + 64 * (wave + NW * i)],
                                             16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < BI; i++) {
            const int s = 64 * (wave + NW * i) + lane, r = s / CPR, c = (s % CPR) ^ chunk_swz<CPR>(r);
            const _Float16 *base;
            const int wr = w_row(r, base);
            __builtin_amdgcn_global_load_lds((const void *)(base + (size_t)wr * k + kk + 8 * c),
                                             (void __attribute__((address_space(3))) *)&s_t[buf * SCH + ACH + 64 * (wave + NW * i)],
                                             16, 0, 0);
        }
    };
    // the lane's fragment slots: A tile i, B tile j, k-step h (chunk 2h + lane/32 of row … + lane%32)
    int ao[TM][H], bo[TN][H];
#pragma unroll
    for (int h = 0; h < H; h++) {
#pragma unroll
        for (int i = 0; i < TM; i++)
            ao[i][h] = chunk_slot<CPR>(wm * TM * 32 + 32 * i + (lane & 31), 2 * h + (lane >> 5));
#pragma unroll
        for (int j = 0; j < TN; j++)
            bo[j][h] = ACH + chunk_slot<CPR>(wn * TN * 32 + 32 * j + (lane & 31), 2 * h + (lane >> 5));
    }
    struct Frag {
        half8 a[2][TM], b[2][TN];
    };
    auto read = [&](Frag &f, int stage) {
        const int4 *st = s_t + (stage % ST) * SCH;
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int i = 0; i < TM; i++) f.a[h][i] = *reinterpret_cast<const half8 *>(st + ao[i][h]);
#pragma unroll
            for (int j = 0; j < TN; j++) f.b[h][j] = *reinterpret_cast<const half8 *>(st + bo[j][h]);
        }
    };
    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    auto mfma_half = [&](const Frag &f, int h) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[h][i], f.b[h][j], acc[i][j], 0, 0, 0);
    };
    if constexpr (KS == 64) {
        // stages of 64 K (each X and W row's 128 bytes of the stage: whole cache lines) in a ring of two: stage kt
        // is computed from one buffer while stage kt + 1 loads into the other. Its four k-steps each read the next
        // k-step's fragments under their MFMAs; before the last, every wave has its reads of stage kt done
        // (lgkmcnt) and its loads of stage kt + 1 in (vmcnt), and the barrier frees stage kt's buffer for stage
        // kt + 2, whose loads go out with the next stage's first fragment reads under the last k-step's MFMAs
        struct Fr {
            half8 a[TM], b[TN];
        };
        auto rd = [&](Fr &f, int stage, int h) {
            const int4 *st = s_t + (stage % ST) * SCH;
#pragma unroll
            for (int i = 0; i < TM; i++) f.a[i] = *reinterpret_cast<const half8 *>(st + ao[i][h]);
#pragma unroll
            for (int j = 0; j < TN; j++) f.b[j] = *reinterpret_cast<const half8 *>(st + bo[j][h]);
        };
        auto mf = [&](const Fr &f) {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
        };
        constexpr int NMF = TM * TN, NVM = AI + BI, NRD = TM + TN;
        // the order pinned: each MFMA followed by one of the k-step's other instructions — a direct load while they
        // last (the last k-step), a fragment read while they last
        auto pin = [&](bool loads) {
#pragma unroll
            for (int q = 0; q < NMF; q++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                if (loads && q < NVM) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one direct load
                if (q < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);           // one LDS read
            }
        };
        issue(0, 0);
        issue(1, 1);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(AI + BI) : "memory");  // stage 0 is in
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        Fr f0, f1;
        rd(f0, 0, 0);
        for (int kt = 0; kt < nk; kt++) {
            rd(f1, kt, 1);
            mf(f0);
            pin(false);
            rd(f0, kt, 2);
            mf(f1);
            pin(false);
            rd(f1, kt, 3);
            mf(f0);
            pin(false);
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            issue(kt + 2, kt % 2);
            rd(f0, kt + 1, 0);
            mf(f1);
            pin(true);
        }
    } else {
#pragma unroll
    for (int s = 0; s < ST - 1; s++) issue(s, s);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((ST - 2) * (AI + BI)) : "memory");  // stage 0 is in
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    Frag f0, f1;
    read(f0, 0);
    // one stage: cur holds its fragments; nxt receives stage kt + 1's. The stages in flight at the wait are kt + 1 …
    // kt + ST − 2 (the one to wait for and ST − 3 later ones); the buffer refilled after the barrier held stage kt − 1,
    // which every wave finished reading in the stage before (the memory clobbers keep the loads and LDS reads after
    // the wait and the barrier; the MFMAs are interleaved with them by the group barriers below, not issued as blocks)
    auto step = [&](Frag &cur, Frag &nxt, int kt) {
        mfma_half(cur, 0);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((ST - 3) * (AI + BI)) : "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        issue(kt + ST - 1, (kt + ST - 1) % ST);
        read(nxt, kt + 1);
        mfma_half(cur, 1);
        // the order after the barrier, pinned: one MFMA, then one of the stage's direct loads, while they last; then
        // one MFMA, then a share of the next stage's fragment reads. Left to itself the scheduler sank the reads to just
        // before their use and waited for each group (lgkmcnt(0) before the MFMAs); pinned, the reads' latency runs
        // under this half-stage's MFMAs. Measured on one MI355X at M = 12100: the FFN GEMM 214–216 → 208 µs
        constexpr int NMF = TM * TN, NVM = AI + BI, NDS = 2 * (TM + TN);
        constexpr int DSPER = NMF > NVM ? (NDS + NMF - NVM - 1) / (NMF - NVM) : NDS;
#pragma unroll
        for (int q = 0; q < NMF; q++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            if (q < NVM)
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one global (direct-to-LDS) load
            else
                __builtin_amdgcn_sched_group_barrier(0x100, DSPER, 0);  // LDS reads
        }
    };
    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
        step(f0, f1, kt);
        step(f1, f0, kt + 1);
    }
    if (kt < nk) step(f0, f1, kt);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no LDS load left in flight when the wave ends

    // epilogue: lane ℓ, register r → row 8(r/4) + 4(ℓ/32) + r%4, column ℓ%32 of each 32 × 32 tile
    if constexpr (EPI == GEMM_FFN) {
        // the wave's TM·32 × 32 f16 outputs go through its own region of the (now idle) stage ring — rows of 32 values
        // 80 bytes apart, so that the two half-waves' rows 4 apart fall on different banks — and leave it as 16-byte
        // row chunks: 2·TM stores a lane instead of 16·TM two-byte ones
        constexpr int RS = 40;                                         // halves a staged row
        static_assert(NW * TM * 32 * RS * 2 <= ST * SCH * 16, "the staging fits the ring");
        __syncthreads();                                               // every wave is done with the ring
        _Float16 *stg = reinterpret_cast<_Float16 *>(s_t) + wave * TM * 32 * RS;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int rr = 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                stg[rr * RS + (lane & 31)] = (_Float16)(silu(acc[i][0][r]) * acc[i][1][r] * a.scale);
            }
        __builtin_amdgcn_wave_barrier();
        const int col0 = tn * (BN / 2) + wn * 32;  // gate tile j = 0, up tile j = 1: the same 32 outputs
#pragma unroll
        for (int t = 0; t < 2 * TM; t++) {
            const int u = lane + 64 * t, rr = u >> 2, c = u & 3;
            const int row = row0 + wm * TM * 32 + rr;
            const int4 v = *reinterpret_cast<const int4 *>(stg + rr * RS + 8 * c);
            if (row < m) *reinterpret_cast<int4 *>(a.y16 + (size_t)row * a.rows[0] + col0 + 8 * c) = v;
        }
        return;
    }
    if constexpr (EPI == GEMM_ACC && !SPLIT) {
        // the residual update as 16-byte row chunks through the wave's own region of the (now idle) stage ring: column
        // tile j's TM·32 × 32 sums are written in the MFMA layout (rows 40 floats apart, so that the two half-waves'
        // rows 4 apart fall on different banks; 32 where 40 does not fit the ring) and read back 4 consecutive columns
        // a lane; a lane then loads, adds and stores 4·TM 16-byte chunks a column tile instead of 16·TM single values
        // (o and down at 12100 rows: 136 → 129 µs for down; the plain store epilogue stays direct: staged, Q/K/V
        // was 1.5 % slower)
        constexpr int RS = NW * TM * 32 * 40 * 4 <= ST * SCH * 16 ? 40 : 32, NC = TM * 32 * 8 / 64;
        static_assert(NW * TM * 32 * RS * 4 <= ST * SCH * 16, "the staging fits the ring");
        __syncthreads();  // every wave is done with the ring
        float *stg = reinterpret_cast<float *>(s_t) + wave * TM * 32 * RS;
        float *y = a.y[wsel];
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int col0 = wrow0 + wn * TN * 32 + 32 * j;  // the column tile's first column (rows a multiple of 64)
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    stg[(32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * RS + (lane & 31)] = acc[i][j][r];
            __builtin_amdgcn_wave_barrier();
            if (col0 < wrows) {  // the part of a last tile past the weight's end is not stored
                float4 v[NC];
#pragma unroll
                for (int t = 0; t < NC; t++) {
                    const int u = lane + 64 * t;
                    v[t] = *reinterpret_cast<const float4 *>(stg + (u >> 3) * RS + 4 * (u & 7));
                }
                // every residual chunk loads before the first sum is stored (rows past M read row M − 1): the stores
                // to y may alias the loads, so the compiler would otherwise chain them one by one
                float4 p[NC];
#pragma unroll
                for (int t = 0; t < NC; t++) {
                    const int u = lane + 64 * t, row = min(row0 + wm * TM * 32 + (u >> 3), m - 1);
                    p[t] = *reinterpret_cast<const float4 *>(y + (size_t)row * wrows + col0 + 4 * (u & 7));
                }
#pragma unroll
                for (int t = 0; t < NC; t++)
                    v[t] = make_float4(p[t].x + v[t].x, p[t].y + v[t].y, p[t].z + v[t].z, p[t].w + v[t].w);
#pragma unroll
                for (int t = 0; t < NC; t++) {
                    const int u = lane + 64 * t, row = row0 + wm * TM * 32 + (u >> 3);
                    if (row < m) *reinterpret_cast<float4 *>(y + (size_t)row * wrows + col0 + 4 * (u & 7)) = v[t];
                }
            }
            __builtin_amdgcn_wave_barrier();  // the reads of this column tile before the next one's writes
        }
        return;
    }
    // F32: the products stored; SPLIT (F32 or ACC): this part of K's product into its own slice [sp][M][N]
    // (k_split_reduce adds the slices)
    float *y = SPLIT ? a.part + (size_t)sp * m * wrows : a.y[wsel];
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int col = wrow0 + wn * TN * 32 + 32 * j + (lane & 31);
        if (col >= wrows) continue;  // the part of a last tile past the weight's end
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = row0 + wm * TM * 32 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < m) y[(size_t)row * wrows + col] = acc[i][j][r];
            }
    }
}

template <class T> int tiles_for(const GemmK &a, int epi, int &tm, int &tn) {
    tm = (a.m + T::BM - 1) / T::BM;
    if (epi == GEMM_FFN) {
        if (a.rows[0] % (T::BN / 2)) return -1;
        tn = a.rows[0] / (T::BN / 2);
        return tm * tn;
    }
    for (int i = 1; i < a.n_w; i++)
        if (a.start[i] % T::BN) return -1;
    tn = (a.start[a.n_w - 1] + a.rows[a.n_w - 1] + T::BN - 1) / T::BN;
    return tm * tn;
}

template <class T> void launch_tile(hipStream_t st, int epi, const GemmK &a) {
    const dim3 grid(a.tiles_m * a.tiles_n * (a.split > 1 ? a.split : 1));
    switch (epi) {
    case GEMM_F32:
        if (a.split > 1) hipLaunchKernelGGL((k_gemm_f16<GEMM_F32, T, true>), grid, dim3(T::GW), 0, st, a);
        else hipLaunchKernelGGL((k_gemm_f16<GEMM_F32, T, false>), grid, dim3(T::GW), 0, st, a);
        break;
    case GEMM_ACC:
        if (a.split > 1) hipLaunchKernelGGL((k_gemm_f16<GEMM_ACC, T, true>), grid, dim3(T::GW), 0, st, a);
        else hipLaunchKernelGGL((k_gemm_f16<GEMM_ACC, T, false>), grid, dim3(T::GW), 0, st, a);
        break;
    default:
        if constexpr (T::TN == 2) hipLaunchKernelGGL((k_gemm_f16<GEMM_FFN, T, false>), grid, dim3(T::GW), 0, st, a);
        break;
    }
}

// the largest tile shape that gives at least half a workgroup per CU; else the one with the most tiles (the FFN: 256
// or 128 — a wave pairs one gate and one up tile)
int launch(htr_device *dev, hipStream_t st, int epi, GemmK &a, bool *normed = nullptr) {
    if (normed) *normed = false;
    if (epi != GEMM_F32 && epi != GEMM_ACC && epi != GEMM_FFN) return htr_fail("gemm_f16: epilogue %d", epi);
    const int want = std::max(1, dev->n_cu / 2);
    int tm, tn;
    // the 256-wide tiles take K in stages of 64
    const int n_tiles[3] = {a.k % 64 ? -1 : tiles_for<T256>(a, epi, tm, tn), tiles_for<T128>(a, epi, tm, tn),
                            epi == GEMM_FFN ? -1 : tiles_for<T64>(a, epi, tm, tn)};
    int pick = -1;
    for (int i = 0; i < 3 && pick < 0; i++)
        if (n_tiles[i] >= want) pick = i;
    // large M: 192-row tiles when they take fewer rows × rounds of one workgroup a CU (M = 12100 at N = 1024: 256
    // tiles in one round against 192 of 256 rows; at N = 3072 three full rounds against 2¼)
    if (pick == 0) {
        const int t192 = tiles_for<T192>(a, epi, tm, tn);
        const long c256 = (long)((n_tiles[0] + dev->n_cu - 1) / dev->n_cu) * 256;
        const long c192 = (long)((t192 + dev->n_cu - 1) / dev->n_cu) * 192;
        if (t192 > 0 && c192 < c256) {
            tiles_for<T192>(a, epi, a.tiles_m, a.tiles_n);
            launch_tile<T192>(st, epi, a);
            return htr_launched(dev, "k_gemm_f16<192>");
        }
    }
    // too few 256 / 128 tiles and a long K (one weight; N a multiple of 4): 128 × 128 tiles with K split over up to 4
    // workgroups (a multiple of 32 each), the products summed in split order by k_split_reduce
    a.split = 1;
    if (pick != 0 && epi != GEMM_FFN && a.n_w == 1 && a.rows[0] % 4 == 0 && n_tiles[1] > 0 && n_tiles[1] < want &&
        a.k >= 1024) {
        int sp = std::min(4, (dev->n_cu + n_tiles[1] - 1) / n_tiles[1]);
        while (sp > 1 && a.k % (32 * sp)) sp--;
        if (sp > 1) {
            void *part = nullptr;
            HTR_TRY(htr_scratch(dev, SCR_GEMM_PART, (size_t)sp * a.m * a.rows[0] * 4, &part));
            a.split = sp;
            a.k_per = a.k / sp;
            a.part = (float *)part;
            tiles_for<T128>(a, epi, a.tiles_m, a.tiles_n);
            launch_tile<T128>(st, epi, a);
            HTR_TRY(htr_launched(dev, "k_gemm_f16<128, split K>"));
            const size_t n4 = (size_t)a.m * a.rows[0] / 4;
            const int nv = a.rows[0] % 1024 ? 0 : a.rows[0] / 1024;
            if (epi == GEMM_ACC && a.norm_w && normed && (nv == 1 || nv == 2 || nv == 4)) {
                const size_t stride = n4 * 4;
                if (nv == 1)
                    hipLaunchKernelGGL(k_split_reduce_norm<1>, dim3(a.m), dim3(256), 0, st, a.part, sp, stride, a.y[0],
                                       a.norm_w, a.eps, a.norm_out);
                else if (nv == 2)
                    hipLaunchKernelGGL(k_split_reduce_norm<2>, dim3(a.m), dim3(256), 0, st, a.part, sp, stride, a.y[0],
                                       a.norm_w, a.eps, a.norm_out);
                else
                    hipLaunchKernelGGL(k_split_reduce_norm<4>, dim3(a.m), dim3(256), 0, st, a.part, sp, stride, a.y[0],
                                       a.norm_w, a.eps, a.norm_out);
                *normed = true;
                return htr_launched(dev, "k_split_reduce_norm");
            }
            const int grid = (int)std::min<size_t>((n4 + 255) / 256, (size_t)dev->n_cu * 8);
            hipLaunchKernelGGL(k_split_reduce, dim3(grid), dim3(256), 0, st, a.part, sp, n4, a.y[0],
                               epi == GEMM_ACC ? 1 : 0);
            return htr_launched(dev, "k_split_reduce");
        }
    }
    for (int i = 0; i < 3 && pick < 0; i++)
        if (n_tiles[i] >= 0 && (pick < 0 || n_tiles[i] > n_tiles[pick])) pick = i;
    if (pick < 0) return htr_fail("gemm_f16: no tile shape fits weights of %d rows", a.rows[0]);
    if (pick == 0) {
        tiles_for<T256>(a, epi, a.tiles_m, a.tiles_n);
        launch_tile<T256>(st, epi, a);
        return htr_launched(dev, "k_gemm_f16<256>");
    }
    if (pick == 1) {
        tiles_for<T128>(a, epi, a.tiles_m, a.tiles_n);
        launch_tile<T128>(st, epi, a);
        return htr_launched(dev, "k_gemm_f16<128>");
    }
    tiles_for<T64>(a, epi, a.tiles_m, a.tiles_n);
    launch_tile<T64>(st, epi, a);
    return htr_launched(dev, "k_gemm_f16<64>");
}

}  // namespace

int launch_gemm_f16(htr_device *dev, hipStream_t st, int epi, const _Float16 *x, int m, const htr_weight *w,
                    const htr_weight *w2, float *y, _Float16 *y16, float scale) {
    if (!w || !w->h) return htr_fail("gemm_f16: the weight has no f16 plane (htr_weight_q8_0_f16)");
    const int n = (int)w->rows, k = (int)w->cols;
    if (m < 1) return htr_fail("gemm_f16: %d rows", m);
    if (n % 64 || k % 32 || (epi == GEMM_FFN && n % 128))
        return htr_fail("gemm_f16: W [%d x %d]: rows a multiple of %d, columns a multiple of 32", n, k,
                        epi == GEMM_FFN ? 128 : 64);
    if (epi == GEMM_FFN && (!w2 || !w2->h || (int)w2->rows != n || (int)w2->cols != k))
        return htr_fail("gemm_f16: the FFN's up weight must match the gate weight [%d x %d]", n, k);
    GemmK a{};
    a.x = x;
    a.w[0] = w->h;
    a.w[1] = epi == GEMM_FFN ? w2->h : w->h;
    a.w[2] = w->h;
    a.n_w = 1;
    a.rows[0] = a.rows[1] = a.rows[2] = n;
    a.y[0] = a.y[1] = a.y[2] = y;
    a.y16 = y16;
    a.m = m;
    a.k = k;
    a.scale = scale;
    return launch(dev, st, epi, a);
}

int launch_gemm_f16_acc_norm(htr_device *dev, hipStream_t st, const _Float16 *x, int m, const htr_weight *w, float *y,
                             const float *norm_w, float eps, _Float16 *h16) {
    if (!w || !w->h) return htr_fail("gemm_f16: the weight has no f16 plane (htr_weight_q8_0_f16)");
    const int n = (int)w->rows, k = (int)w->cols;
    if (m < 1) return htr_fail("gemm_f16: %d rows", m);
    if (n % 64 || k % 32) return htr_fail("gemm_f16: W [%d x %d]: rows a multiple of 64, columns a multiple of 32", n, k);
    if (!norm_w || !h16) return htr_fail("gemm_f16: the norm weight and output are required");
    GemmK a{};
    a.x = x;
    a.w[0] = a.w[1] = a.w[2] = w->h;
    a.n_w = 1;
    a.rows[0] = a.rows[1] = a.rows[2] = n;
    a.y[0] = a.y[1] = a.y[2] = y;
    a.m = m;
    a.k = k;
    a.scale = 1.0f;
    a.norm_w = norm_w;
    a.eps = eps;
    a.norm_out = h16;
    bool normed = false;
    HTR_TRY(launch(dev, st, GEMM_ACC, a, &normed));
    if (!normed) HTR_TRY(launch_rms_norm_f16(dev, st, y, norm_w, h16, m, n, eps));
    return 0;
}

int launch_gemm_f16_qkv(htr_device *dev, hipStream_t st, const _Float16 *x, int m, const htr_weight *wq,
                        const htr_weight *wk, const htr_weight *wv, float *q, float *kk, float *v) {
    const htr_weight *ws[3] = {wq, wk, wv};
    for (const htr_weight *w : ws)
        if (!w || !w->h) return htr_fail("gemm_f16_qkv: a weight has no f16 plane (htr_weight_q8_0_f16)");
    const int k = (int)wq->cols;
    if (m < 1) return htr_fail("gemm_f16_qkv: %d rows", m);
    for (const htr_weight *w : ws)
        if ((int)w->cols != k || w->rows % 64 || k % 32)
            return htr_fail("gemm_f16_qkv: W [%zu x %zu]: rows a multiple of 64, %d columns (a multiple of 32)",
                            w->rows, w->cols, k);
    GemmK a{};
    a.x = x;
    a.n_w = 3;
    int start = 0;
    for (int i = 0; i < 3; i++) {
        a.w[i] = ws[i]->h;
        a.rows[i] = (int)ws[i]->rows;
        a.start[i] = start;
        start += a.rows[i];
    }
    a.y[0] = q;
    a.y[1] = kk;
    a.y[2] = v;
    a.m = m;
    a.k = k;
    a.scale = 1.0f;
    return launch(dev, st, GEMM_F32, a);
}

// ---- ABI ------------------------------------------------------------------------------------------------------------

extern "C" int htr_gemm_f16(htr_device *dev, const uint16_t *d_x, size_t m, const htr_weight *w, float *d_y, int acc) {
    HTR_TRY(htr_check_alive(dev));
    if (!d_x || !d_y || !w) return htr_fail("htr_gemm_f16: null argument");
    if (m > (size_t)INT32_MAX / 2) return htr_fail("htr_gemm_f16: %zu rows", m);
    return launch_gemm_f16(dev, dev->stream, acc ? GEMM_ACC : GEMM_F32, (const _Float16 *)d_x, (int)m, w, nullptr, d_y,
                           nullptr, 1.0f);
}

extern "C" int htr_gemm_ffn_f16(htr_device *dev, const uint16_t *d_x, size_t m, const htr_weight *w_gate,
                                const htr_weight *w_up, float scale, uint16_t *d_g) {
    HTR_TRY(htr_check_alive(dev));
    if (!d_x || !d_g || !w_gate || !w_up) return htr_fail("htr_gemm_ffn_f16: null argument");
    if (m > (size_t)INT32_MAX / 2) return htr_fail("htr_gemm_ffn_f16: %zu rows", m);
    return launch_gemm_f16(dev, dev->stream, GEMM_FFN, (const _Float16 *)d_x, (int)m, w_gate, w_up, nullptr,
                           (_Float16 *)d_g, scale);
}
