// hx_moe_prefill.hip -- routed experts for many tokens on gfx950 (grouped MFMA GEMMs over the
// token-by-expert permutation).
//
// Flow (all stream-ordered, no host synchronisation):
//   plan       expert_count -> per-row expert id and 128/96/64/32-row tile jobs per expert
//   gather     xg[r] = fp16(H(x[token_sorted[r]] . suh_g[e])), xu[r] likewise (H on the matrix
//              cores), and their row sums per 128-column block
//   gate/up    G = xg . W_g[e], U = xu . W_u[e] (quarter-operand MFMA tiles), then in the same
//              workgroup act[r] = fp16(H((act(g) * u) . suh_d)), g = fp16(H(G)) . svh_g ... (fp16
//              chain, transforms on the matrix cores), and the row sums of act
//   gemm d     D = act . W_d[e]                    (fp16 output)
//   combine    y[t] = fp16(sum_j H(D[r_j]) * w_j / sqrt(128) . svh_d[e_j]  + shared[t])
// Reference semantics: src/cuda/quant/exl3_moe_kernel.cuh:57-262, hadamard_inner.cuh:284-481,
// src/engine/glue2.cu:297-306, runner.cpp:957-958.
#include "hx_mfma.hpp"
#include "hx_kernels.hpp"
#include "hx_moe.hpp"

namespace hx {

static size_t al(size_t v) { return (v + 255) & ~(size_t)255; }

struct Job {
    int expert, row0, rows, bm;  // bm: row tile (128, or 96 / 64 / 32 for a remainder of at most that many rows)
};

void MoeWs::prefill_layout(size_t o)
{
    max_jobs = (R + MF_BM - 1) / MF_BM + E;
    const int kmax = hidden > inter ? hidden : inter;
    off_perm = o;       o = al(o + sizeof(int) * 2 * (size_t)((R + 1023) / 1024) * E);
    off_jobs = o;       o = al(o + sizeof(Job) * max_jobs);
    off_njobs = o;      o = al(o + sizeof(int));
    off_row_expert = o; o = al(o + sizeof(int) * R);
    off_xg = o;         o = al(o + sizeof(_Float16) * (size_t)R * hidden);
    off_xu = o;         o = al(o + sizeof(_Float16) * (size_t)R * hidden);
    off_G = o;          o = al(o + sizeof(_Float16) * (size_t)R * inter);
    off_A = o;          o = al(o + sizeof(_Float16) * (size_t)R * inter);
    off_rs = o;         o = al(o + sizeof(float) * (size_t)R * (2 * (hidden / 128) + inter / 128));
    off_D = off_xg;     // D reuses xg (xg is consumed by the gate GEMM before the down GEMM runs)
    off_sh_a = o;       o = al(o + sizeof(_Float16) * (size_t)T * kmax);
    off_sh_g = o;       o = al(o + sizeof(float) * (size_t)T * inter);
    off_sh_u = o;       o = al(o + sizeof(float) * (size_t)T * inter);
    off_sh_act = o;     o = al(o + sizeof(_Float16) * (size_t)T * inter);
    off_sh_d = o;       o = al(o + sizeof(float) * (size_t)T * hidden);
    prefill_end = o;
}

// ------------------------------------------------------------------ plan

// Every block scans the expert counts (E <= 512) in LDS; block 0 writes the tile jobs, and each
// block maps its 256 rows to their expert.
__global__ __launch_bounds__(512) void prefill_plan_kernel(const int64_t* expert_count, int E, int R, Job* jobs,
                                                          int* njobs, int* row_expert)
{
    __shared__ int off[513];   // exclusive scan of the row counts
    __shared__ int joff[513];  // exclusive scan of the job counts
    const int t = threadIdx.x;
    const int c = t < E ? (int)expert_count[t] : 0;
    const int nj = (c + MF_BM - 1) / MF_BM;
    off[t] = c;
    joff[t] = nj;
    __syncthreads();
    for (int d = 1; d < 512; d <<= 1) {  // inclusive Hillis-Steele scans
        const int a = t >= d ? off[t - d] : 0, b = t >= d ? joff[t - d] : 0;
        __syncthreads();
        off[t] += a;
        joff[t] += b;
        __syncthreads();
    }
    const int r0 = off[t] - c, j0 = joff[t] - nj;  // exclusive
    if (blockIdx.x == 0) {
        for (int k = 0; k < nj; ++k) {
            const int rows = min(MF_BM, c - k * MF_BM);
            jobs[j0 + k] = Job{t, r0 + k * MF_BM, rows, rows <= 32 ? 32 : rows <= 64 ? 64 : rows <= 96 ? 96 : MF_BM};
        }
        if (t == 511) *njobs = joff[511];
    }
    __syncthreads();
    off[t] = r0;
    if (t == 0) off[512] = 0x7fffffff;
    __syncthreads();
    const int r = blockIdx.x * 512 + t;
    if (r < R) {
        int lo = 0, hi = E;  // largest e with off[e] <= r
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (off[mid] <= r) lo = mid;
            else hi = mid;
        }
        row_expert[r] = lo;
    }
}

// ------------------------------------------------------------------ gather + input transform

// One wave per (16 sorted rows, 128-column block): the transform is a 16 x 128 by 128 x 128 GEMM on
// the matrix cores, A = fp16(x[token] . suh) (one fp16 rounding, as the reference's __hmul2),
// B = H128 generated in registers, fp32 accumulation (the products
// are exact, so this is the reference's fp32 butterfly up to the order of the fp32 additions), one
// fp16 rounding.  Lane l: A row l % 16, k = 32 kk + 8 (l / 16) + 0..7; B column 16 nb + l % 16 with
// the same k; C rows 4 (l / 16) + i, column 16 nb + l % 16.  Also writes each row's sum of the 128
// outputs (rs[row][block], the codebook-2 map of the grouped GEMMs).
__global__ __launch_bounds__(256, 4) void prefill_gather_kernel(const _Float16* x, const int64_t* token_sorted,
                                                            const int* row_expert, const void* const* suh_g,
                                                            const void* const* suh_u, _Float16* xg, _Float16* xu,
                                                            int hidden, bool gated, float* rs_g, float* rs_u, long R)
{
    const int lane = threadIdx.x & 63;
    const int nblk = hidden >> 7;
    const long unit = (long)blockIdx.x * 4 + (threadIdx.x >> 6);  // (row block, column block)
    const long rb = unit / nblk;
    const int kb = (int)(unit % nblk);
    if (rb * 16 >= R) return;
    const int c = lane & 15, g = lane >> 4;
    const long r = min(rb * 16 + c, R - 1);  // A row of this lane (rows past R repeat the last, not stored)
    const int e = row_expert[r];
    const _Float16* xr = x + (size_t)token_sorted[r] * hidden + kb * 128 + 8 * g;
    const _Float16* sg = static_cast<const _Float16*>(gated ? suh_g[e] : suh_u[e]) + kb * 128 + 8 * g;
    const _Float16* su = static_cast<const _Float16*>(suh_u[e]) + kb * 128 + 8 * g;
    hx_h8 xv[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) xv[kk] = *reinterpret_cast<const hx_h8*>(xr + 32 * kk);
    // H128 B operands: sign of (n, k) = popcount(n & k) & 1 with n = 16 nb + c, k = 32 kk + 8 g + j
    uint32_t f[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t s0 = __builtin_popcount(c & (2 * i) & 7) & 1, s1 = __builtin_popcount(c & (2 * i + 1) & 7) & 1;
        f[i] = (0x3c00u | (s0 << 15)) | ((0x3c00u | (s1 << 15)) << 16);
    }
    const uint32_t base = (uint32_t)((c >> 3) & g & 1);
    __shared__ _Float16 stage[4][2][16][136];
    _Float16 (*sw)[16][136] = stage[threadIdx.x >> 6];
    float sum_g[4] = {0.f, 0.f, 0.f, 0.f}, sum_u[4] = {0.f, 0.f, 0.f, 0.f};
    // the gate's transform, then the up's (one accumulator set at a time)
#pragma unroll 1
    for (int pj = gated ? 0 : 1; pj < 2; ++pj) {
        const _Float16* sp = pj ? su : sg;
        hx_h8 av[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) av[kk] = xv[kk] * *reinterpret_cast<const hx_h8*>(sp + 32 * kk);
        hx_f4 y[8];
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) y[nb] = hx_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) {
                const uint32_t sgn = base ^ ((uint32_t)(nb & 1) & (uint32_t)(g >> 1)) ^ (uint32_t)((nb >> 1) & kk & 1) ^
                                     (uint32_t)((nb >> 2) & (kk >> 1) & 1);
                const uint32_t m = sgn ? 0x80008000u : 0u;
                typedef uint32_t u4v __attribute__((ext_vector_type(4)));
                const u4v bv = {f[0] ^ m, f[1] ^ m, f[2] ^ m, f[3] ^ m};
                y[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[kk], __builtin_bit_cast(hx_h8, bv), y[nb], 0, 0, 0);
            }
        // fp16 outputs staged in LDS (16-byte row stores below); row sums: the 16 lanes of a lane
        // group hold one row's 128 columns
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float t = 0.0f;
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) {
                const _Float16 v = (_Float16)(y[nb][i] * HX_RSQRT128);
                t += (float)v;
                sw[pj][4 * g + i][16 * nb + c] = v;
            }
            if (pj) sum_u[i] = t;
            else sum_g[i] = t;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int row16 = 4 * q + (lane >> 4), c8 = 8 * (lane & 15);
        const long row = rb * 16 + row16;
        if (row < R) {
            const size_t o = (size_t)row * hidden + kb * 128 + c8;
            if (gated) *reinterpret_cast<hx_u4v*>(xg + o) = *reinterpret_cast<const hx_u4v*>(&sw[0][row16][c8]);
            *reinterpret_cast<hx_u4v*>(xu + o) = *reinterpret_cast<const hx_u4v*>(&sw[1][row16][c8]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
            sum_g[i] += __shfl_xor(sum_g[i], o, 64);
            sum_u[i] += __shfl_xor(sum_u[i], o, 64);
        }
    if (c < 4) {
        float vg_ = 0.f, vu_ = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (c == i) vg_ = sum_g[i], vu_ = sum_u[i];
        const long row = rb * 16 + 4 * g + c;
        if (row < R) {
            if (gated) rs_g[(size_t)row * nblk + kb] = vg_;
            rs_u[(size_t)row * nblk + kb] = vu_;
        }
    }
}

// ------------------------------------------------------------------ grouped GEMM

struct GroupedGemmArgs {
    const Job* jobs;
    const int* njobs;
    const _Float16* A[2];
    _Float16* out[2];
    const void* const* tr[2];
    const int32_t* bits_tab[2];
    int bits_uniform[2];
    int K, N, nproj;
    const float* rs[2];  // precomputed row sums of A: rs_n partial sums per row
    int rs_n;
};

template <int BITS, int CB, int BM>
__device__ __forceinline__ void grouped_tile(const GroupedGemmArgs& g, const Job& job, int proj, int cg, MfmaSmemQ& sm)
{
    const _Float16* A = g.A[proj] + (size_t)job.row0 * g.K;
    const uint32_t* tr = static_cast<const uint32_t*>(g.tr[proj][job.expert]);
    hx_f4 acc[BM / 16][2];
    mfma_tile_q<BITS, CB, BM, QT_PF, true>(A, g.K, job.rows, tr, g.K, g.N, cg * 8, sm, acc,
                                            g.rs[proj] + (size_t)job.row0 * g.rs_n, g.rs_n);
    _Float16* out = g.out[proj] + (size_t)job.row0 * g.N + cg * 128;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int half = 0; half < (BM + 63) / 64; ++half) {
        qt_stage_c_half<BM>(acc, half, sm);
        __syncthreads();
        for (int r = wave; r < 64; r += 4) {
            const int row = 64 * half + r;
            if (row >= job.rows) break;
            hx_h2 h = {(_Float16)staged_value<CB>(sm, half, r, 2 * lane), (_Float16)staged_value<CB>(sm, half, r, 2 * lane + 1)};
            *reinterpret_cast<hx_h2*>(out + (size_t)row * g.N + 2 * lane) = h;
        }
        __syncthreads();
    }
}

// (column block, job) of this workgroup, in the XCD-aware order of xcd_group_index: all column
// blocks of a job on one XCD (they all read the job's A rows), the jobs round the XCDs in order.
HX_INLINE bool grouped_tile_index(int njobs, int& bx, int& job)
{
    return xcd_group_index(blockIdx.x + blockIdx.y * gridDim.x, gridDim.x, njobs, bx, job);
}

template <int CB>
__global__ __launch_bounds__(MF_THREADS, qt_occ<CB>()) void grouped_gemm_kernel(GroupedGemmArgs g)
{
    __shared__ MfmaSmemQ sm;
    int bx, job_i;
    if (!grouped_tile_index(*g.njobs, bx, job_i)) return;
    const Job job = g.jobs[job_i];
    const int ntiles = g.N / 128;
    const int proj = bx / ntiles;
    const int cg = bx % ntiles;
    const int bits = g.bits_tab[proj] ? g.bits_tab[proj][job.expert] : g.bits_uniform[proj];
#define HX_GG_CASE(B)                                                                      \
    case B:                                                                                \
        if (job.bm == 32) grouped_tile<B, CB, 32>(g, job, proj, cg, sm);                    \
        else if (job.bm == 64) grouped_tile<B, CB, 64>(g, job, proj, cg, sm);               \
        else if (job.bm == 96) grouped_tile<B, CB, 96>(g, job, proj, cg, sm);               \
        else grouped_tile<B, CB, MF_BM>(g, job, proj, cg, sm);                              \
        break;
    switch (bits) {
        HX_GG_CASE(1) HX_GG_CASE(2) HX_GG_CASE(3) HX_GG_CASE(4)
        HX_GG_CASE(5) HX_GG_CASE(6) HX_GG_CASE(7) HX_GG_CASE(8)
        default: break;
    }
#undef HX_GG_CASE
}

// ------------------------------------------------------------------ fused gate/up + SiLU-gate

struct GuArgs {
    const Job* jobs;
    const int* njobs;
    const _Float16* xg;  // [R][hidden] transformed gate inputs
    const _Float16* xu;
    const void* const* tr[2];
    const void* const* svh[2];
    const void* const* suh_d;
    const int32_t* bits_tab[2];
    int bits_uniform[2];
    int K, N;            // hidden, inter
    float act_limit;
    int act_fn;          // HX_ACT_SILU, HX_ACT_GELU or HX_ACT_RELU2_NOGATE (no gate GEMM)
    _Float16* act;       // [R][inter] down-projection inputs
    _Float16* g_scratch; // [R][inter] fp16 g of the tiles in flight (lane-grouped columns)
    const float* rs_g;   // [R][K / 128] row sums of xg, xu per 128-column block
    const float* rs_u;
    float* rs_act;       // [R][inter / 128] row sums of act per 128-column block
};

// accumulator of the gate/up tiles (quarter-operand layout); LDS: the tile's A buffers, reused as the
// staging block of the matrix-core Hadamard transforms (H128 itself is generated in registers)
template <int BM>
using GuAcc = hx_f4[BM / 16][2];
struct GuSmem {
    union {
        _Float16 ab[QT_NB][MF_BM * MF_LDA];
        _Float16 hx[128 * MF_LDA2];
    };
    float rowsum[MF_BM];
};

template <int BITS, int CB, int BM>
__device__ __forceinline__ void gu_tile(const _Float16* A, int K, int rows, const void* tr, int N, int cg,
                                        GuSmem& sm, GuAcc<BM>& acc, const float* rs)
{
    mfma_tile_q<BITS, CB, BM, QT_PF, true>(A, K, rows, static_cast<const uint32_t*>(tr), K, N, cg * 8, sm, acc, rs,
                                           K / 128);
}

template <int CB, int BM>
__device__ __forceinline__ void gu_tile_bits(int bits, const _Float16* A, int K, int rows, const void* tr, int N,
                                             int cg, GuSmem& sm, GuAcc<BM>& acc, const float* rs)
{
    switch (bits) {
        case 1: gu_tile<1, CB, BM>(A, K, rows, tr, N, cg, sm, acc, rs); break;
        case 2: gu_tile<2, CB, BM>(A, K, rows, tr, N, cg, sm, acc, rs); break;
        case 3: gu_tile<3, CB, BM>(A, K, rows, tr, N, cg, sm, acc, rs); break;
        case 4: gu_tile<4, CB, BM>(A, K, rows, tr, N, cg, sm, acc, rs); break;
        case 5: gu_tile<5, CB, BM>(A, K, rows, tr, N, cg, sm, acc, rs); break;
        case 6: gu_tile<6, CB, BM>(A, K, rows, tr, N, cg, sm, acc, rs); break;
        case 7: gu_tile<7, CB, BM>(A, K, rows, tr, N, cg, sm, acc, rs); break;
        default: gu_tile<8, CB, BM>(A, K, rows, tr, N, cg, sm, acc, rs); break;
    }
}

// Gate and up tiles of one (job, 128-column block), then the SiLU-gate and the down-projection input
// transform on the matrix cores (hadamard_inner.cuh:284-413 op order: G, U rounded to fp16, H,
// fp16, times svh in fp16, fp16 SiLU chain, clamps, times suh_d in fp16, H, fp16).
template <int CB, int BM>
__device__ __forceinline__ void gu_fused(const GuArgs& a, const Job& job, int cg, GuSmem& sm)
{
    constexpr int WM = BM / 2, MB = WM / 16;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int e = job.expert;
    const int bg = a.bits_tab[0] ? a.bits_tab[0][e] : a.bits_uniform[0];
    const int bu = a.bits_tab[1] ? a.bits_tab[1][e] : a.bits_uniform[1];
    _Float16* X = sm.hx;
    auto mapped = [&](int row, float v) -> float {
        if constexpr (CB == 2) return fmaf(v, CB2_SCALE, CB2_BIAS * sm.rowsum[row]);
        else return v;
    };

    GuAcc<BM> acc;
    hx_f4 hacc[MB][4];  // Hadamard results (the matrix-core transform's layout)
    const _Float16* svg = (a.act_fn != HX_ACT_RELU2_NOGATE) ? static_cast<const _Float16*>(a.svh[0][e]) + cg * 128 : nullptr;
    const _Float16* svu = static_cast<const _Float16*>(a.svh[1][e]) + cg * 128;
    const _Float16* sud = static_cast<const _Float16*>(a.suh_d[e]) + cg * 128;
    // g = fp16(H(G)) * svh_g is formed right after the gate tile and waits in global scratch (this
    // workgroup's rows and columns only; it stays in L2) while the up tile runs, which needs the
    // registers.  Scratch layout within a row's 128 columns: a lane's 4 values of the row
    // (columns 64 wn + 16 nb + c, nb = 0..3) sit together at 64 wn + 4 c, one 8-byte access each.
    _Float16* gs = a.g_scratch + (size_t)job.row0 * a.N + cg * 128;
    auto gs_at = [&](int row) { return gs + (size_t)row * a.N + 64 * wn + 4 * (lane & 15); };
    const bool gated = (a.act_fn != HX_ACT_RELU2_NOGATE);
    if (gated) {
        gu_tile_bits<CB, BM>(bg, a.xg + (size_t)job.row0 * a.K, a.K, job.rows, a.tr[0][e], a.N, cg, sm, acc,
                             a.rs_g + (size_t)job.row0 * (a.K / 128));
        // G = fp16(mapped sum), staged for the transform (the A buffers are free between tiles)
        qt_foreach<BM>(acc, [&](int row, int col, float v) { X[row * MF_LDA2 + col] = (_Float16)mapped(row, v); });
        __syncthreads();
        hadamard_mfma_reg<BM>(X, hacc);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = WM * wm + 16 * mb + 4 * (lane >> 4) + r;
                hx_h4 v;
#pragma unroll
                for (int nb = 0; nb < 4; ++nb) v[nb] = (_Float16)hacc[mb][nb][r] * svg[64 * wn + 16 * nb + (lane & 15)];
                if (row < job.rows) *reinterpret_cast<hx_h4*>(gs_at(row)) = v;
            }
        // X is free for the up tile's A buffers (the lanes read back only what they stored
        // themselves, in program order)
        __syncthreads();
    }
    gu_tile_bits<CB, BM>(bu, a.xu + (size_t)job.row0 * a.K, a.K, job.rows, a.tr[1][e], a.N, cg, sm, acc,
                         a.rs_u + (size_t)job.row0 * (a.K / 128));
    // g back from scratch, requested before the up tile's transform
    hx_h4 gv[MB][4];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = WM * wm + 16 * mb + 4 * (lane >> 4) + r;
            gv[mb][r] = hx_h4{(_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
            if (gated && row < job.rows) gv[mb][r] = *reinterpret_cast<const hx_h4*>(gs_at(row));
        }
    // u = fp16(H(U)) * svh_u, kept in registers
    qt_foreach<BM>(acc, [&](int row, int col, float v) { X[row * MF_LDA2 + col] = (_Float16)mapped(row, v); });
    __syncthreads();
    hadamard_mfma_reg<BM>(X, hacc);
    const float L = a.act_limit;
    const _Float16 Lh = (_Float16)L, nLh = (_Float16)(-L);
    __syncthreads();
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
        const int col = 64 * wn + 16 * nb + (lane & 15);
        const _Float16 su = svu[col], sd = sud[col];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = WM * wm + 16 * mb + 4 * (lane >> 4) + r;
                _Float16 g = gv[mb][r][nb];
                _Float16 uu = row < job.rows ? (_Float16)((_Float16)hacc[mb][nb][r] * su) : (_Float16)0.0f;
                g = hx_gate_act(a.act_fn, g, uu);
                if (L != 0.0f) {
                    uu = uu < nLh ? nLh : (uu > Lh ? Lh : uu);
                    g = g > Lh ? Lh : g;
                }
                X[row * MF_LDA2 + col] = (g * uu) * sd;
            }
    }
    __syncthreads();
    // act = fp16(H(p)), staged back to LDS for row-wise stores
    hadamard_mfma_reg<BM>(X, hacc);
    __syncthreads();
    acc_to_lds_f16<BM>(hacc, X, [](int, int, float v) { return v; });
    __syncthreads();
    _Float16* out = a.act + (size_t)job.row0 * a.N + cg * 128;
    const int nblk = a.N >> 7;
    for (int i = threadIdx.x; i < BM * 16; i += MF_THREADS) {
        const int row = i >> 4, c8 = (i & 15) * 8;
        const hx_h8 v = *reinterpret_cast<const hx_h8*>(&X[row * MF_LDA2 + c8]);
        if (row < job.rows) *reinterpret_cast<hx_h8*>(out + (size_t)row * a.N + c8) = v;
        // this block's part of the row sum of act (the down GEMM's codebook-2 map): 16 lanes per row
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) sum += (float)v[j];
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        sum += __shfl_xor(sum, 4, 64);
        sum += __shfl_xor(sum, 8, 64);
        if ((i & 15) == 0 && row < job.rows) a.rs_act[(size_t)(job.row0 + row) * nblk + cg] = sum;
    }
}

template <int CB>
__global__ __launch_bounds__(MF_THREADS, qt_occ<CB>()) void grouped_gu_kernel(GuArgs a)
{
    __shared__ GuSmem sm;
    int cg, job_i;
    if (!grouped_tile_index(*a.njobs, cg, job_i)) return;
    const Job job = a.jobs[job_i];
    if (job.bm == 32) gu_fused<CB, 32>(a, job, cg, sm);
    else if (job.bm == 64) gu_fused<CB, 64>(a, job, cg, sm);
    else if (job.bm == 96) gu_fused<CB, 96>(a, job, cg, sm);
    else gu_fused<CB, MF_BM>(a, job, cg, sm);
}

// ------------------------------------------------------------------ combine

// One wave per (token, 128-column block): contributions H(D[r]) * w / sqrt(128) . svh_d[e] in
// ascending routing rank from +0, then + shared, then fp16.
// One workgroup per token: the token's routes (sorted row, weight, down svh pointer) are staged in
// LDS once; a lane holds 8 consecutive values of a 128-block (16-byte loads), the routes' D blocks
// are loaded 8 at a time and added in routing-rank order (deterministic).
__global__ __launch_bounds__(256) void prefill_combine_kernel(const _Float16* D, const int64_t* r2s,
                                                             const int* row_expert, const _Float16* w_sorted,
                                                             const void* const* svh_d, int T, int topk, int hidden,
                                                             float* contrib, const float* shared_rows, _Float16* y,
                                                             float* y_routed, bool accumulate)
{
    constexpr int J = 8;  // routes loaded together
    __shared__ long rs[64];
    __shared__ float ws[64];
    __shared__ const _Float16* sv[64];
    const int t = blockIdx.x;
    if (threadIdx.x < topk) {
        const long r = r2s[(size_t)t * topk + threadIdx.x];
        rs[threadIdx.x] = r;
        ws[threadIdx.x] = (float)w_sorted[r];
        sv[threadIdx.x] = static_cast<const _Float16*>(svh_d[row_expert[r]]);
    }
    __syncthreads();
    for (int c = 8 * threadIdx.x; c < hidden; c += 8 * 256) {
        float acc[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] = 0.0f;
        for (int j0 = 0; j0 < topk; j0 += J) {
            hx_h8 dv[J];
#pragma unroll
            for (int i = 0; i < J; ++i)
                dv[i] = *reinterpret_cast<const hx_h8*>(D + (size_t)rs[min(j0 + i, topk - 1)] * hidden + c);
#pragma unroll
            for (int i = 0; i < J; ++i) {
                if (j0 + i >= topk) break;
                const hx_h8 sd = *reinterpret_cast<const hx_h8*>(sv[j0 + i] + c);
                float d[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) d[k] = (float)dv[i][k];
                hx_had128_x8(d);
                const float w = ws[j0 + i];
#pragma unroll
                for (int k = 0; k < 8; ++k) d[k] = d[k] * w * (float)sd[k];
                if (contrib) {
                    float* cp = contrib + (size_t)rs[j0 + i] * hidden + c;
                    *reinterpret_cast<float4*>(cp) = make_float4(d[0], d[1], d[2], d[3]);
                    *reinterpret_cast<float4*>(cp + 4) = make_float4(d[4], d[5], d[6], d[7]);
                }
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[k] += d[k];
            }
        }
        const size_t o = (size_t)t * hidden + c;
        if (y_routed) {
            float* yr = y_routed + o;
#pragma unroll
            for (int k = 0; k < 8; ++k) yr[k] = accumulate ? yr[k] + acc[k] : acc[k];
        }
        if (y) {
            hx_h8 out;
#pragma unroll
            for (int k = 0; k < 8; ++k) out[k] = (_Float16)(shared_rows ? acc[k] + shared_rows[o + k] : acc[k]);
            *reinterpret_cast<hx_h8*>(y + o) = out;
        }
    }
}

// The same reduction with the transforms on the matrix cores, for topk dividing 16: one wave per (16
// / topk tokens, 128-column block).  The wave's 16 A rows are the tokens' routes (sorted rows, rank
// order), multiplied by H128 (generated in registers) with fp32 accumulation; the results are staged
// in LDS and each lane then adds its columns over the routes in rank order (the order of
// prefill_combine_kernel and the reference's ordered reduction).
template <int TOPK, int KBC>
__global__ __launch_bounds__(256, 3) void prefill_combine_mfma_kernel(const _Float16* D, const int64_t* r2s,
                                                                      const int* row_expert, const _Float16* w_sorted,
                                                                      const void* const* svh_d, int T, int hidden,
                                                                      float* contrib, const float* shared_rows,
                                                                      _Float16* y, float* y_routed, bool accumulate)
{
    constexpr int TPW = 16 / TOPK;       // tokens per wave
    constexpr int LPT = 64 / TPW;        // lanes per token in the reduction
    constexpr int CPL = 128 / LPT;       // columns per lane in the reduction
    constexpr int SVW = CPL / 2;         // svh words per route and lane
    __shared__ float st[4][16][132];
    __shared__ long srow[4][16];
    __shared__ float sw_[4][16];
    __shared__ const _Float16* ssv[4][16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nblk = hidden >> 7, nchunk = (nblk + KBC - 1) / KBC;
    const long unit = (long)blockIdx.x * 4 + wave;
    const long tg = unit / nchunk;
    const int kb0 = (int)(unit % nchunk) * KBC;
    const long t0 = tg * TPW;
    if (t0 >= T) return;
    const int c = lane & 15, g = lane >> 4;
    const long t = min(t0 + c / TOPK, (long)T - 1);
    const long r = r2s[(size_t)t * TOPK + c % TOPK];
    // the routes' rows, weights and svh rows: looked up once for the wave's KBC column blocks
    if (g == 0) {
        srow[wave][c] = r;
        sw_[wave][c] = (float)w_sorted[r];
        ssv[wave][c] = static_cast<const _Float16*>(svh_d[row_expert[r]]);
    }
    const _Float16* dr = D + (size_t)r * hidden + 8 * g;
    auto load_d = [&](int kb, hx_h8 (&av)[4]) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) av[kk] = *reinterpret_cast<const hx_h8*>(dr + kb * 128 + 32 * kk);
    };
    const int tl = lane / LPT, col = (lane % LPT) * CPL;
    const long tok = t0 + tl;
    auto load_sv = [&](int kb, uint32_t (&sv)[TOPK][SVW]) {
#pragma unroll
        for (int j = 0; j < TOPK; ++j) {
            const uint32_t* p = reinterpret_cast<const uint32_t*>(ssv[wave][tl * TOPK + j] + kb * 128 + col);
#pragma unroll
            for (int w = 0; w < SVW; ++w) sv[j][w] = p[w];
        }
    };
    uint32_t f[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t s0 = __builtin_popcount(c & (2 * i) & 7) & 1, s1 = __builtin_popcount(c & (2 * i + 1) & 7) & 1;
        f[i] = (0x3c00u | (s0 << 15)) | ((0x3c00u | (s1 << 15)) << 16);
    }
    const uint32_t base = (uint32_t)((c >> 3) & g & 1);
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // D and svh of the next column block are requested before this one is transformed and reduced
    hx_h8 av[2][4];
    uint32_t sv[2][TOPK][SVW];
    load_d(kb0, av[0]);
    wave_sync();  // the route tables in LDS
    load_sv(kb0, sv[0]);
#pragma unroll
    for (int i = 0; i < KBC; ++i) {
        const int kb = kb0 + i;
        if (kb >= nblk) break;
        if (i + 1 < KBC && kb + 1 < nblk) {
            load_d(kb + 1, av[(i + 1) & 1]);
            load_sv(kb + 1, sv[(i + 1) & 1]);
        }
        hx_f4 yv[8];
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) yv[nb] = hx_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) {
                const uint32_t sgn = base ^ ((uint32_t)(nb & 1) & (uint32_t)(g >> 1)) ^
                                     (uint32_t)((nb >> 1) & kk & 1) ^ (uint32_t)((nb >> 2) & (kk >> 1) & 1);
                const uint32_t m = sgn ? 0x80008000u : 0u;
                typedef uint32_t u4v __attribute__((ext_vector_type(4)));
                const u4v bv = {f[0] ^ m, f[1] ^ m, f[2] ^ m, f[3] ^ m};
                yv[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i & 1][kk], __builtin_bit_cast(hx_h8, bv), yv[nb],
                                                                0, 0, 0);
            }
        if (i > 0) wave_sync();  // the previous block's reads of st are done
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) st[wave][4 * g + q][16 * nb + c] = yv[nb][q] * HX_RSQRT128;
        wave_sync();
        if (tok < T) {
            float acc[CPL];
#pragma unroll
            for (int k = 0; k < CPL; ++k) acc[k] = 0.0f;
#pragma unroll
            for (int j = 0; j < TOPK; ++j) {
                const int row = tl * TOPK + j;
                const float w = sw_[wave][row];
                float d[CPL];
#pragma unroll
                for (int k = 0; k < CPL; ++k) {
                    const hx_h2 s2 = u32_as_h2(sv[i & 1][j][k >> 1]);
                    d[k] = st[wave][row][col + k] * w * (float)s2[k & 1];
                }
                if (contrib) {
                    float* cp = contrib + (size_t)srow[wave][row] * hidden + kb * 128 + col;
#pragma unroll
                    for (int k = 0; k < CPL; ++k) cp[k] = d[k];
                }
#pragma unroll
                for (int k = 0; k < CPL; ++k) acc[k] += d[k];
            }
            const size_t o = (size_t)tok * hidden + kb * 128 + col;
            if (y_routed) {
                float* yr = y_routed + o;
#pragma unroll
                for (int k = 0; k < CPL; ++k) yr[k] = accumulate ? yr[k] + acc[k] : acc[k];
            }
            if (y) {
                _Float16 out[CPL];
#pragma unroll
                for (int k = 0; k < CPL; ++k) out[k] = (_Float16)(shared_rows ? acc[k] + shared_rows[o + k] : acc[k]);
#pragma unroll
                for (int w = 0; w < SVW; ++w)
                    reinterpret_cast<uint32_t*>(y + o)[w] = h2_as_u32(hx_h2{out[2 * w], out[2 * w + 1]});
            }
        }
    }
}

// Contributions only (no token reduction): one wave per (sorted row, 128-column block).
__global__ __launch_bounds__(256) void prefill_contrib_kernel(const _Float16* D, const int* row_expert,
                                                             const _Float16* w_sorted, const void* const* svh_d,
                                                             long blocks, int hidden, float* contrib)
{
    const int lane = threadIdx.x & 63;
    const long b = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= blocks) return;
    const int per = hidden / 128;
    const long r = b / per;
    const int c = (int)(b % per) * 128 + 2 * lane;
    const int e = row_expert[r];
    const hx_h2 dv = *reinterpret_cast<const hx_h2*>(D + (size_t)r * hidden + c);
    float d0 = (float)dv.x, d1 = (float)dv.y;
    hx_had128_wave(d0, d1);
    const float w = (float)w_sorted[r];
    const hx_h2 sd = *reinterpret_cast<const hx_h2*>(static_cast<const _Float16*>(svh_d[e]) + c);
    *reinterpret_cast<float2*>(contrib + (size_t)r * hidden + c) = make_float2(d0 * w * (float)sd.x, d1 * w * (float)sd.y);
}

// ------------------------------------------------------------------ driver

hipError_t run_moe_prefill(const PrefillArgs& p, float* contrib, const float* shared_rows, _Float16* y,
                           float* y_routed, bool accumulate, hipStream_t st)
{
    const MoeWs& L = *p.lay;
    char* ws = p.ws;
    Job* jobs = reinterpret_cast<Job*>(ws + L.off_jobs);
    int* njobs = reinterpret_cast<int*>(ws + L.off_njobs);
    int* row_expert = reinterpret_cast<int*>(ws + L.off_row_expert);
    _Float16* xg = reinterpret_cast<_Float16*>(ws + L.off_xg);
    _Float16* xu = reinterpret_cast<_Float16*>(ws + L.off_xu);
    _Float16* G = reinterpret_cast<_Float16*>(ws + L.off_G);
    _Float16* A = reinterpret_cast<_Float16*>(ws + L.off_A);
    _Float16* D = reinterpret_cast<_Float16*>(ws + L.off_D);
    float* rs_g = reinterpret_cast<float*>(ws + L.off_rs);
    float* rs_u = rs_g + (size_t)p.R * (p.hidden / 128);
    float* rs_act = rs_u + (size_t)p.R * (p.hidden / 128);
    if (p.E > 512) return hipErrorInvalidValue;

    hipLaunchKernelGGL(prefill_plan_kernel, dim3((unsigned)((p.R + 511) / 512)), dim3(512), 0, st, p.expert_count,
                       p.E, p.R, jobs, njobs, row_expert);
    if (p.R > 0)
        hipLaunchKernelGGL(prefill_gather_kernel, dim3((unsigned)((((long)p.R + 15) / 16 * (p.hidden / 128) + 3) / 4)),
                           dim3(256), 0, st, p.x, p.token_sorted,
                           row_expert, p.suh[0], p.suh[1], xg, xu, p.hidden, p.act_fn != HX_ACT_RELU2_NOGATE, rs_g, rs_u, (long)p.R);

    GuArgs gu{};
    gu.jobs = jobs;
    gu.njobs = njobs;
    gu.xg = xg;
    gu.xu = xu;
    gu.tr[0] = p.tr[0];
    gu.tr[1] = p.tr[1];
    gu.svh[0] = p.svh[0];
    gu.svh[1] = p.svh[1];
    gu.suh_d = p.suh[2];
    gu.bits_tab[0] = p.bits_tab[0];
    gu.bits_tab[1] = p.bits_tab[1];
    gu.bits_uniform[0] = p.bits_uniform[0];
    gu.bits_uniform[1] = p.bits_uniform[1];
    gu.K = p.hidden;
    gu.N = p.inter;
    gu.act_limit = p.act_limit;
    gu.act_fn = p.act_fn;
    gu.act = A;
    gu.g_scratch = G;
    gu.rs_g = rs_g;
    gu.rs_u = rs_u;
    gu.rs_act = rs_act;
    dim3 grid_gu(p.inter / 128, L.max_jobs);
    if (p.cb == 1) hipLaunchKernelGGL(grouped_gu_kernel<1>, grid_gu, dim3(MF_THREADS), 0, st, gu);
    else hipLaunchKernelGGL(grouped_gu_kernel<2>, grid_gu, dim3(MF_THREADS), 0, st, gu);

    GroupedGemmArgs d{};
    d.jobs = jobs;
    d.njobs = njobs;
    d.A[0] = A;
    d.out[0] = D;
    d.tr[0] = p.tr[2];
    d.bits_tab[0] = p.bits_tab[2];
    d.bits_uniform[0] = p.bits_uniform[2];
    d.K = p.inter;
    d.N = p.hidden;
    d.nproj = 1;
    d.rs[0] = rs_act;
    d.rs_n = p.inter / 128;
    dim3 grid_d(p.hidden / 128, L.max_jobs);
    if (p.cb == 1) hipLaunchKernelGGL(grouped_gemm_kernel<1>, grid_d, dim3(MF_THREADS), 0, st, d);
    else hipLaunchKernelGGL(grouped_gemm_kernel<2>, grid_d, dim3(MF_THREADS), 0, st, d);

    if (!y && !y_routed) {
        // contributions only: per sorted row, no route_to_sorted needed
        if (!contrib) return hipErrorInvalidValue;
        const long rblocks = (long)p.R * (p.hidden / 128);
        hipLaunchKernelGGL(prefill_contrib_kernel, dim3((unsigned)((rblocks + 3) / 4)), dim3(256), 0, st, D, row_expert,
                           p.weight_sorted, p.svh[2], rblocks, p.hidden, contrib);
        return hipGetLastError();
    }
    if (!p.r2s) return hipErrorInvalidValue;
    if (p.topk > 64) return hipErrorInvalidValue;
    if (p.T > 0 && (p.topk == 1 || p.topk == 2 || p.topk == 4 || p.topk == 8 || p.topk == 16)) {
        constexpr int KBC = 4;  // 128-column blocks per wave (the route lookups are paid once for them)
        const long units = ((long)p.T * p.topk + 15) / 16 * ((p.hidden / 128 + KBC - 1) / KBC);
        const dim3 grid((unsigned)((units + 3) / 4));
#define HX_CMB(K)                                                                                             \
    case K:                                                                                                   \
        hipLaunchKernelGGL((prefill_combine_mfma_kernel<K, KBC>), grid, dim3(256), 0, st, D, p.r2s, row_expert, \
                           p.weight_sorted, p.svh[2], p.T, p.hidden, contrib, shared_rows, y, y_routed, accumulate); \
        break;
        switch (p.topk) { HX_CMB(1) HX_CMB(2) HX_CMB(4) HX_CMB(8) HX_CMB(16) }
#undef HX_CMB
    } else if (p.T > 0) {
        hipLaunchKernelGGL(prefill_combine_kernel, dim3((unsigned)p.T), dim3(256), 0, st, D, p.r2s, row_expert,
                           p.weight_sorted, p.svh[2], p.T, p.topk, p.hidden, contrib, shared_rows, y, y_routed,
                           accumulate);
    }
    return hipGetLastError();
}

}  // namespace hx
