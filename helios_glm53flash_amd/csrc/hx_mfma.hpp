// hx_mfma.hpp -- EXL3 decode + MFMA tile core for gfx950 (M > 16 paths: the dense linear and the
// grouped expert GEMMs of the prefill), and the Hadamard-128 transform on the matrix cores.
//
// Workgroup = 4 waves, output tile BM x 128 (BM = 128, 64 or 32; 128 columns = one Hadamard block),
// K consumed in chunks of 64.  Each wave owns 32 output columns for all BM rows and decodes those
// columns' trellis words itself, straight into MFMA B operands (mfma_tile_q below); only A (the
// input-transformed activations) goes through LDS, one barrier per chunk: QT_PF chunks ahead, by
// buffer loads that write LDS directly (a ring of QT_NB buffers), or through registers where the
// tile sums A's rows itself.  The trellis words run QT_PT chunks ahead in a register ring.
// Codebook 2 is decoded in affine form (h = 1024 + bytesum, see hx_gemv.hpp): the tile computes
// sum_k a h, and the epilogue adds the map with per-row input sums (accumulated from the staged A, or
// precomputed by the caller).
// Operand layout of v_mfma_f32_16x16x32_f16 (64 lanes): A: lane l holds row l%16,
// k = 8*(l/16)..+7; B: column l%16, same k; C: column l%16, rows 4*(l/16)..+3.
#pragma once
#include "hx_gemv.hpp"

#include <utility>

namespace hx {

constexpr int MF_THREADS = 256;
constexpr int MF_BM = 128;  // largest row tile
constexpr int MF_BN = 128;
constexpr int MF_BK = 64;
constexpr int MF_SWZ = 2;  // LDS swizzle of the A operand rows (below)
// Operand rows of a chunk in LDS (64 halves of k each, 128-byte rows).  Swizzled layout: 16-byte chunk
// c of row r is stored at chunk c ^ f(r), f(r) = (r & 7) ^ ((r >> 3) & 1).  The fragment reads (16
// consecutive rows, one chunk) then touch 8 different 16-byte bank groups in every aligned group of
// 8 rows, and every even and every odd row of the 16 a different one, so they are conflict-free
// whether the LDS serves 8 or 16 lanes of a 16-byte access per cycle; a row's 8 chunk stores are
// conflict-free in any case.  (SWZ 1, f(r) = ((r >> 1) & 7) ^ (((r >> 4) & 1) << 2), suits only the
// 16-lane case and measured 1.3 % slower in the config-4 prefill; SWZ 0 pads rows to 72 halves.)
constexpr int MF_LDA = MF_SWZ ? MF_BK : MF_BK + 8;  // halves per LDS row
constexpr int MF_LDC = MF_BN + 4;  // floats per LDS row in the epilogue

// Chunk permutation of LDS row r (an XOR, so it is its own inverse: slot c of row r holds chunk
// c ^ mf_swz(r)).
HX_INLINE int mf_swz(int r)
{
    if constexpr (MF_SWZ == 2) return (r & 7) ^ ((r >> 3) & 1);
    else if constexpr (MF_SWZ) return ((r >> 1) & 7) ^ (((r >> 4) & 1) << 2);
    else return 0;
}

// Offset (halves) of 16-byte chunk c (8 halves of k) of LDS row r.
HX_INLINE int mf_off(int r, int c) { return r * MF_LDA + 8 * (c ^ mf_swz(r)); }

HX_INLINE __amdgpu_buffer_rsrc_t mf_rsrc(const void* base, size_t bytes)
{
    const uint64_t u = reinterpret_cast<uint64_t>(base);
    const uint64_t b = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(u >> 32)) << 32) |
                       (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)u);
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(b), 0,
                                             (int)(bytes > 0x7fffffffull ? 0x7fffffffull : bytes), 0x00020000);
}

// ---- quarter-operand tile: the decoded weights never leave the registers
//
// Each wave owns 32 columns (tile columns 2w, 2w+1) of the BM x 128 tile for all BM rows and
// decodes its own B: lane l = 16g + 8t + q decodes quarter
// q of the tile in row g (of the chunk's 4 tile rows) and column 2w + t, and the 32 decoded values
// are four MFMA B operands directly (quarter_operand<nh, kh>: column 8nh + q of tile t, k = 16g +
// 8kh + 0..7 of the chunk), as in the GEMV core.  The A fragment of operand (rb, kh) is therefore
// row 16rb + l%16, k = 16(l/16) + 8kh + 0..7.  Only A goes through LDS (stored once, read by the
// 4 waves); no wave decodes a weight another wave uses, and B costs no LDS traffic at all.
// Accumulator acc[rb][nh]: lane l holds rows 16rb + 4(l/16) + i, column 32w + 16t + 8nh + q.
template <int BM>
HX_INLINE void qt_rowcol(int rb, int nh, int i, int& row, int& col)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    row = 16 * rb + 4 * (lane >> 4) + i;
    col = 32 * wave + 16 * ((lane >> 3) & 1) + 8 * nh + (lane & 7);
}

// Chunks of global loads in flight for the quarter-operand tile (2 keeps it at 3 workgroups per CU):
// A chunks (QT_PF) and trellis-word chunks (QT_PT).
constexpr int QT_PF = 2;
constexpr int QT_PT = 2;
// The next chunk's decode runs after the chunk's MFMAs.  (Slicing it between the row blocks' MFMAs,
// so that one wave overlaps its own VALU and matrix work, measured equal on the config-4 prefill:
// 3.14 ms either way; the co-resident waves of a SIMD already overlap the two.)
// workgroups per CU the MFMA-tile kernels are compiled for (their register budget, 512 / QT_OCC
// VGPRs): codebook 2 (the affine decode) fits 168 at 3.  The generic decode of codebooks 0 and 1
// needs a few more registers, and at 3 the allocator spilled the accumulators themselves to scratch
// inside the chunk loop (dense linear 31-53 VGPRs, grouped gate/up 1573): the config-4 prefill with
// MCG experts ran 6.45 ms against 2.91 ms with mul1.  Those codebooks are compiled for 2.
constexpr int QT_OCC = 3;
template <int CB>
constexpr int qt_occ() { return CB == 2 ? QT_OCC : 2; }
// LDS A buffers: with A loaded straight into LDS, the chunks in flight and the one being read
constexpr int QT_NB = QT_PF + 1;
// s_waitcnt immediate that waits until at most n vector-memory instructions are outstanding
// (gfx9 encoding: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left at their no-wait maxima)
constexpr int qt_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
// 1: A by buffer loads that write LDS directly wherever the tile does not sum A's rows itself (those
// read A in registers); 0: always through registers and ds_write (measured 2 % slower, 32 more VGPRs)
constexpr int qt_lcm(int a, int b)
{
    int x = a, y = b;
    while (y) { const int r = x % y; x = y; y = r; }
    return a / x * b;
}

// LDS of a kernel that uses only quarter-operand tiles: the A buffers, the epilogue staging.
struct MfmaSmemQ {
    union {
        _Float16 ab[QT_NB][MF_BM * MF_LDA];
        float c[64 * MF_LDC];
    };
    float rowsum[MF_BM];
};

// XCD-aware renumbering of a grid of ngroups groups of nx workgroups (linear id i, groups of
// consecutive ids).  Workgroups are dispatched to the 8 XCDs round-robin by linear id; the
// renumbering gives all nx members of a group to one XCD, where they run at the same time and share
// that XCD's L2 for what they all read, while the groups still go round the XCDs in order (whole
// rounds of 8 groups; the rest as issued), so every XCD gets the same mix of groups.  Returns false
// for ids past the ngroups * nx real workgroups.
HX_INLINE bool xcd_group_index(int i, int nx, int ngroups, int& member, int& group)
{
    const int total = ngroups * nx;
    if (i >= total) return false;
    int l = i;
    constexpr int NXCD = 8;
    if (i < ngroups / NXCD * NXCD * nx) {
        const int x = i % NXCD, k = i / NXCD;  // k-th workgroup on XCD x: group x + 8 (k / nx)
        l = ((k / nx) * NXCD + x) * nx + k % nx;
    }
    member = l % nx;
    group = l / nx;
    return true;
}

// With rs_src (codebook 2), the row sums of A come precomputed as rs_n fp32 partial sums per row
// (rs_src[r * rs_n + b]) instead of being accumulated from the staged A.
template <int BITS, int CB, int BM, int PF = QT_PF, bool EXT_RS = false, class Smem>
__device__ __forceinline__ void mfma_tile_q(const _Float16* A, long lda, int rows, const uint32_t* trellis, int K,
                                            int N, int tn0, Smem& sm, hx_f4 (&acc)[BM / 16][2],
                                            const float* rs_src = nullptr, int rs_n = 0)
{
    static_assert(BM == 32 || BM == 64 || BM == 96 || BM == 128, "row tile");
    constexpr int RB = BM / 16;
    constexpr int NA = BM / 32;   // 16-byte A loads per thread per chunk
    constexpr int NW = 8 * BITS;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int tiles_n = N >> 4;
#pragma unroll
    for (int i = 0; i < RB; ++i) acc[i][0] = acc[i][1] = hx_f4{0.f, 0.f, 0.f, 0.f};

    const __amdgpu_buffer_rsrc_t ra = mf_rsrc(A, (size_t)max(rows, 0) * lda * sizeof(_Float16));
    const __amdgpu_buffer_rsrc_t rt = mf_rsrc(trellis, (size_t)(K >> 4) * tiles_n * NW * 4);
    int a_voff[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int idx = t + MF_THREADS * i;
        a_voff[i] = (int)(((idx >> 3) * lda + 8 * (idx & 7)) * sizeof(_Float16));
    }
    const int g = lane >> 4, tq = (lane >> 3) & 1, q = lane & 7;
    const int t_off = ((g * tiles_n + tn0 + 2 * wave + tq) * NW) * 4;
    const int voff = t_off + q * BITS * 4;
    const int row_bytes = tiles_n * NW * 4;

    // A and the trellis words have rings of their own: PF chunks of A (16 VGPRs per chunk at BM 128),
    // PT chunks of trellis words (BITS + 1 VGPRs per chunk)
    constexpr int PT = QT_PT;
    // A through LDS by DMA, unless the tile sums A's rows itself (that reads A in registers)
    constexpr bool DMA = EXT_RS || CB != 2;
    static_assert(!DMA || (MF_LDA == MF_BK && PF + 1 <= QT_NB), "A ring in LDS");
    hx_u4v av[DMA ? 1 : PF][NA];
    uint32_t wv[PT][BITS + 1];
    float rs[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) rs[i] = 0.0f;
    auto load_a = [&](int slot, int k0) {
#pragma unroll
        for (int i = 0; i < NA; ++i) av[slot][i] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_voff[i], k0 * 2, 0);
    };
    auto load_t = [&](int slot, int k0) { load_quarter_buf<BITS>(wv[slot], rt, voff, (k0 >> 4) * row_bytes); };
    // A straight into LDS (buffer loads with an LDS destination): instruction i of wave w fills rows
    // 32i + 8w .. +7 of the buffer, lane l 16 bytes at slot l % 8 of row 32i + 8w + l / 8, so the lane
    // fetches the chunk that the swizzle puts in that slot.  Rows past the tile's end read zeros (the
    // buffer resource's range).  The loads use no registers, so with DMA A has QT_NB LDS buffers and
    // no register ring.
    int a_voff_lds[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int r = 32 * i + 8 * wave + (lane >> 3);
        a_voff_lds[i] = (int)(((size_t)r * lda + 8 * ((lane & 7) ^ mf_swz(r))) * sizeof(_Float16));
    }
    // the LDS destination is wave-uniform (it goes to M0): derived from a scalar wave index, it is
    // computed on the scalar unit instead of a v_readfirstlane per load
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    auto load_a_lds = [&](int buf, int k0) {
#pragma unroll
        for (int i = 0; i < NA; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void*)(&sm.ab[buf][(32 * i + 8 * wave_s) * MF_LDA]), 16,
                a_voff_lds[i], k0 * 2, 0, 0);
    };
    auto store_a = [&](int slot, int buf, bool count) {
        _Float16* as = sm.ab[buf];
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int idx = t + MF_THREADS * i;
            *reinterpret_cast<hx_u4v*>(&as[mf_off(idx >> 3, idx & 7)]) = av[slot][i];
            if (CB == 2 && !EXT_RS && count) {
                const hx_h2 one = {(_Float16)1.0f, (_Float16)1.0f};
                float s = rs[i];
                s = __builtin_amdgcn_fdot2(u32_as_h2(av[slot][i].x), one, s, false);
                s = __builtin_amdgcn_fdot2(u32_as_h2(av[slot][i].y), one, s, false);
                s = __builtin_amdgcn_fdot2(u32_as_h2(av[slot][i].z), one, s, false);
                s = __builtin_amdgcn_fdot2(u32_as_h2(av[slot][i].w), one, s, false);
                rs[i] = s;
            }
        }
    };
    auto decode = [&](int slot, uint32_t* d) {
        quarter_wrap<BITS>(wv[slot]);
        if constexpr (CB == 2) quarter_affine<BITS>(wv[slot], d);
        else quarter_decode<BITS, CB>(wv[slot], d);
    };

    const int nk = K / MF_BK;
#pragma unroll
    for (int s = 0; s < (PF > PT ? PF : PT); ++s) {
        if (s < PF) {
            if constexpr (DMA) load_a_lds(s, min(s, nk - 1) * MF_BK);
            else load_a(s, min(s, nk - 1) * MF_BK);
        }
        if (s < PT) load_t(s, min(s, nk - 1) * MF_BK);
    }
    // row t's precomputed sum, requested while the first chunks are in flight (32 independent
    // loads per round trip: one round trip for K up to 4096)
    float rs_ext = 0.0f;
    if constexpr (CB == 2 && EXT_RS) {
        if (t < BM && t < rows)
            for (int b0 = 0; b0 < rs_n; b0 += 32) {
                float v[32];
#pragma unroll
                for (int j = 0; j < 32; ++j) v[j] = b0 + j < rs_n ? rs_src[(size_t)t * rs_n + b0 + j] : 0.0f;
#pragma unroll
                for (int j = 0; j < 32; ++j) rs_ext += v[j];
            }
    }
    // VMEM instructions per chunk: A (DMA) and trellis words; chunk c + 1's A is complete once at
    // most the loads of the PF - 1 later chunks are outstanding (their order within a step is left
    // to the compiler, so the count takes whole chunks)
    constexpr int NT = quarter_buf_vmem(BITS);  // load_t = one load_quarter_buf
    constexpr int A_WAIT = (PF - 1) * (NA + NT);
    static_assert(!DMA || A_WAIT < 64, "vmcnt range");
    // chunk 0: the prologue issued at most the other chunks' loads after it
    if constexpr (DMA) __builtin_amdgcn_s_waitcnt(qt_vmcnt((PF - 1) * NA + (PT - 1) * NT));
    else store_a(0, 0, true);
    // d holds the decoded quarter of the current chunk; the next chunk's quarter is decoded into it
    // after the chunk's MFMAs (their B operands are read before the decode overwrites it)
    constexpr int ND = 1;
    uint32_t d[ND][16];
    decode(0, d[0]);
    hx_lds_barrier();
    // step c: ua = c % PF, ut = c % PT, par = c & 1, all compile-time in the unrolled loops
    auto step = [&](int c, auto ua_, auto ut_, auto par_) {
        constexpr int ua = decltype(ua_)::value, ut = decltype(ut_)::value, par = decltype(par_)::value;
        if constexpr (DMA) load_a_lds((c + PF) % QT_NB, min(c + PF, nk - 1) * MF_BK);
        else load_a(ua, min(c + PF, nk - 1) * MF_BK);
        load_t(ut, min(c + PT, nk - 1) * MF_BK);
        const _Float16* as = sm.ab[DMA ? c % QT_NB : c & 1];
        const uint32_t* dc = d[par % ND];
        uint32_t* dn = d[(par + 1) % ND];
        const hx_h8 b00 = quarter_operand<0, 0>(dc), b01 = quarter_operand<0, 1>(dc);
        const hx_h8 b10 = quarter_operand<1, 0>(dc), b11 = quarter_operand<1, 1>(dc);
        auto read_a = [&](int rb, hx_h8& a0, hx_h8& a1) {
            const int r = 16 * rb + (lane & 15);
            a0 = *reinterpret_cast<const hx_h8*>(&as[mf_off(r, 2 * g)]);
            a1 = *reinterpret_cast<const hx_h8*>(&as[mf_off(r, 2 * g + 1)]);
        };
        auto mfma_ab = [&](int rb, const hx_h8& a0, const hx_h8& a1) {
            acc[rb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b00, acc[rb][0], 0, 0, 0);
            acc[rb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b10, acc[rb][1], 0, 0, 0);
            acc[rb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b01, acc[rb][0], 0, 0, 0);
            acc[rb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b11, acc[rb][1], 0, 0, 0);
        };
        auto mfma_rb = [&](int rb) {
            hx_h8 a0, a1;
            read_a(rb, a0, a1);
            mfma_ab(rb, a0, a1);
        };
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) mfma_rb(rb);
        decode((ut + 1) % PT, dn);
        if constexpr (DMA) __builtin_amdgcn_s_waitcnt(qt_vmcnt(A_WAIT));
        else store_a((ua + 1) % PF, (c + 1) & 1, c + 1 < nk);
        hx_lds_barrier();
    };
    // unrolled period: every ring position and the parity are compile-time constants
    constexpr int PER = qt_lcm(qt_lcm(PF, PT), 2);
    const int nmain = nk - nk % PER;
    for (int c0 = 0; c0 < nmain; c0 += PER) {
        [&]<int... U>(std::integer_sequence<int, U...>) {
            (step(c0 + U, std::integral_constant<int, U % PF>{}, std::integral_constant<int, U % PT>{},
                  std::integral_constant<int, U & 1>{}), ...);
        }(std::make_integer_sequence<int, PER>{});
    }
    [&]<int... U>(std::integer_sequence<int, U...>) {
        ((nmain + U < nk ? step(nmain + U, std::integral_constant<int, U % PF>{},
                                std::integral_constant<int, U % PT>{}, std::integral_constant<int, U & 1>{})
                         : void()), ...);
    }(std::make_integer_sequence<int, PER - 1>{});
    if constexpr (DMA) {
        // the clamped loads past the last chunk still write LDS: drain them before it is reused
        __builtin_amdgcn_s_waitcnt(qt_vmcnt(0));
        hx_lds_barrier();
    }
    if constexpr (CB == 2 && EXT_RS) {
        if (t < BM) sm.rowsum[t] = rs_ext;
        __syncthreads();
    } else if constexpr (CB == 2) {
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            float s = rs[i];
            s += __shfl_xor(s, 1, 64);
            s += __shfl_xor(s, 2, 64);
            s += __shfl_xor(s, 4, 64);
            if ((t & 7) == 0) sm.rowsum[(t + MF_THREADS * i) >> 3] = s;
        }
        __syncthreads();
    }
}

// Calls f(row, col, value) for every accumulator element of a quarter-operand tile.
template <int BM, class F>
HX_INLINE void qt_foreach(const hx_f4 (&acc)[BM / 16][2], F f)
{
#pragma unroll
    for (int rb = 0; rb < BM / 16; ++rb)
#pragma unroll
        for (int nh = 0; nh < 2; ++nh)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int row, col;
                qt_rowcol<BM>(rb, nh, i, row, col);
                f(row, col, acc[rb][nh][i]);
            }
}

// Stage rows [64*half, 64*half + 64) of a quarter-operand tile to LDS (sm.c[row - 64*half][col]).
template <int BM, class Smem>
HX_INLINE void qt_stage_c_half(const hx_f4 (&acc)[BM / 16][2], int half, Smem& sm)
{
#pragma unroll
    for (int rb = 0; rb < BM / 16; ++rb) {
        if (16 * rb >= 64 * half && 16 * rb < 64 * half + 64) {
#pragma unroll
            for (int nh = 0; nh < 2; ++nh)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    int row, col;
                    qt_rowcol<BM>(rb, nh, i, row, col);
                    sm.c[(row - 64 * half) * MF_LDC + col] = acc[rb][nh][i];
                }
        }
    }
}

// Staged value of tile row r (within the half) and column c, with the codebook-2 map applied.
template <int CB, class Smem>
HX_INLINE float staged_value(const Smem& sm, int half, int r, int c)
{
    const float v = sm.c[r * MF_LDC + c];
    if constexpr (CB == 2) return fmaf(v, CB2_SCALE, CB2_BIAS * sm.rowsum[64 * half + r]);
    else return v;
}

}  // namespace hx

namespace hx {

// ---- Hadamard-128 on the matrix cores
//
// Y = X . H128 / sqrt(128) for BM rows of a 128-column block staged in LDS as fp16 (row-major,
// leading dimension MF_LDA2): H128[k][n] = (-1)^popcount(k & n) is exact in fp16 and symmetric, and
// the products are exact in fp32, so this equals the reference's fp32 butterfly up to the order of
// the fp32 additions.  The result lands in the GEMM's accumulator layout (wave (wm, wn) holds rows
// BM/2*wm + 16*mb + 4*(lane/16) + i, columns 64*wn + 16*nb + lane%16).
constexpr int MF_LDA2 = 128 + 8;  // halves per row of a staged 128-column block

// fp16 of a float accumulator tile into X (row-major, MF_LDA2): X[row][col] = fp16(f(row, col, v)).
template <int BM, class F>
HX_INLINE void acc_to_lds_f16(const hx_f4 (&acc)[BM / 32][4], _Float16* x, F f)
{
    constexpr int WM = BM / 2, MB = WM / 16;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = WM * wm + 16 * mb + 4 * (lane >> 4) + r, col = 64 * wn + 16 * nb + (lane & 15);
                x[row * MF_LDA2 + col] = (_Float16)f(row, col, acc[mb][nb][r]);
            }
}

// H128 is generated in registers: for B operand
// (nb, kk) lane l holds n = 64wn + 16nb + c (c = l % 16) and k = kk + 8g + j (g = l / 16, j < 8),
// so popcount(n & k) mod 2 = popcount(c & j & 7) + (c3 g0) + (nb0 g1) + (nb1 kk5) + (wn kk6): a fixed
// per-lane fragment F (the j-dependent part) times a per-lane sign for each (nb, kk), applied as an
// XOR of the fp16 sign bits.
template <int BM>
HX_INLINE void hadamard_mfma_reg(const _Float16* x, hx_f4 (&y)[BM / 32][4])
{
    constexpr int WM = BM / 2, MB = WM / 16;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int c = lane & 15, g = lane >> 4;
    uint32_t f[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t s0 = __builtin_popcount(c & (2 * i) & 7) & 1, s1 = __builtin_popcount(c & (2 * i + 1) & 7) & 1;
        f[i] = (0x3c00u | (s0 << 15)) | ((0x3c00u | (s1 << 15)) << 16);
    }
    const uint32_t base = (uint32_t)(((c >> 3) & g) & 1);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) y[mb][nb] = hx_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 128; kk += 32) {
        hx_h8 af[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
            af[mb] = *reinterpret_cast<const hx_h8*>(&x[(WM * wm + 16 * mb + (lane & 15)) * MF_LDA2 + kk + 8 * g]);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
            const uint32_t sgn = base ^ ((uint32_t)(nb & 1) & (uint32_t)(g >> 1)) ^ (uint32_t)((nb >> 1) & (kk >> 5) & 1) ^
                                 (uint32_t)(wn & (kk >> 6) & 1);
            const uint32_t m = sgn ? 0x80008000u : 0u;
            typedef uint32_t u4v __attribute__((ext_vector_type(4)));
            const u4v bv = {f[0] ^ m, f[1] ^ m, f[2] ^ m, f[3] ^ m};
            const hx_h8 bf = __builtin_bit_cast(hx_h8, bv);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                y[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[mb], bf, y[mb][nb], 0, 0, 0);
        }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) y[mb][nb] = y[mb][nb] * HX_RSQRT128;
}

}  // namespace hx
