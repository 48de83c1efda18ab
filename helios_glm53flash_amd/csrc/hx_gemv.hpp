// hx_gemv.hpp -- small-M (M <= 16) EXL3 GEMV core for gfx950: trellis decode on VALU feeding
// v_mfma_f32_16x16x32_f16, fp32 accumulation.
//
// Work split: one workgroup (4 waves) owns one 128-column group (8 tile columns, one Hadamard
// block of the output) and one K-split range; wave w owns tile columns 2w and 2w+1 and walks the
// range 4 tile rows (64 k) per step.  Lane l = 16*g + 8*t + q decodes quarter q (positions
// 32q..32q+31, i.e. columns q and q+8 of all 16 k) of the tile in row g, column t of the step.
// Those windows all live in tile words [q*bits - 1, q*bits + bits), so each lane loads bits+1
// words and every window is a compile-time funnel shift of its registers (two windows per
// alignbit when bits divides 16).  The 32 decoded fp16 form four MFMA B operands: operand
// (nh, kh) holds column 8nh+q, k = 8kh..8kh+7 of the lane's tile, so the 64 lanes give a 32(k) x
// 16(n) B block whose k-group is the tile row g; the A operand (the transformed activations, rows
// = tokens) comes from LDS.  Codebook decode costs the VALU; the MAC is on the matrix cores and is
// free for any M <= 16.
//
// K-split partials are reduced deterministically: each split writes its 128 x M partial sum to a
// workspace slot and bumps a per-column-group counter; the last arriving workgroup sums the
// splits in split order and runs the output epilogue (Hadamard + scales) for those 128 columns.
// The counter is reset by that workgroup, so the workspace stays reusable without clearing.
#pragma once
#include "hx_device.hpp"
#include <type_traits>

namespace hx {

// Tile-word steps in flight per wave in the dense linear, up to 4 bits / wider.  Fewer steps in
// flight shorten the memory queue that every workgroup's dependent loads (inputs, partial sums,
// arrival counters) wait behind: config 2 (4096 -> 12288, 4-bit) at M = 1 measured 15.6 us with
// 8 steps, 13.9 with 4, 13.4 with 2; the 5-bit lm_head (stream-K, row steps) 96.7-98.3 us with 2,
// 98.0-98.7 with 3, 99.1-99.5 with 4, 122 with 6 (one box, three runs each).
constexpr int LIN_PF = 2;   // up to 4 bits
constexpr int LIN_PFW = 2;  // wider

// Stream-K for one row over more than 1024 column groups that do not spread evenly over the 256 CUs
// (the lm_head, 4096 -> 151552: 1184 groups; one workgroup per group put 4 or 5 on a CU, and the CUs
// with 4 went idle while those with 5 finished): 1024 workgroups (4 on every CU) take equal runs
// of the (column group, 128-k block) units.  lm_head in a graph of 20 calls on one box: 101-104 ->
// 96 us; 2048 workgroups: no gain.  A grid already even over the CUs (K = 16384 -> 32768, 2-bit:
// 4 splits, 1024 workgroups) measured 2 us slower as stream-K, and small linears are bound by their
// chain of dependent steps, not by the work.
constexpr int GEMV_SK_WGS = 1024;
constexpr int GEMV_CUS = 256;
constexpr int GEMV_THREADS = 256;
constexpr int GEMV_WAVES = 4;

// K per split: the largest divisor of K that is a multiple of 128 and at most `cap`, so that a
// workgroup's fixed costs (input transform, split-K handoff) are amortised over many tile rows.
inline int gemv_kc_for(int K, int cap)
{
    int best = 128;
    for (int c = 128; c <= cap && c <= K; c += 128)
        if (K % c == 0) best = c;
    return best;
}

typedef const __attribute__((address_space(1))) uint32_t hx_gu32;

// A lane decodes quarter q of a 16x16 tile from the tile's words q*BITS-1 .. q*BITS+BITS-1 (cyclic;
// NW = 8*BITS words per tile), held in r[0..BITS].  Only words q*BITS .. q*BITS+BITS-1 are loaded,
// through a buffer resource: the per-lane byte offset is fixed for a whole range and the step moves
// only the scalar offset, so a step's loads cost no vector ALU address arithmetic, and a read past
// the tensor's end (num_records) returns zeros instead of faulting.  The first word is the last
// word of quarter q-1, which the neighbouring lane loaded (quarter_wrap).
typedef unsigned int hx_u2 __attribute__((ext_vector_type(2)));
typedef unsigned int hx_u3 __attribute__((ext_vector_type(3)));
typedef unsigned int hx_u4v __attribute__((ext_vector_type(4)));
constexpr int HX_BUF_NT = 2;  // nontemporal: the tile words are read once

template <int N>
HX_INLINE void buf_words(uint32_t* r, __amdgpu_buffer_rsrc_t rs, int voff, int soff)
{
    if constexpr (N >= 4) {
        const hx_u4v v = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, HX_BUF_NT);
        r[0] = v.x, r[1] = v.y, r[2] = v.z, r[3] = v.w;
        if constexpr (N > 4) buf_words<N - 4>(r + 4, rs, voff + 16, soff);
    } else if constexpr (N == 3) {
        const hx_u3 v = __builtin_amdgcn_raw_buffer_load_b96(rs, voff, soff, HX_BUF_NT);
        r[0] = v.x, r[1] = v.y, r[2] = v.z;
    } else if constexpr (N == 2) {
        const hx_u2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff, HX_BUF_NT);
        r[0] = v.x, r[1] = v.y;
    } else if constexpr (N == 1) {
        r[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff, HX_BUF_NT);
    }
}

// VMEM instructions that load_quarter_buf issues: the BITS words in 16-byte pieces (buf_words).  Waits that count loads in flight (the MFMA tile's
// s_waitcnt on its LDS-DMA ring) take their per-chunk count from here.  Each piece is its own
// buffer-load builtin with its own offset register, so the compiler cannot merge pieces into fewer
// instructions (which would make a counted wait too short).
constexpr int quarter_buf_vmem(int bits) { return (bits + 3) / 4; }

// r[1..BITS] = words q*BITS .. q*BITS+BITS-1 of the lane's tile (voff: their byte offset).
template <int BITS>
HX_INLINE void load_quarter_buf(uint32_t* r, __amdgpu_buffer_rsrc_t rs, int voff, int soff)
{
    buf_words<BITS>(r + 1, rs, voff, soff);
}

// r[0] = word q*BITS-1 (cyclic) of the tile, once r[1..BITS] have arrived in every lane of the wave.
// The 8 quarters of a tile are decoded by 8 consecutive lanes (q = lane & 7), so the word is r[BITS]
// of lane q-1, or of lane q+7 for q = 0: a rotation of each 16-lane row by 1 or by 9 (DPP
// row_ror, lane i reads lane (i - n) mod 16 of its row).  A separate load of that word cost as much
// memory throughput as the quarter's own words (a loads-only stream of the lm_head: 115 us with it,
// 83 us without).  Every lane of the wave must be active.
template <int BITS>
HX_INLINE void quarter_wrap(uint32_t* r)
{
    const int w = (int)r[BITS];
    const uint32_t prev = (uint32_t)__builtin_amdgcn_mov_dpp(w, 0x121, 0xf, 0xf, false);  // row_ror:1
    const uint32_t last = (uint32_t)__builtin_amdgcn_mov_dpp(w, 0x129, 0xf, 0xf, false);  // row_ror:9
    r[0] = (threadIdx.x & 7) ? prev : last;
}

// The 32 bits ending at local bit E of the quarter registers (bit 0 = local bit E-1).
template <int E>
HX_INLINE uint32_t quarter_reg(const uint32_t* r)
{
    constexpr int j = E >> 5, rr = E & 31;
    if constexpr (rr == 0) return r[j - 1];
    else return __builtin_amdgcn_alignbit(r[j - 1], r[j], 32 - rr);
}

// Register slot of decoded pair i of a quarter (positions 2i, 2i+1): operand-major, so that the
// four pairs of each MFMA B operand (quarter_operand) sit in consecutive registers.
HX_INLINE constexpr int qpos(int i) { return 4 * (i & 3) + (i >> 2); }

// x = window * 0x83DCD12D mod 2^32 for four 16-bit windows: the low and high halves of ra and rb
// (hi = true) or the low halves of ra, rb, rc, rd (hi = false).  Each product is one
// v_pk_mul_lo_u16 making (w * 0x83DC) << 16 and one v_mad_u32_u16 adding w * 0xD12D (both full-rate
// ops that read only the 16 window bits; v_mul_lo_u32 is quarter rate and would need a masked
// window).  Four products per block keep every dependent pair four instructions apart.
HX_INLINE void mul1_x4_pairs(uint32_t ra, uint32_t rb, uint32_t& x0, uint32_t& x1, uint32_t& x2, uint32_t& x3)
{
    asm("v_pk_mul_lo_u16 %0, %4, %6 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %1, %4, %6 op_sel:[1,0] op_sel_hi:[1,1]\n\t"
        "v_pk_mul_lo_u16 %2, %5, %6 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %3, %5, %6 op_sel:[1,0] op_sel_hi:[1,1]\n\t"
        "v_mad_u32_u16 %0, %4, %7, %0\n\t"
        "v_mad_u32_u16 %1, %4, %7, %1 op_sel:[1,0,0,0]\n\t"
        "v_mad_u32_u16 %2, %5, %7, %2\n\t"
        "v_mad_u32_u16 %3, %5, %7, %3 op_sel:[1,0,0,0]"
        : "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3)
        : "v"(ra), "v"(rb), "s"(0x83dc0000u), "s"(0xd12du));
}

HX_INLINE void mul1_x4_lo(uint32_t ra, uint32_t rb, uint32_t rc, uint32_t rd, uint32_t& x0, uint32_t& x1,
                          uint32_t& x2, uint32_t& x3)
{
    asm("v_pk_mul_lo_u16 %0, %4, %8 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %1, %5, %8 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %2, %6, %8 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %3, %7, %8 op_sel_hi:[0,1]\n\t"
        "v_mad_u32_u16 %0, %4, %9, %0\n\t"
        "v_mad_u32_u16 %1, %5, %9, %1\n\t"
        "v_mad_u32_u16 %2, %6, %9, %2\n\t"
        "v_mad_u32_u16 %3, %7, %9, %3"
        : "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3)
        : "v"(ra), "v"(rb), "v"(rc), "v"(rd), "s"(0x83dc0000u), "s"(0xd12du));
}

// Positions whose window is the low half of a register that also carries position q - D in its high
// half (D = 16 / BITS): the q with (q mod 2D) >= D, in increasing order.
template <int BITS>
struct QuarterRegs {
    static constexpr int D = (16 % BITS == 0) ? 16 / BITS : 0;
    static constexpr int at(int i)
    {
        int n = 0;
        for (int q = 0; q < 32; ++q)
            if (D != 0 && q % (2 * D) >= D) {
                if (n == i) return q;
                ++n;
            }
        return -1;
    }
};

// x of all 32 local positions of a quarter (codebook 2); the window of local position P ends at
// local bit (P+1)*BITS + 32.
template <int BITS, int G = 0>
HX_INLINE void quarter_mul1(const uint32_t* r, uint32_t* x)
{
    constexpr int D = QuarterRegs<BITS>::D;
    if constexpr (D != 0) {
        if constexpr (G < 8) {  // 16 registers, two per block
            constexpr int qa = QuarterRegs<BITS>::at(2 * G), qb = QuarterRegs<BITS>::at(2 * G + 1);
            mul1_x4_pairs(quarter_reg<(qa + 1) * BITS + 32>(r), quarter_reg<(qb + 1) * BITS + 32>(r), x[qa],
                          x[qa - D], x[qb], x[qb - D]);
            quarter_mul1<BITS, G + 1>(r, x);
        }
    } else {
        if constexpr (G < 8) {  // 32 registers, four per block
            constexpr int p = 4 * G;
            mul1_x4_lo(quarter_reg<(p + 1) * BITS + 32>(r), quarter_reg<(p + 2) * BITS + 32>(r),
                       quarter_reg<(p + 3) * BITS + 32>(r), quarter_reg<(p + 4) * BITS + 32>(r), x[p], x[p + 1],
                       x[p + 2], x[p + 3]);
            quarter_mul1<BITS, G + 1>(r, x);
        }
    }
}

// Window of local position P of a quarter: it ends at local bit E = (P+1)*BITS + 32 (MSB first);
// M[j] = the 32 bits ending at local bit 32j + 16, for windows across words j-1 and j.
template <int BITS, int P>
HX_INLINE uint32_t quarter_window(const uint32_t* r, const uint32_t* M)
{
    constexpr int E = (P + 1) * BITS + 32;
    constexpr int j = E >> 5, rr = E & 31;
    if constexpr (rr == 0) return __builtin_amdgcn_ubfe(r[j - 1], 0, 16);
    else if constexpr (rr >= 16) return __builtin_amdgcn_ubfe(r[j], 32 - rr, 16);
    else return __builtin_amdgcn_ubfe(M[j], 16 - rr, 16);
}

// Codebooks 0 and 1: each pair from its two windows (one v_bfe_u32 each, as in the affine decode).
template <int BITS, int CB, int P = 0>
HX_INLINE void quarter_decode_generic(const uint32_t* r, const uint32_t* M, uint32_t* out)
{
    if constexpr (P < 32) {
        out[qpos(P / 2)] = h2_as_u32(hx_decode2<CB>(quarter_window<BITS, P>(r, M), quarter_window<BITS, P + 1>(r, M)));
        quarter_decode_generic<BITS, CB, P + 2>(r, M, out);
    }
}

// Codebook-2 fp16 pairs from eight products x0..x7: pair j = (x_2j, x_2j+1).  h = fp16(0x6400 +
// bytesum(x)) = 1024 + s exactly (s <= 1020, so no carry into the other half); v_sad_u8 against 0
// is the byte sum, and v_sad_hi_u8 adds the second byte sum into the high half directly, so a pair
// costs two ops.  v = fma(h, 0x1eee, 0xc931) rounded once (codebook.cuh:77-90).
HX_INLINE void mul1_dec4(const uint32_t* x, uint32_t& d0, uint32_t& d1, uint32_t& d2, uint32_t& d3)
{
    uint32_t h[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) h[j] = __builtin_amdgcn_sad_u8(x[2 * j], 0u, 0x64006400u);
#pragma unroll
    for (int j = 0; j < 4; ++j) h[j] = __builtin_amdgcn_sad_hi_u8(x[2 * j + 1], 0u, h[j]);
    const hx_h2 c1 = u32_as_h2(0x1eee1eeeu), c0 = u32_as_h2(0xc931c931u);
    d0 = h2_as_u32(__builtin_elementwise_fma(u32_as_h2(h[0]), c1, c0));
    d1 = h2_as_u32(__builtin_elementwise_fma(u32_as_h2(h[1]), c1, c0));
    d2 = h2_as_u32(__builtin_elementwise_fma(u32_as_h2(h[2]), c1, c0));
    d3 = h2_as_u32(__builtin_elementwise_fma(u32_as_h2(h[3]), c1, c0));
}

// Decoded fp16 pairs of a quarter: out[qpos(i)] = positions (2i, 2i+1) = (k, k+1) of one column.
template <int BITS, int CB>
HX_INLINE void quarter_decode(const uint32_t* r, uint32_t* out)
{
    if constexpr (CB == 2) {
        uint32_t x[32];
        quarter_mul1<BITS>(r, x);
#pragma unroll
        for (int o = 0; o < 4; ++o) {  // the pairs of MFMA operand o: pair indices o, o+4, o+8, o+12
            const uint32_t xs[8] = {x[2 * o], x[2 * o + 1], x[2 * o + 8], x[2 * o + 9],
                                    x[2 * o + 16], x[2 * o + 17], x[2 * o + 24], x[2 * o + 25]};
            mul1_dec4(xs, out[4 * o], out[4 * o + 1], out[4 * o + 2], out[4 * o + 3]);
        }
    } else {
        uint32_t M[BITS + 1];
#pragma unroll
        for (int j = 1; j <= BITS; ++j) M[j] = __builtin_amdgcn_alignbit(r[j - 1], r[j], 16);
        quarter_decode_generic<BITS, CB>(r, M, out);
    }
}

// ---- codebook 2 in affine form
//
// The cb2 weight is v = fp16(h * S + B) with h = fp16(0x6400 + bytesum(w * 0x83DCD12D)) = 1024 + s
// and S = fp16 0x1eee, B = fp16 0xc931 (codebook.cuh:77-90).  The GEMV feeds h itself to the matrix
// cores and applies the map once per output: sum_k a_k (h_k S + B) = S sum_k a_k h_k + B sum_k a_k.
// This drops one rounding per weight (|v - (hS + B)| <= 2^-10, against outputs that are sums of
// thousands of terms) and the fma per weight pair.  A window costs one v_bfe_u32 (one v_alignbit_b32
// per word more for the windows that straddle two words) and one v_mul_lo_u32 (full rate on gfx950),
// and a pair of products one v_sad_u8 + one v_sad_hi_u8, which leave h as packed fp16 directly.
constexpr float CB2_SCALE = 0.00676727294921875f;  // fp16 0x1eee
constexpr float CB2_BIAS = -10.3828125f;           // fp16 0xc931

template <int BITS, int P = 0>
HX_INLINE void quarter_affine_pairs(const uint32_t* r, const uint32_t* M, uint32_t* out)
{
    if constexpr (P < 32) {
        const uint32_t x0 = quarter_window<BITS, P>(r, M) * 0x83DCD12Du;
        const uint32_t x1 = quarter_window<BITS, P + 1>(r, M) * 0x83DCD12Du;
        out[qpos(P / 2)] = __builtin_amdgcn_sad_hi_u8(x1, 0u, __builtin_amdgcn_sad_u8(x0, 0u, 0x64006400u));
        quarter_affine_pairs<BITS, P + 2>(r, M, out);
    }
}

// h of a quarter as fp16 pairs: out[qpos(i)] = positions (2i, 2i+1) = (k, k+1) of one column.
template <int BITS>
HX_INLINE void quarter_affine(const uint32_t* r, uint32_t* out)
{
    uint32_t M[BITS + 1];
#pragma unroll
    for (int j = 1; j <= BITS; ++j) M[j] = __builtin_amdgcn_alignbit(r[j - 1], r[j], 16);
    quarter_affine_pairs<BITS>(r, M, out);
}

// MFMA B operand (nh, kh) of a decoded quarter: column 8nh+q, k = 8kh + 0..7, i.e. local positions
// 2kh + 4nh + 8j + {0, 1} for j = 0..3: pairs I0 + 4j, I0 = kh + 2nh, stored at out[4 I0 + j] (qpos),
// so an operand is four consecutive registers and needs no moves.
template <int NH, int KH>
HX_INLINE hx_h8 quarter_operand(const uint32_t* d)
{
    constexpr int I0 = KH + 2 * NH;
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    u4v v;
    v.x = d[4 * I0];
    v.y = d[4 * I0 + 1];
    v.z = d[4 * I0 + 2];
    v.w = d[4 * I0 + 3];
    return __builtin_bit_cast(hx_h8, v);
}

// Input transform of rows [0, M) over k in [k0, k0 + kc) into LDS as fp16:
//   a = fp16(H128(fp16(x . suh)))   (reference had_hf_r_128_inner<true,false>)
// When pre_transformed, x already holds a (copied as is, read with device-coherent loads because
// another workgroup of the same launch may have produced it).
//
// Job j (row m, 128-wide block b) is done by wave j % 4.  The loads of a wave's first IN_PRE jobs are
// issued separately (input_issue) so that a caller can put them ahead of the tile prefetch: the
// vector-memory counter completes in issue order, so an input load issued after the prefetch would
// make the transform wait for every prefetched tile.
constexpr int IN_PRE = 4;

struct InputRegs {
    uint32_t xv[IN_PRE];
    uint32_t sv[IN_PRE];
};

HX_INLINE uint32_t input_word(const _Float16* x, const int* rows, int M, int K, int k0, int blocks, int job, int lane,
                              bool pre_transformed)
{
    const int m = job / blocks, b = job % blocks;
    const int k = k0 + b * 128 + 2 * lane;
    const size_t row = rows ? (size_t)rows[m] : (size_t)m;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(x + row * K + k);
    if (pre_transformed) return __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return *(hx_gu32*)src;
}

HX_INLINE void input_issue(InputRegs& r, const _Float16* x, const int* rows, const _Float16* suh, int M, int K, int k0,
                           int kc, bool pre_transformed)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int blocks = kc >> 7;
#pragma unroll
    for (int i = 0; i < IN_PRE; ++i) {
        const int job = wave + hx_nwaves() * i;
        r.xv[i] = 0;
        r.sv[i] = 0;
        if (job < M * blocks) {
            r.xv[i] = input_word(x, rows, M, K, k0, blocks, job, lane, pre_transformed);
            if (!pre_transformed)
                r.sv[i] = *(hx_gu32*)(suh + k0 + (job % blocks) * 128 + 2 * lane);
        }
    }
}

HX_INLINE uint32_t input_transform(uint32_t xv, uint32_t sv, bool pre_transformed)
{
    if (pre_transformed) return xv;
    hx_h2 p = u32_as_h2(xv) * u32_as_h2(sv);
    float v0 = (float)p.x, v1 = (float)p.y;
    hx_had128_wave(v0, v1);
    hx_h2 r = {(_Float16)v0, (_Float16)v1};
    return h2_as_u32(r);
}

// The input transform of up to 16 rows at once on the matrix cores: per 128-k block, the rows'
// fp16(x . suh) (rows >= M zero) times H128 as one 16 x 128 by 128 x 128 product, H generated in
// registers (sign of (n, k) = popcount(n & k) & 1: a fixed per-lane fragment times one sign per
// operand), fp32 accumulation of the exact +-products, one fp16 rounding after the 1/sqrt(128)
// scale.  The same values as the butterfly (hx_had128_wave) up to the order of the fp32 additions;
// for several rows it replaces a wave-wide butterfly per row and block with 32 MFMAs per block.
// Lane l: A row l % 16, k = 32 kk + 8 (l / 16) + 0..7; C rows 4 (l / 16) + i, column 16 nb + l % 16.
HX_INLINE void input_mfma(uint32_t* a_lds, const _Float16* x, const int* rows, const _Float16* suh, int M, int K,
                          int k0, int kc, int ld = -1)
{
    if (ld < 0) ld = kc;  // row stride of the LDS rows (fp16)
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c = lane & 15, g = lane >> 4;
    const int blocks = kc >> 7;
    uint32_t f[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t s0 = __builtin_popcount(c & (2 * i) & 7) & 1, s1 = __builtin_popcount(c & (2 * i + 1) & 7) & 1;
        f[i] = (0x3c00u | (s0 << 15)) | ((0x3c00u | (s1 << 15)) << 16);
    }
    const uint32_t base = (uint32_t)((c >> 3) & g & 1);
    const bool live = c < M;
    const _Float16* xr = x + (live ? (rows ? (size_t)rows[c] : (size_t)c) : 0) * K + 8 * g;
    _Float16* al = reinterpret_cast<_Float16*>(a_lds);
    for (int b = wave; b < blocks; b += hx_nwaves()) {
        const int kb = k0 + b * 128;
        hx_h8 av[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const hx_h8 sv = *reinterpret_cast<const hx_h8*>(suh + kb + 32 * kk + 8 * g);
            hx_h8 xv = {};
            if (live) xv = *reinterpret_cast<const hx_h8*>(xr + kb + 32 * kk);
            av[kk] = xv * sv;
        }
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
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * g + i;
            if (m < M) {
#pragma unroll
                for (int nb = 0; nb < 8; ++nb) al[m * ld + b * 128 + 16 * nb + c] = (_Float16)(y[nb][i] * HX_RSQRT128);
            }
        }
    }
}

// Transform and store all jobs: the first IN_PRE per wave from r, the rest loaded here.
HX_INLINE void input_finish(uint32_t* a_lds, const InputRegs& r, const _Float16* x, const int* rows,
                            const _Float16* suh, int M, int K, int k0, int kc, bool pre_transformed)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int blocks = kc >> 7;
#pragma unroll
    for (int i = 0; i < IN_PRE; ++i) {
        const int job = wave + hx_nwaves() * i;
        if (job < M * blocks) {
            const int m = job / blocks, b = job % blocks;
            a_lds[(m * kc + b * 128) / 2 + lane] = input_transform(r.xv[i], r.sv[i], pre_transformed);
        }
    }
    for (int job = wave + hx_nwaves() * IN_PRE; job < M * blocks; job += hx_nwaves()) {
        const int m = job / blocks, b = job % blocks;
        const uint32_t xv = input_word(x, rows, M, K, k0, blocks, job, lane, pre_transformed);
        const uint32_t sv =
            pre_transformed ? 0u : *(hx_gu32*)(suh + k0 + b * 128 + 2 * lane);
        a_lds[(m * kc + b * 128) / 2 + lane] = input_transform(xv, sv, pre_transformed);
    }
}

struct NoHook {
    HX_INLINE void operator()() const {}
};

struct GemvArgs {
    const _Float16* x;       // M x K fp16 (or pre-transformed a)
    const int* rows;         // optional row gather: row m of the input is x[rows[m]]
    const uint16_t* trellis; // (K/16, N/16, 16*bits)
    const _Float16* suh;     // K
    int M, K, N;
    int splits;              // K splits
    int kc;                  // K per split (multiple of 128)
    float* partial;          // [splits][M][N] fp32 (unused when splits == 1)
    int* counter;            // [N/128] (unused when splits == 1)
    bool pre_transformed;
    int sk_blocks;           // stream-K: (column group, 128-k block) units in all (0: split-K grid)
};

// LDS scratch of gemv_range: one array per (N, KS), shared by every instantiation of a kernel (a
// __shared__ array inside gemv_range would be allocated once per bit width in mixed-width kernels).
template <int N, int KS>
__device__ __forceinline__ float* gemv_lds()
{
    __shared__ float buf[N * KS];
    return buf;
}

// This workgroup's partial sum of the GEMV over k in [k0, k0 + kc) (kc a multiple of 128): on
// return colsum[m][c] (LDS fp32, MT x 128) holds sum over that range of a[m][k] * W[k][cg*128 + c].
// a_lds must hold MT * kc fp16.  MT <= 16.
//
// KS = 1: 4 waves, wave w owns tile columns 2w, 2w+1 over the whole range.  KS = 4: 16 waves, wave w
// owns tile columns 2(w%4), 2(w%4)+1 over the 128-k blocks j = w/4, w/4 + 4, ... of the range, and
// the four partial sums of a column pair are added in block-subset order through LDS.
//
// ROW (one row, KS = 1): a step of a wave covers ONE tile row of all 8 tiles of the group instead of
// 4 tile rows of 2 tiles, and wave w takes tile rows w, w+4, w+8, ... of the range.  Lane 16p + 8t + q
// then decodes quarter q of tile 2p + t, so a step's loads cover the group's whole tile row
// contiguously (a loads-only stream of the lm_head, 5-bit: 73 us against 83 us for the 4-row step).
// The matrix cores still sum over the four 8-k groups of an MFMA; with one row the groups are kept
// apart through A: row i of A holds the input only in k group i (lanes with lane % 16 == lane / 16),
// zeros elsewhere, so output row p of the MFMA is tile pair p's sum.  The four waves' sums are added
// in wave order through LDS.
//
// before_input() runs after the tile prefetch is issued and before a pre-transformed input is read
// (a consumer waits there for its producer); after_input() runs once the input is in LDS.
// PF4 / PFW: steps of tile words in flight per wave for bit widths up to 4 / wider.
template <int BITS, int CB, int MT, int KS = 1, int PF4 = 8, int PFW = 4, bool ROW = false, class Before = NoHook,
          class After = NoHook>
__device__ __forceinline__ void gemv_range(const GemvArgs& g, int cg, int k0, int kc, uint32_t* a_lds, float* colsum,
                                           Before before_input = Before(), After after_input = After())
{
    static_assert(MT <= 16, "one MFMA holds 16 rows");
    static_assert(KS == 1 || KS == 2 || KS == 4, "k subsets");
    static_assert(!ROW || (MT == 1 && KS == 1), "row steps: one row, no k subsets");
    constexpr bool AFFINE = CB == 2;
    float* asum = gemv_lds<MT, 1>();  // sum of the transformed input over the range, per row (cb2)
    float* kpart = gemv_lds<MT * 128, ROW ? 4 : KS>();
    // wave index as a uniform (scalar) value: the step offsets below stay in SGPRs
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    // tile-column pair of this lane: the wave's (row steps: the lane group's)
    const int pair = ROW ? (lane >> 4) : KS == 1 ? wave : (wave & 3);
    const int ks = KS == 1 ? 0 : (wave >> 2);  // block subset of this wave
    const int gq = ROW ? 0 : (lane >> 4);      // tile row within the 4-row step (MFMA k-group)
    const int t = (lane >> 3) & 1;             // tile column of the pair
    const int q = lane & 7;                    // quarter
    const int tiles_n = g.N >> 4;
    constexpr int NW = 8 * BITS;
    const uint32_t* tw = reinterpret_cast<const uint32_t*>(g.trellis);
    const int tn = cg * 8 + 2 * pair + t;
    const int nblk = kc >> 7;
    // this wave's steps: step s covers k = k0 + 128 * (ks + KS * (s / 2)) + 64 * (s % 2) (row steps:
    // the 16 k of tile row wave + 4s); kc is a multiple of 128, so every wave has kc / 64 row steps
    const int steps = KS == 1 ? (kc >> 6) : 2 * max(0, (nblk - ks + KS - 1) / KS);
    auto step_k = [&](int st) {  // relative to k0
        return ROW ? 16 * (wave + 4 * st) : 128 * (ks + KS * (st >> 1)) + 64 * (st & 1);
    };

    // software pipeline: PF steps of tile words in flight.  The first PF are issued before the input
    // transform (after the input loads themselves) so their HBM latency overlaps it; every step then
    // consumes one ring slot and refills it PF steps ahead (past the end the load repeats the range's
    // last tile row, so the number of loads in flight is the same at every step and each wait is a
    // static count).
    constexpr int PF = BITS <= 4 ? PF4 : PFW;
    uint32_t buf[PF][BITS + 1];
    // byte offsets: lane part (tile row gq of the step, tile column tn, quarter q) and step part
    // (tile rows (k0 + step_k) / 16); the tensor is (K/16) x (N/16) tiles
    // the base is uniform: state it, or every buffer load gets a loop over the lanes' descriptors
    // (readfirstlane returns int: each half goes through uint32_t so the low half is not sign-extended)
    const uint64_t twu = reinterpret_cast<uint64_t>(tw);
    const uint64_t twb = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(twu >> 32)) << 32) |
                         (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)twu);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void*>(twb), 0, (int)min((size_t)0x7fffffff, (size_t)(g.K >> 4) * tiles_n * NW * 4),
        0x00020000);
    const int lane_off = ((gq * tiles_n + tn) * NW) * 4;
    const int voff = lane_off + q * BITS * 4;
    const int row_bytes = tiles_n * NW * 4;
    auto soff = [&](int st) { return ((k0 + step_k(min(st, steps - 1))) >> 4) * row_bytes; };
    InputRegs in;
    // several rows: the transform on the matrix cores (its loads are issued there)
    constexpr bool MF_IN = MT >= 4;
    if (!g.pre_transformed && !MF_IN) input_issue(in, g.x, g.rows, g.suh, g.M, g.K, k0, kc, false);
    if (steps > 0) {
#pragma unroll
        for (int j = 0; j < PF; ++j) load_quarter_buf<BITS>(buf[j], rs, voff, soff(j));
    }

    before_input();
    if (g.pre_transformed) input_issue(in, g.x, g.rows, g.suh, g.M, g.K, k0, kc, true);
    if (MF_IN && !g.pre_transformed) input_mfma(a_lds, g.x, g.rows, g.suh, g.M, g.K, k0, kc);
    else input_finish(a_lds, in, g.x, g.rows, g.suh, g.M, g.K, k0, kc, g.pre_transformed);
    hx_lds_barrier();
    after_input();
    if constexpr (AFFINE) {
        for (int m = wave; m < g.M && m < MT; m += hx_nwaves()) {
            const _Float16* row = reinterpret_cast<const _Float16*>(a_lds) + (size_t)m * kc;
            float v = 0.0f;
            for (int k = lane; k < kc; k += 64) v += (float)row[k];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
            if (lane == 0) asum[m] = v;
        }
    }

    hx_f4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    const int am = min(lane & 15, g.M - 1);  // A row of this lane
    // Only the lanes whose A row carries input read it from LDS; the others keep zero operands, so
    // a read moves 16 bytes per input row and k group instead of 1 KB per wave: with row steps the
    // lanes on the A diagonal, else (MT > 1) the lanes of rows < M (rows >= M of the product are not
    // used).  With MT = 1 and 4-row steps (the MoE decode layer's one-token units) every lane reads:
    // the read's exec-mask branch in each step made that layer slower (47.0 against 46.0-46.5 us).
    const bool diag = (lane & 15) == (lane >> 4);
    const bool a_reads = ROW ? diag : (MT == 1 || (lane & 15) < g.M);
    const _Float16* arow = reinterpret_cast<const _Float16*>(a_lds) + (size_t)am * kc;
    hx_h8 a0 = {}, a1 = {};
    // one group of PF steps; GUARD: the group runs past the range (only the last group can)
    auto group = [&](int st0, auto guard) {
        constexpr bool GUARD = decltype(guard)::value;
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            const int st = st0 + j;
            // progress-based wave priority: a wave entering a group of PF steps outranks the waves
            // of its SIMD that are further into theirs, so co-resident waves advance at the same
            // rate instead of the oldest first (a starved wave would hold back every workgroup that
            // waits for its range)
            if (j == 0) HX_SETPRIO(3);
            if (j == PF / 4) HX_SETPRIO(2);
            if (j == PF / 2) HX_SETPRIO(1);
            if (j == 3 * PF / 4) HX_SETPRIO(0);
            // the decode of a slot past the range is skipped (a range that is not a multiple of PF
            // steps would otherwise decode the repeated last row); every refill is issued (past the
            // range it repeats the last row, an L2 hit), so that the count of loads in flight, and
            // so every wait, is the same at every step
            const bool live = !GUARD || st < steps;
            uint32_t d[16];
            if (live) {
                quarter_wrap<BITS>(buf[j]);
                if constexpr (AFFINE) quarter_affine<BITS>(buf[j], d);
                else quarter_decode<BITS, CB>(buf[j], d);
            }
            load_quarter_buf<BITS>(buf[j], rs, voff, soff(st + PF));
            if (live) {
                const int kl = step_k(st) + 16 * gq;
                if (a_reads) {
                    a0 = *reinterpret_cast<const hx_h8*>(arow + kl);
                    a1 = *reinterpret_cast<const hx_h8*>(arow + kl + 8);
                }
                acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, quarter_operand<0, 0>(d), acc0, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, quarter_operand<0, 1>(d), acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, quarter_operand<1, 0>(d), acc1, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, quarter_operand<1, 1>(d), acc1, 0, 0, 0);
            }
            // keeps each step's decode after the previous step's refill: the scheduler does not see
            // the memory wait a decode implies, and one hoisted into an earlier step waits there for
            // every load in flight
            if (j + 1 < PF) __builtin_amdgcn_sched_barrier(0);
        }
    };
    // whole groups run without per-step branches, so each group is one block
    int st0 = 0;
    for (; st0 + PF <= steps; st0 += PF) group(st0, std::false_type{});
    if (st0 < steps) group(st0, std::true_type{});

    HX_SETPRIO(3);  // the split-K handoff and epilogues are on the critical path
    // C: lane holds rows 4*(lane/16) + i of column label lane%16 = 8t + q; label -> column
    // 16*(2*pair + t) + 8*nh + q of the group
    if constexpr (ROW) {
        // lanes 0..15 hold output rows 0..3 = the sums of tile pairs 0..3 (column label 8t + q)
        if (lane < 16) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                kpart[wave * 128 + 16 * (2 * i + t) + q] = acc0[i];
                kpart[wave * 128 + 16 * (2 * i + t) + 8 + q] = acc1[i];
            }
        }
        hx_lds_barrier();
        for (int i = threadIdx.x; i < 128; i += hx_nthreads()) {
            float v = ((kpart[i] + kpart[128 + i]) + kpart[256 + i]) + kpart[384 + i];
            if constexpr (AFFINE) v = fmaf(v, CB2_SCALE, CB2_BIAS * asum[0]);
            colsum[i] = v;
        }
    } else if constexpr (KS > 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * gq + i;
            if (m < MT && m < g.M) {
                kpart[(ks * MT + m) * 128 + 16 * (2 * pair + t) + q] = acc0[i];
                kpart[(ks * MT + m) * 128 + 16 * (2 * pair + t) + 8 + q] = acc1[i];
            }
        }
        hx_lds_barrier();
        for (int i = threadIdx.x; i < MT * 128; i += hx_nthreads()) {
            const int m = i >> 7;
            if (m < g.M) {
                float v = kpart[i];
#pragma unroll
                for (int sub = 1; sub < KS; ++sub) v += kpart[sub * MT * 128 + i];
                if constexpr (AFFINE) v = fmaf(v, CB2_SCALE, CB2_BIAS * asum[m]);
                colsum[i] = v;
            }
        }
    } else {
        if constexpr (AFFINE) hx_lds_barrier();  // asum of every row is in LDS
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * gq + i;
            if (m < MT && m < g.M) {
                float c0 = acc0[i], c1 = acc1[i];
                if constexpr (AFFINE) {
                    const float b = CB2_BIAS * asum[m];
                    c0 = fmaf(c0, CB2_SCALE, b);
                    c1 = fmaf(c1, CB2_SCALE, b);
                }
                colsum[m * 128 + 16 * (2 * pair + t) + q] = c0;
                colsum[m * 128 + 16 * (2 * pair + t) + 8 + q] = c1;
            }
        }
    }
    hx_lds_barrier();  // colsum is complete (LDS only: the repeated-row refills still in flight need no wait)
}

// Split s of K in chunks of g.kc (the last may be shorter).
template <int BITS, int CB, int MT, class Before = NoHook, class After = NoHook>
__device__ __forceinline__ void gemv_split_sum(const GemvArgs& g, int cg, int s, uint32_t* a_lds, float* colsum,
                                               Before before_input = Before(), After after_input = After())
{
    const int k0 = s * g.kc;
    gemv_range<BITS, CB, MT, 1, LIN_PF, LIN_PFW, MT == 1>(g, cg, k0, min(g.kc, g.K - k0), a_lds, colsum, before_input,
                                                   after_input);
}

// Cross-workgroup handoff of split-K partials.  An agent-scope release/acquire fence pair would
// write back and invalidate the whole L2 of the XCD on every arrival, which costs tens of
// microseconds per launch at thousands of workgroups.  Instead the partials themselves are
// device-coherent (agent-scope atomic stores and loads bypass the non-coherent cache levels), the
// workgroup waits for its stores to complete before it counts its arrival, and the arrival counter
// is a device-scope atomic.

// Store this split's partial (rows < M) to partial[s][m][cg*128 + c].
template <int MT>
HX_INLINE void publish_partial(float* partial, int M, int N, int cg, int s, const float* colsum)
{
    for (int i = threadIdx.x; i < MT * 128; i += hx_nthreads()) {
        const int m = i >> 7, c = i & 127;
        if (m < M)
            __hip_atomic_store(&partial[((size_t)s * M + m) * N + cg * 128 + c], colsum[i], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Count this workgroup's arrival after its device-coherent stores completed; true for the last of
// `target` arrivals, which also resets the counter for the next call.
__device__ inline bool arrive_last(int* counter, int target)
{
    __shared__ int last;
    __builtin_amdgcn_s_waitcnt(0);  // every outstanding memory operation of this wave has completed
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = (old == target - 1);
        if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return last;
}

// colsum[m][c] = sum over splits (in split order) of partial[s][m][cg*128 + c].
template <int MT>
HX_INLINE void gather_partials(const float* partial, int M, int N, int splits, int cg, float* colsum)
{
    // the loads of 8 splits are issued together, then added in split order
    constexpr int B = 8;
    for (int i = threadIdx.x; i < MT * 128; i += hx_nthreads()) {
        const int m = i >> 7, c = i & 127;
        float v = 0.0f;
        if (m < M) {
            const float* p = partial + (size_t)m * N + cg * 128 + c;
            const size_t stride = (size_t)M * N;
            for (int s0 = 0; s0 < splits; s0 += B) {
                float t[B];
#pragma unroll
                for (int j = 0; j < B; ++j)
                    t[j] = __hip_atomic_load(p + (size_t)min(s0 + j, splits - 1) * stride, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                for (int j = 0; j < B; ++j)
                    if (s0 + j < splits) v += t[j];
            }
        }
        colsum[i] = v;
    }
    __syncthreads();
}

}  // namespace hx
