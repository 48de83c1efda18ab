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

namespace hx {

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

// Words q*BITS-1 .. q*BITS+BITS-1 (cyclic) of the tile at `tile`.
template <int BITS>
HX_INLINE void load_quarter(uint32_t* r, const uint32_t* tile, int q)
{
    constexpr int NW = 8 * BITS;
    hx_gu32* t = (hx_gu32*)tile;
    r[0] = __builtin_nontemporal_load(t + (q * BITS + NW - 1) % NW);
#pragma unroll
    for (int i = 0; i < BITS; ++i) r[i + 1] = __builtin_nontemporal_load(t + q * BITS + i);
}

// The 32 bits ending at local bit E of the quarter registers (bit 0 = local bit E-1).
template <int E>
HX_INLINE uint32_t quarter_reg(const uint32_t* r)
{
    constexpr int j = E >> 5, rr = E & 31;
    if constexpr (rr == 0) return r[j - 1];
    else return __builtin_amdgcn_alignbit(r[j - 1], r[j], 32 - rr);
}

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

template <int BITS, int CB, int P = 0>
HX_INLINE void quarter_decode_generic(const uint32_t* r, uint32_t* out)
{
    if constexpr (P < 32) {
        out[P / 2] = h2_as_u32(hx_decode2<CB>(quarter_reg<(P + 1) * BITS + 32>(r) & 0xffffu,
                                              quarter_reg<(P + 2) * BITS + 32>(r) & 0xffffu));
        quarter_decode_generic<BITS, CB, P + 2>(r, out);
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

// Decoded fp16 pairs of a quarter: out[i] = positions (2i, 2i+1) = (k, k+1) of one column.
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
            mul1_dec4(xs, out[o], out[o + 4], out[o + 8], out[o + 12]);
        }
    } else {
        quarter_decode_generic<BITS, CB>(r, out);
    }
}

// MFMA B operand (nh, kh) of a decoded quarter: column 8nh+q, k = 8kh + 0..7, i.e. local positions
// 2kh + 4nh + 8j + {0, 1} for j = 0..3.
template <int NH, int KH>
HX_INLINE hx_h8 quarter_operand(const uint32_t* d)
{
    constexpr int I0 = KH + 2 * NH;  // pair index of positions 2kh + 4nh
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    u4v v;
    v.x = d[I0];
    v.y = d[I0 + 4];
    v.z = d[I0 + 8];
    v.w = d[I0 + 12];
    return __builtin_bit_cast(hx_h8, v);
}

// Input transform of rows [0, M) over k in [k0, k0 + kc) into LDS as fp16:
//   a = fp16(H128(fp16(x . suh)))   (reference had_hf_r_128_inner<true,false>)
// When pre_transformed, x already holds a (copied as is).
HX_INLINE void input_to_lds(uint32_t* a_lds, const _Float16* x, const int* rows, const _Float16* suh, int M,
                            int K, int k0, int kc, bool pre_transformed)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int blocks = kc >> 7;
    for (int job = wave; job < M * blocks; job += GEMV_WAVES) {
        const int m = job / blocks, b = job % blocks;
        const int k = k0 + b * 128 + 2 * lane;
        const size_t row = rows ? (size_t)rows[m] : (size_t)m;
        uint32_t xv = *reinterpret_cast<const uint32_t*>(x + row * K + k);
        uint32_t out;
        if (pre_transformed) {
            out = xv;
        } else {
            hx_h2 s = *reinterpret_cast<const hx_h2*>(suh + k);
            hx_h2 p = u32_as_h2(xv) * s;
            float v0 = (float)p.x, v1 = (float)p.y;
            hx_had128_wave(v0, v1);
            hx_h2 r = {(_Float16)v0, (_Float16)v1};
            out = h2_as_u32(r);
        }
        a_lds[(m * kc + b * 128) / 2 + lane] = out;
    }
}

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
};

// This workgroup's (column group cg, split s) partial sum of the GEMV: on return colsum[m][c]
// (LDS fp32, MT x 128) holds sum over k in the split of a[m][k] * W[k][cg*128 + c].
// a_lds must hold MT * kc fp16.  MT <= 16.
template <int BITS, int CB, int MT>
__device__ void gemv_split_sum(const GemvArgs& g, int cg, int s, uint32_t* a_lds, float* colsum)
{
    static_assert(MT <= 16, "one MFMA holds 16 rows");
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int gq = lane >> 4;             // tile row within the 4-row step (MFMA k-group)
    const int t = (lane >> 3) & 1;        // tile column of the wave's pair
    const int q = lane & 7;               // quarter
    const int k0 = s * g.kc;
    const int kc = min(g.kc, g.K - k0);
    const int tiles_n = g.N >> 4;
    constexpr int NW = 8 * BITS;
    const uint32_t* tw = reinterpret_cast<const uint32_t*>(g.trellis);
    const int tn = cg * 8 + 2 * wave + t;

    // software pipeline: PF steps of tile words in flight.  The first PF are issued before the input
    // transform so their HBM latency overlaps it; every step then consumes one ring slot and refills
    // it PF steps ahead (past the end the load repeats the split's last tile row, so the number of
    // loads in flight is the same at every step and each wait is a static count).
    constexpr int PF = BITS <= 4 ? 8 : 4;
    const int steps = kc >> 6;
    uint32_t buf[PF][BITS + 1];
    const uint32_t* tcol = tw + (size_t)tn * NW;
    const size_t row_stride = (size_t)tiles_n * NW;
    const int tk0 = (k0 >> 4) + gq;
    const int tk_last = (k0 >> 4) + 4 * (steps - 1) + gq;
#pragma unroll
    for (int j = 0; j < PF; ++j) load_quarter<BITS>(buf[j], tcol + (size_t)min(tk0 + 4 * j, tk_last) * row_stride, q);

    input_to_lds(a_lds, g.x, g.rows, g.suh, g.M, g.K, k0, kc, g.pre_transformed);
    hx_lds_barrier();

    hx_f4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    const int am = min(lane & 15, g.M - 1);  // A row of this lane (rows >= M repeat the last row)
    const _Float16* arow = reinterpret_cast<const _Float16*>(a_lds) + (size_t)am * kc;
    for (int st0 = 0; st0 < steps; st0 += PF) {
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            const int st = st0 + j;
            uint32_t d[16];
            quarter_decode<BITS, CB>(buf[j], d);
            load_quarter<BITS>(buf[j], tcol + (size_t)min(tk0 + 4 * (st + PF), tk_last) * row_stride, q);
            if (st < steps) {
                const int kl = 64 * st + 16 * gq;
                const hx_h8 a0 = *reinterpret_cast<const hx_h8*>(arow + kl);
                const hx_h8 a1 = *reinterpret_cast<const hx_h8*>(arow + kl + 8);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, quarter_operand<0, 0>(d), acc0, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, quarter_operand<0, 1>(d), acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, quarter_operand<1, 0>(d), acc1, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, quarter_operand<1, 1>(d), acc1, 0, 0, 0);
            }
        }
    }

    // C: lane holds rows 4*(lane/16) + i of column label lane%16 = 8t + q; label -> column
    // 16*(2*wave + t) + 8*nh + q of the group
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * gq + i;
        if (m < MT && m < g.M) {
            colsum[m * 128 + 16 * (2 * wave + t) + q] = acc0[i];
            colsum[m * 128 + 16 * (2 * wave + t) + 8 + q] = acc1[i];
        }
    }
    __syncthreads();
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
    for (int i = threadIdx.x; i < MT * 128; i += GEMV_THREADS) {
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
    for (int i = threadIdx.x; i < MT * 128; i += GEMV_THREADS) {
        const int m = i >> 7, c = i & 127;
        float v = 0.0f;
        if (m < M)
            for (int sp = 0; sp < splits; ++sp)
                v += __hip_atomic_load(&partial[((size_t)sp * M + m) * N + cg * 128 + c], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        colsum[i] = v;
    }
    __syncthreads();
}

}  // namespace hx
