// hx_gemv.hpp -- small-M (M <= 8) EXL3 GEMV core for gfx950.
//
// Work split: one workgroup (4 waves, 256 lanes) owns one 128-column group (8 tile columns, one
// Hadamard block of the output) and one K-split range.  Inside a wave, lane = 8*ks + tc: lane
// decodes whole 16x16 tiles (tile column tc, tile row ks of an 8-row step) straight from the
// tile words it loaded into registers: every window is one alignbit/bfe on registers, never
// a shuffle.  Positions p, p+1 are the (k, k+1) pair of one column, so each decoded fp16x2 feeds
// one v_dot2_f32_f16 per row with fp32 accumulation.
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

// Tile words of one 16x16 tile into registers (2*BITS 16-byte loads).
typedef const __attribute__((address_space(1))) hx_u4 hx_gu4;

template <int BITS>
HX_INLINE void load_tile(uint32_t* w, const uint32_t* src)
{
    hx_gu4* s4 = (hx_gu4*)(src);
#pragma unroll
    for (int i = 0; i < 2 * BITS; ++i) {
        hx_u4 v = __builtin_nontemporal_load(s4 + i);
        w[4 * i + 0] = v.x;
        w[4 * i + 1] = v.y;
        w[4 * i + 2] = v.z;
        w[4 * i + 3] = v.w;
    }
}

// acc[m][n] += sum_k a[m][k] * W_tile[k][n] for one tile.  xa[m][kp] holds fp16 pair (2kp, 2kp+1).
// Codebook 2 takes the register-level path of hx_mul1_pair (exact fp16 weights).
template <int BITS, int CB, int MT, int P = 0>
HX_INLINE void tile_mac(const uint32_t* w, const uint32_t (*xa)[8], float (*acc)[16])
{
    if constexpr (P < 256) {
        using pos = hx_pos<P>;
        hx_h2 v;
        if constexpr (CB == 2) v = hx_mul1_pair<BITS, P>(w);
        else v = hx_decode2<CB>(hx_window<BITS, P>(w), hx_window<BITS, P + 1>(w));
#pragma unroll
        for (int m = 0; m < MT; ++m)
            acc[m][pos::n] = __builtin_amdgcn_fdot2(v, u32_as_h2(xa[m][pos::kp]), acc[m][pos::n], false);
        tile_mac<BITS, CB, MT, P + 2>(w, xa, acc);
    }
}

// Input transform of rows [0, M) over k in [k0, k0 + kc) into LDS as fp16:
//   a = fp16(H128(fp16(x . suh)))   (reference had_hf_r_128_inner<true,false>)
// When pre_transformed, x already holds a (copied as is).
HX_INLINE void input_to_lds(uint32_t* a_lds, const _Float16* x, const int64_t* rows, const _Float16* suh, int M,
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
    const int64_t* rows;     // optional row gather: row m of the input is x[rows[m]]
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
// a_lds must hold MT * kc fp16; red must hold GEMV_WAVES * MT * 128 floats.
template <int BITS, int CB, int MT>
__device__ void gemv_split_sum(const GemvArgs& g, int cg, int s, uint32_t* a_lds, float* red,
                               float* colsum)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int tc = lane & 7, ks = lane >> 3;
    const int k0 = s * g.kc;
    const int kc = min(g.kc, g.K - k0);
    const int tiles_n = g.N >> 4;

    input_to_lds(a_lds, g.x, g.rows, g.suh, g.M, g.K, k0, kc, g.pre_transformed);
    __syncthreads();

    float acc[MT][16];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int n = 0; n < 16; ++n) acc[m][n] = 0.0f;

    const uint32_t* tw = reinterpret_cast<const uint32_t*>(g.trellis);
    const int tn = cg * 8 + tc;
    const int tk_begin = k0 >> 4, tk_end = (k0 + kc) >> 4;

    uint32_t w[8 * BITS];
    int tk = tk_begin + wave * 8 + ks;
    if (tk < tk_end) load_tile<BITS>(w, tw + ((size_t)tk * tiles_n + tn) * (8 * BITS));
    for (; tk < tk_end; tk += GEMV_WAVES * 8) {
        uint32_t xa[MT][8];
        const int kl = (tk << 4) - k0;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < g.M) {
                const uint4* src = reinterpret_cast<const uint4*>(a_lds + (m * kc + kl) / 2);
                uint4 q0 = src[0], q1 = src[1];
                xa[m][0] = q0.x; xa[m][1] = q0.y; xa[m][2] = q0.z; xa[m][3] = q0.w;
                xa[m][4] = q1.x; xa[m][5] = q1.y; xa[m][6] = q1.z; xa[m][7] = q1.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) xa[m][i] = 0;
            }
        }
        uint32_t cur[8 * BITS];
#pragma unroll
        for (int i = 0; i < 8 * BITS; ++i) cur[i] = w[i];
        const int tk_next = tk + GEMV_WAVES * 8;
        if (tk_next < tk_end) load_tile<BITS>(w, tw + ((size_t)tk_next * tiles_n + tn) * (8 * BITS));
        tile_mac<BITS, CB, MT>(cur, xa, acc);
    }

    // reduce over the 8 tile rows of a wave (lanes with equal tc)
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int n = 0; n < 16; ++n) {
            float v = acc[m][n];
            v += __shfl_xor(v, 8, 64);
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            acc[m][n] = v;
        }
    if (ks == 0) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int n = 0; n < 16; ++n) red[(wave * MT + m) * 128 + tc * 16 + n] = acc[m][n];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < MT * 128; i += GEMV_THREADS) {
        float v = 0.0f;
#pragma unroll
        for (int wv = 0; wv < GEMV_WAVES; ++wv) v += red[wv * MT * 128 + i];
        colsum[i] = v;
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
