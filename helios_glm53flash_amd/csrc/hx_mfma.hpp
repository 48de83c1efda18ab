// hx_mfma.hpp -- EXL3 decode-to-LDS + MFMA tile core for gfx950 (M >= 16 path).
//
// Workgroup = 4 waves, output tile 128 rows x 128 columns (one Hadamard block wide), K consumed
// in chunks of 64.  Per chunk:
//   * A (128 x 64 fp16, already input-transformed) is staged to LDS with 16-byte loads;
//   * B (64 x 128) is decoded from 4 x 8 trellis tiles straight into LDS as fp16 in [n][k] order:
//     8 threads per tile, thread q of a tile owns positions 32q..32q+31 (columns q and q+8, all 16
//     k).  Those windows live in stream words [q*bits - 1, q*bits + bits) of the tile, so each
//     thread loads bits+1 words and every window offset is a compile-time constant;
//   * each wave computes a 64 x 64 quarter with v_mfma_f32_16x16x32_f16 (fp32 accumulate).
// Operand layout of v_mfma_f32_16x16x32_f16 (64 lanes): A: lane l holds row l%16,
// k = 8*(l/16)..+7; B: column l%16, same k; C: column l%16, rows 4*(l/16)..+3.
#pragma once
#include "hx_device.hpp"

namespace hx {

constexpr int MF_THREADS = 256;
constexpr int MF_BM = 128;
constexpr int MF_BN = 128;
constexpr int MF_BK = 64;
constexpr int MF_LDA = MF_BK + 8;  // halves per LDS row (pad against bank conflicts)
constexpr int MF_LDC = MF_BN + 4;  // floats per LDS row in the epilogue

struct MfmaSmem {
    union {
        struct {
            _Float16 a[MF_BM * MF_LDA];
            _Float16 b[MF_BN * MF_LDA];
        } ab;
        float c[64 * MF_LDC];
    };
};

// Thread-local decode of 32 positions of one tile: r[0..BITS] are stream words q*BITS-1 .. q*BITS+BITS-1.
template <int BITS, int CB, int I = 0>
HX_INLINE void decode_quarter(const uint32_t* r, int q, _Float16* bcol /* Bs + (16*tc)*LDA + 16*tr */)
{
    if constexpr (I < 32) {
        constexpr int e0 = (I + 1) * BITS + 32, e1 = (I + 2) * BITS + 32;
        constexpr int s0 = e0 - 16, s1 = e1 - 16;
        uint32_t w0, w1;
        if constexpr ((s0 & 31) <= 16) w0 = (r[s0 >> 5] >> (16 - (s0 & 31))) & 0xffffu;
        else w0 = __builtin_amdgcn_alignbit(r[s0 >> 5], r[(s0 >> 5) + 1], 48 - (s0 & 31)) & 0xffffu;
        if constexpr ((s1 & 31) <= 16) w1 = (r[s1 >> 5] >> (16 - (s1 & 31))) & 0xffffu;
        else w1 = __builtin_amdgcn_alignbit(r[s1 >> 5], r[(s1 >> 5) + 1], 48 - (s1 & 31)) & 0xffffu;
        hx_h2 v = hx_decode2<CB>(w0, w1);
        constexpr int j = I & 7;
        constexpr int k = 2 * ((I >> 3) & 3) + 8 * ((j >> 1) & 1);
        constexpr int nn = 8 * (j >> 2);
        *reinterpret_cast<hx_h2*>(bcol + (nn + q) * MF_LDA + k) = v;
        decode_quarter<BITS, CB, I + 2>(r, q, bcol);
    }
}

// acc[mb][nb] (float4) for this wave's 64 x 64 quarter of the 128 x 128 tile.
//   A: rows [0, rows) of an fp16 row-major matrix with leading dimension lda (k offset 0 = k 0)
//   trellis: tile words of the weight; tn0 = first tile column (8 tiles = 128 columns); N columns total.
template <int BITS, int CB>
__device__ void mfma_tile(const _Float16* A, long lda, int rows, const uint32_t* trellis, int K, int N, int tn0,
                          MfmaSmem& sm, hx_f4 (&acc)[4][4])
{
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int tiles_n = N >> 4;
    constexpr int NW = 8 * BITS;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = hx_f4{0.f, 0.f, 0.f, 0.f};

    // decode role: tile (tr, tc) of the 4 x 8 chunk, quarter q
    const int dtile = t >> 3, q = t & 7;
    const int tr = dtile >> 3, tc = dtile & 7;

    for (int k0 = 0; k0 < K; k0 += MF_BK) {
        // stage A
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = t + MF_THREADS * i;
            const int row = idx >> 3, c = idx & 7;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (row < rows) v = *reinterpret_cast<const uint4*>(A + (size_t)row * lda + k0 + 8 * c);
            *reinterpret_cast<uint4*>(&sm.ab.a[row * MF_LDA + 8 * c]) = v;
        }
        // decode B
        {
            const int tk = (k0 >> 4) + tr;
            const uint32_t* tw = trellis + ((size_t)tk * tiles_n + tn0 + tc) * NW;
            uint32_t r[BITS + 1];
            r[0] = tw[(q * BITS + NW - 1) % NW];
#pragma unroll
            for (int i = 0; i < BITS; ++i) r[i + 1] = tw[q * BITS + i];
            decode_quarter<BITS, CB>(r, q, &sm.ab.b[(16 * tc) * MF_LDA + 16 * tr]);
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < MF_BK; kk += 32) {
            hx_h8 af[4], bf[4];
#pragma unroll
            for (int mb = 0; mb < 4; ++mb)
                af[mb] = *reinterpret_cast<const hx_h8*>(&sm.ab.a[(64 * wm + 16 * mb + (lane & 15)) * MF_LDA + kk + 8 * (lane >> 4)]);
#pragma unroll
            for (int nb = 0; nb < 4; ++nb)
                bf[nb] = *reinterpret_cast<const hx_h8*>(&sm.ab.b[(64 * wn + 16 * nb + (lane & 15)) * MF_LDA + kk + 8 * (lane >> 4)]);
#pragma unroll
            for (int mb = 0; mb < 4; ++mb)
#pragma unroll
                for (int nb = 0; nb < 4; ++nb)
                    acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[mb], bf[nb], acc[mb][nb], 0, 0, 0);
        }
        __syncthreads();
    }
}

// Stage rows [64*half, 64*half + 64) of the accumulated tile to LDS (sm.c[row - 64*half][col]).
HX_INLINE void stage_c_half(const hx_f4 (&acc)[4][4], int half, MfmaSmem& sm)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    if (wm == half) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int nb = 0; nb < 4; ++nb)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sm.c[(16 * mb + 4 * (lane >> 4) + r) * MF_LDC + 64 * wn + 16 * nb + (lane & 15)] = acc[mb][nb][r];
    }
}

}  // namespace hx
