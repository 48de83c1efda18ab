#pragma once
// hx_linear_impl.hpp -- EXL3 quantized linear y = svh . H_N(H_K(x . suh) . W_hat) on gfx950,
// small-M path (M <= 8): fused trellis decode + GEMV + split-K + output Hadamard epilogue in one
// launch.  Reference semantics: src/cuda/quant/exl3_gemv_kernel.cuh:138-402 and
// exl3_gemm_kernel.cuh:8-80 (input transform, GEMM, output transform + svh).
#include "hx_gemv.hpp"
#include "hx_kernels.hpp"

namespace hx {

// This lane's two svh entries of column group cg (columns cg*128 + 2*lane, +1).  Requested when the
// group's work starts: read in the epilogue, the load would be one more dependent round trip after
// the split-K arrival and gather.
HX_INLINE hx_h2 svh_pair(const _Float16* svh, int cg)
{
    return *reinterpret_cast<const hx_h2*>(svh + cg * 128 + 2 * (threadIdx.x & 63));
}

// Output epilogue for one 128-column group: y[m][cg*128 + c] = svh . H128(colsum[m][:]), sv = svh_pair
//   fp32 out: had_ff_r_128_inner<false,true> (transform in fp32, times float(svh))
//   fp16 out: had_fh_r_128_inner<false,true> (transform, round to fp16, fp16 multiply by svh)
template <int MT>
__device__ void linear_epilogue(const float* colsum, hx_h2 sv, void* y, int M, int N, int cg, bool y_fp32)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c = cg * 128 + 2 * lane;
    for (int m = wave; m < M && m < MT; m += hx_nwaves()) {
        float v0 = colsum[m * 128 + 2 * lane], v1 = colsum[m * 128 + 2 * lane + 1];
        hx_had128_wave(v0, v1);
        if (y_fp32) {
            float2 o = make_float2(v0 * (float)sv.x, v1 * (float)sv.y);
            *reinterpret_cast<float2*>(static_cast<float*>(y) + (size_t)m * N + c) = o;
        } else {
            hx_h2 h = {(_Float16)v0, (_Float16)v1};
            h = h * sv;
            *reinterpret_cast<hx_h2*>(static_cast<_Float16*>(y) + (size_t)m * N + c) = h;
        }
    }
}

template <int BITS, int CB, int MT>
__global__ __launch_bounds__(GEMV_THREADS) void linear_gemv_kernel(GemvArgs g, const _Float16* svh, void* y,
                                                                  bool y_fp32)
{
    extern __shared__ uint32_t a_lds[];
    __shared__ float colsum[MT * 128];
    const int groups = g.N >> 7;
    const int cg = blockIdx.x % groups;
    const int s = blockIdx.x / groups;
    const hx_h2 sv = svh_pair(svh, cg);
    gemv_split_sum<BITS, CB, MT>(g, cg, s, a_lds, colsum);
    if (g.splits > 1) {
        publish_partial<MT>(g.partial, g.M, g.N, cg, s, colsum);
        if (!arrive_last(&g.counter[cg], g.splits)) return;
        gather_partials<MT>(g.partial, g.M, g.N, g.splits, cg, colsum);
    }
    linear_epilogue<MT>(colsum, sv, y, g.M, g.N, cg, y_fp32);
}

// Workgroup owning unit b of `units` split evenly over `wgs` workgroups (workgroup i takes units
// [i*units/wgs, (i+1)*units/wgs)): the largest i whose first unit is <= b.  units * wgs < 2^31.
HX_INLINE unsigned stream_owner(unsigned b, unsigned units, unsigned wgs) { return ((b + 1) * wgs - 1) / units; }

// One row, stream-K: workgroup i runs the (column group, 128-k block) units [i*T/G, (i+1)*T/G) of
// T = (N/128) * (K/128), group by group.  A group met by several workgroups is finished by the last
// to arrive, which adds the partials in workgroup order (deterministic); the others publish theirs.
template <int BITS, int CB>
__global__ __launch_bounds__(GEMV_THREADS) void linear_gemv_stream_kernel(GemvArgs g, const _Float16* svh, void* y,
                                                                         bool y_fp32)
{
    extern __shared__ uint32_t a_lds[];
    __shared__ float colsum[128];
    const unsigned T = g.sk_blocks, G = gridDim.x, nb = g.K >> 7, i = blockIdx.x;
    const unsigned b1 = (i + 1) * T / G;
    for (unsigned b = i * T / G; b < b1;) {
        const unsigned cg = b / nb, e = min(b1, (cg + 1) * nb);
        const hx_h2 sv = svh_pair(svh, cg);
        gemv_range<BITS, CB, 1, 1, LIN_PF, LIN_PFW, true>(g, cg, (b - cg * nb) * 128, (e - b) * 128, a_lds, colsum);
        const unsigned first = stream_owner(cg * nb, T, G), last = stream_owner(cg * nb + nb - 1, T, G);
        bool finish = true;
        if (last > first) {
            publish_partial<1>(g.partial, 1, g.N, cg, i - first, colsum);
            finish = arrive_last(&g.counter[cg], last - first + 1);
            if (finish) gather_partials<1>(g.partial, 1, g.N, last - first + 1, cg, colsum);
        }
        if (finish) linear_epilogue<1>(colsum, sv, y, 1, g.N, cg, y_fp32);
        __syncthreads();  // colsum is read before the next group overwrites it
        b = e;
    }
}

template <int BITS, int CB, int MT>
hipError_t launch_gemv_t(const GemvArgs& g, const _Float16* svh, void* y, bool y_fp32, hipStream_t st)
{
    const int groups = g.N >> 7;
    const size_t lds = (size_t)MT * g.kc * sizeof(_Float16);
    hipLaunchKernelGGL((linear_gemv_kernel<BITS, CB, MT>), dim3(groups * g.splits), dim3(GEMV_THREADS), lds, st, g,
                       svh, y, y_fp32);
    return hipGetLastError();
}

template <int BITS, int CB>
hipError_t launch_gemv_b(const GemvArgs& g, const _Float16* svh, void* y, bool y_fp32, hipStream_t st)
{
    if (g.sk_blocks) {  // one row (gemv_plan): the grid is the plan's workgroup count
        hipLaunchKernelGGL((linear_gemv_stream_kernel<BITS, CB>), dim3(GEMV_SK_WGS), dim3(GEMV_THREADS),
                           (size_t)g.kc * sizeof(_Float16), st, g, svh, y, y_fp32);
        return hipGetLastError();
    }
    if (g.M <= 1) return launch_gemv_t<BITS, CB, 1>(g, svh, y, y_fp32, st);
    if (g.M <= 4) return launch_gemv_t<BITS, CB, 4>(g, svh, y, y_fp32, st);
    if (g.M <= 8) return launch_gemv_t<BITS, CB, 8>(g, svh, y, y_fp32, st);
    return launch_gemv_t<BITS, CB, 16>(g, svh, y, y_fp32, st);
}

template <int BITS>
hipError_t launch_gemv_cb(int cb, const GemvArgs& g, const _Float16* svh, void* y, bool y_fp32, hipStream_t st)
{
    switch (cb) {
        case 0: return launch_gemv_b<BITS, 0>(g, svh, y, y_fp32, st);
        case 1: return launch_gemv_b<BITS, 1>(g, svh, y, y_fp32, st);
        default: return launch_gemv_b<BITS, 2>(g, svh, y, y_fp32, st);
    }
}

}  // namespace hx
