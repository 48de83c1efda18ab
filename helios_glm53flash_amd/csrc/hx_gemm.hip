// hx_gemm.hip -- EXL3 quantized linear for M > 8 on MFMA (gfx950): input transform kernel, then
// quarter-operand MFMA tiles (hx_mfma.hpp) with the output Hadamard + svh epilogue fused.
// Reference semantics: src/cuda/quant/exl3_gemm_kernel.cuh:8-80, exl3_gemm_inner.cuh:456-480.
#include "hx_mfma.hpp"
#include "hx_kernels.hpp"

namespace hx {

// a = fp16(H128(fp16(x . suh))) row-wise (had_hf_r_128_inner<true,false>); one wave per 128 block.
__global__ __launch_bounds__(256) void input_had_kernel(const _Float16* x, const _Float16* suh, _Float16* a,
                                                        long blocks, int K)
{
    const int lane = threadIdx.x & 63;
    const long b = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= blocks) return;
    const long row = b / (K / 128);
    const int c = (int)(b % (K / 128)) * 128 + 2 * lane;
    hx_h2 v = *reinterpret_cast<const hx_h2*>(x + row * K + c) * *reinterpret_cast<const hx_h2*>(suh + c);
    float v0 = (float)v.x, v1 = (float)v.y;
    hx_had128_wave(v0, v1);
    hx_h2 o = {(_Float16)v0, (_Float16)v1};
    *reinterpret_cast<hx_h2*>(a + row * K + c) = o;
}

hipError_t launch_input_had(const _Float16* x, const _Float16* suh, _Float16* a, long rows, int K, hipStream_t st)
{
    long blocks = rows * (K / 128);
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(input_had_kernel, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, st, x, suh, a, blocks, K);
    return hipGetLastError();
}

// Output epilogue for a staged 64-row half: y[row][cg*128 + c] = svh . H128(C[row][:]).
template <int CB, class Smem>
__device__ void linear_tile_epilogue(const Smem& sm, int half, int rows, const _Float16* svh, void* y, int N,
                                     int cg, bool y_fp32)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = cg * 128 + 2 * lane;
    const hx_h2 sv = *reinterpret_cast<const hx_h2*>(svh + c);
    for (int r = wave; r < 64; r += 4) {
        const int row = 64 * half + r;
        if (row >= rows) break;
        float v0 = staged_value<CB>(sm, half, r, 2 * lane), v1 = staged_value<CB>(sm, half, r, 2 * lane + 1);
        hx_had128_wave(v0, v1);
        if (y_fp32) {
            *reinterpret_cast<float2*>(static_cast<float*>(y) + (size_t)row * N + c) =
                make_float2(v0 * (float)sv.x, v1 * (float)sv.y);
        } else {
            hx_h2 h = {(_Float16)v0, (_Float16)v1};
            *reinterpret_cast<hx_h2*>(static_cast<_Float16*>(y) + (size_t)row * N + c) = h * sv;
        }
    }
}

// Quarter-operand tile (each wave decodes its own 32 columns into MFMA B operands; only A is staged
// in LDS), three workgroups per CU.
template <int BITS, int CB>
__global__ __launch_bounds__(MF_THREADS, qt_occ<CB>()) void linear_mfma_kernel(const _Float16* a, const uint32_t* trellis,
                                                                const _Float16* svh, void* y, int M, int K, int N,
                                                                bool y_fp32)
{
    __shared__ MfmaSmemQ sm;
    // the row tiles of a column group on one XCD: its trellis words come from memory once and the
    // other row tiles read them from that XCD's L2
    int mt, cg;
    xcd_group_index(blockIdx.x + blockIdx.y * gridDim.x, gridDim.y, gridDim.x, mt, cg);
    const int m0 = mt * MF_BM;
    const int rows = min(MF_BM, M - m0);
    hx_f4 acc[MF_BM / 16][2];
    mfma_tile_q<BITS, CB, MF_BM>(a + (size_t)m0 * K, K, rows, trellis, K, N, cg * 8, sm, acc);
    void* yt = y_fp32 ? (void*)(static_cast<float*>(y) + (size_t)m0 * N) : (void*)(static_cast<_Float16*>(y) + (size_t)m0 * N);
    for (int half = 0; half < 2; ++half) {
        qt_stage_c_half<MF_BM>(acc, half, sm);
        __syncthreads();
        linear_tile_epilogue<CB>(sm, half, rows, svh, yt, N, cg, y_fp32);
        __syncthreads();
    }
}

template <int BITS>
static hipError_t launch_mfma_b(int cb, const _Float16* a, const uint32_t* tr, const _Float16* svh, void* y, int M,
                                int K, int N, bool y_fp32, hipStream_t st)
{
    dim3 grid(N / 128, (M + MF_BM - 1) / MF_BM);
    switch (cb) {
        case 0: hipLaunchKernelGGL((linear_mfma_kernel<BITS, 0>), grid, dim3(MF_THREADS), 0, st, a, tr, svh, y, M, K, N, y_fp32); break;
        case 1: hipLaunchKernelGGL((linear_mfma_kernel<BITS, 1>), grid, dim3(MF_THREADS), 0, st, a, tr, svh, y, M, K, N, y_fp32); break;
        default: hipLaunchKernelGGL((linear_mfma_kernel<BITS, 2>), grid, dim3(MF_THREADS), 0, st, a, tr, svh, y, M, K, N, y_fp32); break;
    }
    return hipGetLastError();
}

hipError_t launch_linear_mfma(const _Float16* a_had, const uint16_t* trellis, const _Float16* svh, void* y, int M,
                              int K, int N, int bits, int cb, bool y_fp32, hipStream_t st)
{
    const uint32_t* tr = reinterpret_cast<const uint32_t*>(trellis);
    switch (bits) {
        case 1: return launch_mfma_b<1>(cb, a_had, tr, svh, y, M, K, N, y_fp32, st);
        case 2: return launch_mfma_b<2>(cb, a_had, tr, svh, y, M, K, N, y_fp32, st);
        case 3: return launch_mfma_b<3>(cb, a_had, tr, svh, y, M, K, N, y_fp32, st);
        case 4: return launch_mfma_b<4>(cb, a_had, tr, svh, y, M, K, N, y_fp32, st);
        case 5: return launch_mfma_b<5>(cb, a_had, tr, svh, y, M, K, N, y_fp32, st);
        case 6: return launch_mfma_b<6>(cb, a_had, tr, svh, y, M, K, N, y_fp32, st);
        case 7: return launch_mfma_b<7>(cb, a_had, tr, svh, y, M, K, N, y_fp32, st);
        case 8: return launch_mfma_b<8>(cb, a_had, tr, svh, y, M, K, N, y_fp32, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace hx
