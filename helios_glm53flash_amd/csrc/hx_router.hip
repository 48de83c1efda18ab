// hx_router.hip -- dense fp16 NT GEMM y[m][n] = sum_k x[m][k] * w[n][k] (w row-major [N][K], fp32
// accumulate), the router-logits front end of the MoE layer on gfx950.  Reference semantics:
// helios::glue::gemm_nt_f16 / gemv_nt_f16 (src/engine/glue2.cu:9-65,165-182): fp16 output rounded
// once from the fp32 sum, or fp32 output (optionally added to y).
//
//   M <= 8   gemv: one workgroup per output column n; its 4 waves split K, each lane takes 8
//            consecutive k per step (16-byte loads of w and x), v_dot2_f32_f16 accumulation, the
//            wave sums added in wave order.
//   M > 8    direct-load MFMA: each wave computes a 32 x 32 block with v_mfma_f32_16x16x32_f16; both
//            operands are contiguous along k, so a lane's MFMA fragment (8 halves) is one 16-byte
//            load from L2, no LDS staging.
#include "hx_device.hpp"
#include "hx_kernels.hpp"

namespace hx {

namespace {

typedef uint32_t u4v __attribute__((ext_vector_type(4)));

HX_INLINE float dot8(u4v a, u4v b, float acc)
{
    acc = __builtin_amdgcn_fdot2(u32_as_h2(a.x), u32_as_h2(b.x), acc, false);
    acc = __builtin_amdgcn_fdot2(u32_as_h2(a.y), u32_as_h2(b.y), acc, false);
    acc = __builtin_amdgcn_fdot2(u32_as_h2(a.z), u32_as_h2(b.z), acc, false);
    acc = __builtin_amdgcn_fdot2(u32_as_h2(a.w), u32_as_h2(b.w), acc, false);
    return acc;
}

HX_INLINE void store_out(void* y, size_t idx, float v, bool y_fp32, bool add)
{
    if (y_fp32) {
        float* yf = static_cast<float*>(y);
        yf[idx] = add ? yf[idx] + v : v;
    } else {
        static_cast<_Float16*>(y)[idx] = (_Float16)v;
    }
}

}  // namespace

template <int MT>
__global__ __launch_bounds__(256) void gemv_nt_kernel(const _Float16* x, const _Float16* w, void* y, int M, int N,
                                                      int K, bool y_fp32, bool add)
{
    __shared__ float part[4][MT];
    const int n = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int kq = (K / 4 + 7) & ~7;  // k range of a wave, a multiple of 8
    const int k0 = wave * kq, k1 = min(K, k0 + kq);
    const _Float16* wr = w + (size_t)n * K;
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    for (int k = k0 + 8 * lane; k < k1; k += 512) {
        const u4v wv = *reinterpret_cast<const u4v*>(wr + k);
#pragma unroll
        for (int m = 0; m < MT; ++m)
            if (m < M) acc[m] = dot8(*reinterpret_cast<const u4v*>(x + (size_t)m * K + k), wv, acc[m]);
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        float v = acc[m];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
        if (lane == 0) part[wave][m] = v;
    }
    __syncthreads();
    if (threadIdx.x < M) {
        const int m = threadIdx.x;
        const float v = ((part[0][m] + part[1][m]) + part[2][m]) + part[3][m];
        store_out(y, (size_t)m * N + n, v, y_fp32, add);
    }
}

// Workgroup = 4 waves stacked along m: rows 128*bx + 32*wave .. +31, columns 32*by .. +31.
__global__ __launch_bounds__(256) void gemm_nt_mfma_kernel(const _Float16* x, const _Float16* w, void* y, int M,
                                                           int N, int K, bool y_fp32, bool add)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r0 = 128 * blockIdx.x + 32 * wave, c0 = 32 * blockIdx.y;
    if (r0 >= M) return;  // whole wave past the last row (uniform)
    const int lr = lane & 15, lk = 8 * (lane >> 4);
    // fragment rows / columns of this lane (clamped: out-of-range rows and columns are not stored)
    const _Float16* ap[2];
    const _Float16* bp[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        ap[i] = x + (size_t)min(r0 + 16 * i + lr, M - 1) * K + lk;
        bp[i] = w + (size_t)min(c0 + 16 * i + lr, N - 1) * K + lk;
    }
    hx_f4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = hx_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int k = 0; k < K; k += 32) {
        hx_h8 a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            a[i] = *reinterpret_cast<const hx_h8*>(ap[i] + k);
            b[i] = *reinterpret_cast<const hx_h8*>(bp[i] + k);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    // C: lane holds column lane % 16, rows 4 * (lane / 16) + r of each 16 x 16 block
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = r0 + 16 * i + 4 * (lane >> 4) + r, n = c0 + 16 * j + lr;
                if (m < M && n < N) store_out(y, (size_t)m * N + n, acc[i][j][r], y_fp32, add);
            }
}

hipError_t launch_gemm_nt_f16(const _Float16* x, const _Float16* w, void* y, int M, int N, int K, bool y_fp32,
                              bool add, hipStream_t st)
{
    if (M <= 0 || N <= 0) return hipSuccess;
    if (M <= 8) {
        if (M <= 1)
            hipLaunchKernelGGL((gemv_nt_kernel<1>), dim3(N), dim3(256), 0, st, x, w, y, M, N, K, y_fp32, add);
        else
            hipLaunchKernelGGL((gemv_nt_kernel<8>), dim3(N), dim3(256), 0, st, x, w, y, M, N, K, y_fp32, add);
    } else {
        hipLaunchKernelGGL(gemm_nt_mfma_kernel, dim3((M + 127) / 128, (N + 31) / 32), dim3(256), 0, st, x, w, y, M,
                           N, K, y_fp32, add);
    }
    return hipGetLastError();
}

}  // namespace hx
