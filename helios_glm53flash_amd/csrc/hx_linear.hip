// hx_linear.hip -- small-M linear dispatch (kernels in hx_linear_impl.hpp, one translation unit per
// bit width: hx_linear_b<bits>.hip).
#include "hx_gemv.hpp"
#include "hx_kernels.hpp"

namespace hx {

template <int BITS>
hipError_t launch_gemv_cb(int cb, const GemvArgs& g, const _Float16* svh, void* y, bool y_fp32, hipStream_t st);

// Split-K plan: at least 4 tile-row steps of 8 tiles per split so every wave has work, and enough
// workgroups (>= ~2048) to cover 256 CUs several times.
void gemv_plan(int M, int K, int N, int* splits, int* kc)
{
    const int groups = N / 128;
    const int kblocks = K / 128;                 // 128-wide k blocks
    int max_splits = kblocks / 4 > 0 ? kblocks / 4 : 1;
    int want = (2048 + groups - 1) / groups;
    int s = want < max_splits ? want : max_splits;
    if (s < 1) s = 1;
    int blocks_per = (kblocks + s - 1) / s;
    s = (kblocks + blocks_per - 1) / blocks_per;
    *splits = s;
    *kc = blocks_per * 128;
}

size_t gemv_workspace_bytes(int M, int K, int N)
{
    int s, kc;
    gemv_plan(M, K, N, &s, &kc);
    return HX_COUNTER_BYTES + (size_t)s * M * N * sizeof(float);
}

hipError_t launch_linear_gemv(const _Float16* x, const uint16_t* trellis, const _Float16* suh, const _Float16* svh,
                              void* y, int M, int K, int N, int bits, int cb, bool y_fp32, void* ws, hipStream_t st)
{
    GemvArgs g;
    g.x = x;
    g.rows = nullptr;
    g.trellis = trellis;
    g.suh = suh;
    g.M = M;
    g.K = K;
    g.N = N;
    gemv_plan(M, K, N, &g.splits, &g.kc);
    if ((size_t)(N / 128) * sizeof(int) > HX_COUNTER_BYTES) return hipErrorInvalidValue;
    g.counter = static_cast<int*>(ws);
    g.partial = reinterpret_cast<float*>(static_cast<char*>(ws) + HX_COUNTER_BYTES);
    g.pre_transformed = false;
    switch (bits) {
        case 1: return launch_gemv_cb<1>(cb, g, svh, y, y_fp32, st);
        case 2: return launch_gemv_cb<2>(cb, g, svh, y, y_fp32, st);
        case 3: return launch_gemv_cb<3>(cb, g, svh, y, y_fp32, st);
        case 4: return launch_gemv_cb<4>(cb, g, svh, y, y_fp32, st);
        case 5: return launch_gemv_cb<5>(cb, g, svh, y, y_fp32, st);
        case 6: return launch_gemv_cb<6>(cb, g, svh, y, y_fp32, st);
        case 7: return launch_gemv_cb<7>(cb, g, svh, y, y_fp32, st);
        case 8: return launch_gemv_cb<8>(cb, g, svh, y, y_fp32, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace hx
