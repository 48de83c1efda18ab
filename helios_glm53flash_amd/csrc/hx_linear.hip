// hx_linear.hip -- small-M linear dispatch (kernels in hx_linear_impl.hpp, one translation unit per
// bit width: hx_linear_b<bits>.hip).
#include "hx_gemv.hpp"
#include "hx_kernels.hpp"

#include <algorithm>

namespace hx {

template <int BITS>
hipError_t launch_gemv_cb(int cb, const GemvArgs& g, const _Float16* svh, void* y, bool y_fp32, hipStream_t st);

// Split-K plan: grid = (N / 128) column groups x (K / kc) splits.  kc shrinks from the largest
// chunk whose activation block (M x kc fp16) fits 32 KiB of LDS, in two stages:
//  1. toward 2048 workgroups (8 per CU) while the chunks stay at least 2048 long: a long stream
//     wants the occupancy (2-bit K = 16384 -> N = 32768: 2 splits 81.3-82.3 us, 4 splits 77.1-77.4,
//     8 splits 73.2, graphs of 20 calls on one box);
//  2. toward 512 workgroups (2 per CU), not below 512: each split adds a partial sum that the last
//     arriver gathers, on the critical path of a small linear.  Measured at K = 4096, M = 1:
//     config 1 (N = 2048, 16 column groups) 13.2 us with 32 splits of 128, 9.0 us with 8 splits of
//     512, 11.5 us with 4 of 1024; config 2 (N = 12288) best at 8 splits too (13.4 us; 13.8 us with 16).
constexpr int GEMV_KC_FLOOR = 512;
constexpr int GEMV_LONG_KC = 2048;

static void split_plan(int M, int K, int N, int* splits, int* kc)
{
    const int groups = N / 128;
    const int cap = 16384 / (M < 1 ? 1 : M);
    int c = gemv_kc_for(K, cap);
    while (c > GEMV_LONG_KC && (long)groups * (K / c) < 8 * GEMV_CUS) {
        const int smaller = gemv_kc_for(K, c - 128);
        if (smaller == c || smaller < GEMV_LONG_KC) break;
        c = smaller;
    }
    const int min_wg = 2 * GEMV_CUS, floor_kc = GEMV_KC_FLOOR;
    while (c > 128 && c > floor_kc && (long)groups * (K / c) < min_wg) {
        // one shrink step can skip past the floor when K has no multiple-of-128 divisor in
        // [floor_kc, c) (K = 1152: 1152 -> 384): stop at c then
        const int smaller = gemv_kc_for(K, c - 128);
        if (smaller == c || smaller < floor_kc) break;
        c = smaller;
    }
    *kc = c;
    *splits = K / c;
}

GemvPlan gemv_plan(int M, int K, int N)
{
    GemvPlan p{};
    split_plan(M, K, N, &p.splits, &p.kc);
    const int groups = N / 128;
    const long long nb = K / 128, blocks = (long long)groups * nb;
    // unit and workgroup indices are multiplied in 32 bits in the kernel: blocks * wgs < 2^31
    if (M == 1 && groups > GEMV_SK_WGS && groups % GEMV_CUS != 0 &&
        blocks * GEMV_SK_WGS < (1LL << 31) &&
        (blocks + GEMV_SK_WGS - 1) / GEMV_SK_WGS <= 16384 / 128) {
        p.sk_wgs = GEMV_SK_WGS;
        p.sk_blocks = (int)blocks;
        // a workgroup covers at least blocks / wgs blocks, so a column group's nb blocks meet at most
        // nb / (blocks / wgs) + 2 workgroups
        p.slots = (int)(nb / (blocks / GEMV_SK_WGS) + 2);
        p.kc = (int)std::min<long long>(nb, (blocks + GEMV_SK_WGS - 1) / GEMV_SK_WGS) * 128;  // LDS per workgroup
    }
    return p;
}

size_t gemv_workspace_bytes(int M, int K, int N)
{
    const GemvPlan p = gemv_plan(M, K, N);
    const int parts = p.sk_wgs ? p.slots : p.splits;
    return HX_COUNTER_BYTES + (size_t)parts * M * N * sizeof(float);
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
    const GemvPlan p = gemv_plan(M, K, N);
    g.splits = p.splits;
    g.kc = p.kc;
    g.sk_blocks = p.sk_wgs ? p.sk_blocks : 0;
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
