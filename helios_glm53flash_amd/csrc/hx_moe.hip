// hx_moe.hip -- host orchestration of the MoE layer on gfx950: router top-k, deterministic
// permutation, fused few-token expert kernels (hx_moe_decode.hpp) or the grouped MFMA prefill
// (hx_moe_prefill.hip), the ordered reduction and the shared-expert combine.
#include "hx_moe_decode.hpp"
#include "hx_kernels.hpp"
#include "hx_moe.hpp"

#include <stdlib.h>

namespace hx {

hipError_t launch_moe_decode_phase_m1(const MoeDecodeArgs& a, int cb, bool gu, int bits, hipStream_t st);
hipError_t launch_moe_decode_phase_m4(const MoeDecodeArgs& a, int cb, bool gu, int bits, hipStream_t st);
hipError_t launch_moe_decode_phase_m8(const MoeDecodeArgs& a, int cb, bool gu, int bits, hipStream_t st);

// ------------------------------------------------------------------ combine

// y[t][c] = fp16( (sum_j contrib[r2s[t*topk + j]][c], ascending j from +0) + shared[t][c] )
// (glue2.cu:297-306 then runner.cpp:957-958); y_routed (optional) gets the fp32 routed sum, added to
// its previous contents when accumulate is set (the reference's y += contributions contract).
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* contrib, const int64_t* r2s, int T, int topk,
                                                         int hidden, bool has_shared, _Float16* y, float* y_routed,
                                                         bool accumulate)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)T * hidden) return;
    const int t = (int)(i / hidden), c = (int)(i % hidden);
    float acc = 0.0f;
    for (int j = 0; j < topk; ++j) acc += contrib[(size_t)r2s[(size_t)t * topk + j] * hidden + c];
    if (y_routed) y_routed[i] = accumulate ? y_routed[i] + acc : acc;
    if (has_shared) acc += contrib[((size_t)T * topk + t) * hidden + c];
    if (y) y[i] = (_Float16)acc;
}

static size_t al(size_t v) { return (v + 255) & ~(size_t)255; }

// Split-K plan for `groups` column groups over K: each split covers >= 4 k-blocks of 128 (one
// 8-tile step for each of the 4 waves) and the grid aims at >= 2048 workgroups.
static void split_plan(int K, int groups, int* splits, int* kc, const char* env)
{
    const int kblocks = K / 128;
    int max_s = kblocks / 4 > 0 ? kblocks / 4 : 1;
    int want = (2048 + groups - 1) / groups;
    int s = want < max_s ? want : max_s;
    if (const char* v = getenv(env)) {  // tuning override: fixed number of K splits
        int f = atoi(v);
        if (f > 0) s = f < kblocks ? f : kblocks;
    }
    if (s < 1) s = 1;
    const int per = (kblocks + s - 1) / s;
    *splits = (kblocks + per - 1) / per;
    *kc = per * 128;
}

void MoeWs::plan(int T_, int hidden_, int inter_, int E_, int topk_, bool shared_)
{
    T = T_;
    hidden = hidden_;
    inter = inter_;
    E = E_;
    topk = topk_;
    R = T * topk;
    routed_slots = R < E ? R : E;
    slots = routed_slots + 1;
    split_plan(hidden, slots * 2 * (inter / 128), &splits_gu, &kc_gu, "HX_MOE_SPLITS_GU");
    split_plan(inter, slots * (hidden / 128), &splits_d, &kc_d, "HX_MOE_SPLITS_D");
    size_t o = HX_COUNTER_BYTES;
    off_idx = o;      o = al(o + sizeof(int64_t) * R);
    off_w = o;        o = al(o + sizeof(_Float16) * R);
    off_count = o;    o = al(o + sizeof(int64_t) * (E + 1));
    off_tsorted = o;  o = al(o + sizeof(int64_t) * R);
    off_wsorted = o;  o = al(o + sizeof(_Float16) * R);
    off_r2s = o;      o = al(o + sizeof(int64_t) * R);
    if (T <= 8) {
        off_pg = o;   o = al(o + sizeof(float) * slots * splits_gu * 8 * inter);
        off_pu = o;   o = al(o + sizeof(float) * slots * splits_gu * 8 * inter);
        off_pd = o;   o = al(o + sizeof(float) * slots * splits_d * 8 * hidden);
        off_act = o;  o = al(o + sizeof(_Float16) * slots * 8 * inter);
        off_contrib = o; o = al(o + sizeof(float) * (size_t)(R + T) * hidden);
    } else {
        prefill_layout(o);
        o = prefill_end;
    }
    total = o;
}

MoeDecodeArgs MoeWs::decode_args(char* base) const
{
    MoeDecodeArgs a{};
    a.T = T;
    a.hidden = hidden;
    a.inter = inter;
    a.E = E;
    a.topk = topk;
    a.routed_slots = routed_slots;
    a.splits_gu = splits_gu;
    a.kc_gu = kc_gu;
    a.splits_d = splits_d;
    a.kc_d = kc_d;
    a.counter_gu = reinterpret_cast<int*>(base);
    a.counter_d = reinterpret_cast<int*>(base) + 8192;
    a.partial_g = reinterpret_cast<float*>(base + off_pg);
    a.partial_u = reinterpret_cast<float*>(base + off_pu);
    a.partial_d = reinterpret_cast<float*>(base + off_pd);
    a.act = reinterpret_cast<_Float16*>(base + off_act);
    return a;
}

static hipError_t decode_phase(const MoeDecodeArgs& a, int cb, bool gu, int bits, hipStream_t st)
{
    if (a.T <= 1) return launch_moe_decode_phase_m1(a, cb, gu, bits, st);
    if (a.T <= 4) return launch_moe_decode_phase_m4(a, cb, gu, bits, st);
    return launch_moe_decode_phase_m8(a, cb, gu, bits, st);
}

hipError_t run_moe_decode(MoeDecodeArgs& a, int cb, uint32_t mask_gu, uint32_t mask_d, hipStream_t st)
{
    if (a.T > 8) return hipErrorInvalidValue;
    if (a.routed_slots + 1 > 8192 / (a.inter / 128) || a.routed_slots + 1 > 8192 / (a.hidden / 128))
        return hipErrorInvalidValue;
    hipError_t e = hipSuccess;
    for (int b = 1; b <= 8 && e == hipSuccess; ++b)
        if (mask_gu & (1u << b)) e = decode_phase(a, cb, true, b, st);
    for (int b = 1; b <= 8 && e == hipSuccess; ++b)
        if (mask_d & (1u << b)) e = decode_phase(a, cb, false, b, st);
    return e;
}

hipError_t launch_moe_combine(const float* contrib, const int64_t* r2s, int T, int topk, int hidden, bool has_shared,
                              _Float16* y, float* y_routed, bool accumulate, hipStream_t st)
{
    const size_t n = (size_t)T * hidden;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, contrib, r2s, T, topk,
                       hidden, has_shared, y, y_routed, accumulate);
    return hipGetLastError();
}

}  // namespace hx
