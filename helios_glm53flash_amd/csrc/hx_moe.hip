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

static size_t al(size_t v) { return (v + 255) & ~(size_t)255; }

// Split-K plan: K per split = largest multiple-of-128 divisor of K up to `cap` (HX_MOE_KC overrides
// the cap for tuning); the activation block (8 x kc fp16) stays within LDS.
static void split_plan(int K, int max_bits, int* splits, int* kc)
{
    (void)max_bits;
    int cap = 1024;
    if (const char* v = getenv("HX_MOE_KC")) cap = atoi(v) > 0 ? atoi(v) : cap;
    if (cap > 2048) cap = 2048;
    *kc = gemv_kc_for(K, cap);
    *splits = K / *kc;
}

void MoeWs::plan(int T_, int hidden_, int inter_, int E_, int topk_, bool shared_, int max_bits)
{
    T = T_;
    hidden = hidden_;
    inter = inter_;
    E = E_;
    topk = topk_;
    R = T * topk;
    routed_slots = R < E ? R : E;
    slots = routed_slots + 1;
    split_plan(hidden, max_bits, &splits_gu, &kc_gu);
    split_plan(inter, max_bits, &splits_d, &kc_d);
    size_t o = HX_COUNTER_BYTES;
    off_idx = o;      o = al(o + sizeof(int64_t) * R);
    off_w = o;        o = al(o + sizeof(_Float16) * R);
    off_count = o;    o = al(o + sizeof(int64_t) * (E + 1));
    off_tsorted = o;  o = al(o + sizeof(int64_t) * R);
    off_wsorted = o;  o = al(o + sizeof(_Float16) * R);
    off_r2s = o;      o = al(o + sizeof(int64_t) * R);
    if (T <= 8 && R <= 64) {
        off_plan = o;     o = al(o + sizeof(DecodePlan));
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
    a.counter_d = reinterpret_cast<int*>(base) + 6144;
    a.counter_y = reinterpret_cast<int*>(base) + 12288;
    a.plan = reinterpret_cast<DecodePlan*>(base + off_plan);
    a.contrib = reinterpret_cast<float*>(base + off_contrib);
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
    if (a.T > 8 || a.T * a.topk > DEC_MAX_R) return hipErrorInvalidValue;
    if ((a.routed_slots + 1) * (a.inter / 128) > 6144 || (a.routed_slots + 1) * (a.hidden / 128) > 6144 ||
        a.hidden / 128 > 4096)
        return hipErrorInvalidValue;
    hipError_t e = hipSuccess;
    for (int b = 1; b <= 8 && e == hipSuccess; ++b)
        if (mask_gu & (1u << b)) e = decode_phase(a, cb, true, b, st);
    for (int b = 1; b <= 8 && e == hipSuccess; ++b)
        if (mask_d & (1u << b)) e = decode_phase(a, cb, false, b, st);
    return e;
}


}  // namespace hx
