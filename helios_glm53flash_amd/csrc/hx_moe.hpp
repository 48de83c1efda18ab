// hx_moe.hpp -- MoE layer workspace layout and host entry points shared by hx_moe*.hip / hx_capi.hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace hx {

struct MoeDecodeArgs;

// Workspace layout of one MoE layer call (all offsets in bytes from the workspace base; the first
// HX_COUNTER_BYTES are the zero-initialised arrival counters).
struct MoeWs {
    int T = 0, hidden = 0, inter = 0, E = 0, topk = 0, R = 0;
    int routed_slots = 0, slots = 0;
    size_t off_idx = 0, off_w = 0, off_count = 0, off_tsorted = 0, off_wsorted = 0, off_r2s = 0;
    // few-token path
    size_t off_pg = 0, off_pu = 0, off_pd = 0, off_act = 0, off_contrib = 0;
    // prefill path
    int max_jobs = 0;
    size_t off_perm = 0, off_jobs = 0, off_njobs = 0, off_row_expert = 0, off_xg = 0, off_xu = 0, off_G = 0,
           off_A = 0, off_rs = 0, off_D = 0, off_sh_a = 0, off_sh_g = 0, off_sh_u = 0, off_sh_act = 0, off_sh_d = 0;
    size_t prefill_end = 0;
    size_t total = 0;

    void plan(int T, int hidden, int inter, int E, int topk, bool shared, int max_bits = 8);
    bool few_tokens() const { return T <= 8 && R <= 64; }
    void prefill_layout(size_t start);
    MoeDecodeArgs decode_args(char* base) const;
};

struct PrefillArgs {
    const _Float16* x;
    int T, hidden, inter, E, topk, R;
    const int64_t* expert_count;
    const int64_t* token_sorted;
    const _Float16* weight_sorted;
    const int64_t* r2s;
    const void* const* tr[3];
    const void* const* suh[3];
    const void* const* svh[3];
    const int32_t* bits_tab[3];
    int bits_uniform[3];
    float act_limit;
    int act_fn;        // HX_ACT_* of the routed experts
    int cb;
    char* ws;
    const MoeWs* lay;
};

// Few-token layer (one persistent launch); bits_mask has bit b set for every bit width b in use.
hipError_t run_moe_decode(MoeDecodeArgs& a, int cb, uint32_t bits_mask, hipStream_t st);
// Sets a.units_gu / a.units_d (the decode layer's grid; `resident` = workgroups that fit at once)
// and returns the longest unit's k extent.
int decode_units(MoeDecodeArgs& a, int resident);
int resident_blocks(const void* kernel, int threads, size_t lds);
int decode_resident(const void* kernel, int threads, size_t lds, int max_per_cu);
size_t decode_lds_pad(const void* kernel, size_t lds, int max_per_cu);
// Routed experts for T > 8 tokens: writes per-row fp32 contributions (sorted order) when contrib is
// non-null, y = fp16(routed + shared_rows) when y is non-null, and the fp32 routed sum into
// y_routed (added to its contents when accumulate) when y_routed is non-null.
hipError_t run_moe_prefill(const PrefillArgs& p, float* contrib, const float* shared_rows, _Float16* y,
                           float* y_routed, bool accumulate, hipStream_t st);

}  // namespace hx
