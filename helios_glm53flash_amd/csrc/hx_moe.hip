// hx_moe.hip -- host orchestration of the MoE layer on gfx950: router top-k, deterministic
// permutation, fused few-token expert kernels (hx_moe_decode.hpp) or the grouped MFMA prefill
// (hx_moe_prefill.hip), the ordered reduction and the shared-expert combine.
#include "hx_moe_decode.hpp"
#include "hx_kernels.hpp"
#include "hx_moe.hpp"

#include <stdlib.h>



namespace hx {

hipError_t launch_moe_decode_m1(const MoeDecodeArgs& a, int cb, int bits, hipStream_t st);
hipError_t launch_moe_decode_m4(const MoeDecodeArgs& a, int cb, int bits, hipStream_t st);
hipError_t launch_moe_decode_m8(const MoeDecodeArgs& a, int cb, int bits, hipStream_t st);

static size_t al(size_t v) { return (v + 255) & ~(size_t)255; }

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
    (void)max_bits;
    size_t o = HX_COUNTER_BYTES;
    off_idx = o;      o = al(o + sizeof(int64_t) * R);
    off_w = o;        o = al(o + sizeof(_Float16) * R);
    off_count = o;    o = al(o + sizeof(int64_t) * (E + 1));
    off_tsorted = o;  o = al(o + sizeof(int64_t) * R);
    off_wsorted = o;  o = al(o + sizeof(_Float16) * R);
    off_r2s = o;      o = al(o + sizeof(int64_t) * R);
    if (T <= 8 && R <= 64) {
        off_plan = o;     o = al(o + sizeof(DecodePlan));
        // partial sums: one 8 x 128 slot per (slot, column group, segment); a column group has at
        // most K/128 segments (every share holds at least one 128-k block)
        const size_t seg_g = (size_t)slots * (inter / 128) * (hidden / 128 + 1) * 8 * 128;
        const size_t seg_d = (size_t)slots * (hidden / 128) * (inter / 128 + 1) * 8 * 128;
        off_pg = o;   o = al(o + sizeof(float) * seg_g);
        off_pu = o;   o = al(o + sizeof(float) * seg_g);
        off_pd = o;   o = al(o + sizeof(float) * seg_d);
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
    a.counter_gu = reinterpret_cast<int*>(base);
    int* ctr = reinterpret_cast<int*>(base);
    a.counter_d = ctr + 4096;
    a.counter_y = ctr + 8192;
    a.exit_count = ctr + 10240;
    a.ready = ctr + 10304;
    a.status = reinterpret_cast<int*>(base + off_plan);
    a.contrib = reinterpret_cast<float*>(base + off_contrib);
    a.partial_g = reinterpret_cast<float*>(base + off_pg);
    a.partial_u = reinterpret_cast<float*>(base + off_pu);
    a.partial_d = reinterpret_cast<float*>(base + off_pd);
    a.act = reinterpret_cast<_Float16*>(base + off_act);
    return a;
}

// Units of the decode layer: gate/up per (slot, projection, column group, k-split of kc_gu), down
// per (slot, column group, k-split of kc_d), kc = the largest multiple-of-128 divisor of K up to
// 1024 (HX_MOE_KC overrides the cap, for tuning), so that every unit is one segment of one column
// group: 1152 + 576 workgroups for 9 slots at hidden 4096, intermediate 2048, i.e. a little under
// two rounds of resident workgroups (1024 on MI355X).  Measured (config-3 layer): cap 512 81 us,
// 1024 62-64 us, 2048 65 us, 4096 72 us; unaligned units sized to whole rounds of resident
// workgroups 61-68 us.  Returns the longest unit's k extent.
int decode_units(MoeDecodeArgs& a)
{
    int cap = 1024;
    if (const char* v = getenv("HX_MOE_KC")) cap = atoi(v) > 0 ? atoi(v) : cap;
    const int kg = gemv_kc_for(a.hidden, cap), kd = gemv_kc_for(a.inter, cap);
    const int slots = a.routed_slots + 1;
    a.units_gu = slots * 2 * (a.inter / 128) * (a.hidden / kg);
    a.units_d = slots * (a.hidden / 128) * (a.inter / kd);
    return kg > kd ? kg : kd;
}

hipError_t run_moe_decode(MoeDecodeArgs& a, int cb, uint32_t bits_mask, hipStream_t st)
{
    if (a.T > 8 || a.T * a.topk > DEC_MAX_R) return hipErrorInvalidValue;
    // counter area (ints): counter_gu [0, 4096), counter_d [4096, 8192), counter_y [8192, 10240),
    // exit 10240, prefill permutation arrival 10250, ready [10304, 16384)
    const int slots = a.routed_slots + 1;
    if (slots * (a.inter / 128) > 4096 || slots * (a.hidden / 128) > 4096 || a.hidden / 128 > 2048 ||
        slots * (a.inter / 128) > 6080)
        return hipErrorInvalidValue;
    // one bit width everywhere -> the fixed-width kernel; several -> per-unit dispatch
    const int bits = (bits_mask & (bits_mask - 1)) ? 0 : __builtin_ctz(bits_mask);
    if (a.T <= 1) return launch_moe_decode_m1(a, cb, bits, st);
    if (a.T <= 4) return launch_moe_decode_m4(a, cb, bits, st);
    return launch_moe_decode_m8(a, cb, bits, st);
}

}  // namespace hx
