// hx_moe.hip -- host orchestration of the MoE layer on gfx950: router top-k, deterministic
// permutation, fused few-token expert kernels (hx_moe_decode.hpp) or the grouped MFMA prefill
// (hx_moe_prefill.hip), the ordered reduction and the shared-expert combine.
#include "hx_moe_decode.hpp"
#include "hx_kernels.hpp"
#include "hx_moe.hpp"

#include <stdio.h>
#include <stdlib.h>

#include <mutex>
#include <utility>
#include <vector>



namespace hx {

template <int MT>
hipError_t launch_moe_decode_mt(const MoeDecodeArgs& a, int cb, int bits, hipStream_t st);  // hx_moe_decode_m*.hip

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
    a.status = ctr + DEC_STATUS_INT;  // counter area: zero between calls unless a wait gave up
    a.contrib = reinterpret_cast<float*>(base + off_contrib);
    a.partial_g = reinterpret_cast<float*>(base + off_pg);
    a.partial_u = reinterpret_cast<float*>(base + off_pu);
    a.partial_d = reinterpret_cast<float*>(base + off_pd);
    a.act = reinterpret_cast<_Float16*>(base + off_act);
    return a;
}

// Workgroups of `kernel` that fit on the current device at once (CU count x blocks per CU), cached
// per (device, kernel, threads, lds).
int resident_blocks(const void* kernel, int threads, size_t lds)
{
    struct Key {
        int dev;
        const void* k;
        int threads;
        size_t lds;
        int n;
    };
    static std::mutex mu;
    static std::vector<Key> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(mu);
    for (const Key& c : cache)
        if (c.dev == dev && c.k == kernel && c.threads == threads && c.lds == lds) return c.n;
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, lds) != hipSuccess || per <= 0) per = 1;
    cache.push_back({dev, kernel, threads, lds, cus * per});
    return cus * per;
}

// Occupancy of a decode launch: the decode kernels are tuned for 4 workgroups per CU (16 waves:
// one round of gate/up units, then the down units as those retire).  When the kernel needs fewer
// registers, more would fit: the down units of the second round would then be resident from the
// start, spinning on their inputs, and the streaming units slow down (measured 58 against 51 us at
// config 3).  decode_resident is the resident count with that cap; decode_lds_pad raises the
// dynamic LDS so that each workgroup takes more than 1/(max_per_cu + 1) of the CU's 160 KB, which
// enforces it in hardware (the runtime's occupancy query is not relied on for the LDS size per CU).
constexpr size_t DEC_LDS_PER_CU = 160 * 1024;

static int device_cus()
{
    static std::mutex mu;
    static std::vector<std::pair<int, int>> cache;  // (device, CUs)
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lock(mu);
    for (const auto& c : cache)
        if (c.first == dev) return c.second;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 0;
    cache.push_back({dev, cus});
    return cus;
}

int decode_resident(const void* kernel, int threads, size_t lds, int max_per_cu)
{
    const int res = resident_blocks(kernel, threads, lds);
    const int cus = device_cus();
    if (cus <= 0) return res;
    const int cap = max_per_cu * cus;
    return res < cap ? res : cap;
}

size_t decode_lds_pad(const void* kernel, size_t lds, int max_per_cu)
{
    static std::mutex mu;
    static std::vector<std::pair<const void*, size_t>> cache;  // (kernel, static LDS bytes)
    size_t stat = 0;
    {
        std::lock_guard<std::mutex> lock(mu);
        bool found = false;
        for (const auto& c : cache)
            if (c.first == kernel) {
                stat = c.second;
                found = true;
            }
        if (!found) {
            hipFuncAttributes fa;
            if (hipFuncGetAttributes(&fa, kernel) != hipSuccess) return lds;
            stat = fa.sharedSizeBytes;
            cache.push_back({kernel, stat});
        }
    }
    const size_t total = DEC_LDS_PER_CU / (size_t)(max_per_cu + 1) + 1024;
    const size_t dyn = total > stat ? total - stat : 0;
    return lds > dyn ? lds : dyn;
}

// Units of the decode layer (the grid): gate/up units first, then down units (a second round,
// dispatched as the first one's workgroups finish).  Each phase has as many units as one round of
// resident workgroups holds, clamped to [column groups, blocks] of the phase; a column group gets
// U / C or U / C + 1 units (equal k ranges within it, one segment each).  Measured (config-3 layer,
// 1024 resident, 4-step ring): 1024 + 1024 units (3 or 4 per column group, every CU holds 4
// gate/up workgroups) 46.3 us; 864 + 864 (3 per column group, so 96 CUs hold 4 and the others 3)
// 48.3 us; 960 + 1024 47.7 us; 1024 + 1280 48.4 us; 576 + 864 49.1 us; and for the down phase
// alone (1024 gate/up): 1024 46.1-46.5 us, 992 45.9, 960 45.8, 928 46.1, 832 47.3 us, so the down
// phase takes 15/16 of the resident count (its units, a little longer, gather fewer partials).
// (With the earlier ring, whose waits drained every load in flight once per group, 864 + 864 was
// the faster one.)
// A fused variant (workgroup w runs gate/up unit w then down unit w, reusing its plan) took 60 us.
// Returns the longest unit's k extent.
int decode_units(MoeDecodeArgs& a, int resident)
{
    const long slots = a.routed_slots + 1;
    const long cg_gu = slots * 2 * (a.inter / 128), kb_gu = a.hidden / 128;
    const long cg_d = slots * (a.hidden / 128), kb_d = a.inter / 128;
    auto clampu = [](long u, long c, long kb) { return u < c ? c : (u > c * kb ? c * kb : u); };
    long ug = clampu(resident, cg_gu, kb_gu), ud = clampu(resident - resident / 16, cg_d, kb_d);
    a.units_gu = (int)ug;
    a.units_d = (int)ud;
    const long bg = (kb_gu + ug / cg_gu - 1) / (ug / cg_gu), bd = (kb_d + ud / cg_d - 1) / (ud / cg_d);
    return (int)(128 * (bg > bd ? bg : bd));
}

hipError_t run_moe_decode(MoeDecodeArgs& a, int cb, uint32_t bits_mask, hipStream_t st)
{
    if (a.T > 8 || a.T * a.topk > DEC_MAX_R) return hipErrorInvalidValue;
    // counter area (ints): counter_gu [0, 4096), counter_d [4096, 8192), counter_y [8192, 10240),
    // exit 10240, wait status 10242, prefill permutation arrival 10250, ready [10304, 16384)
    const int slots = a.routed_slots + 1;
    if (slots * (a.inter / 128) > 4096 || slots * (a.hidden / 128) > 4096 || a.hidden / 128 > 2048 ||
        slots * (a.inter / 128) > 6080)
        return hipErrorInvalidValue;
    // one bit width everywhere -> the fixed-width kernel; several, or the non-gated relu2 (whose gate
    // units skip their stream) -> per-unit dispatch
    const bool one = (bits_mask & (bits_mask - 1)) == 0 && a.act_fn != HX_ACT_RELU2_NOGATE;
    const int bits = one ? __builtin_ctz(bits_mask) : 0;
    if (a.T <= 1) return launch_moe_decode_mt<1>(a, cb, bits, st);
    if (a.T <= 4) return launch_moe_decode_mt<4>(a, cb, bits, st);
    return launch_moe_decode_mt<8>(a, cb, bits, st);
}

}  // namespace hx
