// hx_moe_decode.hpp -- fused MoE layer for few tokens (T <= 8, T*topk <= 64) on gfx950 in ONE
// launch, without host synchronisation.  Every workgroup computes the router top-k and the
// token-by-expert permutation from the fp16 scores (a few hundred bytes), then runs one unit:
//
//   gate/up unit  one k range of one expert's gate or up GEMV with the trellis decode fused; the
//                 last-arriving unit of a (slot, column group) adds the partial sums, runs the
//                 SiLU-gate epilogue, stores the down-projection input and raises its ready flag.
//   down unit     requests its tile words, waits for the ready flags of its k range, then one k
//                 range of one expert's down GEMV; the last unit of a (slot, column group) writes
//                 the weighted contribution rows; the last of all slots of a column group reduces
//                 the contributions in routing-rank order, adds the shared expert and writes y.
//
// Reference semantics: src/cuda/aux/routing.cu:211-329 (router), src/engine/glue2.cu:244-311
// (permutation, ordered reduction), src/cuda/quant/exl3_moe_kernel.cuh:57-262 and
// hadamard_inner.cuh:284-481 (experts), src/engine/runner.cpp:723-738,957-958 (shared expert,
// combine).  Slot j is the j-th expert, in expert-index order, with a nonzero token count (the
// reference's ticket numbering, exl3_moe_kernel.cuh:57-69); one extra slot holds the shared expert.
#pragma once
#include "hx_gemv.hpp"


namespace hx {

constexpr int DEC_MAX_R = 64;  // T * topk rows handled by the few-token path
constexpr int DEC_SHARED = -2;  // build_plan: the workgroup's slot is the shared expert
constexpr int DEC_STATUS_INT = 10242;  // int index of the wait-status word in the counter area
constexpr int DEC_STATUS_TIMEOUT = 1;  // status bits: a bounded wait gave up
constexpr int DEC_STATUS_BAD_BITS = 2; // a per-expert bit table held a width outside 1..8

// Routing plan of one call: sorted rows and active-expert slots.
// Tables of a workgroup's slot's expert (or of the shared expert) that its unit uses: trellis and
// suh of the projection it streams, and the scale rows of its epilogue (gate/up units: svh of gate,
// svh of up, suh of down; down units: svh of down).
constexpr int DEC_TABS = 5;
struct SlotTables {
    const void* tr;
    const void* suh;
    const void* ep[3];
};

struct DecodePlan {
    int n;                     // active routed experts
    int expert[DEC_MAX_R];
    int start[DEC_MAX_R];
    int count[DEC_MAX_R];
    int token[DEC_MAX_R];      // token of sorted row r
    float weight[DEC_MAX_R];   // routing weight of sorted row r
    int r2s[DEC_MAX_R];        // flat routing index -> sorted row
    SlotTables tab;            // tables of the workgroup's own slot and projection
};

struct MoeDecodeArgs {
    const _Float16* x;             // [T][hidden]
    int T, hidden, inter, E, topk;
    // layer mode: router scores (fp16 [T][E]) and optional bias
    const _Float16* scores;
    const _Float16* bias;
    float routed_scale;
    // grouped mode (scores == null): the caller's permutation
    const int64_t* expert_count;   // [E+1]
    const int64_t* token_sorted;   // [T*topk]
    const _Float16* weight_sorted; // [T*topk]
    const int64_t* route_to_sorted;// [T*topk] (needed only when combining)
    // routed expert tables (device arrays of device pointers), per-expert bits (nullable)
    const void* const* tr[3];
    const void* const* suh[3];
    const void* const* svh[3];
    const int32_t* bits_tab[3];
    int bits_uniform[3];
    // shared expert (null trellis -> none)
    const void* sh_tr[3];
    const void* sh_suh[3];
    const void* sh_svh[3];
    int sh_bits[3];
    float act_limit;
    int act_fn;                    // routed experts: HX_ACT_SILU, HX_ACT_GELU or HX_ACT_RELU2_NOGATE
    int routed_slots;              // upper bound of active experts = min(E, T*topk)
    // workspace
    int* counter_gu;               // [slots][inter/128]
    int* counter_d;                // [slots][hidden/128]
    int* counter_y;                // [hidden/128]
    float* partial_g;              // [slots][inter/128][hidden/128 + 1 segments][8][128]
    float* partial_u;
    float* partial_d;              // [slots][hidden/128][inter/128 + 1 segments][8][128]
    _Float16* act;                 // [slots][8][inter]  (down-projection input, already transformed)
    int* exit_count;               // workgroups that finished (zero between calls)
    int units_gu, units_d;         // workgroups of the gate/up and down phases (grid = their sum)
    int* ready;                    // [slots][inter/128] 1 once the guad epilogue stored that block
    int* status;                   // DEC_STATUS_* bits (never expected to be set); read and cleared by
                                   // hx_moe_check_status
    // outputs
    int64_t* out_idx;              // optional router outputs [T][topk]
    _Float16* out_w;
    float* contrib;                // [T*topk (+ T)][hidden]: sorted routed rows, then shared rows
    bool combine;                  // kernel B reduces contributions into y / y_routed
    _Float16* y;                   // fp16(routed + shared), optional
    float* y_routed;               // fp32 routed sum, optional
    bool y_accumulate;             // y_routed += sum instead of =
};

struct SlotInfo {
    int expert;  // -1: shared slot
    int start;   // first sorted row
    int count;   // rows
    bool valid;
};

HX_INLINE float sigmoid_stable(float x)
{
    const float ez = __expf(-fabsf(x));
    const float base = ez / (1.0f + ez);
    return x >= 0.0f ? 1.0f - base : base;
}

// Top-k of one token's scores by one wave (routing.cu:211-329: key = logit, or sigmoid + bias;
// larger first under the monotone unsigned encoding of the fp32 key, ties to the lower index;
// weights sigmoid(payload) * scale / (sum + 1e-20) rounded to fp16).  Lane k < topk returns
// selection k in (e, w).
struct NoTopkHook {
    HX_INLINE void operator()() const {}
};

// after_loads() runs once the score loads are issued (a caller issues its own loads there, so that
// their latencies overlap).
template <class Hook = NoTopkHook>
HX_INLINE void wave_topk(const _Float16* scores, const _Float16* bias, int E, int topk, float scale, int& e_out,
                         float& w_out, Hook after_loads = Hook())
{
    const int lane = threadIdx.x & 63;
    constexpr int PER = 8;  // candidates per lane: E <= 512
    if (!bias) {
        // key = the fp16 logit itself: its monotone 16-bit encoding and the complemented index fit
        // one u32 (larger = higher logit, then lower index; +0 above -0 as in the fp32 encoding)
        uint32_t c[PER];
        uint16_t raw[PER];
        // all loads first (clamped addresses, no branches) so their latencies overlap
#pragma unroll
        for (int i = 0; i < PER; ++i) raw[i] = h_as_u16(scores[min(lane + 64 * i, E - 1)]);
        after_loads();
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = lane + 64 * i;
            uint32_t h = raw[i];
            h = (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
            c[i] = e < E ? (h << 16) | (0xffffu - (uint32_t)e) : 0u;
        }
        // each lane's candidates in descending order (Batcher's 19-comparator network for 8), so a
        // round only compares the lanes' heads: the wave's largest head is selection k, and its lane
        // (keys are unique) drops its head
        auto cas = [&](int i, int j) {
            const uint32_t hi = max(c[i], c[j]), lo = min(c[i], c[j]);
            c[i] = hi;
            c[j] = lo;
        };
        cas(0, 1); cas(2, 3); cas(4, 5); cas(6, 7);
        cas(0, 2); cas(1, 3); cas(4, 6); cas(5, 7);
        cas(1, 2); cas(5, 6);
        cas(0, 4); cas(1, 5); cas(2, 6); cas(3, 7);
        cas(2, 4); cas(3, 5);
        cas(1, 2); cas(3, 4); cas(5, 6);
        uint32_t sel = 0;
        for (int k = 0; k < topk; ++k) {
            const uint32_t best = hx_wave_max_u32(c[0]);
            const bool own = c[0] == best;
#pragma unroll
            for (int i = 0; i + 1 < PER; ++i) c[i] = own ? c[i + 1] : c[i];
            c[PER - 1] = own ? 0u : c[PER - 1];
            sel = lane == k ? best : sel;
        }
        // the sigmoid of selection k on lane k; their sum in selection order
        uint32_t h = sel >> 16;
        h = (h & 0x8000u) ? (h & 0x7fffu) : (~h & 0xffffu);
        const float o = sigmoid_stable((float)u16_as_h((uint16_t)h));
        float sum = 0.0f;
        for (int k = 0; k < topk; ++k) sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, o), k));
        sum += 1e-20f;
        e_out = lane < topk ? (int)(0xffffu - (sel & 0xffffu)) : 0;
        w_out = lane < topk ? (float)(_Float16)(o * scale / sum) : 0.0f;
        return;
    }
    uint64_t cand[PER];
    float payload[PER];
    _Float16 sv[PER], bv[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = min(lane + 64 * i, E - 1);
        sv[i] = scores[e];
        bv[i] = bias[e];
    }
    after_loads();
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = lane + 64 * i;
        cand[i] = 0;
        payload[i] = 0.0f;
        if (e < E) {
            payload[i] = sigmoid_stable((float)sv[i]);
            const float key = payload[i] + (float)bv[i];
            uint32_t u = __float_as_uint(key);
            u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
            cand[i] = ((uint64_t)u << 32) | (uint64_t)(0xfffffu - (uint32_t)e + 1u);
        }
    }
    float sum = 0.0f;
    e_out = 0;
    w_out = 0.0f;
    for (int k = 0; k < topk; ++k) {
        uint64_t b = 0;
        float bp = 0.0f;
#pragma unroll
        for (int i = 0; i < PER; ++i)
            if (cand[i] > b) {
                b = cand[i];
                bp = payload[i];
            }
        // the wave's largest 64-bit key in two 32-bit DPP reductions: the largest key word, then
        // the largest index word (lowest expert) among the lanes holding that key word
        const uint32_t hi = hx_wave_max_u32((uint32_t)(b >> 32));
        const uint32_t lo = hx_wave_max_u32((uint32_t)(b >> 32) == hi ? (uint32_t)b : 0u);
        const uint64_t best = ((uint64_t)hi << 32) | lo;
        const uint64_t owner = __ballot(b == best);
        const float o = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bp),
                                                                            (int)__ffsll((unsigned long long)owner) - 1));
#pragma unroll
        for (int i = 0; i < PER; ++i)
            if (cand[i] == best) cand[i] = 0;
        sum += o;
        if (lane == k) {
            e_out = (int)(0xfffffu + 1u - lo);
            w_out = o;
        }
    }
    sum += 1e-20f;
    w_out = (float)(_Float16)(w_out * scale / sum);
}

// Element `i` of a 3-array member of the kernel arguments, by selects rather than a run-time index:
// indexing an argument array at run time makes the compiler copy the whole argument block into
// per-lane scratch memory.
// The loaded values pass through an empty asm so that the compiler cannot turn the selects back
// into one load from a computed address.
template <class T>
HX_INLINE T opaque_value(T v)
{
    static_assert(sizeof(T) == 8 || sizeof(T) == 4, "pointer or 32-bit value");
    if constexpr (sizeof(T) == 8) {
        uint64_t u = __builtin_bit_cast(uint64_t, v);
        asm volatile("" : "+s"(u));
        return __builtin_bit_cast(T, u);
    } else {
        uint32_t u = __builtin_bit_cast(uint32_t, v);
        asm volatile("" : "+s"(u));
        return __builtin_bit_cast(T, u);
    }
}

template <class T>
HX_INLINE T pick3(const T (&v)[3], int i)
{
    const T v0 = opaque_value(v[0]), v1 = opaque_value(v[1]), v2 = opaque_value(v[2]);
    return i == 0 ? v0 : (i == 1 ? v1 : v2);
}

HX_INLINE uint64_t ptr_bits(const void* p) { return reinterpret_cast<uint64_t>(p); }
HX_INLINE const void* bits_ptr(uint64_t u) { return reinterpret_cast<const void*>(u); }

// Table q (SlotTables order: tr, suh, ep[0..2]) of a unit streaming projection proj: the per-expert
// pointer array, or null where the unit needs none.
HX_INLINE const void* const* tab_base(const MoeDecodeArgs& a, int q, int proj)
{
    const bool gu = proj < 2;
    switch (q) {
        case 0: return pick3(a.tr, proj);
        case 1: return gu ? pick3(a.suh, proj) : nullptr;
        case 2: return gu ? a.svh[0] : a.svh[2];
        case 3: return gu ? a.svh[1] : nullptr;
        default: return gu ? a.suh[2] : nullptr;
    }
}

HX_INLINE const void* sh_tab(const MoeDecodeArgs& a, int q, int proj)
{
    const bool gu = proj < 2;
    switch (q) {
        case 0: return pick3(a.sh_tr, proj);
        case 1: return gu ? pick3(a.sh_suh, proj) : nullptr;
        case 2: return gu ? a.sh_svh[0] : a.sh_svh[2];
        case 3: return gu ? a.sh_svh[1] : nullptr;
        default: return gu ? a.sh_suh[2] : nullptr;
    }
}

HX_INLINE void set_tab(SlotTables& t, int q, const void* v)
{
    if (q == 0) t.tr = v;
    else if (q == 1) t.suh = v;
    else t.ep[q - 2] = v;
}

// Tables of a unit streaming projection proj of expert e (e < 0: the shared expert).
HX_INLINE void load_slot_tables(const MoeDecodeArgs& a, SlotTables& t, int e, int proj)
{
#pragma unroll
    for (int q = 0; q < DEC_TABS; ++q) {
        const void* const* b = tab_base(a, q, proj);
        set_tab(t, q, e < 0 ? sh_tab(a, q, proj) : (b ? b[e] : nullptr));
    }
}

// Build the plan in LDS (every workgroup computes the same plan), and the tables of projection
// proj of the workgroup's own slot: routed slot my_slot >= 0 if it is active, the shared expert for
// my_slot == DEC_SHARED, none for -1.  Layer mode routes the tokens; grouped mode reads the caller's
// expert_count / token_sorted / weight_sorted.
template <int MT>
__device__ __forceinline__ void build_plan(const MoeDecodeArgs& a, DecodePlan& p, int my_slot, int proj)
{
    __shared__ int sel_e[DEC_MAX_R];
    __shared__ float sel_w[DEC_MAX_R];
    constexpr int TAB_MAX_E = 320, TPL = TAB_MAX_E / 64;
    __shared__ uint64_t tab_lds[DEC_TABS][TAB_MAX_E];  // table entries of every expert
    const int wave = hx_vwave(), lane = threadIdx.x & 63;
    const int R = a.T * a.topk;
    if (a.scores) {
        // The slot's table entries would be one more dependent load after the ranking.  Instead
        // they are loaded for every expert while the scores are in flight and parked in LDS: wave 0
        // loads trellis and suh (parked after its selection, which then waits for the scores only,
        // as loads complete in order), wave 1 the epilogue tables.  The owning lane of the slot's
        // expert takes trellis and suh after the ranking, thread 0 the rest after the plan barrier.
        const bool pf_tab = my_slot >= 0 && a.E <= TAB_MAX_E;
        auto load_tabs = [&](int q0, int q1, uint64_t (*v)[TPL]) {
#pragma unroll
            for (int q = q0; q < q1; ++q) {
                const void* const* b = tab_base(a, q, proj);
#pragma unroll
                for (int i = 0; i < TPL; ++i) v[q - q0][i] = b ? ptr_bits(b[min(lane + 64 * i, a.E - 1)]) : 0;
            }
        };
        auto park_tabs = [&](int q0, int q1, uint64_t (*v)[TPL]) {
#pragma unroll
            for (int q = q0; q < q1; ++q)
#pragma unroll
                for (int i = 0; i < TPL; ++i) tab_lds[q][lane + 64 * i] = v[q - q0][i];
        };
        uint64_t v_main[2][TPL];
        auto prefetch = [&]() {
            if (pf_tab && wave == 0) load_tabs(0, 2, v_main);
        };
        if (pf_tab && wave == 1) {
            uint64_t v_ep[DEC_TABS - 2][TPL];
            load_tabs(2, DEC_TABS, v_ep);
            park_tabs(2, DEC_TABS, v_ep);
        }
        // one token: wave 0 selects and sorts in registers; more: one wave per token, then LDS
        // (token 0 is peeled off: only its wave issues the table prefetch; MT = 1 has no loop)
        int e1 = 0;
        float w1 = 0.0f;
        if (wave == 0) {
            wave_topk(a.scores, a.bias, a.E, a.topk, a.routed_scale, e1, w1, prefetch);
            if (pf_tab) {
                park_tabs(0, 2, v_main);
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            }
            if (a.T > 1 && lane < a.topk) {
                sel_e[lane] = e1;
                sel_w[lane] = w1;
            }
        }
        if constexpr (MT > 1) {
            for (int t = wave == 0 ? hx_nwaves() : wave; t < a.T; t += hx_nwaves()) {
                int e;
                float w;
                wave_topk(a.scores + (size_t)t * a.E, a.bias, a.E, a.topk, a.routed_scale, e, w);
                if (lane < a.topk) {
                    sel_e[t * a.topk + lane] = e;
                    sel_w[t * a.topk + lane] = w;
                }
            }
            if (a.T > 1) __syncthreads();
        }
        if (wave == 0) {
            // stable counting sort of the R <= 64 selections by expert (ascending flat index within an
            // expert, glue2.cu:244-293 with a deterministic cursor); selection j is read from lane j
            const int i = lane;
            const int ei = i < R ? (a.T == 1 ? e1 : sel_e[i]) : 0x7fffffff;
            const float wi = a.T == 1 ? w1 : (i < R ? sel_w[i] : 0.0f);
            int less = 0, eqb = 0, cnt = 0, dless = 0, n = 0;
            if (a.T == 1) {
                // one token: its selections are distinct experts, so a selection's rank is the
                // number of selected experts below it, read from a bitmap of the selection in LDS
                // (a few independent instructions instead of two loops of R dependent readlanes)
                __shared__ __align__(16) uint32_t sel_bits[16];  // E <= 512
                if (lane < 16) sel_bits[lane] = 0u;
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                if (i < R) __hip_atomic_fetch_or(&sel_bits[ei >> 5], 1u << (ei & 31), __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_WAVEFRONT);
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                if (i < R) {
                    const int wd = ei >> 5;
                    const uint32_t below = (1u << (ei & 31)) - 1u;
#pragma unroll
                    for (int q = 0; q < 16; ++q) {
                        const uint32_t m = sel_bits[q];
                        less += __builtin_popcount(q < wd ? m : (q == wd ? (m & below) : 0u));
                    }
                }
                dless = less;
                cnt = 1;
                n = R;
            } else {
                for (int j = 0; j < R; ++j) {
                    const int ej = __builtin_amdgcn_readlane(ei, j);
                    less += ej < ei;
                    eqb += (ej == ei) && (j < i);
                    cnt += ej == ei;
                }
                const uint64_t fm = __ballot(i < R && eqb == 0);  // first selection of each expert
                for (int j = 0; j < R; ++j)                        // distinct experts below ei
                    if ((fm >> j) & 1) dless += __builtin_amdgcn_readlane(ei, j) < ei;
                n = __popcll(fm);
            }
            if (i < R) {
                const int pos = less + eqb;
                p.token[pos] = i / a.topk;
                p.weight[pos] = wi;
                p.r2s[i] = pos;
                if (eqb == 0) {
                    p.expert[dless] = ei;
                    p.start[dless] = less;
                    p.count[dless] = cnt;
                    if (dless == my_slot) {
                        if (pf_tab) {
                            p.tab.tr = bits_ptr(tab_lds[0][ei]);
                            p.tab.suh = bits_ptr(tab_lds[1][ei]);
                        } else {
                            load_slot_tables(a, p.tab, ei, proj);
                        }
                    }
                }
            }
            if (lane == 0) {
                p.n = n;
                if (my_slot == DEC_SHARED) load_slot_tables(a, p.tab, -1, proj);
            }
        }
    } else {
        if (wave == 0) {
            // active experts in index order from expert_count (all loads issued together)
            constexpr int PER = 8;
            int c[PER];
#pragma unroll
            for (int q = 0; q < PER; ++q) {
                const int e = lane + 64 * q;
                c[q] = e < a.E ? (int)a.expert_count[e] : 0;
            }
            int seen = 0, base = 0;
#pragma unroll
            for (int q = 0; q < PER; ++q) {
                int cs = c[q];
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const int v = __shfl_up(cs, o, 64);
                    if (lane >= o) cs += v;
                }
                const uint64_t act = __ballot(c[q] > 0);
                const int before = __popcll(act & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
                if (c[q] > 0 && seen + before < DEC_MAX_R) {
                    // clamp to the R sorted rows so an inconsistent expert_count cannot index past them
                    const int st = min(base + cs - c[q], R);
                    p.expert[seen + before] = lane + 64 * q;
                    p.start[seen + before] = st;
                    p.count[seen + before] = min(c[q], R - st);
                }
                seen += __popcll(act);
                base += __shfl(cs, 63, 64);
            }
            if (lane == 0) {
                p.n = min(seen, DEC_MAX_R);
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                if (my_slot >= 0 && my_slot < p.n) load_slot_tables(a, p.tab, p.expert[my_slot], proj);
                else if (my_slot == DEC_SHARED) load_slot_tables(a, p.tab, -1, proj);
            }
            if (lane < R) {
                p.token[lane] = min(max((int)a.token_sorted[lane], 0), a.T - 1);
                p.weight[lane] = (float)a.weight_sorted[lane];
                p.r2s[lane] = a.route_to_sorted ? min(max((int)a.route_to_sorted[lane], 0), R - 1) : lane;
            }
        }
    }
    __syncthreads();
    // the slot's epilogue tables (the epilogues read them after later barriers)
    if (a.scores && hx_vtid() == 0 && my_slot >= 0 && my_slot < p.n && a.E <= TAB_MAX_E) {
        const int e = p.expert[my_slot];
#pragma unroll
        for (int q = 2; q < DEC_TABS; ++q) {
            set_tab(p.tab, q, bits_ptr(tab_lds[q][e]));
        }
    }
}

HX_INLINE SlotInfo slot_info(const MoeDecodeArgs& a, const DecodePlan& p, int slot)
{
    SlotInfo si{0, 0, 0, false};
    if (slot == a.routed_slots) {
        si.expert = -1;
        si.count = a.T;
        si.valid = a.sh_tr[0] != nullptr;
    } else if (slot < p.n) {
        si.expert = p.expert[slot];
        si.start = p.start[slot];
        si.count = p.count[slot];
        si.valid = si.count > 0;
    }
    return si;
}

HX_INLINE int proj_bits(const MoeDecodeArgs& a, int proj, int expert)
{
    if (expert < 0) return pick3(a.sh_bits, proj);
    const int32_t* bt = pick3(a.bits_tab, proj);
    return bt ? bt[expert] : pick3(a.bits_uniform, proj);
}

// ------------------------------------------------------------------ epilogues

// guad epilogue for rows m < count of one 128-column group (hadamard_inner.cuh:284-413 for routed
// experts; swiglu_clamp + down-input transform for the shared expert, runner.cpp:723-738).
template <int MT>
// sg, su, sd: this lane's pairs (columns cg*128 + 2*lane, +1) of svh_gate, svh_up and suh_down.
__device__ __forceinline__ void guad_epilogue(const MoeDecodeArgs& a, const DecodePlan& p, const SlotInfo& si, int slot,
                                              int cg, const float* cs_g, const float* cs_u, hx_h2 sg, hx_h2 su,
                                              hx_h2 sd)
{
    const int wave = hx_vwave(), lane = threadIdx.x & 63;
    const int c = cg * 128 + 2 * lane;
    const bool shared = si.expert < 0;
    const float L = a.act_limit;
    for (int m = wave; m < si.count && m < MT; m += hx_nwaves()) {
        hx_h2 p;
        if (!shared) {
            // G, U as fp16 (the reference GEMM writes fp16), transform, fp16, times svh (fp16)
            // (the non-gated relu2 has no gate sums: its gate lane comes from u)
            hx_h2 U = {(_Float16)cs_u[m * 128 + 2 * lane], (_Float16)cs_u[m * 128 + 2 * lane + 1]};
            float u0 = (float)U.x, u1 = (float)U.y;
            hx_had128_wave(u0, u1);
            hx_h2 u = hx_h2{(_Float16)u0, (_Float16)u1} * su;
            hx_h2 g = {(_Float16)0.0f, (_Float16)0.0f};
            if (a.act_fn != HX_ACT_RELU2_NOGATE) {
                hx_h2 G = {(_Float16)cs_g[m * 128 + 2 * lane], (_Float16)cs_g[m * 128 + 2 * lane + 1]};
                float g0 = (float)G.x, g1 = (float)G.y;
                hx_had128_wave(g0, g1);
                g = hx_h2{(_Float16)g0, (_Float16)g1} * sg;
            }
            g.x = hx_gate_act(a.act_fn, g.x, u.x);
            g.y = hx_gate_act(a.act_fn, g.y, u.y);
            if (L != 0.0f) {
                const _Float16 Lh = (_Float16)L, nLh = (_Float16)(-L);
                u.x = u.x < nLh ? nLh : (u.x > Lh ? Lh : u.x);
                u.y = u.y < nLh ? nLh : (u.y > Lh ? Lh : u.y);
                g.x = g.x > Lh ? Lh : g.x;
                g.y = g.y > Lh ? Lh : g.y;
            }
            p = (g * u) * sd;
        } else {
            float g0 = cs_g[m * 128 + 2 * lane], g1 = cs_g[m * 128 + 2 * lane + 1];
            float u0 = cs_u[m * 128 + 2 * lane], u1 = cs_u[m * 128 + 2 * lane + 1];
            hx_had128_wave(g0, g1);
            hx_had128_wave(u0, u1);
            g0 = fminf(g0 * (float)sg.x, L);
            g1 = fminf(g1 * (float)sg.y, L);
            u0 = fminf(fmaxf(u0 * (float)su.x, -L), L);
            u1 = fminf(fmaxf(u1 * (float)su.y, -L), L);
            hx_h2 act = {(_Float16)(g0 / (1.0f + __expf(-g0)) * u0), (_Float16)(g1 / (1.0f + __expf(-g1)) * u1)};
            p = act * sd;
        }
        float p0 = (float)p.x, p1 = (float)p.y;
        hx_had128_wave(p0, p1);
        hx_h2 o = {(_Float16)p0, (_Float16)p1};
        // read by the down-projection units of other workgroups of this launch
        __hip_atomic_store(reinterpret_cast<uint32_t*>(a.act + ((size_t)slot * 8 + m) * a.inter + c), h2_as_u32(o),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}


// Weighted contribution rows of one 128-column group (hadamard_inner.cuh:418-481: D rounded to fp16,
// transform, times weight / sqrt(128) and svh_d in fp32; the shared expert keeps D in fp32).
template <int MT>
__device__ __forceinline__ void down_epilogue(const MoeDecodeArgs& a, const DecodePlan& p, const SlotInfo& si, int cg,
                              const float* cs)
{
    const int wave = hx_vwave(), lane = threadIdx.x & 63;
    const int c = cg * 128 + 2 * lane;
    const bool shared = si.expert < 0;
    const hx_h2 sd = *reinterpret_cast<const hx_h2*>(static_cast<const _Float16*>(p.tab.ep[0]) + c);
    const int R = a.T * a.topk;
    for (int m = wave; m < si.count && m < MT; m += hx_nwaves()) {
        float d0, d1, wgt;
        size_t row;
        if (!shared) {
            d0 = (float)(_Float16)cs[m * 128 + 2 * lane];
            d1 = (float)(_Float16)cs[m * 128 + 2 * lane + 1];
            wgt = p.weight[si.start + m];
            row = (size_t)(si.start + m);
        } else {
            d0 = cs[m * 128 + 2 * lane];
            d1 = cs[m * 128 + 2 * lane + 1];
            wgt = 1.0f;
            row = (size_t)(R + m);
        }
        hx_had128_wave(d0, d1);
        d0 = d0 * wgt * (float)sd.x;
        d1 = d1 * wgt * (float)sd.y;
        float* dst = a.contrib + row * a.hidden + c;
        __hip_atomic_store(dst, d0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(dst + 1, d1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// y[t][c] = fp16((sum_j contrib[r2s[t*topk + j]][c], ascending j from +0) + shared[t][c])
// (glue2.cu:297-306 then runner.cpp:957-958) for one 128-column group.
__device__ __forceinline__ void combine_columns(const MoeDecodeArgs& a, const DecodePlan& p, int cg, bool has_shared)
{
    const int R = a.T * a.topk;
    for (int i = threadIdx.x; i < a.T * 128; i += hx_nthreads()) {
        const int t = i >> 7;
        const int c = cg * 128 + (i & 127);
        // the loads of 8 contributions (and the shared row) are issued together, then added in
        // routing-rank order
        constexpr int B = 8;
        float acc = 0.0f;
        for (int j0 = 0; j0 < a.topk; j0 += B) {
            float v[B];
#pragma unroll
            for (int j = 0; j < B; ++j)
                v[j] = __hip_atomic_load(a.contrib + (size_t)p.r2s[t * a.topk + min(j0 + j, a.topk - 1)] * a.hidden + c,
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int j = 0; j < B; ++j)
                if (j0 + j < a.topk) acc += v[j];
        }
        const float sh = has_shared ? __hip_atomic_load(a.contrib + (size_t)(R + t) * a.hidden + c, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT)
                                    : 0.0f;
        const size_t o = (size_t)t * a.hidden + c;
        if (a.y_routed) a.y_routed[o] = a.y_accumulate ? a.y_routed[o] + acc : acc;
        if (has_shared) acc += sh;
        if (a.y) a.y[o] = (_Float16)acc;
    }
}


// ------------------------------------------------------------------ the layer kernel
//
// One launch per layer call.  Work is cut in 128-k blocks: the gate/up blocks of every possible
// slot (ordered slot, projection, column group, k) in units_gu equal contiguous units, then the
// down blocks (slot, column group, k) in units_d units; workgroup w < units_gu runs gate/up unit w,
// the others down unit w - units_gu.  The grid is larger than what fits at once, and the hardware
// dispatches workgroups in increasing index order as earlier ones finish, so faster CUs take more
// units (no work queue, no atomics).  Every gate/up workgroup has a lower index than every down
// workgroup and never waits; the dispatcher of each XCD takes its own workgroups in index order,
// so it dispatches a down workgroup only after all of its gate/up workgroups, which then hold no
// slot that a producer would need: every producer a down workgroup waits for gets dispatched and
// finishes, and the waits end.  A unit's partial sum
// goes to its own workspace slot; the last of the units of a column group adds them in unit order
// (deterministic) and runs the epilogue.  A down workgroup requests its tile words first and only
// then waits for the activations it needs (per slot and 128-column block), so the down
// projection's HBM latency overlaps the end of the gate/up phase.  Units of slots beyond the
// active ones (fewer distinct experts than routed rows) return at once.

// Workgroup shape: 4 waves.  (Measured on MI355X, config-3 layer, 1 token, with an earlier unit
// scheme: 4 waves x 4 workgroups per CU 73 us, 8 x 2 76 us, 16 x 1 83 us -- fewer, larger workgroups
// wait longer at their barriers than they save in handoffs.)
// Tile-word steps in flight per wave in the layer kernel (up to 4 bits).  Every resident unit's ring
// is in flight at once, and the queue that builds up in the memory system delays each unit's own
// dependent loads (scores, inputs, flags, partial sums): measured at config 3 (layer time), 8 steps
// 51.1 us, 6 steps 49.8 us, 5 steps 49.6 us, 4 steps 49.4 us, 3 steps 50.5 us, 2 steps 51.7 us.
// Since a step loads only the quarter's own words (one load per lane at 2 bits, the wrapped word
// comes from the neighbouring lane), 5 steps are best: 45.9-46.0 us against 46.4-46.5 us with 4 and
// 3, 46.3-46.5 us with 6 (one box, two runs each).
// Since the down units poll their flags at once and the gate/up finisher gathers in one round trip,
// the gate/up units gain from one step more: 6 steps 43.86-43.95 us, 7 steps 43.82-44.08 us, 5 steps
// 44.13-44.33 us (one box, four runs each); the down units keep 5 (8: slower, 3: no change).
// (The linear GEMV keeps its own ring depth: it streams alone.)
constexpr int DEC_PF = 5;
constexpr int DEC_PF_GU = 6;
constexpr int DEC_THREADS = 256;

// Bounded wait of one wave for flags[i] >= target, i < n <= 64: lane i polls flag i and the wave
// goes on once all are set (polled one after another, the flags cost one dependent round trip each
// even when all were already set, as they are for the down units that start late).  The producers
// are resident workgroups that do not wait for anything themselves, so the wait ends; the bound
// only turns a bug into a flagged wrong result instead of a hung device.
HX_INLINE void wait_flags(const int* flags, int n, int target, int* status)
{
    const int lane = threadIdx.x & 63;
    int spins = 0;
    while (__ballot(lane < n && __hip_atomic_load(&flags[min(lane, n - 1)], __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT) < target) != 0) {
        // back off: device-coherent loads of a few flags from a thousand workgroups all go to the
        // memory channels of those flags, which the weight streams go through too
        if (spins < 4) __builtin_amdgcn_s_sleep(4);
        else if (spins < 16) __builtin_amdgcn_s_sleep(16);
        else __builtin_amdgcn_s_sleep(64);
        if ((++spins & 1023) == 0 &&
            (__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & DEC_STATUS_TIMEOUT))
            break;  // another wait already gave up: do not add its bound to every later wait
        if (spins > (1 << 22)) {
            if (lane == 0) __hip_atomic_fetch_or(status, DEC_STATUS_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
    }
}

// Units of a phase: C column groups of KB 128-k blocks in U units, C <= U <= C * KB.  The first
// r = U % C column groups get q + 1 = U / C + 1 units, the others q; the units of a column group
// are equal contiguous k ranges, numbered in k order (the order their partial sums are added in).
struct Split {
    int C, KB, q, r;
    HX_INLINE static Split make(int C, int KB, int U)
    {
        U = max(C, min(U, C * KB));
        return Split{C, KB, U / C, U % C};
    }
    HX_INLINE int count(long c) const { return q + (c < r ? 1 : 0); }
    // unit w -> column group of the unit
    HX_INLINE int ucg(int w) const
    {
        const int big = r * (q + 1);
        return w < big ? w / (q + 1) : r + (w - big) / q;
    }
    // unit w -> index of the unit within its column group
    HX_INLINE int uidx(int w) const
    {
        const int big = r * (q + 1);
        return w < big ? w % (q + 1) : (w - big) % q;
    }
    HX_INLINE int kb_begin(long c, int j) const { return j * KB / count(c); }
};

// Slot of unit slot position us: with a shared expert, position 0 is the shared expert (its units
// come first, and need no routing) and position 1 + s routed slot s; -1 for an inactive position.
HX_INLINE int unit_slot(const MoeDecodeArgs& a, const DecodePlan& p, int us)
{
    if (a.sh_tr[0] != nullptr) {
        if (us == 0) return a.routed_slots;
        return us - 1 < p.n ? us - 1 : -1;
    }
    return us < p.n ? us : -1;
}

// Arrival of a gate/up unit; the last of a column group's units adds the partial sums and runs the
// epilogue.  The gate partials exist for all but the routed experts of the non-gated relu2, which
// only the run-time-width kernel (RT) runs.
template <int MT, bool RT>
__device__ __forceinline__ void gu_finish(const MoeDecodeArgs& a, const DecodePlan& plan, const Split& sp, long c,
                                          int slot, float* cs_g, float* cs_u)
{
    const int gg = a.inter >> 7, KB = a.hidden >> 7;
    const int proj = (int)((c / gg) & 1), cg = (int)(c % gg);
    const SlotInfo si = slot_info(a, plan, slot);
    const bool gated = !RT || si.expert < 0 || a.act_fn != HX_ACT_RELU2_NOGATE;
    const long cgate = c - proj * gg, cup = cgate + gg;
    const int ng = sp.count(cgate), nu = sp.count(cup);
    if (!arrive_last(&a.counter_gu[slot * gg + cg], ng + nu)) return;
    // the epilogue's scale pairs and both projections' partial sums in one round trip: the scale
    // loads go first, the gate and up sums are gathered side by side (with one row, threads 0-127
    // take the gate's columns and 128-255 the up's); the gate's svh of a non-gated expert need not
    // exist
    const int lane = threadIdx.x & 63;
    const int col = cg * 128 + 2 * lane;
    auto ep = [&](int q) { return *reinterpret_cast<const hx_h2*>(static_cast<const _Float16*>(plan.tab.ep[q]) + col); };
    const hx_h2 sg = si.expert < 0 || a.act_fn != HX_ACT_RELU2_NOGATE ? ep(0) : hx_h2{(_Float16)0.0f, (_Float16)0.0f};
    const hx_h2 su = ep(1), sd = ep(2);
    const float* pg = a.partial_g + (size_t)(slot * gg + cg) * (KB + 1) * 8 * 128;
    const float* pu = a.partial_u + (size_t)(slot * gg + cg) * (KB + 1) * 8 * 128;
    for (int i = threadIdx.x; i < 2 * MT * 128; i += hx_nthreads()) {
        const bool up = i >= MT * 128;
        const int k = up ? i - MT * 128 : i, m = k >> 7;
        const int n = up ? nu : ng;
        float v = 0.0f;
        if (m < si.count && (up || gated)) {
            // segment s, row m of the partial sums: (s * rows + m) * 128 + column; 8 segments' loads
            // together, added in segment order
            const float* p = (up ? pu : pg) + (size_t)m * 128 + (k & 127);
            const size_t stride = (size_t)si.count * 128;
            constexpr int B = 8;
            for (int s0 = 0; s0 < n; s0 += B) {
                float t[B];
#pragma unroll
                for (int j = 0; j < B; ++j)
                    t[j] = __hip_atomic_load(p + (size_t)min(s0 + j, n - 1) * stride, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                for (int j = 0; j < B; ++j)
                    if (s0 + j < n) v += t[j];
            }
        }
        (up ? cs_u : cs_g)[k] = v;
    }
    __syncthreads();
    guad_epilogue<MT>(a, plan, si, slot, cg, cs_g, cs_u, sg, su, sd);
    // the activations of this block are stored (device-coherent): flag them for the down phase
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (hx_vtid() == 0) __hip_atomic_store(&a.ready[slot * gg + cg], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Streams gate/up unit (c, j) and publishes its partial sum (gu_finish follows).
template <int BITS, int CB, int MT>
__device__ __forceinline__ void gu_segment(const MoeDecodeArgs& a, const DecodePlan& plan, const Split& sp, long c,
                                           int j, int slot, uint32_t* a_lds, float* cs_g, float* cs_u, int* rows)
{
    const int kb0 = sp.kb_begin(c, j), kb1 = sp.kb_begin(c, j + 1);
    const int gg = a.inter >> 7, KB = a.hidden >> 7;
    const int proj = (int)((c / gg) & 1), cg = (int)(c % gg);
    const SlotInfo si = slot_info(a, plan, slot);
    const bool shared = si.expert < 0;
    if (threadIdx.x < 8)
        rows[threadIdx.x] = shared ? (int)threadIdx.x : plan.token[si.start + min((int)threadIdx.x, si.count - 1)];
    hx_lds_barrier();

    GemvArgs g;
    g.x = a.x;
    g.rows = rows;
    g.trellis = static_cast<const uint16_t*>(plan.tab.tr);
    g.suh = static_cast<const _Float16*>(plan.tab.suh);
    g.M = si.count;
    g.K = a.hidden;
    g.N = a.inter;
    g.pre_transformed = false;
    gemv_range<BITS, CB, MT, 1, DEC_PF_GU>(g, cg, kb0 * 128, (kb1 - kb0) * 128, a_lds, cs_g);

    // partial of segment i of (slot, proj, cg): partial_{g,u}[((slot*gg + cg) * (KB + 1) + i) * 8 + m][128]
    float* pbase = (proj == 0 ? a.partial_g : a.partial_u) + (size_t)(slot * gg + cg) * (KB + 1) * 8 * 128;
    publish_partial<MT>(pbase, si.count, 128, 0, j, cs_g);
}

template <int BITS, int CB, int MT>
__device__ __forceinline__ void d_segment(const MoeDecodeArgs& a, const DecodePlan& plan, const Split& sp, long c,
                                          int j, int slot, uint32_t* a_lds, float* cs)
{
    const int kb0 = sp.kb_begin(c, j), kb1 = sp.kb_begin(c, j + 1);
    const int gd = a.hidden >> 7, gg = a.inter >> 7, KB = a.inter >> 7;
    const int cg = (int)(c % gd);
    const SlotInfo si = slot_info(a, plan, slot);
    const bool shared = si.expert < 0;

    GemvArgs g;
    g.x = a.act + (size_t)slot * 8 * a.inter;
    g.rows = nullptr;
    g.trellis = static_cast<const uint16_t*>(plan.tab.tr);
    g.suh = nullptr;
    g.M = si.count;
    g.K = a.inter;
    g.N = a.hidden;
    g.pre_transformed = true;
    // the input blocks kb0..kb1-1 of this slot are the guad outputs of gate/up column groups kb0..kb1-1
    auto wait_inputs = [&]() {
        if (hx_vwave() == 0) wait_flags(&a.ready[slot * gg + kb0], kb1 - kb0, 1, a.status);
        hx_lds_barrier();
    };
    gemv_range<BITS, CB, MT, 1, DEC_PF>(g, cg, kb0 * 128, (kb1 - kb0) * 128, a_lds, cs, wait_inputs);
}

// Split-K handoff of a down unit: publish, arrive; the last unit of the column group runs the down
// epilogue and, as the last slot of the column, the combine.
template <int MT>
__device__ __forceinline__ void d_finish(const MoeDecodeArgs& a, const DecodePlan& plan, const Split& sp, long c,
                                         int j, int slot, float* cs)
{
    const int gd = a.hidden >> 7, KB = a.inter >> 7;
    const int cg = (int)(c % gd);
    const SlotInfo si = slot_info(a, plan, slot);
    const int count = sp.count(c);
    float* pbase = a.partial_d + (size_t)(slot * gd + cg) * (KB + 1) * 8 * 128;
    publish_partial<MT>(pbase, si.count, 128, 0, j, cs);
    if (!arrive_last(&a.counter_d[slot * gd + cg], count)) return;
    gather_partials<MT>(pbase, si.count, 128, count, 0, cs);
    down_epilogue<MT>(a, plan, si, cg, cs);
    if (!a.combine) return;
    const bool has_shared = a.sh_tr[0] != nullptr;
    if (!arrive_last(&a.counter_y[cg], plan.n + (has_shared ? 1 : 0))) return;
    combine_columns(a, plan, cg, has_shared);
}

// Bits of a projection of a slot's expert (the shared slot uses the shared expert's).
HX_INLINE int slot_bits(const MoeDecodeArgs& a, const DecodePlan& p, int slot, int proj)
{
    const SlotInfo si = slot_info(a, p, slot);
    return proj_bits(a, proj, si.valid ? si.expert : 0);
}

// Runs unit (c, j) of a phase (one segment of one column group); units of inactive slots return.
template <int BITS, int CB, int MT>
__device__ __forceinline__ void run_unit(const MoeDecodeArgs& a, const DecodePlan& plan, const Split& sp, bool gu,
                                         long c, int j, uint32_t* a_lds, float* cs_g, float* cs_u, int* rows)
{
    const int gg = a.inter >> 7, gd = a.hidden >> 7;
    const int slot = unit_slot(a, plan, (int)(gu ? c / (2 * gg) : c / gd));
    if (slot < 0) return;
    // the non-gated relu2 (run on the BITS = 0 kernel only) has no routed gate GEMM: its gate units
    // only arrive
    const bool stream =
        BITS != 0 || !gu || a.act_fn != HX_ACT_RELU2_NOGATE || slot == a.routed_slots || ((c / gg) & 1) == 1;
    int bits = BITS;
    if constexpr (BITS == 0) bits = slot_bits(a, plan, slot, gu ? (int)((c / gg) & 1) : 2);
    if (stream) {
        switch (bits) {
#define HX_SEG_CASE(B)                                                                             \
    case B:                                                                                        \
        if constexpr (BITS == 0 || BITS == B) {                                                    \
            if (gu) gu_segment<B, CB, MT>(a, plan, sp, c, j, slot, a_lds, cs_g, cs_u, rows);         \
            else d_segment<B, CB, MT>(a, plan, sp, c, j, slot, a_lds, cs_g);                         \
        }                                                                                          \
        break;
            HX_SEG_CASE(1) HX_SEG_CASE(2) HX_SEG_CASE(3) HX_SEG_CASE(4)
            HX_SEG_CASE(5) HX_SEG_CASE(6) HX_SEG_CASE(7) HX_SEG_CASE(8)
#undef HX_SEG_CASE
            default:
                // a per-expert width outside 1..8 in the device bit tables: flagged for
                // hx_moe_check_status; the unit still takes part in its handoff below, so no
                // consumer waits for it and every counter returns to zero
                if (threadIdx.x == 0)
                    __hip_atomic_fetch_or(a.status, DEC_STATUS_BAD_BITS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
        }
    }
    if (gu) gu_finish<MT, BITS == 0>(a, plan, sp, c, slot, cs_g, cs_u);
    else d_finish<MT>(a, plan, sp, c, j, slot, cs_g);
}

// BITS = 0 dispatches each segment on its projection's bit width at run time (mixed-bit layers, and
// every layer of the non-gated relu2).
template <int BITS, int CB, int MT>
__device__ __forceinline__ void moe_decode_body(const MoeDecodeArgs& a)
{
    extern __shared__ uint32_t a_lds[];
    __shared__ float cs_g[MT * 128];
    __shared__ float cs_u[MT * 128];
    __shared__ DecodePlan plan;
    __shared__ int rows[8];
    HX_SETPRIO(3);  // the routing plan gates every workgroup
    const int gg = a.inter >> 7, gd = a.hidden >> 7;
    const int w = blockIdx.x, G = gridDim.x;
    const int nslots = a.routed_slots + 1;  // units exist for every possible slot
    const bool gu = w < a.units_gu;
    const Split sp = gu ? Split::make(nslots * 2 * gg, a.hidden >> 7, a.units_gu)
                        : Split::make(nslots * gd, a.inter >> 7, a.units_d);
    const int u = gu ? w : w - a.units_gu;
    const int c = sp.ucg(u), j = sp.uidx(u);
    const bool has_shared = a.sh_tr[0] != nullptr;
    const int us = gu ? c / (2 * gg) : c / gd;   // unit slot position (0: the shared expert, if any)
    const bool shared_unit = has_shared && us == 0;
    const int proj = gu ? (c / gg) & 1 : 2;       // the projection this unit streams
    if (gu && shared_unit && !(w == 0 && a.out_idx)) {
        // the shared expert's gate/up needs no routing: its tables are arguments, its rows every token
        if (hx_vtid() == 0) {
            plan.n = 0;
            load_slot_tables(a, plan.tab, -1, proj);
        }
        __syncthreads();
    } else {
        // every workgroup routes for itself: the scores are a few plain (cached) loads, whereas a
        // plan published by one workgroup would be read by all with device-coherent loads of the
        // same few lines (measured: 54 -> 97 us for the config-3 layer, the weight streams through
        // those lines' memory channel stall)
        build_plan<MT>(a, plan, shared_unit ? DEC_SHARED : (has_shared ? us - 1 : us), proj);
    }
    if (blockIdx.x == 0 && a.out_idx) {
        const int R = a.T * a.topk;
        for (int i = threadIdx.x; i < R; i += hx_nthreads()) {
            const int pos = plan.r2s[i];
            int e = 0;
            for (int qq = 0; qq < plan.n; ++qq)
                if (pos >= plan.start[qq] && pos < plan.start[qq] + plan.count[qq]) e = plan.expert[qq];
            a.out_idx[i] = e;
            a.out_w[i] = (_Float16)plan.weight[pos];
        }
    }
    run_unit<BITS, CB, MT>(a, plan, sp, gu, c, j, a_lds, cs_g, cs_u, rows);
    // the last workgroup to finish clears the activation flags for the next call
    __shared__ bool last;
    if (hx_vtid() == 0)
        last = __hip_atomic_fetch_add(a.exit_count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1;
    __syncthreads();
    if (last) {
        for (int i = threadIdx.x; i < (a.routed_slots + 1) * gg; i += hx_nthreads())
            __hip_atomic_store(&a.ready[i], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (hx_vtid() == 0) __hip_atomic_store(a.exit_count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Fixed bit width: at most 128 VGPRs so that 16 waves (4 workgroups) share a CU, and
// exactly that occupancy as the scheduling target (4 waves per SIMD).  Without the upper bound the
// compiler trades the streaming loop's latency hiding for registers to reach 6 waves per SIMD,
// which the launch never uses (measured 58 against 51 us at config 3).
template <int BITS, int CB, int MT>
__global__ __launch_bounds__(DEC_THREADS, 4) __attribute__((amdgpu_waves_per_eu(4, 4)))
void moe_decode_kernel(MoeDecodeArgs a)
{
    moe_decode_body<BITS, CB, MT>(a);
}

// Mixed bit widths (per-segment dispatch); the larger code keeps the default register budget.
template <int CB, int MT>
__global__ __launch_bounds__(DEC_THREADS) void moe_decode_mixed_kernel(MoeDecodeArgs a)
{
    moe_decode_body<0, CB, MT>(a);
}

}  // namespace hx
