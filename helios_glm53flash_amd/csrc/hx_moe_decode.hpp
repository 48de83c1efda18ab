// hx_moe_decode.hpp -- fused MoE layer for few tokens (T <= 8) on gfx950: every active expert's
// gate/up GEMV, the SiLU-gate, the down GEMV and the weighted contribution rows, with trellis decode
// fused into the GEMVs, in two launches without host synchronisation.
//
// Reference semantics: src/cuda/quant/exl3_moe_kernel.cuh:57-262 (per expert: gather, input
// Hadamard with suh_g/suh_u, G/U GEMMs with fp16 outputs, guad epilogue, down GEMM with fp16
// output, d epilogue with weight/sqrt(128) and svh_d), hadamard_inner.cuh:284-481, and for the
// shared expert src/engine/runner.cpp:723-738 + glue2.cu:406-414.
//
// Slots: slot j < n_routed_slots is the j-th expert (in expert-index order) with a nonzero count in
// expert_count (the reference's ticket numbering, exl3_moe_kernel.cuh:57-69); its rows are the
// expert's sorted routing rows [start, start + count).  With a shared expert, one extra slot holds
// all T tokens.  Each workgroup finds its slot's expert by a wave scan of expert_count, so the launch
// grid is sized by the upper bound min(E, T*topk) and surplus workgroups exit.
#pragma once
#include "hx_gemv.hpp"

namespace hx {

struct MoeDecodeArgs {
    const _Float16* x;             // [T][hidden]
    int T, hidden, inter, E, topk;
    const int64_t* expert_count;   // [E+1]
    const int64_t* token_sorted;   // [T*topk]
    const _Float16* weight_sorted; // [T*topk]
    // routed expert tables (device arrays of device pointers), per-expert bits (nullable)
    const void* const* tr[3];
    const void* const* suh[3];
    const void* const* svh[3];
    const int32_t* bits_tab[3];
    int bits_uniform[3];
    // shared expert (nullable trellis -> none)
    const void* sh_tr[3];
    const void* sh_suh[3];
    const void* sh_svh[3];
    int sh_bits[3];
    float act_limit;
    int routed_slots;              // upper bound of active experts
    int splits_gu, kc_gu, splits_d, kc_d;
    // workspace
    int* counter_gu;               // [slots][inter/128]
    int* counter_d;                // [slots][hidden/128]
    float* partial_g;              // [slots][splits_gu][8][inter]
    float* partial_u;
    float* partial_d;              // [slots][splits_d][8][hidden]
    _Float16* act;                 // [slots][8][inter]  (down-projection input, already transformed)
    // outputs
    float* contrib;                // [T*topk (+ T)][hidden]: sorted routed rows, then shared rows
};

struct SlotInfo {
    int expert;  // -1: shared slot
    int start;   // first sorted row
    int count;   // rows
    bool valid;
};

// Wave-uniform scan of expert_count for the slot-th active expert.
HX_INLINE SlotInfo find_slot(const MoeDecodeArgs& a, int slot)
{
    SlotInfo si{0, 0, 0, false};
    if (slot == a.routed_slots) {  // shared
        si.expert = -1;
        si.start = 0;
        si.count = a.T;
        si.valid = a.sh_tr[0] != nullptr;
        return si;
    }
    const int lane = threadIdx.x & 63;
    int seen = 0, base = 0;
    for (int e0 = 0; e0 < a.E; e0 += 64) {
        const int e = e0 + lane;
        const int c = e < a.E ? (int)a.expert_count[e] : 0;
        // inclusive scan of counts and of "active" flags across the wave
        int cs = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            int v = __shfl_up(cs, o, 64);
            if (lane >= o) cs += v;
        }
        const uint64_t act = __ballot(c > 0);
        const int before = __popcll(act & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
        const bool hit = c > 0 && seen + before == slot;
        const uint64_t hm = __ballot(hit);
        if (hm) {
            const int l = __ffsll((unsigned long long)hm) - 1;
            si.expert = e0 + l;
            si.start = base + __shfl(cs - c, l, 64);
            si.count = __shfl(c, l, 64);
            si.valid = true;
            return si;
        }
        seen += __popcll(act);
        base += __shfl(cs, 63, 64);
    }
    return si;
}

HX_INLINE int proj_bits(const MoeDecodeArgs& a, int proj, int expert)
{
    if (expert < 0) return a.sh_bits[proj];
    return a.bits_tab[proj] ? a.bits_tab[proj][expert] : a.bits_uniform[proj];
}

// ------------------------------------------------------------------ kernel A: gate/up + SiLU-gate

// guad epilogue for rows m < count of one 128-column group (hadamard_inner.cuh:284-413 for routed
// experts; swiglu_clamp + down-input transform for the shared expert).
template <int MT>
__device__ void guad_epilogue(const MoeDecodeArgs& a, const SlotInfo& si, int slot, int cg, const float* cs_g,
                              const float* cs_u)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c = cg * 128 + 2 * lane;
    const bool shared = si.expert < 0;
    const _Float16* svg = static_cast<const _Float16*>(shared ? a.sh_svh[0] : a.svh[0][si.expert]);
    const _Float16* svu = static_cast<const _Float16*>(shared ? a.sh_svh[1] : a.svh[1][si.expert]);
    const _Float16* sud = static_cast<const _Float16*>(shared ? a.sh_suh[2] : a.suh[2][si.expert]);
    const hx_h2 sg = *reinterpret_cast<const hx_h2*>(svg + c);
    const hx_h2 su = *reinterpret_cast<const hx_h2*>(svu + c);
    const hx_h2 sd = *reinterpret_cast<const hx_h2*>(sud + c);
    const float L = a.act_limit;
    for (int m = wave; m < si.count && m < MT; m += GEMV_WAVES) {
        hx_h2 p;
        if (!shared) {
            // G, U as fp16 (the reference GEMM writes fp16), transform, fp16, times svh (fp16)
            hx_h2 G = {(_Float16)cs_g[m * 128 + 2 * lane], (_Float16)cs_g[m * 128 + 2 * lane + 1]};
            hx_h2 U = {(_Float16)cs_u[m * 128 + 2 * lane], (_Float16)cs_u[m * 128 + 2 * lane + 1]};
            float g0 = (float)G.x, g1 = (float)G.y, u0 = (float)U.x, u1 = (float)U.y;
            hx_had128_wave(g0, g1);
            hx_had128_wave(u0, u1);
            hx_h2 g = hx_h2{(_Float16)g0, (_Float16)g1} * sg;
            hx_h2 u = hx_h2{(_Float16)u0, (_Float16)u1} * su;
            g.x = hx_silu_h(g.x);
            g.y = hx_silu_h(g.y);
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
        *reinterpret_cast<hx_h2*>(a.act + ((size_t)slot * 8 + m) * a.inter + c) = o;
    }
}

template <int BITS, int CB, int MT>
__global__ __launch_bounds__(GEMV_THREADS) void moe_decode_gu_kernel(MoeDecodeArgs a)
{
    extern __shared__ uint32_t a_lds[];
    __shared__ float red[GEMV_WAVES * MT * 128];
    __shared__ float cs_g[MT * 128];
    __shared__ float cs_u[MT * 128];
    const int groups = a.inter >> 7;
    const int per_slot = 2 * groups * a.splits_gu;
    const int slot = blockIdx.x / per_slot;
    int r = blockIdx.x % per_slot;
    const int s = r / (2 * groups);
    r %= 2 * groups;
    const int proj = r / groups;  // 0 gate, 1 up
    const int cg = r % groups;
    const SlotInfo si = find_slot(a, slot);
    if (!si.valid) return;
    if (proj_bits(a, proj, si.expert) != BITS) return;
    const bool shared = si.expert < 0;

    GemvArgs g;
    g.x = a.x;
    g.rows = shared ? nullptr : a.token_sorted + si.start;
    g.trellis = static_cast<const uint16_t*>(shared ? a.sh_tr[proj] : a.tr[proj][si.expert]);
    g.suh = static_cast<const _Float16*>(shared ? a.sh_suh[proj] : a.suh[proj][si.expert]);
    g.M = si.count;
    g.K = a.hidden;
    g.N = a.inter;
    g.splits = a.splits_gu;
    g.kc = a.kc_gu;
    g.pre_transformed = false;
    float* partial = (proj == 0 ? a.partial_g : a.partial_u) + (size_t)slot * a.splits_gu * 8 * a.inter;
    g.partial = partial;

    gemv_split_sum<BITS, CB, MT>(g, cg, s, a_lds, red, cs_g);
    publish_partial<MT>(partial, g.M, g.N, cg, s, cs_g);
    if (!arrive_last(&a.counter_gu[slot * groups + cg], 2 * a.splits_gu)) return;
    gather_partials<MT>(a.partial_g + (size_t)slot * a.splits_gu * 8 * a.inter, g.M, g.N, a.splits_gu, cg, cs_g);
    gather_partials<MT>(a.partial_u + (size_t)slot * a.splits_gu * 8 * a.inter, g.M, g.N, a.splits_gu, cg, cs_u);
    guad_epilogue<MT>(a, si, slot, cg, cs_g, cs_u);
}

// ------------------------------------------------------------------ kernel B: down + contributions

template <int MT>
__device__ void down_epilogue(const MoeDecodeArgs& a, const SlotInfo& si, int cg, const float* cs)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c = cg * 128 + 2 * lane;
    const bool shared = si.expert < 0;
    const _Float16* svd = static_cast<const _Float16*>(shared ? a.sh_svh[2] : a.svh[2][si.expert]);
    const hx_h2 sd = *reinterpret_cast<const hx_h2*>(svd + c);
    const int R = a.T * a.topk;
    for (int m = wave; m < si.count && m < MT; m += GEMV_WAVES) {
        float d0, d1, wgt;
        size_t row;
        if (!shared) {
            // D as fp16 (reference GEMM output), transform, times weight / sqrt(128) and svh_d in fp32
            d0 = (float)(_Float16)cs[m * 128 + 2 * lane];
            d1 = (float)(_Float16)cs[m * 128 + 2 * lane + 1];
            wgt = (float)a.weight_sorted[si.start + m];
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
        *reinterpret_cast<float2*>(a.contrib + row * a.hidden + c) = make_float2(d0, d1);
    }
}

template <int BITS, int CB, int MT>
__global__ __launch_bounds__(GEMV_THREADS) void moe_decode_d_kernel(MoeDecodeArgs a)
{
    extern __shared__ uint32_t a_lds[];
    __shared__ float red[GEMV_WAVES * MT * 128];
    __shared__ float cs[MT * 128];
    const int groups = a.hidden >> 7;
    const int per_slot = groups * a.splits_d;
    const int slot = blockIdx.x / per_slot;
    const int r = blockIdx.x % per_slot;
    const int s = r / groups;
    const int cg = r % groups;
    const SlotInfo si = find_slot(a, slot);
    if (!si.valid) return;
    if (proj_bits(a, 2, si.expert) != BITS) return;
    const bool shared = si.expert < 0;

    GemvArgs g;
    g.x = a.act + (size_t)slot * 8 * a.inter;
    g.rows = nullptr;
    g.trellis = static_cast<const uint16_t*>(shared ? a.sh_tr[2] : a.tr[2][si.expert]);
    g.suh = nullptr;
    g.M = si.count;
    g.K = a.inter;
    g.N = a.hidden;
    g.splits = a.splits_d;
    g.kc = a.kc_d;
    g.pre_transformed = true;
    float* partial = a.partial_d + (size_t)slot * a.splits_d * 8 * a.hidden;
    g.partial = partial;

    gemv_split_sum<BITS, CB, MT>(g, cg, s, a_lds, red, cs);
    if (a.splits_d > 1) {
        publish_partial<MT>(partial, g.M, g.N, cg, s, cs);
        if (!arrive_last(&a.counter_d[slot * groups + cg], a.splits_d)) return;
        gather_partials<MT>(partial, g.M, g.N, a.splits_d, cg, cs);
    }
    down_epilogue<MT>(a, si, cg, cs);
}

}  // namespace hx
