// helios/exl3_compat.hpp -- header-only C++ layer that re-creates the reference engine's EXL3,
// router and MoE-glue signatures on top of the C ABI in hx/exl3.h, so the engine's call sites
// (src/engine/runner.cpp) compile unchanged against libhx_exl3.so.
//
// Differences a caller sees: errors throw helios::exl3::Error (the reference aborts); the fused
// kernels need a workspace, which this layer keeps per (device, stream) (allocated on first use, zeroed
// once, never freed while the process runs) unless the caller installs one with set_workspace().
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <stdexcept>
#include <string>
#include <map>

#include "../hx/exl3.h"

namespace helios {

using Stream = hipStream_t;

namespace exl3 {

// reference: src/cuda/quant/helios_shim.cuh:120-124
enum class DType : int { Half = HX_DTYPE_HALF, Float = HX_DTYPE_FLOAT };

struct Error : std::runtime_error {
    explicit Error(const std::string& s) : std::runtime_error(s) {}
};

inline int check(int code, const char* what)
{
    if (code < 0) throw Error(std::string(what) + ": " + hx_last_error());
    return code;
}

// Workspace of one (device, stream) pair (the reference keeps one lock buffer per device,
// src/cuda/quant/exl3_devctx.cu:60-71, and is unsafe across streams).  Calls on different streams get
// different buffers, so their arrival counters and ready flags never meet.  A buffer that must grow is
// replaced after a device-wide synchronisation, since kernels queued on any stream may still use it.
// Grow outside graph capture: run each call shape once on the capturing stream first.
class Workspace {
public:
    struct View {
        void* ptr;
        size_t bytes;
    };
    static Workspace& get()
    {
        static Workspace w;
        return w;
    }
    View acquire(size_t bytes, Stream s)
    {
        std::lock_guard<std::mutex> g(mu_);
        int dev = 0;
        (void)hipGetDevice(&dev);
        auto it = installed_.find(dev);
        if (it != installed_.end()) {
            if (it->second.bytes < bytes) throw Error("installed workspace is smaller than the call needs");
            return View{it->second.ptr, it->second.bytes};
        }
        Slot& slot = slots_[Key{dev, s}];
        if (slot.bytes < bytes) {
            if (slot.ptr) {
                if (hipDeviceSynchronize() != hipSuccess) throw Error("device synchronisation failed");
                (void)hipFree(slot.ptr);
                slot = Slot{};
            }
            if (hipMalloc(&slot.ptr, bytes) != hipSuccess) throw Error("workspace allocation failed");
            slot.bytes = bytes;
            check(hx_workspace_init(slot.ptr, bytes, (hx_stream_t)s), "hx_workspace_init");
        }
        return View{slot.ptr, slot.bytes};
    }
    // Install a caller-owned, zero-filled workspace for every call on the current device; the caller
    // then keeps calls on different streams from overlapping.
    void set(void* ptr, size_t bytes)
    {
        std::lock_guard<std::mutex> g(mu_);
        int dev = 0;
        (void)hipGetDevice(&dev);
        installed_[dev] = Slot{ptr, bytes};
    }

private:
    struct Slot {
        void* ptr = nullptr;
        size_t bytes = 0;
    };
    struct Key {
        int dev;
        Stream stream;
        bool operator<(const Key& o) const { return dev != o.dev ? dev < o.dev : stream < o.stream; }
    };
    std::mutex mu_;
    std::map<Key, Slot> slots_;
    std::map<int, Slot> installed_;
};

inline void set_workspace(void* ptr, size_t bytes) { Workspace::get().set(ptr, bytes); }

// reference: src/cuda/quant/exl3_gemm.cuh:30-36
struct GroupWords {
    const uint16_t* trellis;
    const void* suh;
    const void* svh;
    int mul1;
};

// reference: src/cuda/quant/exl3_gemm.cuh:51-66 (force_shape_idx / force_num_sms are accepted and
// ignored: the kernel choice is by M)
inline int gemm(void* y, const void* x, const GroupWords& w, int M, int N, int K, int bits, bool y_fp32 = false,
                Stream s = 0, void* a_had = nullptr, bool mcg = false, int force_shape_idx = 0, int force_num_sms = 0)
{
    (void)force_shape_idx;
    (void)force_num_sms;
    const hx_group_words g{w.trellis, w.suh, w.svh, w.mul1};
    const size_t ws_bytes = hx_exl3_gemm_workspace_size(M, N, K);
    const Workspace::View ws = Workspace::get().acquire(ws_bytes, s);
    return check(hx_exl3_gemm(y, x, &g, M, N, K, bits, y_fp32, (hx_stream_t)s, a_had, mcg, ws.ptr,
                              ws.bytes),
                 "helios::exl3::gemm");
}

// reference: src/cuda/quant/exl3_gemm.cuh:70-83 (small-M path; M <= 16 here)
inline void gemv(void* y, const void* x, const GroupWords& w, int M, int N, int K, int bits, bool y_fp32 = false,
                 Stream s = 0, void* a_had = nullptr, bool mcg = false)
{
    if (M > 16) throw Error("helios::exl3::gemv: M must be <= 16");
    gemm(y, x, w, M, N, K, bits, y_fp32, s, a_had, mcg);
}

// reference: src/cuda/quant/reconstruct.cuh:15-63
inline void reconstruct_slice(void* unpacked, const void* packed, int packed_rows, int packed_cols, int unpacked_cols,
                              int K, bool mcg, bool mul1, int64_t n_offset, Stream s = 0)
{
    check(hx_exl3_reconstruct_slice(unpacked, packed, packed_rows, packed_cols, unpacked_cols, K, mcg, mul1, n_offset,
                                    (hx_stream_t)s),
          "helios::exl3::reconstruct_slice");
}
inline void reconstruct(void* unpacked, const void* packed, int packed_rows, int packed_cols, int unpacked_cols, int K,
                        bool mcg, bool mul1, Stream s = 0)
{
    reconstruct_slice(unpacked, packed, packed_rows, packed_cols, unpacked_cols, K, mcg, mul1, 0, s);
}
// reference: src/cuda/quant/reconstruct.cuh:37-63
inline void reconstruct_had_slice(void* unpacked, const void* packed, const void* suh, const void* svh, int packed_rows,
                                  int packed_cols, int unpacked_rows, int unpacked_cols, int K, bool mcg, bool mul1,
                                  int64_t n_offset, Stream s = 0)
{
    check(hx_exl3_reconstruct_had_slice(unpacked, packed, suh, svh, packed_rows, packed_cols, unpacked_rows,
                                        unpacked_cols, K, mcg, mul1, n_offset, (hx_stream_t)s),
          "helios::exl3::reconstruct_had_slice");
}
// reference: src/cuda/quant/pack.cuh:9-33
inline void pack_trellis(void* packed, const void* unpacked, int rows, int cols, int K, Stream s = 0)
{
    check(hx_exl3_pack_trellis(packed, unpacked, rows, cols, K, (hx_stream_t)s), "helios::exl3::pack_trellis");
}
inline void unpack_trellis(void* unpacked, const void* packed, int rows, int cols, int K, Stream s = 0)
{
    check(hx_exl3_unpack_trellis(unpacked, packed, rows, cols, K, (hx_stream_t)s), "helios::exl3::unpack_trellis");
}

// reference: src/cuda/quant/pack.cuh:36-44 (packed[c] bit i = sign of unpacked[16 c + i])
inline void pack_signs(void* packed, const void* unpacked, int cols, Stream s = 0)
{
    check(hx_pack_signs(packed, unpacked, cols, (hx_stream_t)s), "helios::exl3::pack_signs");
}

// reference: src/cuda/quant/util.cuh:9-19 (y[0] += infinities, y[1] += NaNs; the caller zeroes y)
inline void count_inf_nan(const void* x, unsigned long long* y, uint64_t numel, DType dt, Stream s = 0)
{
    check(hx_count_inf_nan(x, y, numel, (int)dt, (hx_stream_t)s), "helios::exl3::count_inf_nan");
}

// reference: src/cuda/quant/exl3_moe.cuh:35
inline int moe_max_concurrency(int device) { return check(hx_moe_max_concurrency(device), "helios::exl3::moe_max_concurrency"); }

// reference: src/cuda/quant/exl3_moe.cuh:20-31
struct ExpertTables {
    const uint16_t** gate_trellis;
    const void** gate_suh;
    const void** gate_svh;
    const uint16_t** up_trellis;
    const void** up_suh;
    const void** up_svh;
    const uint16_t** down_trellis;
    const void** down_suh;
    const void** down_svh;
};

// reference: src/cuda/quant/exl3_moe.cuh:74-105.  Without sorted_contributions the reference
// accumulates into y atomically; this build adds the routed sum in routing-rank order, which needs
// the permutation's route_to_sorted (pass it as the last argument).
inline void moe_grouped(const void* x, void* y, const int64_t* expert_count, const int64_t* token_sorted,
                        const void* weight_sorted, void* temp_state_g, void* temp_state_u, void* temp_intermediate_g,
                        void* temp_intermediate_u, const ExpertTables& tables, int tokens, int hidden_dim,
                        int intermediate_dim, int num_experts, int topk, int max_tokens_per_expert, int concurrency,
                        int K_gate, int K_up, int K_down, bool mcg = false, bool mul1 = false, float act_limit = 10.0f,
                        int act_function = 0, int num_active = -1, Stream s = 0,
                        float* sorted_contributions = nullptr, const int64_t* route_to_sorted = nullptr)
{
    const hx_expert_tables t{reinterpret_cast<const void* const*>(tables.gate_trellis),
                             reinterpret_cast<const void* const*>(tables.gate_suh),
                             reinterpret_cast<const void* const*>(tables.gate_svh),
                             reinterpret_cast<const void* const*>(tables.up_trellis),
                             reinterpret_cast<const void* const*>(tables.up_suh),
                             reinterpret_cast<const void* const*>(tables.up_svh),
                             reinterpret_cast<const void* const*>(tables.down_trellis),
                             reinterpret_cast<const void* const*>(tables.down_suh),
                             reinterpret_cast<const void* const*>(tables.down_svh),
                             nullptr, nullptr, nullptr, 0u};
    const size_t ws_bytes = hx_moe_workspace_size(tokens, hidden_dim, intermediate_dim, num_experts, topk);
    const Workspace::View ws = Workspace::get().acquire(ws_bytes, s);
    check(hx_moe_grouped(x, static_cast<float*>(y), expert_count, token_sorted, weight_sorted, temp_state_g,
                         temp_state_u, temp_intermediate_g, temp_intermediate_u, &t, tokens, hidden_dim,
                         intermediate_dim, num_experts, topk, max_tokens_per_expert, concurrency, K_gate, K_up, K_down,
                         mcg, mul1, act_limit, act_function, num_active, (hx_stream_t)s, sorted_contributions,
                         route_to_sorted, ws.ptr, ws.bytes),
          "helios::exl3::moe_grouped");
}

// The whole single-GPU MoE FFN layer in one call (router, permutation, routed experts, shared
// expert, ordered combine; hx_moe_layer).  No reference counterpart: it replaces the sequence of
// runner.cpp:711-959 (Runner::moe_ffn) for one GPU.  shared may be null (no shared expert).
inline void moe_layer(void* y, float* y_routed, const void* x, const void* scores, const void* bias,
                      const ExpertTables& tables, const GroupWords* shared, const int* shared_bits, int tokens,
                      int hidden_dim, int intermediate_dim, int num_experts, int topk, int K_gate, int K_up,
                      int K_down, float routed_scale, float act_limit = 10.0f, bool mcg = false, bool mul1 = true,
                      Stream s = 0)
{
    const hx_expert_tables t{reinterpret_cast<const void* const*>(tables.gate_trellis),
                             reinterpret_cast<const void* const*>(tables.gate_suh),
                             reinterpret_cast<const void* const*>(tables.gate_svh),
                             reinterpret_cast<const void* const*>(tables.up_trellis),
                             reinterpret_cast<const void* const*>(tables.up_suh),
                             reinterpret_cast<const void* const*>(tables.up_svh),
                             reinterpret_cast<const void* const*>(tables.down_trellis),
                             reinterpret_cast<const void* const*>(tables.down_suh),
                             reinterpret_cast<const void* const*>(tables.down_svh),
                             nullptr, nullptr, nullptr, 0u};
    hx_group_words sh[3];
    if (shared)
        for (int i = 0; i < 3; ++i) sh[i] = hx_group_words{shared[i].trellis, shared[i].suh, shared[i].svh, shared[i].mul1};
    const size_t ws_bytes = hx_moe_workspace_size(tokens, hidden_dim, intermediate_dim, num_experts, topk);
    const Workspace::View ws = Workspace::get().acquire(ws_bytes, s);
    check(hx_moe_layer(y, y_routed, x, scores, bias, &t, shared ? sh : nullptr, shared_bits, tokens, hidden_dim,
                       intermediate_dim, num_experts, topk, K_gate, K_up, K_down, routed_scale, act_limit, mcg, mul1,
                       ws.ptr, ws.bytes, (hx_stream_t)s),
          "helios::exl3::moe_layer");
}

// reference: src/cuda/quant/hadamard.cuh:14-25 (the kernel multiplies by scale / sqrt(128); fp16 or fp32
// data; pre_scale and post_scale are exclusive)
inline void had_r_128(const void* input, void* output, const void* pre_scale, const void* post_scale, int rows,
                      int cols, DType dt, float scale, Stream s = 0)
{
    check(hx_had_r_128(input, output, pre_scale, post_scale, rows, cols, (int)dt, scale, (hx_stream_t)s),
          "helios::exl3::had_r_128");
}

// reference: src/cuda/quant/hadamard.cuh:27-43
inline void had_r_128_dual(const void* input1, void* output1, const void* pre_scale1, const void* post_scale1,
                           const void* input2, void* output2, const void* pre_scale2, const void* post_scale2, int rows,
                           int cols, DType dt, float scale, Stream s = 0)
{
    check(hx_had_r_128_dual(input1, output1, pre_scale1, post_scale1, input2, output2, pre_scale2, post_scale2, rows,
                            cols, (int)dt, scale, (hx_stream_t)s),
          "helios::exl3::had_r_128_dual");
}

}  // namespace exl3

namespace aux {
// reference: src/cuda/aux/routing.cuh:36-49
inline void routing_ds3_nogroup(const void* scores, const void* bias, int64_t* topk_indices, void* topk_weights,
                                int bsz, int num_experts, int K, float scaling_factor, bool use_topk = true,
                                int act_fn = 0, Stream s = 0)
{
    exl3::check(hx_routing_ds3_nogroup(scores, bias, topk_indices, topk_weights, bsz, num_experts, K, scaling_factor,
                                       use_topk, act_fn, (hx_stream_t)s),
                "helios::aux::routing_ds3_nogroup");
}

// reference: src/cuda/aux/routing.cuh:9-17
enum RoutingAct : int { ROUTING_ACT_SIGMOID = 0, ROUTING_ACT_SQRTSP = 1 };

// reference: src/cuda/aux/routing.cuh:19-29
inline void routing_gemv(const void* x, const void* gate_t, void* scores, int k, int E, Stream s = 0)
{
    exl3::check(hx_routing_gemv(x, gate_t, scores, k, E, (hx_stream_t)s), "helios::aux::routing_gemv");
}

// reference: src/cuda/aux/routing.cuh:51-66
inline void routing_ds3_nogroup_hidden(const void* hidden, const void* gate_t, void* scores, const void* bias,
                                       int64_t* topk_indices, void* topk_weights, int k, int num_experts, int K,
                                       float scaling_factor, int act_fn = ROUTING_ACT_SIGMOID, Stream s = 0)
{
    exl3::check(hx_routing_ds3_nogroup_hidden(hidden, gate_t, scores, bias, topk_indices, topk_weights, k, num_experts,
                                              K, scaling_factor, act_fn, (hx_stream_t)s),
                "helios::aux::routing_ds3_nogroup_hidden");
}
}  // namespace aux

namespace glue {
// reference: src/engine/glue2.cuh:44-49, :64
inline void moe_permute(const int64_t* ids, const void* weights, int M, int topk, int E, int64_t* expert_count,
                        int64_t* token_sorted, void* weight_sorted, int64_t* workspace, Stream s = 0,
                        int64_t* route_to_sorted = nullptr)
{
    exl3::check(hx_moe_permute(ids, weights, M, topk, E, expert_count, token_sorted, weight_sorted, workspace,
                               (hx_stream_t)s, route_to_sorted),
                "helios::glue::moe_permute");
}
inline void moe_reduce_sorted(float* y, const float* contributions, const int64_t* route_to_sorted, int M, int topk,
                              int hidden, Stream s = 0)
{
    exl3::check(hx_moe_reduce_sorted(y, contributions, route_to_sorted, M, topk, hidden, (hx_stream_t)s),
                "helios::glue::moe_reduce_sorted");
}
inline void swiglu_clamp(const float* gate, const float* up, void* out, size_t n, float limit, Stream s = 0)
{
    exl3::check(hx_swiglu_clamp(gate, up, out, n, limit, (hx_stream_t)s), "helios::glue::swiglu_clamp");
}
// reference: src/engine/glue.cuh:14-17 (the dense-MoE fallback, runner.cpp:902-907)
inline void gather_rows(const void* src, const int64_t* idx, void* dst, int n, int h, Stream s = 0)
{
    exl3::check(hx_gather_rows(src, idx, dst, n, h, (hx_stream_t)s), "helios::glue::gather_rows");
}
inline void scatter_add_rows(float* y, const float* src, const int64_t* idx, const void* w, int n, int h,
                             Stream s = 0)
{
    exl3::check(hx_scatter_add_rows(y, src, idx, w, n, h, (hx_stream_t)s), "helios::glue::scatter_add_rows");
}
// reference: src/engine/glue2.cuh:9-10 (router logits and other dense fp16 NT products)
inline void gemm_nt_f16(void* y, const void* x, const void* w, int M, int N, int K, bool y_fp32, bool add,
                        Stream s = 0)
{
    exl3::check(hx_gemm_nt_f16(y, x, w, M, N, K, y_fp32 ? 1 : 0, add ? 1 : 0, (hx_stream_t)s),
                "helios::glue::gemm_nt_f16");
}
}  // namespace glue

}  // namespace helios
