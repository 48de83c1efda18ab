// hx_kernels.hpp -- host-side launchers shared by the kernel translation units and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace hx {

// Every workspace starts with a fixed counter area (arrival counters of the split-K / last-arriver
// epilogues).  It is zero-filled once by the caller, every kernel leaves the counters it used at
// zero, and no call ever stores data into it, so calls of different shapes can share a workspace.
constexpr size_t HX_COUNTER_BYTES = 64 * 1024;

// Largest M served by the decode-GEMV kernels (one MFMA row block); larger M uses the MFMA GEMM.
constexpr int GEMV_MAX_M = 16;

// small-M linear (hx_linear.hip)
// Grid of the small-M linear: either column groups x `splits` k chunks of `kc`, or (one row, many
// 128-k blocks) `sk_wgs` workgroups over equal runs of (column group, block) units, whose column
// groups are shared by at most `slots` workgroups (stream-K).
struct GemvPlan {
    int splits, kc;
    int sk_wgs, sk_blocks, slots;
};
GemvPlan gemv_plan(int M, int K, int N);
size_t gemv_workspace_bytes(int M, int K, int N);
hipError_t launch_linear_gemv(const _Float16* x, const uint16_t* trellis, const _Float16* suh, const _Float16* svh,
                              void* y, int M, int K, int N, int bits, int cb, bool y_fp32, void* ws, hipStream_t st);

// large-M linear on MFMA (hx_gemm.hip)
hipError_t launch_input_had(const _Float16* x, const _Float16* suh, _Float16* a, long rows, int K, hipStream_t st);
hipError_t launch_linear_mfma(const _Float16* a_had, const uint16_t* trellis, const _Float16* svh, void* y,
                              int M, int K, int N, int bits, int cb, bool y_fp32, hipStream_t st);

// utilities (hx_misc.hip)
hipError_t launch_reconstruct(_Float16* out, const uint16_t* packed, int packed_rows, int packed_cols,
                              int unpacked_cols, int bits, int cb, long n_offset, hipStream_t st);
hipError_t launch_pack_signs(uint16_t* packed, const uint16_t* unpacked, int cols, hipStream_t st);
hipError_t launch_count_inf_nan(const void* x, unsigned long long* counts, uint64_t numel, bool fp32, hipStream_t st);
hipError_t launch_had_r_128(const void* in1, void* out1, const void* scale1, const void* in2, void* out2,
                            const void* scale2, int scale_mode, long rows, int cols, bool fp32, float r_scale,
                            hipStream_t st);
hipError_t launch_routing(const _Float16* scores, const _Float16* bias, int64_t* idx, _Float16* w, int bsz, int E,
                          int K, float scale, hipStream_t st, bool use_topk = true, int act_fn = 0);
hipError_t launch_permute(const int64_t* ids, const _Float16* w, int M, int topk, int E, int64_t* expert_count,
                          int64_t* token_sorted, _Float16* weight_sorted, int64_t* route_to_sorted,
                          int64_t* workspace, hipStream_t st);
// Chunked permutation for many routes (same result as launch_permute): scratch holds
// 2 * ceil(M*topk/1024) * E ints, arrive is a zero-initialised counter (left zero).
hipError_t launch_permute_chunked(const int64_t* ids, const _Float16* w, int M, int topk, int E, int64_t* expert_count,
                                  int64_t* token_sorted, _Float16* weight_sorted, int64_t* route_to_sorted,
                                  int* scratch, int* arrive, hipStream_t st);
hipError_t launch_reduce_sorted(float* y, const float* contrib, const int64_t* route_to_sorted, int M, int topk,
                                int hidden, hipStream_t st);
hipError_t launch_swiglu_clamp(const float* g, const float* u, _Float16* out, size_t n, float limit, hipStream_t st);
hipError_t launch_pack_trellis(uint16_t* packed, const uint16_t* unpacked, long blocks, int K, hipStream_t st);
hipError_t launch_unpack_trellis(uint16_t* unpacked, const uint16_t* packed, long blocks, int K, hipStream_t st);
hipError_t launch_reconstruct_had(_Float16* out, const uint16_t* packed, const _Float16* suh, const _Float16* svh,
                                  int packed_rows, int packed_cols, int unpacked_rows, int unpacked_cols, int bits,
                                  int cb, long n_offset, hipStream_t st);
hipError_t launch_gather_rows(const _Float16* src, const int64_t* idx, _Float16* dst, int n, int h, hipStream_t st);
hipError_t launch_scatter_add_rows(float* y, const float* src, const int64_t* idx, const _Float16* w, int n, int h,
                                   hipStream_t st);
hipError_t launch_gemm_nt_f16(const _Float16* x, const _Float16* w, void* y, int M, int N, int K, bool y_fp32,
                              bool add, hipStream_t st);

}  // namespace hx
