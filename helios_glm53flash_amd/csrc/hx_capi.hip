// hx_capi.hip -- extern "C" boundary of libhx_exl3.so (declarations in include/hx/exl3.h).
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include "../../include/hx/exl3.h"
#include "hx_kernels.hpp"

namespace {
thread_local char g_err[256] = "";

int fail(int code, const char* what)
{
    snprintf(g_err, sizeof(g_err), "%s", what);
    return code;
}

int hip_status(hipError_t e, const char* where)
{
    if (e == hipSuccess) return 0;
    snprintf(g_err, sizeof(g_err), "%s: %s", where, hipGetErrorString(e));
    return HX_ERR_HIP;
}

int codebook(int mcg, int mul1) { return mcg ? 1 : (mul1 ? 2 : 0); }

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
}  // namespace

extern "C" {

const char* hx_version(void) { return "hx_exl3 0.1 gfx950"; }
const char* hx_last_error(void) { return g_err; }

int hx_workspace_init(void* workspace, size_t bytes, hx_stream_t stream)
{
    if (!workspace && bytes) return fail(HX_ERR_INVALID, "hx_workspace_init: null workspace");
    return hip_status(hipMemsetAsync(workspace, 0, bytes, (hipStream_t)stream), "hx_workspace_init");
}

size_t hx_exl3_gemm_workspace_size(int M, int N, int K)
{
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    if (M <= 8) return hx::gemv_workspace_bytes(M, K, N);
    return hx::HX_COUNTER_BYTES + align256((size_t)M * K * sizeof(_Float16));
}

int hx_exl3_gemm(void* y, const void* x, const hx_group_words* w, int M, int N, int K, int bits, int y_fp32,
                 hx_stream_t stream, void* a_had, int mcg, void* workspace, size_t workspace_bytes)
{
    if (!w || !y || !x || !w->trellis || !w->suh || !w->svh) return fail(HX_ERR_INVALID, "hx_exl3_gemm: null pointer");
    if (M < 0 || N <= 0 || K <= 0 || N % 128 || K % 128) return fail(HX_ERR_INVALID, "hx_exl3_gemm: K and N must be positive multiples of 128");
    if (bits < 1 || bits > 8) return fail(HX_ERR_INVALID, "hx_exl3_gemm: bits must be in [1, 8]");
    if (w->mul1 && (uint32_t)w->mul1 != 0x83DCD12Du) return fail(HX_ERR_INVALID, "hx_exl3_gemm: unsupported mul1 constant");
    if (M == 0) return HX_GEMM_PATH_GEMV;
    const int cb = codebook(mcg, w->mul1);
    hipStream_t st = (hipStream_t)stream;
    const _Float16* xh = static_cast<const _Float16*>(x);
    const uint16_t* tr = static_cast<const uint16_t*>(w->trellis);
    const _Float16* suh = static_cast<const _Float16*>(w->suh);
    const _Float16* svh = static_cast<const _Float16*>(w->svh);
    if (M <= 8) {
        if (!workspace || workspace_bytes < hx::gemv_workspace_bytes(M, K, N))
            return fail(HX_ERR_WORKSPACE, "hx_exl3_gemm: workspace smaller than hx_exl3_gemm_workspace_size");
        int r = hip_status(hx::launch_linear_gemv(xh, tr, suh, svh, y, M, K, N, bits, cb, y_fp32 != 0, workspace, st),
                           "hx_exl3_gemm(gemv)");
        return r ? r : HX_GEMM_PATH_GEMV;
    }
    _Float16* ah = static_cast<_Float16*>(a_had);
    if (!ah) {
        if (!workspace || workspace_bytes < hx::HX_COUNTER_BYTES + (size_t)M * K * sizeof(_Float16))
            return fail(HX_ERR_WORKSPACE, "hx_exl3_gemm: a_had is null and the workspace cannot hold M*K fp16");
        ah = reinterpret_cast<_Float16*>(static_cast<char*>(workspace) + hx::HX_COUNTER_BYTES);
    }
    int r = hip_status(hx::launch_input_had(xh, suh, ah, M, K, st), "hx_exl3_gemm(input transform)");
    if (r) return r;
    r = hip_status(hx::launch_linear_mfma(ah, tr, svh, y, M, K, N, bits, cb, y_fp32 != 0, st), "hx_exl3_gemm(mfma)");
    return r ? r : HX_GEMM_PATH_MFMA;
}

int hx_exl3_reconstruct_slice(void* unpacked, const void* packed, int packed_rows, int packed_cols,
                              int unpacked_cols, int bits, int mcg, int mul1, int64_t n_offset, hx_stream_t stream)
{
    if (!unpacked || !packed) return fail(HX_ERR_INVALID, "hx_exl3_reconstruct_slice: null pointer");
    if (bits < 1 || bits > 8) return fail(HX_ERR_INVALID, "hx_exl3_reconstruct_slice: bits must be in [1, 8]");
    if (unpacked_cols % 128 || n_offset % 128 || n_offset < 0 || n_offset + unpacked_cols > (int64_t)packed_cols * 16)
        return fail(HX_ERR_INVALID, "hx_exl3_reconstruct_slice: slice must be 128-aligned and inside the tensor");
    return hip_status(hx::launch_reconstruct(static_cast<_Float16*>(unpacked), static_cast<const uint16_t*>(packed),
                                             packed_rows, packed_cols, unpacked_cols, bits, codebook(mcg, mul1),
                                             (long)n_offset, (hipStream_t)stream),
                      "hx_exl3_reconstruct_slice");
}

int hx_had_r_128(const void* input, void* output, const void* pre_scale, const void* post_scale, int64_t rows,
                 int cols, float r_scale, hx_stream_t stream)
{
    if (!input || !output || rows < 0 || cols <= 0 || cols % 128) return fail(HX_ERR_INVALID, "hx_had_r_128: bad arguments");
    return hip_status(hx::launch_had_r_128(static_cast<const _Float16*>(input), static_cast<_Float16*>(output),
                                           static_cast<const _Float16*>(pre_scale),
                                           static_cast<const _Float16*>(post_scale), (long)rows, cols, r_scale,
                                           (hipStream_t)stream),
                      "hx_had_r_128");
}

int hx_routing_ds3_nogroup(const void* scores, const void* bias, int64_t* topk_indices, void* topk_weights,
                           int bsz, int num_experts, int K, float scaling_factor, int use_topk, int act_fn,
                           hx_stream_t stream)
{
    if (!use_topk || act_fn != 0) return fail(HX_ERR_UNSUPPORTED, "hx_routing_ds3_nogroup: only use_topk=1 with sigmoid");
    if (!scores || !topk_indices || !topk_weights || bsz < 0 || num_experts < 1 || num_experts > 512 || K < 1 ||
        K > 64 || K > num_experts)
        return fail(HX_ERR_INVALID, "hx_routing_ds3_nogroup: bad arguments");
    return hip_status(hx::launch_routing(static_cast<const _Float16*>(scores), static_cast<const _Float16*>(bias),
                                         topk_indices, static_cast<_Float16*>(topk_weights), bsz, num_experts, K,
                                         scaling_factor, (hipStream_t)stream),
                      "hx_routing_ds3_nogroup");
}

int hx_moe_permute(const int64_t* ids, const void* weights, int M, int topk, int E, int64_t* expert_count,
                   int64_t* token_sorted, void* weight_sorted, int64_t* workspace, hx_stream_t stream,
                   int64_t* route_to_sorted)
{
    if (!ids || !weights || !expert_count || !token_sorted || !weight_sorted || M < 0 || topk < 1 || E < 1 || E > 512)
        return fail(HX_ERR_INVALID, "hx_moe_permute: bad arguments");
    return hip_status(hx::launch_permute(ids, static_cast<const _Float16*>(weights), M, topk, E, expert_count,
                                         token_sorted, static_cast<_Float16*>(weight_sorted), route_to_sorted,
                                         workspace, (hipStream_t)stream),
                      "hx_moe_permute");
}

int hx_moe_reduce_sorted(float* y, const float* contributions, const int64_t* route_to_sorted, int M, int topk,
                         int hidden, hx_stream_t stream)
{
    if (!y || !contributions || !route_to_sorted || M < 0 || topk < 1 || hidden <= 0 || hidden % 4)
        return fail(HX_ERR_INVALID, "hx_moe_reduce_sorted: bad arguments");
    return hip_status(hx::launch_reduce_sorted(y, contributions, route_to_sorted, M, topk, hidden, (hipStream_t)stream),
                      "hx_moe_reduce_sorted");
}

int hx_swiglu_clamp(const float* gate, const float* up, void* out, size_t n, float limit, hx_stream_t stream)
{
    if (!gate || !up || !out) return fail(HX_ERR_INVALID, "hx_swiglu_clamp: null pointer");
    return hip_status(hx::launch_swiglu_clamp(gate, up, static_cast<_Float16*>(out), n, limit, (hipStream_t)stream),
                      "hx_swiglu_clamp");
}

}  // extern "C"
