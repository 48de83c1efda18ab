// hx_capi.hip -- extern "C" boundary of libhx_exl3.so (declarations in include/hx/exl3.h).
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "../../include/hx/exl3.h"
#include "hx_kernels.hpp"
#include "hx_moe.hpp"
#include "hx_moe_decode.hpp"

namespace {
thread_local char g_err[512] = "";

// Optional phase profiler: HIP events recorded around each phase of hx_moe_layer on its stream.
struct Prof {
    bool on = false;
    struct Rec {
        int phase;
        hipEvent_t a, b;
    };
    std::vector<Rec> recs;
    std::vector<hipEvent_t> pool;
    hipEvent_t take()
    {
        if (!pool.empty()) {
            hipEvent_t e = pool.back();
            pool.pop_back();
            return e;
        }
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        return e;
    }
};
Prof g_prof;
const char* const k_phase_names[] = {"route", "permute", "experts_gate_up", "experts_down", "combine",
                                     "shared_expert", "prefill_plan_gather", "prefill_gemm_gate_up",
                                     "prefill_guad", "prefill_gemm_down", "prefill_combine", "moe_decode"};
constexpr int k_nphases = sizeof(k_phase_names) / sizeof(k_phase_names[0]);

struct Phase {
    int id;
    hipStream_t st;
    hipEvent_t a = nullptr;
    Phase(int id_, hipStream_t st_) : id(id_), st(st_)
    {
        if (g_prof.on) {
            a = g_prof.take();
            if (a) hipEventRecord(a, st);
        }
    }
    ~Phase()
    {
        if (a) {
            hipEvent_t b = g_prof.take();
            if (b) {
                hipEventRecord(b, st);
                g_prof.recs.push_back({id, a, b});
            }
        }
    }
};

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

namespace hx {
// Error text for hx_last_error from the other translation units of the library.
void set_error(const char* msg) { snprintf(g_err, sizeof(g_err), "%s", msg); }
}  // namespace hx

extern "C" {

const char* hx_version(void) { return "hx_exl3 0.1 gfx950"; }
const char* hx_last_error(void) { return g_err; }

int hx_profile_enable(int on)
{
    g_prof.on = on != 0;
    return 0;
}

int hx_profile_read(double* ms_total, int* counts, int max_phases)
{
    if (hipDeviceSynchronize() != hipSuccess) return fail(HX_ERR_HIP, "hx_profile_read: synchronize failed");
    for (int i = 0; i < max_phases; ++i) {
        ms_total[i] = 0.0;
        counts[i] = 0;
    }
    for (auto& r : g_prof.recs) {
        float ms = 0.0f;
        hipEventElapsedTime(&ms, r.a, r.b);
        if (r.phase < max_phases) {
            ms_total[r.phase] += ms;
            counts[r.phase] += 1;
        }
        g_prof.pool.push_back(r.a);
        g_prof.pool.push_back(r.b);
    }
    g_prof.recs.clear();
    return k_nphases;
}

const char* hx_profile_phase_name(int phase)
{
    return (phase >= 0 && phase < k_nphases) ? k_phase_names[phase] : "";
}

int hx_workspace_init(void* workspace, size_t bytes, hx_stream_t stream)
{
    if (!workspace && bytes) return fail(HX_ERR_INVALID, "hx_workspace_init: null workspace");
    return hip_status(hipMemsetAsync(workspace, 0, bytes, (hipStream_t)stream), "hx_workspace_init");
}

int hx_moe_max_concurrency(int device)
{
    int cus = 0;
    const int r = hip_status(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device),
                             "hx_moe_max_concurrency");
    if (r != 0) return r;
    return cus / 8 > 0 ? cus / 8 : 1;
}

int hx_moe_check_status(void* workspace, hx_stream_t stream)
{
    if (!workspace) return fail(HX_ERR_INVALID, "hx_moe_check_status: null workspace");
    int* status = static_cast<int*>(workspace) + hx::DEC_STATUS_INT;  // in the counter area
    int v = 0;
    int r = hip_status(hipMemcpyAsync(&v, status, sizeof(int), hipMemcpyDeviceToHost, (hipStream_t)stream),
                       "hx_moe_check_status");
    if (r == 0) r = hip_status(hipStreamSynchronize((hipStream_t)stream), "hx_moe_check_status");
    if (r != 0) return r;
    if (!v) return 0;
    const int zero = 0;
    r = hip_status(hipMemcpyAsync(status, &zero, sizeof(int), hipMemcpyHostToDevice, (hipStream_t)stream),
                   "hx_moe_check_status");
    if (r == 0) r = hip_status(hipStreamSynchronize((hipStream_t)stream), "hx_moe_check_status");
    if (r != 0) return r;
    if (v & hx::DEC_STATUS_TIMEOUT)
        return fail(HX_ERR_TIMEOUT, "hx_moe_check_status: a bounded wait of the few-token MoE layer gave up");
    return fail(HX_ERR_UNSUPPORTED, "hx_moe_check_status: a per-expert bit table holds a width outside 1..8");
}

// Debug option: with HX_MOE_SYNC_CHECK=1 in the environment, every few-token MoE call synchronizes
// its stream and reports a given-up bounded wait (hx_moe_check_status) as its own return value.
// Skipped while the stream is being captured into a graph (no synchronization is possible there).
static int decode_checked(int r, void* workspace, hx_stream_t stream)
{
    if (r != 0) return r;
    const char* v = getenv("HX_MOE_SYNC_CHECK");
    if (!v || atoi(v) == 0) return 0;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return 0;
    return hx_moe_check_status(workspace, stream);
}

size_t hx_exl3_gemm_workspace_size(int M, int N, int K)
{
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    if (M <= hx::GEMV_MAX_M) return hx::gemv_workspace_bytes(M, K, N);
    return hx::HX_COUNTER_BYTES + align256((size_t)M * K * sizeof(_Float16));
}

int hx_exl3_gemm(void* y, const void* x, const hx_group_words* w, int M, int N, int K, int bits, int y_fp32,
                 hx_stream_t stream, void* a_had, int mcg, void* workspace, size_t workspace_bytes)
{
    if (!w || !w->trellis || !w->suh || !w->svh || (M != 0 && (!y || !x)))
        return fail(HX_ERR_INVALID, "hx_exl3_gemm: null pointer");
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
    if (M <= hx::GEMV_MAX_M) {
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

}  // extern "C"

// ---- the allocation-free linear: its workspace is a device array of this library, not an argument
//
// `scratch` is the workspace of hx_exl3_gemm_noalloc on every GPU this library runs on (each holds
// its own copy until the process ends).  Host code uses the address hipGetSymbolAddress returns for
// the current device, never the array's name (on the host that name is not a device address).  The
// first HX_COUNTER_BYTES are arrival counters: zero when the code object loads (static storage) and
// left at zero by every kernel that uses them, so no call clears them; the rest (split-K partials,
// or the transformed activations of the MFMA path) is written before it is read in every call.
namespace {

constexpr size_t HX_NOALLOC_SCRATCH_BYTES = 8u << 20;
constexpr int HX_NOALLOC_MAX_DEVICES = 64;
__device__ __align__(256) static unsigned char scratch[HX_NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
void* g_scratch_ptr[HX_NOALLOC_MAX_DEVICES];

// The current device's copy of `scratch`, looked up once per device (with that device current).
int scratch_ptr(void** out)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= HX_NOALLOC_MAX_DEVICES)
        return fail(HX_ERR_HIP, "hx_exl3_gemm_noalloc: no current device (or more than 64 devices)");
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_status(e != hipSuccess ? e : hipErrorInvalidSymbol, "hx_exl3_gemm_noalloc(scratch)");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace

extern "C" {

size_t hx_exl3_gemm_noalloc_max_bytes(void) { return HX_NOALLOC_SCRATCH_BYTES; }

int hx_exl3_gemm_noalloc(void* y, const void* x, const hx_group_words* w, int M, int N, int K, int bits, int y_fp32,
                         hx_stream_t stream, int mcg)
{
    if (M < 0 || N <= 0 || K <= 0) return fail(HX_ERR_INVALID, "hx_exl3_gemm_noalloc: bad extents");
    const size_t need = hx_exl3_gemm_workspace_size(M, N, K);
    if (need > HX_NOALLOC_SCRATCH_BYTES) {
        snprintf(g_err, sizeof(g_err),
                 "hx_exl3_gemm_noalloc: M=%d N=%d K=%d needs %zu bytes of scratch, more than its %zu (use hx_exl3_gemm "
                 "with a workspace)",
                 M, N, K, need, HX_NOALLOC_SCRATCH_BYTES);
        return HX_ERR_WORKSPACE;
    }
    void* ws = nullptr;
    if (M > 0) {
        const int r = scratch_ptr(&ws);
        if (r) return r;
    }
    return hx_exl3_gemm(y, x, w, M, N, K, bits, y_fp32, stream, nullptr, mcg, ws, HX_NOALLOC_SCRATCH_BYTES);
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

int hx_exl3_reconstruct_had_slice(void* unpacked, const void* packed, const void* suh, const void* svh,
                                  int packed_rows, int packed_cols, int unpacked_rows, int unpacked_cols, int bits,
                                  int mcg, int mul1, int64_t n_offset, hx_stream_t stream)
{
    if (!unpacked || !packed || !suh || !svh) return fail(HX_ERR_INVALID, "hx_exl3_reconstruct_had_slice: null pointer");
    if (bits < 1 || bits > 8) return fail(HX_ERR_INVALID, "hx_exl3_reconstruct_had_slice: bits must be in [1, 8]");
    if (unpacked_rows % 128 || unpacked_cols % 128 || n_offset % 128 || n_offset < 0 || unpacked_rows < 0 ||
        unpacked_cols < 0 || n_offset + unpacked_cols > (int64_t)packed_cols * 16 || unpacked_rows > packed_rows * 16)
        return fail(HX_ERR_INVALID, "hx_exl3_reconstruct_had_slice: dimensions must be 128-aligned and inside the tensor");
    return hip_status(hx::launch_reconstruct_had(static_cast<_Float16*>(unpacked), static_cast<const uint16_t*>(packed),
                                                 static_cast<const _Float16*>(suh), static_cast<const _Float16*>(svh),
                                                 packed_rows, packed_cols, unpacked_rows, unpacked_cols, bits,
                                                 codebook(mcg, mul1), (long)n_offset, (hipStream_t)stream),
                      "hx_exl3_reconstruct_had_slice");
}

int hx_exl3_pack_trellis(void* packed, const void* unpacked, int rows, int cols, int K, hx_stream_t stream)
{
    if (!packed || !unpacked || rows < 0 || cols < 0 || K < 1 || K > 8)
        return fail(HX_ERR_INVALID, "hx_exl3_pack_trellis: bad arguments");
    return hip_status(hx::launch_pack_trellis(static_cast<uint16_t*>(packed), static_cast<const uint16_t*>(unpacked),
                                              (long)rows * cols, K, (hipStream_t)stream),
                      "hx_exl3_pack_trellis");
}

int hx_exl3_unpack_trellis(void* unpacked, const void* packed, int rows, int cols, int K, hx_stream_t stream)
{
    if (!packed || !unpacked || rows < 0 || cols < 0 || K < 1 || K > 8)
        return fail(HX_ERR_INVALID, "hx_exl3_unpack_trellis: bad arguments");
    return hip_status(hx::launch_unpack_trellis(static_cast<uint16_t*>(unpacked), static_cast<const uint16_t*>(packed),
                                                (long)rows * cols, K, (hipStream_t)stream),
                      "hx_exl3_unpack_trellis");
}

int hx_pack_signs(void* packed, const void* unpacked, int cols, hx_stream_t stream)
{
    if (cols < 0 || (cols > 0 && (!packed || !unpacked))) return fail(HX_ERR_INVALID, "hx_pack_signs: bad arguments");
    if (cols == 0) return 0;
    return hip_status(hx::launch_pack_signs(static_cast<uint16_t*>(packed), static_cast<const uint16_t*>(unpacked), cols,
                                            (hipStream_t)stream),
                      "hx_pack_signs");
}

int hx_count_inf_nan(const void* x, unsigned long long* counts, uint64_t numel, int dtype, hx_stream_t stream)
{
    if (!counts || (numel > 0 && !x)) return fail(HX_ERR_INVALID, "hx_count_inf_nan: null pointer");
    if (dtype != HX_DTYPE_HALF && dtype != HX_DTYPE_FLOAT)
        return fail(HX_ERR_INVALID, "hx_count_inf_nan: dtype must be HX_DTYPE_HALF or HX_DTYPE_FLOAT");
    if (numel == 0) return 0;
    return hip_status(hx::launch_count_inf_nan(x, counts, numel, dtype == HX_DTYPE_FLOAT, (hipStream_t)stream),
                      "hx_count_inf_nan");
}

int hx_had_r_128(const void* input, void* output, const void* pre_scale, const void* post_scale, int64_t rows,
                 int cols, int dtype, float scale, hx_stream_t stream)
{
    return hx_had_r_128_dual(input, output, pre_scale, post_scale, nullptr, nullptr, nullptr, nullptr, rows, cols, dtype,
                             scale, stream);
}

int hx_had_r_128_dual(const void* input1, void* output1, const void* pre_scale1, const void* post_scale1,
                      const void* input2, void* output2, const void* pre_scale2, const void* post_scale2,
                      int64_t rows, int cols, int dtype, float scale, hx_stream_t stream)
{
    const bool dual = input2 != nullptr || output2 != nullptr;
    if (!input1 || !output1 || (dual && (!input2 || !output2)) || rows < 0 || cols <= 0 || cols % 128)
        return fail(HX_ERR_INVALID, "hx_had_r_128: bad arguments (cols must be a positive multiple of 128)");
    if (dtype != HX_DTYPE_HALF && dtype != HX_DTYPE_FLOAT)
        return fail(HX_ERR_INVALID, "hx_had_r_128: dtype must be HX_DTYPE_HALF or HX_DTYPE_FLOAT");
    if ((pre_scale1 && post_scale1) || (pre_scale2 && post_scale2))
        return fail(HX_ERR_INVALID, "hx_had_r_128: pre_scale and post_scale are exclusive");
    if (dual && (!pre_scale1 != !pre_scale2 || !post_scale1 != !post_scale2))
        return fail(HX_ERR_INVALID, "hx_had_r_128_dual: both tensors need the same scaling mode");
    const int mode = pre_scale1 ? 1 : post_scale1 ? 2 : 0;
    const void* s1 = pre_scale1 ? pre_scale1 : post_scale1;
    const void* s2 = pre_scale2 ? pre_scale2 : post_scale2;
    return hip_status(hx::launch_had_r_128(input1, output1, s1, input2, output2, s2, mode, (long)rows, cols,
                                           dtype == HX_DTYPE_FLOAT, scale * HX_HAD_RSQRT128, (hipStream_t)stream),
                      "hx_had_r_128");
}

int hx_routing_ds3_nogroup(const void* scores, const void* bias, int64_t* topk_indices, void* topk_weights,
                           int bsz, int num_experts, int K, float scaling_factor, int use_topk, int act_fn,
                           hx_stream_t stream)
{
    if (act_fn != 0 && act_fn != 1) return fail(HX_ERR_UNSUPPORTED, "hx_routing_ds3_nogroup: act_fn must be 0 (sigmoid) or 1 (sqrt-softplus)");
    if (!scores || !topk_indices || !topk_weights || bsz < 0 || num_experts < 1 || num_experts > 512 || K < 1 ||
        K > 64 || K > num_experts)
        return fail(HX_ERR_INVALID, "hx_routing_ds3_nogroup: bad arguments");
    return hip_status(hx::launch_routing(static_cast<const _Float16*>(scores), static_cast<const _Float16*>(bias),
                                         topk_indices, static_cast<_Float16*>(topk_weights), bsz, num_experts, K,
                                         scaling_factor, (hipStream_t)stream, use_topk != 0, act_fn),
                      "hx_routing_ds3_nogroup");
}

int hx_routing_gemv(const void* x, const void* gate_t, void* scores, int k, int E, hx_stream_t stream)
{
    if (!x || !gate_t || !scores || k <= 0 || E < 1 || (k & 1))
        return fail(HX_ERR_INVALID, "hx_routing_gemv: bad arguments (k must be even)");
    if (k % 32) return fail(HX_ERR_UNSUPPORTED, "hx_routing_gemv: k must be a multiple of 32 here");
    return hip_status(hx::launch_gemm_nt_f16(static_cast<const _Float16*>(x), static_cast<const _Float16*>(gate_t),
                                             scores, 1, E, k, false, false, (hipStream_t)stream),
                      "hx_routing_gemv");
}

int hx_routing_ds3_nogroup_hidden(const void* hidden, const void* gate_t, void* scores, const void* bias,
                                  int64_t* topk_indices, void* topk_weights, int k, int num_experts, int K,
                                  float scaling_factor, int act_fn, hx_stream_t stream)
{
    if (act_fn != 0 && act_fn != 1)
        return fail(HX_ERR_UNSUPPORTED, "hx_routing_ds3_nogroup_hidden: act_fn must be 0 (sigmoid) or 1 (sqrt-softplus)");
    if (!topk_indices || !topk_weights || num_experts > 512 || K < 1 || K > 64 || K > num_experts)
        return fail(HX_ERR_INVALID, "hx_routing_ds3_nogroup_hidden: bad arguments");
    if (int r = hx_routing_gemv(hidden, gate_t, scores, k, num_experts, stream)) return r;
    return hx_routing_ds3_nogroup(scores, bias, topk_indices, topk_weights, 1, num_experts, K, scaling_factor, 1,
                                  act_fn, stream);
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

int hx_gather_rows(const void* src, const int64_t* idx, void* dst, int n, int h, hx_stream_t stream)
{
    if (n < 0 || h < 0) return fail(HX_ERR_INVALID, "hx_gather_rows: negative extent");
    if (n > 0 && h > 0 && (!src || !idx || !dst)) return fail(HX_ERR_INVALID, "hx_gather_rows: null pointer");
    return hip_status(hx::launch_gather_rows(static_cast<const _Float16*>(src), idx, static_cast<_Float16*>(dst), n, h,
                                             (hipStream_t)stream),
                      "hx_gather_rows");
}

int hx_scatter_add_rows(float* y, const float* src, const int64_t* idx, const void* w, int n, int h,
                        hx_stream_t stream)
{
    if (n < 0 || h < 0) return fail(HX_ERR_INVALID, "hx_scatter_add_rows: negative extent");
    if (n > 0 && h > 0 && (!y || !src || !idx || !w)) return fail(HX_ERR_INVALID, "hx_scatter_add_rows: null pointer");
    return hip_status(hx::launch_scatter_add_rows(y, src, idx, static_cast<const _Float16*>(w), n, h,
                                                  (hipStream_t)stream),
                      "hx_scatter_add_rows");
}

int hx_gemm_nt_f16(void* y, const void* x, const void* w, int M, int N, int K, int y_fp32, int add,
                   hx_stream_t stream)
{
    if (!y || !x || !w || M < 0 || N < 0 || K <= 0 || K % 32)
        return fail(HX_ERR_INVALID, "hx_gemm_nt_f16: bad arguments (K must be a positive multiple of 32)");
    return hip_status(hx::launch_gemm_nt_f16(static_cast<const _Float16*>(x), static_cast<const _Float16*>(w), y, M,
                                             N, K, y_fp32 != 0, add != 0, (hipStream_t)stream),
                      "hx_gemm_nt_f16");
}

// ------------------------------------------------------------------ MoE

size_t hx_moe_workspace_size(int tokens, int hidden_dim, int intermediate_dim, int num_experts, int topk)
{
    if (tokens < 0 || hidden_dim <= 0 || intermediate_dim <= 0 || num_experts <= 0 || topk <= 0) return 0;
    hx::MoeWs L;
    L.plan(tokens, hidden_dim, intermediate_dim, num_experts, topk, true);
    return L.total;
}

namespace {

int moe_check(const hx_expert_tables* t, int tokens, int hidden, int inter, int E, int topk, int Kg, int Ku, int Kd,
              int mcg, int mul1, const char* who)
{
    if (!t || !t->gate_trellis || !t->gate_suh || !t->gate_svh || !t->up_trellis || !t->up_suh || !t->up_svh ||
        !t->down_trellis || !t->down_suh || !t->down_svh)
        return fail(HX_ERR_INVALID, who);
    if (tokens < 0 || hidden <= 0 || inter <= 0 || hidden % 128 || inter % 128 || E < 1 || E > 512 || topk < 1 ||
        topk > E || topk > 64)
        return fail(HX_ERR_INVALID, who);
    if (!!mcg == !!mul1) return fail(HX_ERR_INVALID, who);  // exactly one of mcg / mul1 (reference contract)
    const bool tab = t->gate_bits || t->up_bits || t->down_bits;
    if (tab && !(t->gate_bits && t->up_bits && t->down_bits && t->bits_mask)) return fail(HX_ERR_INVALID, who);
    if (!tab && (Kg < 1 || Kg > 8 || Ku < 1 || Ku > 8 || Kd < 1 || Kd > 8)) return fail(HX_ERR_INVALID, who);
    return 0;
}

void fill_tables(const hx_expert_tables* t, const void* const* (&tr)[3], const void* const* (&suh)[3],
                 const void* const* (&svh)[3], const int32_t* (&bits)[3], int (&uni)[3], int Kg, int Ku, int Kd)
{
    tr[0] = t->gate_trellis; tr[1] = t->up_trellis; tr[2] = t->down_trellis;
    suh[0] = t->gate_suh; suh[1] = t->up_suh; suh[2] = t->down_suh;
    svh[0] = t->gate_svh; svh[1] = t->up_svh; svh[2] = t->down_svh;
    bits[0] = t->gate_bits; bits[1] = t->up_bits; bits[2] = t->down_bits;
    uni[0] = Kg; uni[1] = Ku; uni[2] = Kd;
}

int max_bits_of(const hx_expert_tables* t, int Kg, int Ku, int Kd, const int* shared_bits)
{
    int m = 0;
    if (t->gate_bits) {
        for (int b = 1; b <= 8; ++b)
            if (t->bits_mask & (1u << b)) m = b;
    } else {
        m = Kg > Ku ? Kg : Ku;
        m = m > Kd ? m : Kd;
    }
    if (shared_bits)
        for (int i = 0; i < 3; ++i) m = shared_bits[i] > m ? shared_bits[i] : m;
    return m;
}

uint32_t phase_mask(const hx_expert_tables* t, int Ka, int Kb)
{
    if (t->gate_bits) return t->bits_mask;
    uint32_t m = 1u << Ka;
    if (Kb > 0) m |= 1u << Kb;
    return m;
}

}  // namespace

int hx_moe_grouped(const void* x, float* y, const int64_t* expert_count, const int64_t* token_sorted,
                   const void* weight_sorted, void* temp_state_g, void* temp_state_u, void* temp_intermediate_g,
                   void* temp_intermediate_u, const hx_expert_tables* tables, int tokens, int hidden_dim,
                   int intermediate_dim, int num_experts, int topk, int max_tokens_per_expert, int concurrency,
                   int K_gate, int K_up, int K_down, int mcg, int mul1, float act_limit, int act_function,
                   int num_active, hx_stream_t stream, float* sorted_contributions, const int64_t* route_to_sorted,
                   void* workspace, size_t workspace_bytes)
{
    (void)temp_state_g; (void)temp_state_u; (void)temp_intermediate_g; (void)temp_intermediate_u;
    (void)max_tokens_per_expert; (void)concurrency; (void)num_active;
    if (int r = moe_check(tables, tokens, hidden_dim, intermediate_dim, num_experts, topk, K_gate, K_up, K_down, mcg,
                          mul1, "hx_moe_grouped: bad arguments"))
        return r;
    if (act_function < HX_ACT_SILU || act_function > HX_ACT_RELU2_NOGATE)
        return fail(HX_ERR_UNSUPPORTED, "hx_moe_grouped: act_function must be 0 (SiLU), 1 (GELU) or 2 (relu2, no gate)");
    if (tokens == 0) return 0;  // an empty batch is a no-op (its activation pointers may be null)
    if (!x || !expert_count || !token_sorted || !weight_sorted) return fail(HX_ERR_INVALID, "hx_moe_grouped: null input");
    if (!sorted_contributions && (!y || !route_to_sorted))
        return fail(HX_ERR_INVALID, "hx_moe_grouped: y and route_to_sorted are needed without sorted_contributions");
    hx::MoeWs L;
    L.plan(tokens, hidden_dim, intermediate_dim, num_experts, topk, false,
           max_bits_of(tables, K_gate, K_up, K_down, nullptr));
    if (!workspace || workspace_bytes < L.total) return fail(HX_ERR_WORKSPACE, "hx_moe_grouped: workspace too small");
    char* base = static_cast<char*>(workspace);
    hipStream_t st = (hipStream_t)stream;
    const int cb = mcg ? 1 : 2;
    const _Float16* xh = static_cast<const _Float16*>(x);
    const _Float16* ws_sorted = static_cast<const _Float16*>(weight_sorted);
    if (L.few_tokens()) {
        hx::MoeDecodeArgs a = L.decode_args(base);
        a.x = xh;
        a.expert_count = expert_count;
        a.token_sorted = token_sorted;
        a.weight_sorted = ws_sorted;
        a.route_to_sorted = route_to_sorted;
        fill_tables(tables, a.tr, a.suh, a.svh, a.bits_tab, a.bits_uniform, K_gate, K_up, K_down);
        a.act_limit = act_limit;
        a.act_fn = act_function;
        if (sorted_contributions) {
            a.contrib = sorted_contributions;
        } else {
            a.combine = true;
            a.y_routed = y;
            a.y_accumulate = true;
        }
        return decode_checked(hip_status(hx::run_moe_decode(a, cb, phase_mask(tables, K_gate, K_up) | phase_mask(tables, K_down, 0), st),
                                         "hx_moe_grouped(decode)"),
                              workspace, stream);
    }
    hx::PrefillArgs p{};
    p.x = xh;
    p.T = tokens;
    p.hidden = hidden_dim;
    p.inter = intermediate_dim;
    p.E = num_experts;
    p.topk = topk;
    p.R = tokens * topk;
    p.expert_count = expert_count;
    p.token_sorted = token_sorted;
    p.weight_sorted = ws_sorted;
    p.r2s = route_to_sorted;
    fill_tables(tables, p.tr, p.suh, p.svh, p.bits_tab, p.bits_uniform, K_gate, K_up, K_down);
    p.act_limit = act_limit;
    p.act_fn = act_function;
    p.cb = cb;
    p.ws = base;
    p.lay = &L;
    if (sorted_contributions) {
        // contributions only: combine writes them; no y
        return hip_status(hx::run_moe_prefill(p, sorted_contributions, nullptr, nullptr, nullptr, false, st),
                          "hx_moe_grouped(prefill)");
    }
    return hip_status(hx::run_moe_prefill(p, nullptr, nullptr, nullptr, y, true, st), "hx_moe_grouped(prefill)");
}

int hx_moe_layer(void* y, float* y_routed, const void* x, const void* scores, const void* bias,
                 const hx_expert_tables* tables, const hx_group_words* shared, const int* shared_bits, int tokens,
                 int hidden_dim, int intermediate_dim, int num_experts, int topk, int K_gate, int K_up, int K_down,
                 float routed_scale, float act_limit, int mcg, int mul1, void* workspace, size_t workspace_bytes,
                 hx_stream_t stream)
{
    if (int r = moe_check(tables, tokens, hidden_dim, intermediate_dim, num_experts, topk, K_gate, K_up, K_down, mcg,
                          mul1, "hx_moe_layer: bad arguments"))
        return r;
    if (tokens == 0) return 0;  // an empty batch is a no-op (its activation pointers may be null)
    if (!x || !scores || (!y && !y_routed)) return fail(HX_ERR_INVALID, "hx_moe_layer: null input/output");
    if (shared) {
        if (!shared_bits) return fail(HX_ERR_INVALID, "hx_moe_layer: shared_bits required with a shared expert");
        for (int i = 0; i < 3; ++i)
            if (!shared[i].trellis || !shared[i].suh || !shared[i].svh || shared_bits[i] < 1 || shared_bits[i] > 8)
                return fail(HX_ERR_INVALID, "hx_moe_layer: bad shared expert");
        // the shared expert is decoded with the routed experts' codebook (mcg / mul1)
        for (int i = 0; i < 3; ++i)
            if ((shared[i].mul1 != 0) != (mul1 != 0))
                return fail(HX_ERR_INVALID, "hx_moe_layer: the shared expert's codebook (mul1) differs from the "
                                            "routed experts'");
        if (act_limit <= 0.0f) return fail(HX_ERR_INVALID, "hx_moe_layer: the shared-expert swiglu needs act_limit > 0");
    }
    hx::MoeWs L;
    L.plan(tokens, hidden_dim, intermediate_dim, num_experts, topk, shared != nullptr,
           max_bits_of(tables, K_gate, K_up, K_down, shared ? shared_bits : nullptr));
    if (!workspace || workspace_bytes < L.total) return fail(HX_ERR_WORKSPACE, "hx_moe_layer: workspace too small");
    char* base = static_cast<char*>(workspace);
    hipStream_t st = (hipStream_t)stream;
    const int cb = mcg ? 1 : 2;
    const _Float16* xh = static_cast<const _Float16*>(x);
    int64_t* idx = reinterpret_cast<int64_t*>(base + L.off_idx);
    _Float16* wt = reinterpret_cast<_Float16*>(base + L.off_w);
    int64_t* cnt = reinterpret_cast<int64_t*>(base + L.off_count);
    int64_t* ts = reinterpret_cast<int64_t*>(base + L.off_tsorted);
    _Float16* wsorted = reinterpret_cast<_Float16*>(base + L.off_wsorted);
    int64_t* r2s = reinterpret_cast<int64_t*>(base + L.off_r2s);

    int r;
    if (L.few_tokens()) {
        hx::MoeDecodeArgs a = L.decode_args(base);
        a.x = xh;
        a.scores = static_cast<const _Float16*>(scores);
        a.bias = static_cast<const _Float16*>(bias);
        a.routed_scale = routed_scale;
        fill_tables(tables, a.tr, a.suh, a.svh, a.bits_tab, a.bits_uniform, K_gate, K_up, K_down);
        uint32_t mgu = phase_mask(tables, K_gate, K_up), md = phase_mask(tables, K_down, 0);
        if (shared) {
            for (int i = 0; i < 3; ++i) {
                a.sh_tr[i] = shared[i].trellis;
                a.sh_suh[i] = shared[i].suh;
                a.sh_svh[i] = shared[i].svh;
                a.sh_bits[i] = shared_bits[i];
            }
            mgu |= (1u << shared_bits[0]) | (1u << shared_bits[1]);
            md |= 1u << shared_bits[2];
        }
        a.act_limit = act_limit;
        a.out_idx = idx;
        a.out_w = wt;
        a.combine = true;
        a.y = static_cast<_Float16*>(y);
        a.y_routed = y_routed;
        Phase ph(11, st);
        return decode_checked(hip_status(hx::run_moe_decode(a, cb, mgu | md, st), "hx_moe_layer(decode)"), workspace,
                              stream);
    }
    {
        Phase ph(0, st);
        r = hip_status(hx::launch_routing(static_cast<const _Float16*>(scores), static_cast<const _Float16*>(bias), idx,
                                          wt, tokens, num_experts, topk, routed_scale, st),
                       "hx_moe_layer(routing)");
    }
    if (r) return r;
    {
        Phase ph(1, st);
        r = hip_status(hx::launch_permute_chunked(idx, wt, tokens, topk, num_experts, cnt, ts, wsorted, r2s,
                                                  reinterpret_cast<int*>(base + L.off_perm),
                                                  reinterpret_cast<int*>(base) + 10250, st),
                       "hx_moe_layer(permute)");
    }
    if (r) return r;

    const float* shared_rows = nullptr;
    if (shared) {
        Phase ph(5, st);
        _Float16* sh_a = reinterpret_cast<_Float16*>(base + L.off_sh_a);
        float* sh_g = reinterpret_cast<float*>(base + L.off_sh_g);
        float* sh_u = reinterpret_cast<float*>(base + L.off_sh_u);
        _Float16* sh_act = reinterpret_cast<_Float16*>(base + L.off_sh_act);
        float* sh_d = reinterpret_cast<float*>(base + L.off_sh_d);
        auto H = [](const void* p) { return static_cast<const _Float16*>(p); };
        auto U16 = [](const void* p) { return static_cast<const uint16_t*>(p); };
        hipError_t e = hx::launch_input_had(xh, H(shared[0].suh), sh_a, tokens, hidden_dim, st);
        if (!e) e = hx::launch_linear_mfma(sh_a, U16(shared[0].trellis), H(shared[0].svh), sh_g, tokens, hidden_dim,
                                           intermediate_dim, shared_bits[0], cb, true, st);
        if (!e) e = hx::launch_input_had(xh, H(shared[1].suh), sh_a, tokens, hidden_dim, st);
        if (!e) e = hx::launch_linear_mfma(sh_a, U16(shared[1].trellis), H(shared[1].svh), sh_u, tokens, hidden_dim,
                                           intermediate_dim, shared_bits[1], cb, true, st);
        if (!e) e = hx::launch_swiglu_clamp(sh_g, sh_u, sh_act, (size_t)tokens * intermediate_dim, act_limit, st);
        if (!e) e = hx::launch_input_had(sh_act, H(shared[2].suh), sh_a, tokens, intermediate_dim, st);
        if (!e) e = hx::launch_linear_mfma(sh_a, U16(shared[2].trellis), H(shared[2].svh), sh_d, tokens,
                                           intermediate_dim, hidden_dim, shared_bits[2], cb, true, st);
        if ((r = hip_status(e, "hx_moe_layer(shared expert)"))) return r;
        shared_rows = sh_d;
    }
    hx::PrefillArgs p{};
    p.x = xh;
    p.T = tokens;
    p.hidden = hidden_dim;
    p.inter = intermediate_dim;
    p.E = num_experts;
    p.topk = topk;
    p.R = tokens * topk;
    p.expert_count = cnt;
    p.token_sorted = ts;
    p.weight_sorted = wsorted;
    p.r2s = r2s;
    fill_tables(tables, p.tr, p.suh, p.svh, p.bits_tab, p.bits_uniform, K_gate, K_up, K_down);
    p.act_limit = act_limit;
    p.cb = cb;
    p.ws = base;
    p.lay = &L;
    Phase ph(7, st);
    return hip_status(hx::run_moe_prefill(p, nullptr, shared_rows, static_cast<_Float16*>(y), y_routed, false, st),
                      "hx_moe_layer(prefill)");
}

}  // extern "C"
