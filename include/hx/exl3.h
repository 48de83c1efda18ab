/*
 * hx/exl3.h -- C ABI of the MI355X (gfx950) EXL3 quantized expert-GEMM path (libhx_exl3.so).
 *
 * Every entry point replaces one reference interface (file:line in the reference repository,
 * neron82/helios-glm53flash) with the same argument meaning; the differences are C linkage,
 * POD descriptors, caller-owned workspaces with size queries, and int status codes instead of
 * abort():
 *   >= 0  success (hx_exl3_gemm returns which path ran, see below)
 *   HX_ERR_INVALID     argument outside the supported domain (nothing was launched)
 *   HX_ERR_WORKSPACE   workspace missing or smaller than the size query
 *   HX_ERR_HIP         a HIP launch failed (hx_last_error() names it)
 *   HX_ERR_UNSUPPORTED an option the reference has that this build does not implement
 *   HX_ERR_TIMEOUT     a bounded in-kernel wait of the few-token MoE layer gave up (hx_moe_check_status)
 *
 * Conventions: all data pointers are device pointers on the current HIP device; fp16 data is
 * IEEE binary16; `stream` may be 0 (null stream).  Calls are asynchronous on `stream`.
 * Workspaces: caller-owned device memory, zero-filled once before first use (hx_workspace_init
 * or any zero fill).  The first 64 KiB hold arrival counters that every kernel leaves at zero and
 * no call writes data into, so one workspace serves calls of any shape without clearing.  Two
 * calls in flight at once must not share a workspace.
 */
#ifndef HX_EXL3_H
#define HX_EXL3_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hx_stream_t; /* == hipStream_t */

#define HX_ERR_INVALID (-1)
#define HX_ERR_WORKSPACE (-2)
#define HX_ERR_HIP (-3)
#define HX_ERR_UNSUPPORTED (-4)
#define HX_ERR_TIMEOUT (-5)

#define HX_GEMM_PATH_MFMA 1
#define HX_GEMM_PATH_GEMV 90 /* same value the reference returns when its GEMV ran */

/* One EXL3 linear W[out=N][in=K]: trellis uint16 (K/16, N/16, 16*bits), suh fp16 [K],
 * svh fp16 [N], mul1 != 0 selects codebook 2 (mul1 must then be 0x83DCD12D).
 * Replaces helios::exl3::GroupWords (src/cuda/quant/exl3_gemm.cuh:30-36). */
typedef struct hx_group_words {
    const void* trellis;
    const void* suh;
    const void* svh;
    int mul1;
} hx_group_words;

/* Per-expert device pointer tables, each a device array of num_experts pointers, plus optional
 * per-expert bit widths (device int32 arrays, or NULL to use the call's uniform widths) and
 * bits_mask, the host-side union of the widths those arrays hold (bit b set when some expert
 * uses b bits).  Replaces helios::exl3::ExpertTables (src/cuda/quant/exl3_moe.cuh:20-31); the
 * bits arrays and mask are an extension for layers that mix bit widths across experts. */
typedef struct hx_expert_tables {
    const void* const* gate_trellis;
    const void* const* gate_suh;
    const void* const* gate_svh;
    const void* const* up_trellis;
    const void* const* up_suh;
    const void* const* up_svh;
    const void* const* down_trellis;
    const void* const* down_suh;
    const void* const* down_svh;
    const int32_t* gate_bits;
    const int32_t* up_bits;
    const int32_t* down_bits;
    uint32_t bits_mask;
} hx_expert_tables;

/* ---- library ---------------------------------------------------------------------------- */
const char* hx_version(void);
const char* hx_last_error(void);
int hx_workspace_init(void* workspace, size_t bytes, hx_stream_t stream);

/* Whether a bounded wait inside the few-token MoE layer (hx_moe_layer / hx_moe_grouped with T <= 8:
 * a down-projection workgroup waiting for its activations) gave up since the last check: synchronizes
 * `stream`, clears the flag, returns HX_ERR_TIMEOUT if it was set (the results of those calls are
 * then not to be trusted), HX_ERR_UNSUPPORTED if a per-expert bit table held a width outside 1..8,
 * else 0.  With HX_MOE_SYNC_CHECK=1 in the environment every few-token
 * hx_moe_layer / hx_moe_grouped call runs this check itself (outside graph capture) and returns its
 * result (debug option).  No counterpart in the reference, whose kernels cannot wait on each other. */
int hx_moe_check_status(void* workspace, hx_stream_t stream);

/* Phase profiler (no reference counterpart; the reference times phases with HELIOS_PROF host/event
 * timers, src/engine/runner.cpp:1006-1058): while enabled, hx_moe_layer records HIP events around
 * each phase on its stream.  hx_profile_read synchronizes the device, writes the summed
 * milliseconds and the number of records per phase (arrays of max_phases), clears the records and
 * returns the number of phases; hx_profile_phase_name names phase i. */
int hx_profile_enable(int on);
int hx_profile_read(double* ms_total, int* counts, int max_phases);
const char* hx_profile_phase_name(int phase);

/* ---- quantized linear ------------------------------------------------------------------- */

/* y[M][N] = svh . H_N( H_K(x . suh) . W_hat ), x fp16 [M][K], y fp32 (y_fp32) or fp16.
 * Replaces helios::exl3::gemm (src/cuda/quant/exl3_gemm.cuh:51-66, exl3_gemm.cu:81-243).
 * M <= 16 runs the fused decode-GEMV (returns HX_GEMM_PATH_GEMV), else the MFMA GEMM (returns
 * HX_GEMM_PATH_MFMA), which needs a_had (M*K fp16 scratch, as in the reference) or, when
 * a_had is NULL, takes it from the workspace.  K % 128 == 0, N % 128 == 0, bits 1..8.  M == 0 is
 * a no-op (x and y may then be NULL). */
size_t hx_exl3_gemm_workspace_size(int M, int N, int K);
int hx_exl3_gemm(void* y, const void* x, const hx_group_words* w, int M, int N, int K, int bits, int y_fp32,
                 hx_stream_t stream, void* a_had, int mcg, void* workspace, size_t workspace_bytes);

/* hx_exl3_gemm without a workspace argument and without any allocation: the scratch memory (arrival
 * counters, split-K partials, the MFMA path's transformed activations) is a fixed device array of
 * the library, hx_exl3_gemm_noalloc_max_bytes() = 8 MiB per GPU, held until the process ends.
 * Calls whose hx_exl3_gemm_workspace_size(M, N, K) exceeds it return HX_ERR_WORKSPACE.  Every call
 * on one GPU uses that GPU's array: calls that overlap on one GPU (two streams, two host threads)
 * race.  No counterpart in the reference; it is for callers that cannot allocate, such as code
 * under graph capture or serving loops that forbid hipMalloc. */
size_t hx_exl3_gemm_noalloc_max_bytes(void);
int hx_exl3_gemm_noalloc(void* y, const void* x, const hx_group_words* w, int M, int N, int K, int bits, int y_fp32,
                         hx_stream_t stream, int mcg);

/* Bit-exact decode of a trellis slice to W_hat fp16 [packed_rows*16][unpacked_cols] (no
 * Hadamard).  Replaces helios::exl3::reconstruct_slice (src/cuda/quant/reconstruct.cuh:15-35,
 * reconstruct.cu:97-142); bits is the reference's K argument. */
int hx_exl3_reconstruct_slice(void* unpacked, const void* packed, int packed_rows, int packed_cols,
                              int unpacked_cols, int bits, int mcg, int mul1, int64_t n_offset, hx_stream_t stream);

/* Original-basis weights W = diag(suh) . H128 . W_hat . H128 . diag(svh) / 128 per 128 x 128 tile,
 * fp16 [unpacked_rows][unpacked_cols]; unpacked_rows, unpacked_cols and n_offset multiples of 128;
 * suh holds >= unpacked_rows entries, svh >= unpacked_cols (already offset by n_offset).
 * Replaces helios::exl3::reconstruct_had_slice (src/cuda/quant/reconstruct.cuh:37-63,
 * reconstruct.cu:320-374). */
int hx_exl3_reconstruct_had_slice(void* unpacked, const void* packed, const void* suh, const void* svh,
                                  int packed_rows, int packed_cols, int unpacked_rows, int unpacked_cols, int bits,
                                  int mcg, int mul1, int64_t n_offset, hx_stream_t stream);

/* rows*cols blocks of 256 K-bit symbols (uint16 each, low K bits used) <-> 16*K uint16 trellis
 * words per block.  Replace helios::exl3::pack_trellis / unpack_trellis (src/cuda/quant/pack.cuh:9-33,
 * pack.cu:7-176); unpack writes symbols with the bits above K zero. */
int hx_exl3_pack_trellis(void* packed, const void* unpacked, int rows, int cols, int K, hx_stream_t stream);
int hx_exl3_unpack_trellis(void* unpacked, const void* packed, int rows, int cols, int K, hx_stream_t stream);
/* Sign bits of fp16 values, 16 per column: packed[c] (uint16) bit i = sign bit of unpacked[16 c + i]
 * (fp16), c < cols.  Replaces helios::exl3::pack_signs (src/cuda/quant/pack.cuh:36-44, pack.cu:180-233;
 * the bit order is that of the reference kernel, which puts value i in bit i, whatever the comment in
 * pack.cuh:36 says about bit 15). */
int hx_pack_signs(void* packed, const void* unpacked, int cols, hx_stream_t stream);
/* counts[0] += the number of infinities, counts[1] += the number of NaNs among numel values of x
 * (dtype HX_DTYPE_HALF or HX_DTYPE_FLOAT); the caller zeroes counts first.  Replaces
 * helios::exl3::count_inf_nan (src/cuda/quant/util.cuh:9-19, util.cu:54-116). */
int hx_count_inf_nan(const void* x, unsigned long long* counts, uint64_t numel, int dtype, hx_stream_t stream);

/* Row-wise Hadamard-128: y = H128(x) * scale / sqrt(128) on each consecutive 128-element group of a
 * rows x cols tensor of `dtype` (HX_DTYPE_HALF fp16, HX_DTYPE_FLOAT fp32; in place when
 * input == output), with an optional fp16 scale of `cols` entries applied before (pre_scale) or after
 * (post_scale) the transform, not both.  Replaces helios::exl3::had_r_128 (src/cuda/quant/
 * hadamard.cuh:14-25, hadamard.cu:86-170); dtype codes are the reference's DType values. */
#define HX_DTYPE_HALF 0
#define HX_DTYPE_FLOAT 1
#define HX_HAD_RSQRT128 0.088388347648f
int hx_had_r_128(const void* input, void* output, const void* pre_scale, const void* post_scale, int64_t rows,
                 int cols, int dtype, float scale, hx_stream_t stream);
/* The same transform on two tensors of one shape in one launch; both use the same scaling mode.
 * Replaces helios::exl3::had_r_128_dual (src/cuda/quant/hadamard.cuh:27-43, hadamard.cu:173-290). */
int hx_had_r_128_dual(const void* input1, void* output1, const void* pre_scale1, const void* post_scale1,
                      const void* input2, void* output2, const void* pre_scale2, const void* post_scale2,
                      int64_t rows, int cols, int dtype, float scale, hx_stream_t stream);

/* ---- router / permutation / reduction ----------------------------------------------------- */

/* Router top-k: topk_indices int64 [bsz][K], topk_weights fp16 [bsz][K].  act_fn 0 = sigmoid
 * (ROUTING_ACT_SIGMOID), 1 = sqrt(softplus) (ROUTING_ACT_SQRTSP); use_topk 0 selects the sorting
 * variant's key (the activated score; exactly tied activated keys are ordered lower index first,
 * where the reference's radix network uses its lane order).  E <= 512, K <= 64.
 * Replaces helios::aux::routing_ds3_nogroup (src/cuda/aux/routing.cuh:36-49, routing.cu:528-540). */
int hx_routing_ds3_nogroup(const void* scores, const void* bias, int64_t* topk_indices, void* topk_weights,
                           int bsz, int num_experts, int K, float scaling_factor, int use_topk, int act_fn,
                           hx_stream_t stream);

/* Single-token router GEMV: scores[e] = fp16(sum_j x[j] * gate_t[e][j]) (fp32 accumulate), gate_t
 * (E, k) row-major; k even, and a multiple of 32 here (HX_ERR_UNSUPPORTED otherwise).
 * Replaces helios::aux::routing_gemv (src/cuda/aux/routing.cuh:19-29, routing.cu:148-204). */
int hx_routing_gemv(const void* x, const void* gate_t, void* scores, int k, int E, hx_stream_t stream);

/* Decode fast path (one token): scores = hidden . gate_t^T into the scratch `scores`, then the top-k
 * variant of hx_routing_ds3_nogroup.  Replaces helios::aux::routing_ds3_nogroup_hidden
 * (src/cuda/aux/routing.cuh:51-66, routing.cu:547-567). */
int hx_routing_ds3_nogroup_hidden(const void* hidden, const void* gate_t, void* scores, const void* bias,
                                  int64_t* topk_indices, void* topk_weights, int k, int num_experts, int K,
                                  float scaling_factor, int act_fn, hx_stream_t stream);

/* Token-by-expert permutation: expert_count int64 [E+1], token_sorted int64 [M*topk],
 * weight_sorted fp16 [M*topk], route_to_sorted int64 [M*topk] (optional).  Within an expert the
 * order is ascending flat routing index (deterministic; the reference uses an atomic cursor).
 * Replaces helios::glue::moe_permute (src/engine/glue2.cuh:44-46, glue2.cu:280-293); workspace
 * is accepted for signature parity and unused. */
int hx_moe_permute(const int64_t* ids, const void* weights, int M, int topk, int E, int64_t* expert_count,
                   int64_t* token_sorted, void* weight_sorted, int64_t* workspace, hx_stream_t stream,
                   int64_t* route_to_sorted);

/* y[t][c] = sum_j contributions[route_to_sorted[t*topk+j]][c] in ascending j from +0, fp32.
 * Replaces helios::glue::moe_reduce_sorted (src/engine/glue2.cuh:48-49, glue2.cu:297-311). */
int hx_moe_reduce_sorted(float* y, const float* contributions, const int64_t* route_to_sorted, int M, int topk,
                         int hidden, hx_stream_t stream);

/* out = fp16(silu(min(g, L)) * clamp(u, -L, L)).
 * Replaces helios::glue::swiglu_clamp (src/engine/glue2.cuh:64, glue2.cu:406-414). */
int hx_swiglu_clamp(const float* gate, const float* up, void* out, size_t n, float limit, hx_stream_t stream);

/* dst[r][:] = src[idx[r]][:] for r < n, fp16 rows of h elements (the dense-MoE fallback's row
 * gather).  Replaces helios::glue::gather_rows (src/engine/glue.cuh:14, glue.cu:48-60). */
int hx_gather_rows(const void* src, const int64_t* idx, void* dst, int n, int h, hx_stream_t stream);

/* y[idx[r]][:] += float(w[r]) * src[r][:] for r < n (fp32 y and src, fp16 w), the product and the sum
 * each rounded once; idx must hold distinct rows within a call, and calls that share y must be
 * ordered on one stream.  Replaces helios::glue::scatter_add_rows (src/engine/glue.cuh:16-17,
 * glue.cu:62-82). */
int hx_scatter_add_rows(float* y, const float* src, const int64_t* idx, const void* w, int n, int h,
                        hx_stream_t stream);

/* Dense fp16 NT GEMM y[m][n] = sum_k x[m][k] * w[n][k] (x [M][K], w [N][K] row-major, fp32
 * accumulate): fp16 output rounded once (y_fp32 = 0) or fp32 output, added to y when add != 0.  The
 * MoE router logits (w = the router gate [E][hidden]) are its main use.  K % 32 == 0.
 * Replaces helios::glue::gemm_nt_f16 (src/engine/glue2.cuh:9-10, glue2.cu:9-65,165-182). */
int hx_gemm_nt_f16(void* y, const void* x, const void* w, int M, int N, int K, int y_fp32, int add,
                   hx_stream_t stream);

/* ---- MoE layer ---------------------------------------------------------------------------- */

/* Number of expert groups the engine's moe_grouped temp buffers are sized for ([concurrency,
 * max_tokens_per_expert, dim]): CU count / 8 of `device` (negative status on error).  This build's
 * experts do not use those buffers (hx_moe_grouped takes a workspace instead); the value keeps the
 * engine's buffer sizing valid.  Replaces helios::exl3::moe_max_concurrency
 * (src/cuda/quant/exl3_moe.cuh:35, exl3_moe.cu:52-56). */
int hx_moe_max_concurrency(int device);

/* Workspace bytes for hx_moe_grouped / hx_moe_layer with these extents. */
size_t hx_moe_workspace_size(int tokens, int hidden_dim, int intermediate_dim, int num_experts, int topk);

/* Routed experts of one MoE layer: per expert, gather its rows, input Hadamard with suh_g/suh_u,
 * gate/up GEMMs, activation gate with act_limit clamp, down GEMM, times the routing weight and svh_d.
 * With sorted_contributions (fp32 [tokens*topk][hidden_dim], token_sorted order) each weighted row
 * is written once for a fixed-order reduction (hx_moe_reduce_sorted); without it y (fp32
 * [tokens][hidden_dim]) receives y += the routed sum in ascending routing rank (deterministic;
 * route_to_sorted is then required).  tokens <= 8 runs the fused decode-GEMV kernels, larger
 * batches the grouped MFMA path.  Replaces helios::exl3::moe_grouped
 * (src/cuda/quant/exl3_moe.cuh:74-105, exl3_moe.cu:58-265).  temp_* buffers, max_tokens_per_expert,
 * concurrency and num_active are accepted for signature parity and unused (all scratch comes from
 * the workspace; there is no token cap per expert).  Codebooks: mcg or mul1 (as the reference);
 * act_function (exl3_moe_common.cuh:6-8): 0 SiLU, 1 tanh-form GELU, 2 non-gated relu2 (the gate GEMM
 * and gate input are skipped; the gate tables must still be valid arrays, their per-expert pointers
 * are not read).  tokens == 0 is a no-op (the activation pointers may then be NULL). */
int hx_moe_grouped(const void* x, float* y, const int64_t* expert_count, const int64_t* token_sorted,
                   const void* weight_sorted, void* temp_state_g, void* temp_state_u, void* temp_intermediate_g,
                   void* temp_intermediate_u, const hx_expert_tables* tables, int tokens, int hidden_dim,
                   int intermediate_dim, int num_experts, int topk, int max_tokens_per_expert, int concurrency,
                   int K_gate, int K_up, int K_down, int mcg, int mul1, float act_limit, int act_function,
                   int num_active, hx_stream_t stream, float* sorted_contributions, const int64_t* route_to_sorted,
                   void* workspace, size_t workspace_bytes);

/* A whole MoE FFN layer without host synchronisation: sigmoid top-k over scores (fp16
 * [tokens][E], optional bias), deterministic permutation, routed experts, shared expert (three
 * hx_group_words gate/up/down with bit widths shared_bits[3], decoded with the layer's codebook, so
 * their mul1 must agree with it (HX_ERR_INVALID otherwise), or NULL), ordered reduction and
 * y = fp16(routed + shared) [tokens][hidden_dim]; y_routed (fp32, optional) receives the routed
 * sum.  Replaces the single-GPU part of helios Runner::moe_ffn (src/engine/runner.cpp:711-959:
 * shared expert :723-738, router :759-762, permute :764, moe_grouped + reduce :918-922,
 * combine :957-958).  tokens == 0 is a no-op (the activation pointers may then be NULL). */
int hx_moe_layer(void* y, float* y_routed, const void* x, const void* scores, const void* bias,
                 const hx_expert_tables* tables, const hx_group_words* shared, const int* shared_bits, int tokens,
                 int hidden_dim, int intermediate_dim, int num_experts, int topk, int K_gate, int K_up, int K_down,
                 float routed_scale, float act_limit, int mcg, int mul1, void* workspace, size_t workspace_bytes,
                 hx_stream_t stream);

/* ---- checkpoint loading (host side) -------------------------------------------------------- */

/* A directory of safetensors shards, headers parsed (the index file's weight map names the shards,
 * else every *.safetensors file by name); tensor data is read on demand.  Replaces
 * helios::ShardSet::load_dir / find / read (src/core/safetensors.hpp:28-44, safetensors.cpp:35-120). */
typedef struct hx_ckpt hx_ckpt;
int hx_ckpt_open(const char* dir, hx_ckpt** out);
void hx_ckpt_close(hx_ckpt* ckpt);
int hx_ckpt_tensor_count(const hx_ckpt* ckpt);
/* dtype codes: 0 F16, 1 BF16, 2 F32, 3 F64, 4 I32, 5 I16, 6 I8, 7 U8, 8 BOOL, 9 I64 */
int hx_ckpt_tensor_info(const hx_ckpt* ckpt, const char* name, int* dtype, int64_t* shape, int max_dims, int* ndim,
                        uint64_t* bytes);
int hx_ckpt_read(const hx_ckpt* ckpt, const char* name, void* host_dst, uint64_t bytes);

/* Slab layout of one layer's routed experts: expert e occupies [e * stride, (e + 1) * stride) of the
 * slab, piece q = 4 * projection + (0 trellis, 1 suh, 2 svh, 3 mul1) at off[q] with piece[q] bytes,
 * each projection 64-byte aligned.  Replaces helios::ExpertLayout (src/core/expert_layout.hpp:8-16). */
typedef struct hx_expert_layout {
    uint64_t off[12];
    uint64_t piece[12];
    int bits[3];
    uint64_t stride;
} hx_expert_layout;

/* Validates every routed expert of `layer` (names model.language_model.layers.<l>.mlp.experts.<e>.
 * {gate,up,down}_proj.{trellis,suh,svh,mul1}, shapes, dtypes, byte sizes, mul1 == 0x83DCD12D, one bit
 * width per projection across the layer) and returns the slab layout; HX_ERR_INVALID with the tensor's
 * name otherwise.  Replaces helios::expert_layout (src/core/expert_layout.cpp:6-55); 7-bit experts are
 * accepted (the reference refuses them: its fused kernels are not built for 7 bits). */
int hx_ckpt_expert_layout(const hx_ckpt* ckpt, int layer, int experts, int hidden, int intermediate,
                          hx_expert_layout* out);

/* Copies the layer's experts into a device slab of >= experts * layout.stride bytes (pinned staging,
 * `readers` reader threads, asynchronous copies on `stream`; returns once the copies are done).
 * Replaces the expert part of helios Model::load (src/core/model.cpp:254-340), which fills a host
 * arena for PCIe streaming: here every expert stays resident in HBM. */
int hx_ckpt_load_experts(const hx_ckpt* ckpt, int layer, int experts, const hx_expert_layout* layout, void* slab,
                         size_t slab_bytes, int readers, hx_stream_t stream);

/* Writes the nine per-expert pointer arrays of a loaded slab into table_storage (device memory of
 * 9 * experts pointers) and fills *out for hx_moe_layer / hx_moe_grouped (uniform bit widths:
 * bits arrays NULL).  The engine's per-layer ExpertTables build (src/engine/runner.cpp:845-866). */
int hx_ckpt_expert_tables(const hx_expert_layout* layout, const void* slab, int experts, void* table_storage,
                          hx_expert_tables* out, hx_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
