/*
 * exl3_oracle.h -- CPU restatement of the EXL3 expert-GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product library (libhx_exl3.so) never links or calls it.
 *
 * Every function names the reference file:line whose behaviour it restates
 * (paths relative to the reference repository root).  Pinning status of each
 * function (which known-answer test / invariant / fixture checks it) is listed
 * in the header comment of exl3_oracle.c.
 *
 * Conventions: all pointers are host pointers; fp16 values are passed as their
 * IEEE binary16 bit patterns (uint16_t).  cb: 0 = 3INST, 1 = MCG, 2 = MUL1.
 */
#ifndef HX_EXL3_ORACLE_H
#define HX_EXL3_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- exact fp16 <-> fp64 (IEEE binary16, round to nearest even) ---- */
double   hx_or_h2d(uint16_t h);
uint16_t hx_or_d2h(double v);

/* ---- trellis bitstream / codebook (src/cuda/quant/exl3_dq.cuh, codebook.cuh) ---- */
uint32_t hx_or_window(const uint16_t* tile, int bits, int p);
uint16_t hx_or_decode(int cb, uint32_t window);
void     hx_or_codebook_table(int cb, uint16_t* out /* 65536 */);
void     hx_or_pack_tile(const uint16_t* sym /* 256 */, int bits, uint16_t* out /* 16*bits */);
void     hx_or_unpack_tile(const uint16_t* tile, int bits, uint16_t* windows /* 256 */);
void     hx_or_reconstruct(uint16_t* out /* K*N */, const uint16_t* trellis, int K, int N, int bits, int cb);

/* ---- Hadamard-128 (src/cuda/quant/hadamard_inner.cuh) ---- */
void     hx_or_had128(double* v, long n /* multiple of 128 */);
void     hx_or_had_r_128_f16(uint16_t* out, const uint16_t* in, long rows, long cols,
                             const uint16_t* pre_scale, const uint16_t* post_scale, double r_scale);

/* ---- quantized linear y = svh . H_N(H_K(x . suh) . W_hat)  (exl3_gemm_kernel.cuh) ---- */
void     hx_or_linear(double* y /* M*N */, const uint16_t* x /* M*K fp16 */, int M, int K, int N,
                      const uint16_t* trellis, const uint16_t* suh, const uint16_t* svh,
                      int bits, int cb, int out_f16);

/* ---- router / permutation / reduction (routing.cu, glue2.cu) ---- */
void     hx_or_routing(const uint16_t* scores /* bsz*E */, const uint16_t* bias /* E or NULL */,
                       int64_t* topk_idx, uint16_t* topk_w, int bsz, int E, int K, double scale);
void     hx_or_routing2(const uint16_t* scores, const uint16_t* bias, int64_t* topk_idx, uint16_t* topk_w,
                        int bsz, int E, int K, double scale, int use_topk, int act);
void     hx_or_permute(const int64_t* ids, const uint16_t* w, int M, int topk, int E,
                       int64_t* expert_count /* E+1 */, int64_t* token_sorted, uint16_t* weight_sorted,
                       int64_t* route_to_sorted);
void     hx_or_reduce_sorted(float* y, const float* contrib, const int64_t* route_to_sorted,
                             int M, int topk, int hidden);
void     hx_or_swiglu_clamp(const float* g, const float* u, uint16_t* out, long n, float limit);

/* ---- one MoE layer for a subset of tokens (exl3_moe_kernel.cuh + runner.cpp moe_ffn) ----
 * tables: per expert e, gate/up/down trellis, suh, svh pointers and bits (host arrays of length E).
 * rows:   the tokens to evaluate (indices into x); results y_routed[r][hidden] (fp64, routed sum
 *         in rank order) and, when shared != NULL, y_out16[r][hidden] = f16(routed + shared).   */
typedef struct {
    const uint16_t* const* trellis[3];  /* [proj][e] gate, up, down */
    const uint16_t* const* suh[3];
    const uint16_t* const* svh[3];
    const int* bits[3];
    int cb;
} hx_or_experts;

typedef struct {
    const uint16_t* trellis[3];
    const uint16_t* suh[3];
    const uint16_t* svh[3];
    int bits[3];
    int cb;
} hx_or_dense_mlp;

void     hx_or_moe_rows(double* y_routed, uint16_t* y_out16, const uint16_t* x, int hidden, int inter,
                        const int64_t* topk_idx, const uint16_t* topk_w, int topk,
                        const int* rows, int n_rows, const hx_or_experts* ex,
                        const hx_or_dense_mlp* shared, float act_limit, int act);

/* ---- CPU baseline: fp32-accumulate decode + GEMV, OpenMP (threads<=0: all) ----
 * returns wall seconds of one call. */
double   hx_cpu_linear_f32(float* y, const uint16_t* x, int M, int K, int N,
                           const uint16_t* trellis, const uint16_t* suh, const uint16_t* svh,
                           int bits, int cb, int threads);
int      hx_cpu_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
