/*
 * exl3_oracle.c -- CPU restatement of the reference EXL3 expert-GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the CPU baseline.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it;
 * the shipped library never does.
 *
 * Reference files restated (paths relative to the reference repository root):
 *   src/cuda/quant/codebook.cuh:57-124     codebooks cb0 / cb1 / cb2      -> hx_or_decode
 *   src/cuda/quant/exl3_dq.cuh:17-32,188-293 bitstream windows            -> hx_or_window
 *   src/cuda/quant/pack.cu:6-54            symbol packer                  -> hx_or_pack_tile
 *   src/cuda/quant/reconstruct.cu:8-81     trellis -> W_hat fp16 [K][N]   -> hx_or_reconstruct
 *   src/cuda/quant/hadamard_inner.cuh:93-279 Hadamard-128                 -> hx_or_had128
 *   src/cuda/quant/exl3_gemm_kernel.cuh:14-31, exl3_gemm_inner.cuh:456-480 -> hx_or_linear
 *   src/cuda/aux/routing.cu:18-76,211-329  sigmoid top-k router           -> hx_or_routing
 *   src/cuda/aux/routing.cu:18-36,211-443  both activations, both kernels -> hx_or_routing2
 *   src/engine/glue2.cu:244-311,406-414    permute / reduce / swiglu      -> hx_or_permute, ...
 *   src/cuda/quant/exl3_moe_kernel.cuh:57-262, hadamard_inner.cuh:284-481,
 *   src/engine/runner.cpp:723-738,918-958  one MoE layer                  -> hx_or_moe_rows
 *
 * Pinning (what checks each function independently of retyping it; see tests/test_oracle.py):
 *   hx_or_h2d/d2h      exhaustive round trip of all 65536 fp16 patterns; numpy float16 agreement
 *   hx_or_window       impulse tests (a single stream bit reaches exactly the 16 windows whose
 *                      span covers it, at the bit predicted by MSB-first order); window low bits
 *                      == packed symbol (round trip with hx_or_pack_tile)
 *   hx_or_pack_tile    worked bit-level example; round trip; SWAP16 word order
 *   hx_or_decode       exhaustive 65536-entry tables: numpy re-derivation via float16 arithmetic,
 *                      SHA-256 of each table committed as a fixture, cb2 range and affine form
 *   hx_or_reconstruct  lane-layout derivation from the MMA B-fragment layout (k, n map), checked
 *                      through per-position impulse tests and the committed fixture
 *   hx_or_had128       H*H = I, agreement with scipy.linalg.hadamard (Sylvester order)
 *   hx_or_linear       equality with an independent numpy dense pipeline built from the decoded
 *                      W_hat (tests/test_oracle.py), linearity in x
 *   hx_or_routing      brute-force sorted order on small cases, tie rule (lower index first,
 *                      +0 above -0), weight formula sums to scale; with a correction bias: brute
 *                      force on key sigmoid + bias, a biased low logit selected with its unbiased weight
 *   hx_or_permute      definition (stable counting sort), multiset equality with the atomic version
 *   hx_or_reduce_sorted reference fixture test_deterministic_reductions.cu:49-66 ({1e20,-1e20,1,1})
 *   hx_or_moe_rows     dense numpy restatement of the layer from decoded W_hat and scipy Hadamard on
 *                      a tiny layer; exact linearity in the routing weight; row selection
 */
#include "exl3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ fp16 */

double hx_or_h2d(uint16_t h)
{
    int s = (h >> 15) & 1, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexp((double)(m | 0x400), e - 25);
    return s ? -v : v;
}

uint16_t hx_or_d2h(double v)
{
    uint16_t sign = signbit(v) ? 0x8000 : 0;
    double a = fabs(v);
    if (isnan(v)) return 0x7e00;
    if (a >= 65520.0) return sign | 0x7c00;
    if (a < ldexp(1.0, -14)) {
        double q = nearbyint(ldexp(a, 24));  /* round half even (default mode) */
        return sign | (uint16_t)q;
    }
    int ex;
    double m = frexp(a, &ex);                /* a = m * 2^ex, m in [0.5, 1) */
    int E = ex - 1;
    double q = nearbyint((ldexp(m, 1) - 1.0) * 1024.0);
    if (q >= 1024.0) { q = 0.0; E += 1; }
    if (E > 15) return sign | 0x7c00;
    return sign | (uint16_t)(((E + 15) << 10) | (int)q);
}

static inline uint16_t rh(double v) { return hx_or_d2h(v); }
static inline double hd(uint16_t h) { return hx_or_h2d(h); }

/* ------------------------------------------------------------------ bitstream */

/* Stream bit b of a tile: bit 31 - (b % 32) of the little-endian uint32 word b / 32
 * (MSB-first uint16 stream with halves swapped per uint32: pack.cu:27-53). */
static inline int stream_bit(const uint16_t* tile, int b)
{
    int wi = b >> 5;
    uint32_t w = (uint32_t)tile[2 * wi] | ((uint32_t)tile[2 * wi + 1] << 16);
    return (w >> (31 - (b & 31))) & 1;
}

/* Window p: the 16 stream bits ending at bit (p + 1) * bits, read MSB-first, indices cyclic
 * modulo 256 * bits (tail-biting trellis).  exl3_dq.cuh:17-32 (dq), :188-208 (2-bit form). */
uint32_t hx_or_window(const uint16_t* tile, int bits, int p)
{
    int total = 256 * bits;
    int start = (p + 1) * bits - 16;
    uint32_t w = 0;
    for (int i = 0; i < 16; ++i) {
        int b = ((start + i) % total + total) % total;
        w = (w << 1) | (uint32_t)stream_bit(tile, b);
    }
    return w;
}

/* codebook.cuh:57-90.  Arithmetic is uint32 modulo 2^32; every fp16 operation is one rounding of
 * the exact value, which double holds exactly for these operands. */
uint16_t hx_or_decode(int cb, uint32_t w)
{
    uint32_t x = w & 0xffffu;
    if (cb == 2) {
        x *= 0x83DCD12Du;
        uint32_t s = (x & 0xff) + ((x >> 8) & 0xff) + ((x >> 16) & 0xff) + (x >> 24);
        /* fp16 (0x6400 + s) == 1024 + s exactly (s <= 1020); hfma(h, 0x1eee, 0xc931) */
        return rh((1024.0 + (double)s) * hd(0x1eee) + hd(0xc931));
    }
    if (cb == 1) x *= 0xCBAC1FEDu;
    else x = x * 89226354u + 64248484u;
    /* lop3 immediate 0x6a over (a=x, b=0x8fff8fff, c=0x3b603b60) is (a & b) ^ c */
    x = (x & 0x8fff8fffu) ^ 0x3b603b60u;
    return rh(hd((uint16_t)(x & 0xffff)) + hd((uint16_t)(x >> 16)));
}

void hx_or_codebook_table(int cb, uint16_t* out)
{
    for (uint32_t w = 0; w < 65536; ++w) out[w] = hx_or_decode(cb, w);
}

/* pack.cu:6-54: symbol p occupies stream bits [p*bits, (p+1)*bits), MSB first. */
void hx_or_pack_tile(const uint16_t* sym, int bits, uint16_t* out)
{
    int nwords = 8 * bits;
    uint32_t* words = (uint32_t*)calloc((size_t)nwords, sizeof(uint32_t));
    for (int p = 0; p < 256; ++p) {
        uint32_t v = sym[p] & ((1u << bits) - 1u);
        for (int i = 0; i < bits; ++i) {
            int b = p * bits + i;
            if ((v >> (bits - 1 - i)) & 1) words[b >> 5] |= 1u << (31 - (b & 31));
        }
    }
    for (int i = 0; i < nwords; ++i) {
        out[2 * i] = (uint16_t)(words[i] & 0xffff);
        out[2 * i + 1] = (uint16_t)(words[i] >> 16);
    }
    free(words);
}

void hx_or_unpack_tile(const uint16_t* tile, int bits, uint16_t* windows)
{
    for (int p = 0; p < 256; ++p) windows[p] = (uint16_t)hx_or_window(tile, bits, p);
}

/* Position p -> (k, n) inside a 16x16 tile.  dq_dispatch(ptr, 8 * lane) yields positions
 * 8*lane..+7 as two m16n8k16 B fragments (exl3_dq.cuh:188-208); reconstruct.cu:36-81 stores
 * fragment element (lane, j) at row k = 2*(lane%4) + (j&1) + 8*((j>>1)&1), column
 * n = lane/4 + 8*(j>>2). */
static inline void pos_to_kn(int p, int* k, int* n)
{
    int l = p >> 3, j = p & 7;
    *k = 2 * (l & 3) + (j & 1) + 8 * ((j >> 1) & 1);
    *n = 8 * (j >> 2) + (l >> 2);
}

static void decode_tile_h(const uint16_t* tile, int bits, int cb, uint16_t w16[16][16])
{
    for (int p = 0; p < 256; ++p) {
        int k, n;
        pos_to_kn(p, &k, &n);
        w16[k][n] = hx_or_decode(cb, hx_or_window(tile, bits, p));
    }
}

/* reconstruct.cu:8-81 / :97-142: tile (tk, tn) at uint16 offset (tk*(N/16)+tn)*16*bits. */
void hx_or_reconstruct(uint16_t* out, const uint16_t* trellis, int K, int N, int bits, int cb)
{
    int tiles_n = N / 16, tw = 16 * bits;
#pragma omp parallel for schedule(static)
    for (int tk = 0; tk < K / 16; ++tk) {
        uint16_t w16[16][16];
        for (int tn = 0; tn < tiles_n; ++tn) {
            decode_tile_h(trellis + ((size_t)tk * tiles_n + tn) * tw, bits, cb, w16);
            for (int k = 0; k < 16; ++k)
                for (int n = 0; n < 16; ++n)
                    out[(size_t)(16 * tk + k) * N + 16 * tn + n] = w16[k][n];
        }
    }
}

/* ------------------------------------------------------------------ Hadamard */

/* Sylvester-order 128-point transform per 128-element block, scaled by 1/sqrt(128)
 * (hadamard_inner.cuh:93-147: element 4*lane + r; butterflies pair index bits low to high). */
void hx_or_had128(double* v, long n)
{
    const double rs = 1.0 / sqrt(128.0);
    for (long base = 0; base < n; base += 128) {
        double* b = v + base;
        for (int h = 1; h < 128; h <<= 1)
            for (int j = 0; j < 128; j += h << 1)
                for (int k = j; k < j + h; ++k) {
                    double a = b[k], c = b[k + h];
                    b[k] = a + c;
                    b[k + h] = a - c;
                }
        for (int j = 0; j < 128; ++j) b[j] *= rs;
    }
}

/* hadamard.cu had_r_128: f16 in, optional f16 pre-scale (hmul), transform, * r_scale, f16,
 * optional f16 post-scale (hmul).  Evaluated exactly, one rounding per reference rounding point. */
void hx_or_had_r_128_f16(uint16_t* out, const uint16_t* in, long rows, long cols,
                         const uint16_t* pre, const uint16_t* post, double r_scale)
{
    double buf[128];
    for (long r = 0; r < rows; ++r)
        for (long c0 = 0; c0 < cols; c0 += 128) {
            for (int j = 0; j < 128; ++j) {
                uint16_t h = in[r * cols + c0 + j];
                if (pre) h = rh(hd(h) * hd(pre[c0 + j]));
                buf[j] = hd(h);
            }
            hx_or_had128(buf, 128);
            for (int j = 0; j < 128; ++j) {
                uint16_t h = rh(buf[j] * sqrt(128.0) * r_scale);
                if (post) h = rh(hd(h) * hd(post[c0 + j]));
                out[r * cols + c0 + j] = h;
            }
        }
}

/* ------------------------------------------------------------------ linear */

/* a_had = f16(H(f16(x . suh)))  (had_hf_r_128_inner<true,false>, exl3_gemm_kernel.cuh:14-31) */
static void input_had(uint16_t* a, const uint16_t* x, const uint16_t* suh, long n)
{
    double buf[128];
    for (long c0 = 0; c0 < n; c0 += 128) {
        for (int j = 0; j < 128; ++j) buf[j] = hd(rh(hd(x[c0 + j]) * hd(suh[c0 + j])));
        hx_or_had128(buf, 128);
        for (int j = 0; j < 128; ++j) a[c0 + j] = rh(buf[j]);
    }
}

/* acc[M][N] = a[M][K] . W_hat[K][N] in fp64 */
static void matmul_trellis(double* acc, const uint16_t* a, int M, int K, int N,
                           const uint16_t* trellis, int bits, int cb)
{
    int tiles_n = N / 16, tw = 16 * bits;
    memset(acc, 0, sizeof(double) * (size_t)M * N);
#pragma omp parallel for schedule(static)
    for (int tn = 0; tn < tiles_n; ++tn) {
        uint16_t w16[16][16];
        double wd[16][16];
        for (int tk = 0; tk < K / 16; ++tk) {
            decode_tile_h(trellis + ((size_t)tk * tiles_n + tn) * tw, bits, cb, w16);
            for (int k = 0; k < 16; ++k)
                for (int n = 0; n < 16; ++n) wd[k][n] = hd(w16[k][n]);
            for (int m = 0; m < M; ++m) {
                double* y = acc + (size_t)m * N + 16 * tn;
                const uint16_t* am = a + (size_t)m * K + 16 * tk;
                for (int k = 0; k < 16; ++k) {
                    double av = hd(am[k]);
                    for (int n = 0; n < 16; ++n) y[n] += av * wd[k][n];
                }
            }
        }
    }
}

/* y = svh . H_N(acc)  (fp32 output: had_ff_r_128_inner<false,true>); out_f16 rounds after the
 * transform and again after the svh multiply (had_fh_r_128_inner<false,true>). */
void hx_or_linear(double* y, const uint16_t* x, int M, int K, int N,
                  const uint16_t* trellis, const uint16_t* suh, const uint16_t* svh,
                  int bits, int cb, int out_f16)
{
    uint16_t* a = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)M * K);
    for (int m = 0; m < M; ++m) input_had(a + (size_t)m * K, x + (size_t)m * K, suh, K);
    matmul_trellis(y, a, M, K, N, trellis, bits, cb);
    for (int m = 0; m < M; ++m) {
        double* ym = y + (size_t)m * N;
        hx_or_had128(ym, N);
        for (int n = 0; n < N; ++n)
            ym[n] = out_f16 ? hd(rh(hd(rh(ym[n])) * hd(svh[n]))) : ym[n] * hd(svh[n]);
    }
    free(a);
}

/* ------------------------------------------------------------------ router */

/* Monotone unsigned encoding of an fp32 key used by warp_reduce_best_f32 (routing.cu:45-56):
 * larger encoding = larger key, +0 ranks above -0; equal encodings -> lower expert index. */
static inline uint32_t key_enc(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }

/* Score activation (routing.cu:18-36): act 0 = sigmoid, act 1 = sqrt(softplus(x)) with softplus's
 * threshold 20 (x itself above it), both in double then rounded to fp32 as the kernels hold them. */
static double route_act(double x, int act)
{
    if (act == 1) return sqrt(x > 20.0 ? x : log1p(exp(x)));
    return sigmoid_d(x);
}

/* routing.cu:211-329 (routing_ds3_nogroup_topk_kernel, use_topk) and routing.cu:333-443
 * (routing_ds3_nogroup_kernel, the sorting variant), for both score activations (routing.cu:18-36).
 * Selection key: with a bias, act(logit) + bias in fp32 (both variants); without, the fp16 logit
 * (use_topk) or act(logit) (sorting variant).  Larger key first; equal keys: lower expert index
 * first.  Weights: act(logit) normalised over the selection, o * scale / (sum + 1e-20) (use_topk) or
 * o * (scale / (sum + 1e-20)) (sorting variant), rounded to fp16. */
void hx_or_routing2(const uint16_t* scores, const uint16_t* bias, int64_t* topk_idx, uint16_t* topk_w,
                    int bsz, int E, int K, double scale, int use_topk, int act)
{
    uint32_t* enc = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)E);
    char* used = (char*)malloc((size_t)E);
    for (int r = 0; r < bsz; ++r) {
        const uint16_t* s = scores + (size_t)r * E;
        for (int e = 0; e < E; ++e) {
            float logit = (float)hd(s[e]);
            float a = (float)route_act(logit, act);
            float key = bias ? a + (float)hd(bias[e]) : (use_topk ? logit : a);
            enc[e] = key_enc(key);
            used[e] = 0;
        }
        float o[64];
        float sum = 0.0f;
        for (int k = 0; k < K; ++k) {
            int best = -1;
            for (int e = 0; e < E; ++e)
                if (!used[e] && (best < 0 || enc[e] > enc[best])) best = e;
            used[best] = 1;
            topk_idx[(size_t)r * K + k] = best;
            o[k] = (float)route_act(hd(s[best]), act);
            sum += o[k];
        }
        sum += 1e-20f;
        for (int k = 0; k < K; ++k)
            topk_w[(size_t)r * K + k] = use_topk ? rh((double)(o[k] * (float)scale / sum))
                                                 : rh((double)(o[k] * ((float)scale / sum)));
    }
    free(enc);
    free(used);
}

/* routing.cu:211-329 (routing_ds3_nogroup_topk_kernel, sigmoid activation). */
void hx_or_routing(const uint16_t* scores, const uint16_t* bias, int64_t* topk_idx, uint16_t* topk_w,
                   int bsz, int E, int K, double scale)
{
    uint32_t* enc = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)E);
    char* used = (char*)malloc((size_t)E);
    for (int r = 0; r < bsz; ++r) {
        const uint16_t* s = scores + (size_t)r * E;
        for (int e = 0; e < E; ++e) {
            float logit = (float)hd(s[e]);
            float key = bias ? (float)sigmoid_d(logit) + (float)hd(bias[e]) : logit;
            enc[e] = key_enc(key);
            used[e] = 0;
        }
        double o[64], sum = 0.0;
        for (int k = 0; k < K; ++k) {
            int best = -1;
            for (int e = 0; e < E; ++e)
                if (!used[e] && (best < 0 || enc[e] > enc[best])) best = e;
            used[best] = 1;
            topk_idx[(size_t)r * K + k] = best;
            o[k] = sigmoid_d(hd(s[best]));
            sum += o[k];
        }
        sum += 1e-20;
        for (int k = 0; k < K; ++k) topk_w[(size_t)r * K + k] = rh(o[k] * scale / sum);
    }
    free(enc);
    free(used);
}

/* glue2.cu:244-293 with the canonical within-expert order: ascending flat routing index. */
void hx_or_permute(const int64_t* ids, const uint16_t* w, int M, int topk, int E,
                   int64_t* expert_count, int64_t* token_sorted, uint16_t* weight_sorted,
                   int64_t* route_to_sorted)
{
    int total = M * topk;
    int64_t* cur = (int64_t*)calloc((size_t)E + 1, sizeof(int64_t));
    for (int e = 0; e <= E; ++e) expert_count[e] = 0;
    for (int i = 0; i < total; ++i) expert_count[ids[i]]++;
    int64_t acc = 0;
    for (int e = 0; e < E; ++e) { cur[e] = acc; acc += expert_count[e]; }
    for (int i = 0; i < total; ++i) {
        int64_t pos = cur[ids[i]]++;
        token_sorted[pos] = i / topk;
        weight_sorted[pos] = w[i];
        if (route_to_sorted) route_to_sorted[i] = pos;
    }
    free(cur);
}

/* glue2.cu:297-306: fp32 sum in ascending routing rank from +0. */
void hx_or_reduce_sorted(float* y, const float* contrib, const int64_t* route_to_sorted,
                         int M, int topk, int hidden)
{
    for (int t = 0; t < M; ++t)
        for (int c = 0; c < hidden; ++c) {
            float acc = 0.0f;
            for (int j = 0; j < topk; ++j)
                acc += contrib[(size_t)route_to_sorted[t * topk + j] * hidden + c];
            y[(size_t)t * hidden + c] = acc;
        }
}

/* glue2.cu:406-414 */
void hx_or_swiglu_clamp(const float* g, const float* u, uint16_t* out, long n, float limit)
{
    for (long i = 0; i < n; ++i) {
        double gv = fmin((double)g[i], limit);
        double uv = fmin(fmax((double)u[i], -limit), limit);
        out[i] = rh(gv / (1.0 + exp(-gv)) * uv);
    }
}

/* ------------------------------------------------------------------ MoE */

/* fp16 silu chain of had_hf_r_128_guad_inner (hadamard_inner.cuh:331-340), each op one
 * rounding of the exact value. */
static uint16_t silu_h(uint16_t g)
{
    uint16_t e = rh(exp(-hd(g)));
    uint16_t s = rh(1.0 + hd(e));
    uint16_t r = rh(1.0 / hd(s));
    return rh(hd(g) * hd(r));
}

/* tanh-form GELU of an fp16 value, rounded to fp16 (hadamard_inner.cuh:342-349; the reference's
 * fp32 tanh approximation is restated as the exact function) */
static uint16_t gelu_h(uint16_t g)
{
    double x = hd(g);
    return rh(0.5 * x * (1.0 + tanh(0.797884560803 * (x + 0.044715 * x * x * x))));
}

/* act: 0 SiLU, 1 GELU, 2 non-gated relu2 (exl3_moe_common.cuh:6-8; the gate GEMM is skipped and the
 * gate lane is relu(u), hadamard_inner.cuh:378-382) */
static void expert_row(double* c_out, const uint16_t* xt, int hidden, int inter,
                       const hx_or_experts* ex, int e, uint16_t wt, float L, int act)
{
    uint16_t* ag = (uint16_t*)malloc(2 * (size_t)hidden);
    uint16_t* au = (uint16_t*)malloc(2 * (size_t)hidden);
    uint16_t* ad = (uint16_t*)malloc(2 * (size_t)inter);
    double* G = (double*)malloc(sizeof(double) * (size_t)inter);
    double* U = (double*)malloc(sizeof(double) * (size_t)inter);
    double* D = (double*)malloc(sizeof(double) * (size_t)hidden);
    double buf[128];

    /* 1. gather + input Hadamard (exl3_moe_kernel.cuh:85-112) */
    const int gated = act != 2;
    if (gated) input_had(ag, xt, ex->suh[0][e], hidden);
    input_had(au, xt, ex->suh[1][e], hidden);
    /* 2. G, U with fp16 output, no output transform (exl3_gemm_kernel_inner<..., false>) */
    if (gated) matmul_trellis(G, ag, 1, hidden, inter, ex->trellis[0][e], ex->bits[0][e], ex->cb);
    else for (int i = 0; i < inter; ++i) G[i] = 0.0;
    matmul_trellis(U, au, 1, hidden, inter, ex->trellis[1][e], ex->bits[1][e], ex->cb);
    /* 3-6. guad (hadamard_inner.cuh:284-413) */
    const uint16_t* svg = gated ? ex->svh[0][e] : NULL;
    const uint16_t* svu = ex->svh[1][e];
    const uint16_t* sud = ex->suh[2][e];
    uint16_t Lh = rh(L), nLh = rh(-L);
    for (int c0 = 0; c0 < inter; c0 += 128) {
        uint16_t g16[128], u16[128], p16[128];
        for (int j = 0; j < 128; ++j) buf[j] = hd(rh(G[c0 + j]));
        hx_or_had128(buf, 128);
        for (int j = 0; j < 128; ++j) g16[j] = gated ? rh(hd(rh(buf[j])) * hd(svg[c0 + j])) : 0;
        for (int j = 0; j < 128; ++j) buf[j] = hd(rh(U[c0 + j]));
        hx_or_had128(buf, 128);
        for (int j = 0; j < 128; ++j) u16[j] = rh(hd(rh(buf[j])) * hd(svu[c0 + j]));
        for (int j = 0; j < 128; ++j) {
            uint16_t u = u16[j];
            uint16_t g = act == 1 ? gelu_h(g16[j]) : act == 2 ? (hd(u) > 0.0 ? u : 0) : silu_h(g16[j]);
            if (L != 0.0f) {
                if (hd(u) < hd(nLh)) u = nLh;
                if (hd(u) > hd(Lh)) u = Lh;
                if (hd(g) > hd(Lh)) g = Lh;
            }
            p16[j] = rh(hd(rh(hd(g) * hd(u))) * hd(sud[c0 + j]));
            buf[j] = hd(p16[j]);
        }
        hx_or_had128(buf, 128);
        for (int j = 0; j < 128; ++j) ad[c0 + j] = rh(buf[j]);
    }
    /* 7. D with fp16 output */
    matmul_trellis(D, ad, 1, inter, hidden, ex->trellis[2][e], ex->bits[2][e], ex->cb);
    for (int c = 0; c < hidden; ++c) D[c] = hd(rh(D[c]));
    /* 8. c = H(D) * w / sqrt(128) . svh_d  (hadamard_inner.cuh:418-481) */
    hx_or_had128(D, hidden);
    const uint16_t* svd = ex->svh[2][e];
    for (int c = 0; c < hidden; ++c) c_out[c] = D[c] * hd(wt) * hd(svd[c]);
    free(ag); free(au); free(ad); free(G); free(U); free(D);
}

void hx_or_moe_rows(double* y_routed, uint16_t* y_out16, const uint16_t* x, int hidden, int inter,
                    const int64_t* topk_idx, const uint16_t* topk_w, int topk,
                    const int* rows, int n_rows, const hx_or_experts* ex,
                    const hx_or_dense_mlp* shared, float act_limit, int act)
{
    double* c = (double*)malloc(sizeof(double) * (size_t)hidden);
    for (int r = 0; r < n_rows; ++r) {
        int t = rows[r];
        const uint16_t* xt = x + (size_t)t * hidden;
        double* yr = y_routed + (size_t)r * hidden;
        float* yf = (float*)calloc((size_t)hidden, sizeof(float));
        for (int j = 0; j < topk; ++j) {
            expert_row(c, xt, hidden, inter, ex, (int)topk_idx[(size_t)t * topk + j],
                       topk_w[(size_t)t * topk + j], act_limit, act);
            /* ordered fp32 reduction, ascending rank (glue2.cu:297-306) */
            for (int i = 0; i < hidden; ++i) yf[i] += (float)c[i];
        }
        for (int i = 0; i < hidden; ++i) yr[i] = yf[i];
        if (shared && y_out16) {
            /* runner.cpp:723-738: gate/up fp32 out, swiglu_clamp -> fp16, down fp32 out */
            double* g = (double*)malloc(sizeof(double) * (size_t)inter);
            double* u = (double*)malloc(sizeof(double) * (size_t)inter);
            double* d = (double*)malloc(sizeof(double) * (size_t)hidden);
            uint16_t* act = (uint16_t*)malloc(2 * (size_t)inter);
            hx_or_linear(g, xt, 1, hidden, inter, shared->trellis[0], shared->suh[0], shared->svh[0],
                         shared->bits[0], shared->cb, 0);
            hx_or_linear(u, xt, 1, hidden, inter, shared->trellis[1], shared->suh[1], shared->svh[1],
                         shared->bits[1], shared->cb, 0);
            for (int i = 0; i < inter; ++i) {
                double gv = fmin(g[i], act_limit);
                double uv = fmin(fmax(u[i], -act_limit), act_limit);
                act[i] = rh(gv / (1.0 + exp(-gv)) * uv);
            }
            hx_or_linear(d, act, 1, inter, hidden, shared->trellis[2], shared->suh[2], shared->svh[2],
                         shared->bits[2], shared->cb, 0);
            /* runner.cpp:957-958: y = y_routed + y_shared (fp32), cast to fp16 */
            for (int i = 0; i < hidden; ++i)
                y_out16[(size_t)r * hidden + i] = rh((double)(yf[i] + (float)d[i]));
            free(g); free(u); free(d); free(act);
        }
        free(yf);
    }
    free(c);
}

/* ------------------------------------------------------------------ CPU baseline */

int hx_cpu_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static float* g_cb_table[3];

static const float* cb_table_f32(int cb)
{
    if (!g_cb_table[cb]) {
        float* t = (float*)malloc(sizeof(float) * 65536);
        for (uint32_t w = 0; w < 65536; ++w) t[w] = (float)hd(hx_or_decode(cb, w));
        g_cb_table[cb] = t;
    }
    return g_cb_table[cb];
}

static void had128_f32(float* b)
{
    for (int h = 1; h < 128; h <<= 1)
        for (int j = 0; j < 128; j += h << 1)
            for (int k = j; k < j + h; ++k) {
                float a = b[k], c = b[k + h];
                b[k] = a + c;
                b[k + h] = a - c;
            }
    for (int j = 0; j < 128; ++j) b[j] *= 0.088388347648f;
}

/* A plain CPU implementation of the same linear: per-codebook 64K-entry fp32 decode table,
 * window extraction from a 64-bit stream register, fp32 accumulation, OpenMP over column
 * tiles.  This is the timed CPU baseline, not the parity oracle (hx_or_linear is). */
double hx_cpu_linear_f32(float* y, const uint16_t* x, int M, int K, int N,
                         const uint16_t* trellis, const uint16_t* suh, const uint16_t* svh,
                         int bits, int cb, int threads)
{
    const float* tab = cb_table_f32(cb);
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    float* a = (float*)malloc(sizeof(float) * (size_t)M * K);
    for (int m = 0; m < M; ++m)
        for (int c0 = 0; c0 < K; c0 += 128) {
            float* b = a + (size_t)m * K + c0;
            for (int j = 0; j < 128; ++j)
                b[j] = (float)hd(rh(hd(x[(size_t)m * K + c0 + j]) * hd(suh[c0 + j])));
            had128_f32(b);
            for (int j = 0; j < 128; ++j) b[j] = (float)hd(rh(b[j]));
        }
    int tiles_n = N / 16, tw = 16 * bits;
    int nt = threads > 0 ? threads : hx_cpu_max_threads();
    (void)nt;
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int tn = 0; tn < tiles_n; ++tn)
    for (int m0 = 0; m0 < M; m0 += 8) {
        int mc = M - m0 < 8 ? M - m0 : 8;
        float acc[8][16];
        memset(acc, 0, sizeof(acc));
        for (int tk = 0; tk < K / 16; ++tk) {
            const uint16_t* t = trellis + ((size_t)tk * tiles_n + tn) * tw;
            uint32_t words[64];
            for (int i = 0; i < 8 * bits; ++i) words[i] = (uint32_t)t[2 * i] | ((uint32_t)t[2 * i + 1] << 16);
            int total = 256 * bits;
            for (int p = 0; p < 256; ++p) {
                int end = (p + 1) * bits;            /* window = stream bits [end-16, end) */
                int s = (end - 16 + total) % total;
                int wi = s >> 5, off = s & 31;
                uint64_t pair = ((uint64_t)words[wi] << 32) | words[(wi + 1) % (8 * bits)];
                uint32_t w = (uint32_t)(pair >> (48 - off)) & 0xffff;
                float v = tab[w];
                int l = p >> 3, j = p & 7;
                int k = 2 * (l & 3) + (j & 1) + 8 * ((j >> 1) & 1);
                int n = 8 * (j >> 2) + (l >> 2);
                for (int m = 0; m < mc; ++m) acc[m][n] += a[(size_t)(m0 + m) * K + 16 * tk + k] * v;
            }
        }
        for (int m = 0; m < mc; ++m)
            for (int n = 0; n < 16; ++n) y[(size_t)(m0 + m) * N + 16 * tn + n] = acc[m][n];
    }
    for (int m = 0; m < M; ++m)
        for (int c0 = 0; c0 < N; c0 += 128) {
            float* b = y + (size_t)m * N + c0;
            had128_f32(b);
            for (int j = 0; j < 128; ++j) b[j] *= (float)hd(svh[c0 + j]);
        }
    free(a);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}
