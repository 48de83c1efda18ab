// hx_misc.hip -- trellis reconstruct, standalone Hadamard-128, sigmoid top-k router, deterministic
// MoE permutation, ordered reduction and swiglu for gfx950.
#include "hx_device.hpp"
#include <type_traits>
#include "hx_kernels.hpp"

namespace hx {

// ------------------------------------------------------------------ reconstruct

// One workgroup per (tile row tk, 8 consecutive tile columns): thread t writes 8 consecutive
// fp16 of row 16*tk + t/16.  Reference: reconstruct.cu:8-81 (same W_hat [K][N] row-major output).
template <int CB>
__global__ __launch_bounds__(256) void reconstruct_kernel(_Float16* out, const uint16_t* packed, int packed_cols,
                                                          int packed_n_offset, int out_cols, int bits)
{
    __shared__ uint32_t words[8][64];
    const int t = threadIdx.x;
    const int tk = blockIdx.y;
    const int tn0 = blockIdx.x * 8;  // first output tile column of this group
    const int nw = 8 * bits;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(packed) +
                          ((size_t)tk * packed_cols + packed_n_offset + tn0) * nw;
    for (int i = t; i < 8 * nw; i += 256) words[i / nw][i % nw] = src[i];
    __syncthreads();
    const int k = t >> 4, c0 = (t & 15) * 8;
    const int tile = c0 >> 4, n0 = c0 & 15;
    hx_h8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = hx_decode1<CB>(window_rt(words[tile], bits, hx_kn_to_pos(k, n0 + i)));
    *reinterpret_cast<hx_h8*>(out + (size_t)(16 * tk + k) * out_cols + tn0 * 16 + c0) = v;
}

hipError_t launch_reconstruct(_Float16* out, const uint16_t* packed, int packed_rows, int packed_cols,
                              int unpacked_cols, int bits, int cb, long n_offset, hipStream_t st)
{
    if (bits < 1 || bits > 8 || unpacked_cols % 128 || n_offset % 128 || n_offset < 0 ||
        n_offset + unpacked_cols > (long)packed_cols * 16)
        return hipErrorInvalidValue;
    if (unpacked_cols == 0 || packed_rows == 0) return hipSuccess;
    dim3 grid(unpacked_cols / 128, packed_rows);
    const int off = (int)(n_offset / 16);
    switch (cb) {
        case 0: hipLaunchKernelGGL(reconstruct_kernel<0>, grid, dim3(256), 0, st, out, packed, packed_cols, off, unpacked_cols, bits); break;
        case 1: hipLaunchKernelGGL(reconstruct_kernel<1>, grid, dim3(256), 0, st, out, packed, packed_cols, off, unpacked_cols, bits); break;
        default: hipLaunchKernelGGL(reconstruct_kernel<2>, grid, dim3(256), 0, st, out, packed, packed_cols, off, unpacked_cols, bits); break;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ had_r_128

// Row-wise Hadamard-128 with an optional fp16 scale per column, applied before (SCALE 1) or after
// (SCALE 2) the transform, on one or two tensors of rows x cols (reference hadamard.cu had_r_128 /
// had_r_128_dual, hadamard_inner.cuh:93-225).  fp16 data: pre-scale by an fp16 multiply, transform
// in fp32, times r_scale, round to fp16, post-scale by an fp16 multiply.  fp32 data: the scales are
// widened and every step stays in fp32.  One wave per 128-element block, two elements per lane;
// blocks past the first tensor's belong to the second.
struct HadPair {
    const void* in[2];
    void* out[2];
    const _Float16* scale[2];
};

template <typename T, int SCALE>
__global__ __launch_bounds__(256) void had_r_128_kernel(HadPair job, long blocks, int cols, float r_scale)
{
    const int lane = threadIdx.x & 63;
    long b = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= 2 * blocks || (b >= blocks && !job.in[1])) return;
    const int which = b >= blocks;
    b -= which * blocks;
    const long row = b / (cols / 128);
    const int c = (int)(b % (cols / 128)) * 128 + 2 * lane;
    const T* in = static_cast<const T*>(job.in[which]) + row * cols + c;
    T* out = static_cast<T*>(job.out[which]) + row * cols + c;
    const _Float16* sc = job.scale[which];
    const float rs = r_scale / HX_RSQRT128;  // hx_had128_wave already applies 1/sqrt(128)
    if constexpr (std::is_same<T, float>::value) {
        float v0 = in[0], v1 = in[1];
        if (SCALE == 1) v0 *= (float)sc[c], v1 *= (float)sc[c + 1];
        hx_had128_wave(v0, v1);
        v0 *= rs, v1 *= rs;
        if (SCALE == 2) v0 *= (float)sc[c], v1 *= (float)sc[c + 1];
        out[0] = v0, out[1] = v1;
    } else {
        hx_h2 v = *reinterpret_cast<const hx_h2*>(in);
        if (SCALE == 1) v = v * *reinterpret_cast<const hx_h2*>(sc + c);
        float v0 = (float)v.x, v1 = (float)v.y;
        hx_had128_wave(v0, v1);
        hx_h2 o = {(_Float16)(v0 * rs), (_Float16)(v1 * rs)};
        if (SCALE == 2) o = o * *reinterpret_cast<const hx_h2*>(sc + c);
        *reinterpret_cast<hx_h2*>(out) = o;
    }
}

template <typename T>
static void had_launch(const HadPair& job, int scale_mode, long blocks, int cols, float r_scale, hipStream_t st)
{
    const long total = (job.in[1] ? 2 : 1) * blocks;
    const dim3 grid((unsigned)((total + 3) / 4));
    if (scale_mode == 1) hipLaunchKernelGGL((had_r_128_kernel<T, 1>), grid, dim3(256), 0, st, job, blocks, cols, r_scale);
    else if (scale_mode == 2) hipLaunchKernelGGL((had_r_128_kernel<T, 2>), grid, dim3(256), 0, st, job, blocks, cols, r_scale);
    else hipLaunchKernelGGL((had_r_128_kernel<T, 0>), grid, dim3(256), 0, st, job, blocks, cols, r_scale);
}

hipError_t launch_had_r_128(const void* in1, void* out1, const void* scale1, const void* in2, void* out2,
                            const void* scale2, int scale_mode, long rows, int cols, bool fp32, float r_scale,
                            hipStream_t st)
{
    if (cols % 128) return hipErrorInvalidValue;
    const long blocks = rows * (cols / 128);
    if (blocks == 0) return hipSuccess;
    HadPair job{{in1, in2}, {out1, out2}, {(const _Float16*)scale1, (const _Float16*)scale2}};
    if (fp32) had_launch<float>(job, scale_mode, blocks, cols, r_scale, st);
    else had_launch<_Float16>(job, scale_mode, blocks, cols, r_scale, st);
    return hipGetLastError();
}

// ------------------------------------------------------------------ router

// Router top-k, one wave per token: reference routing_ds3_nogroup_topk_kernel (routing.cu:211-329,
// use_topk) and routing_ds3_nogroup_kernel (routing.cu:333-443, the sorting variant), for both score
// activations (ACT 0 sigmoid, 1 sqrt(softplus) with softplus's threshold 20; routing.cu:18-36).
// Selection key: with a bias act(logit) + bias, else the fp16 logit (use_topk) or act(logit)
// (sorting variant).  Order: larger key first using the monotone unsigned encoding of the fp32 key
// (so +0 ranks above -0), ties to the lower expert index.  Weights: act(logit) of the selection,
// normalised as o * scale / (sum o + 1e-20) (use_topk) or o * (scale / (sum + 1e-20)), in fp16.
// The reference's sorting variant orders exactly equal activated keys by its radix network's lane
// order instead; only keys that tie in fp32 can differ.
HX_INLINE float sigmoid_stable(float x)
{
    float ez = __expf(-fabsf(x));
    float base = ez / (1.0f + ez);
    return x >= 0.0f ? 1.0f - base : base;
}

template <int ACT>
HX_INLINE float route_act(float x)
{
    if constexpr (ACT == 1) return sqrtf(x > 20.0f ? x : log1pf(__expf(x)));
    else return sigmoid_stable(x);
}

template <int ACT, bool SORT>
__global__ __launch_bounds__(64) void routing_topk_kernel(const _Float16* scores, const _Float16* bias, int64_t* idx,
                                                          _Float16* w, int E, int K, float scale)
{
    const int lane = threadIdx.x;
    const int row = blockIdx.x;
    scores += (size_t)row * E;
    constexpr int PER = 8;  // E <= 512
    uint64_t cand[PER];
    float act[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = lane + 64 * i;
        cand[i] = 0;
        act[i] = 0.0f;
        if (e < E) {
            const float logit = (float)scores[e];
            act[i] = route_act<ACT>(logit);
            const float key = bias ? act[i] + (float)bias[e] : (SORT ? act[i] : logit);
            uint32_t u = __float_as_uint(key);
            u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
            // larger is better: key high, lower index wins ties; +1 keeps valid candidates nonzero
            cand[i] = ((uint64_t)u << 32) | (uint64_t)(0xfffffu - (uint32_t)e + 1u);
        }
    }
    float o_sel = 0.0f;
    int e_sel = 0;
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) {
        uint64_t b = 0;
        float ba = 0.0f;
#pragma unroll
        for (int i = 0; i < PER; ++i)
            if (cand[i] > b) { b = cand[i]; ba = act[i]; }
        // the wave's largest 64-bit key in two 32-bit DPP reductions (the key word, then the index
        // word among the lanes holding that key word); its activation from the owning lane (K <= E
        // valid candidates, so the key is nonzero and has one owner)
        const uint32_t hi = hx_wave_max_u32((uint32_t)(b >> 32));
        const uint32_t lo = hx_wave_max_u32((uint32_t)(b >> 32) == hi ? (uint32_t)b : 0u);
        const uint64_t best = ((uint64_t)hi << 32) | lo;
        const uint64_t owner = __ballot(b == best);
        const float best_a = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ba), (int)__ffsll((unsigned long long)owner) - 1));
        const int e = (int)(0xfffffu + 1u - lo);
#pragma unroll
        for (int i = 0; i < PER; ++i)
            if (cand[i] == best) cand[i] = 0;
        sum += best_a;
        if (lane == k) { o_sel = best_a; e_sel = e; }
    }
    sum += 1e-20f;
    if (lane < K) {
        idx[(size_t)row * K + lane] = e_sel;
        w[(size_t)row * K + lane] = (_Float16)(SORT ? o_sel * (scale / sum) : o_sel * scale / sum);
    }
}

hipError_t launch_routing(const _Float16* scores, const _Float16* bias, int64_t* idx, _Float16* w, int bsz, int E,
                          int K, float scale, hipStream_t st, bool use_topk, int act_fn)
{
    if (E > 512 || K > 64 || K > E || K < 1 || act_fn < 0 || act_fn > 1) return hipErrorInvalidValue;
    if (bsz == 0) return hipSuccess;
    auto kernel = act_fn == 1 ? (use_topk ? routing_topk_kernel<1, false> : routing_topk_kernel<1, true>)
                              : (use_topk ? routing_topk_kernel<0, false> : routing_topk_kernel<0, true>);
    hipLaunchKernelGGL(kernel, dim3(bsz), dim3(64), 0, st, scores, bias, idx, w, E, K, scale);
    return hipGetLastError();
}

// ------------------------------------------------------------------ permutation

// Deterministic counting sort of routing slots by expert (reference glue2.cu:244-293 computes the
// same expert_count / token_sorted / weight_sorted / route_to_sorted, but places slots within an
// expert with an atomic cursor).  Here slot i of expert e lands at offset[e] + (number of slots
// i' < i with ids[i'] == e): ascending flat index within each expert.  One 1024-lane workgroup per
// chunk of 1024 slots (permute_kernel: one workgroup for all chunks, in order).
constexpr int PERM_THREADS = 1024;
constexpr int PERM_EMAX = 512;

// Scatter of the routes [base, base + PERM_THREADS) given each expert's next free position in
// cursor[] (LDS, advanced past the chunk on return): each wave ranks its lanes by ballot and counts
// its routes per expert; a wave's group of an expert starts after the groups of the waves before it,
// so positions ascend with the flat index within each expert.
__device__ __forceinline__ void permute_scatter_chunk(const int64_t* ids, const _Float16* w, int total, int topk, int E,
                                                      int base, int* cursor, int64_t* token_sorted,
                                                      _Float16* weight_sorted, int64_t* route_to_sorted)
{
    constexpr int NW = PERM_THREADS / 64;
    __shared__ int wfirst[NW * PERM_EMAX];  // [wave][expert]: the wave's group size, then its first position
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int i = base + t;
    const int64_t e64 = i < total ? ids[i] : -1;
    const bool valid = e64 >= 0 && e64 < E;
    const int e = valid ? (int)e64 : -1;
    for (int k = t; k < NW * E; k += PERM_THREADS) wfirst[(k / E) * PERM_EMAX + k % E] = 0;
    int rank = 0, group = 0;
    bool leader = false;
    uint64_t remaining = __ballot(valid);
    while (remaining) {
        const int ld = __ffsll((unsigned long long)remaining) - 1;
        const int le = __shfl(e, ld, 64);
        const uint64_t m = __ballot(valid && e == le);
        if (valid && e == le) {
            rank = __popcll(m & lt_mask);
            group = __popcll(m);
            leader = (lane == ld);
        }
        remaining &= ~m;
    }
    __syncthreads();
    if (leader) wfirst[wave * PERM_EMAX + e] = group;
    __syncthreads();
    for (int x = t; x < E; x += PERM_THREADS) {
        int run = cursor[x];
#pragma unroll
        for (int wv = 0; wv < NW; ++wv) {
            const int g = wfirst[wv * PERM_EMAX + x];
            wfirst[wv * PERM_EMAX + x] = run;
            run += g;
        }
        cursor[x] = run;
    }
    __syncthreads();
    if (valid) {
        const int pos = wfirst[wave * PERM_EMAX + e] + rank;
        token_sorted[pos] = i / topk;
        weight_sorted[pos] = w[i];
        if (route_to_sorted) route_to_sorted[i] = pos;
    }
    __syncthreads();  // wfirst and cursor are read before a next chunk rewrites them
}

__global__ __launch_bounds__(PERM_THREADS) void permute_kernel(const int64_t* ids, const _Float16* w, int total,
                                                               int topk, int E, int64_t* expert_count,
                                                               int64_t* token_sorted, _Float16* weight_sorted,
                                                               int64_t* route_to_sorted)
{
    __shared__ int cnt[PERM_EMAX];
    __shared__ int cursor[PERM_EMAX];
    const int t = threadIdx.x;
    for (int e = t; e < PERM_EMAX; e += PERM_THREADS) cnt[e] = 0;
    __syncthreads();
    for (int i = t; i < total; i += PERM_THREADS) {
        const int64_t e = ids[i];
        if (e >= 0 && e < E) atomicAdd(&cnt[(int)e], 1);
    }
    __syncthreads();
    if (t == 0) {
        int acc = 0;
        for (int e = 0; e < E; ++e) {
            cursor[e] = acc;
            acc += cnt[e];
        }
    }
    __syncthreads();
    for (int e = t; e <= E; e += PERM_THREADS) expert_count[e] = e < E ? cnt[e] : 0;
    for (int base = 0; base < total; base += PERM_THREADS)
        permute_scatter_chunk(ids, w, total, topk, E, base, cursor, token_sorted, weight_sorted, route_to_sorted);
}

// Many routes: per-chunk histograms, then (last chunk to arrive) each chunk's starting position
// per expert, then an independent scatter per chunk.  Same positions as permute_kernel.
__global__ __launch_bounds__(PERM_THREADS) void permute_count_kernel(const int64_t* ids, int total, int E,
                                                                     int* counts, int* offs, int* arrive,
                                                                     int64_t* expert_count)
{
    __shared__ int hist[PERM_EMAX];
    __shared__ bool last;
    const int t = threadIdx.x, chunks = gridDim.x;
    for (int e = t; e < PERM_EMAX; e += PERM_THREADS) hist[e] = 0;
    __syncthreads();
    const int i = blockIdx.x * PERM_THREADS + t;
    if (i < total) {
        const int64_t e = ids[i];
        if (e >= 0 && e < E) atomicAdd(&hist[(int)e], 1);
    }
    __syncthreads();
    for (int e = t; e < E; e += PERM_THREADS)
        __hip_atomic_store(&counts[blockIdx.x * E + e], hist[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0) {
        last = __hip_atomic_fetch_add(arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == chunks - 1;
        if (last) __hip_atomic_store(arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    // one expert per thread (E <= PERM_EMAX <= PERM_THREADS); the chunk counts are read PB at a time,
    // all PB loads in flight together (one round trip per PB chunks instead of one per chunk)
    constexpr int PB = 16;
    static_assert(PERM_EMAX <= PERM_THREADS, "one expert per thread");
    auto load_counts = [&](int c0, int (&v)[PB]) {
#pragma unroll
        for (int j = 0; j < PB; ++j)
            v[j] = c0 + j < chunks ? __hip_atomic_load(&counts[(c0 + j) * E + t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                   : 0;
    };
    int n_e = 0;  // routes of expert t over all chunks
    if (t < E)
        for (int c0 = 0; c0 < chunks; c0 += PB) {
            int v[PB];
            load_counts(c0, v);
#pragma unroll
            for (int j = 0; j < PB; ++j) n_e += v[j];
        }
    // exclusive scan over the experts: inclusive scan per wave, then the totals of the waves below
    __shared__ int wave_sum[PERM_THREADS / 64];
    const int lane = t & 63, wave = t >> 6;
    int inc = n_e;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(inc, o, 64);
        if (lane >= o) inc += u;
    }
    if (lane == 63) wave_sum[wave] = inc;
    __syncthreads();
    int first = inc - n_e;
    for (int k = 0; k < wave; ++k) first += wave_sum[k];
    if (t <= E) expert_count[t] = t < E ? n_e : 0;
    // each chunk's first position per expert: the expert's first position plus the routes of the
    // chunks before (the counts again, now cached)
    if (t < E)
        for (int c0 = 0; c0 < chunks; c0 += PB) {
            int v[PB];
            load_counts(c0, v);
#pragma unroll
            for (int j = 0; j < PB; ++j)
                if (c0 + j < chunks) {
                    offs[(c0 + j) * E + t] = first;
                    first += v[j];
                }
        }
}

__global__ __launch_bounds__(PERM_THREADS) void permute_scatter_kernel(const int64_t* ids, const _Float16* w, int total,
                                                                       int topk, int E, const int* offs,
                                                                       int64_t* token_sorted, _Float16* weight_sorted,
                                                                       int64_t* route_to_sorted)
{
    __shared__ int cursor[PERM_EMAX];
    for (int e = threadIdx.x; e < E; e += PERM_THREADS) cursor[e] = offs[blockIdx.x * E + e];
    __syncthreads();
    permute_scatter_chunk(ids, w, total, topk, E, blockIdx.x * PERM_THREADS, cursor, token_sorted, weight_sorted,
                          route_to_sorted);
}

hipError_t launch_permute_chunked(const int64_t* ids, const _Float16* w, int M, int topk, int E, int64_t* expert_count,
                                  int64_t* token_sorted, _Float16* weight_sorted, int64_t* route_to_sorted,
                                  int* scratch, int* arrive, hipStream_t st)
{
    if (E > PERM_EMAX || E < 1) return hipErrorInvalidValue;
    const int total = M * topk;
    const int chunks = (total + PERM_THREADS - 1) / PERM_THREADS;
    if (chunks == 0) return hipSuccess;
    int* counts = scratch;
    int* offs = scratch + (size_t)chunks * E;
    hipLaunchKernelGGL(permute_count_kernel, dim3(chunks), dim3(PERM_THREADS), 0, st, ids, total, E, counts, offs, arrive,
                       expert_count);
    hipLaunchKernelGGL(permute_scatter_kernel, dim3(chunks), dim3(PERM_THREADS), 0, st, ids, w, total, topk, E, offs,
                       token_sorted, weight_sorted, route_to_sorted);
    return hipGetLastError();
}

hipError_t launch_permute(const int64_t* ids, const _Float16* w, int M, int topk, int E, int64_t* expert_count,
                          int64_t* token_sorted, _Float16* weight_sorted, int64_t* route_to_sorted,
                          int64_t* workspace, hipStream_t st)
{
    (void)workspace;
    if (E > PERM_EMAX || E < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(PERM_THREADS), 0, st, ids, w, M * topk, topk, E, expert_count,
                       token_sorted, weight_sorted, route_to_sorted);
    return hipGetLastError();
}

// ------------------------------------------------------------------ ordered reduction / swiglu

// y[t][c] = sum_j contrib[route_to_sorted[t*topk + j]][c], ascending j, from +0 (glue2.cu:297-306).
__global__ __launch_bounds__(256) void reduce_sorted_kernel(float* y, const float* contrib, const int64_t* r2s, int M,
                                                            int topk, int hidden)
{
    const size_t i4 = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t total4 = (size_t)M * hidden / 4;
    if (i4 >= total4) return;
    const int t = (int)(i4 * 4 / hidden);
    const int c = (int)(i4 * 4 % hidden);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j = 0; j < topk; ++j) {
        const float4 v = *reinterpret_cast<const float4*>(contrib + (size_t)r2s[(size_t)t * topk + j] * hidden + c);
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
    }
    *reinterpret_cast<float4*>(y + i4 * 4) = acc;
}

hipError_t launch_reduce_sorted(float* y, const float* contrib, const int64_t* route_to_sorted, int M, int topk,
                                int hidden, hipStream_t st)
{
    if (hidden % 4) return hipErrorInvalidValue;
    size_t total4 = (size_t)M * hidden / 4;
    if (total4 == 0) return hipSuccess;
    hipLaunchKernelGGL(reduce_sorted_kernel, dim3((unsigned)((total4 + 255) / 256)), dim3(256), 0, st, y, contrib,
                       route_to_sorted, M, topk, hidden);
    return hipGetLastError();
}

// out = fp16(silu(min(g, L)) * clamp(u, -L, L))  (glue2.cu:406-414)
__global__ __launch_bounds__(256) void swiglu_clamp_kernel(const float* g, const float* u, _Float16* out, size_t n,
                                                           float limit)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float gv = fminf(g[i], limit);
    const float uv = fminf(fmaxf(u[i], -limit), limit);
    out[i] = (_Float16)(gv / (1.0f + __expf(-gv)) * uv);
}

hipError_t launch_swiglu_clamp(const float* g, const float* u, _Float16* out, size_t n, float limit, hipStream_t st)
{
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_clamp_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u, out, n, limit);
    return hipGetLastError();
}

// ------------------------------------------------------------------ dense-MoE row glue

// dst[r][:] = src[idx[r]][:] (fp16 rows of h).  Reference glue::gather_rows (src/engine/glue.cu:48-60).
// 16-byte accesses when h % 8 == 0, else one element per thread.
__global__ __launch_bounds__(256) void gather_rows_kernel(const _Float16* src, const int64_t* idx, _Float16* dst,
                                                          long n, int h)
{
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if ((h & 7) == 0) {
        const int hv = h >> 3;
        if (i >= n * hv) return;
        const long r = i / hv, d = i % hv;
        reinterpret_cast<hx_u4*>(dst)[r * hv + d] = reinterpret_cast<const hx_u4*>(src)[idx[r] * hv + d];
    } else {
        if (i >= n * h) return;
        const long r = i / h, d = i % h;
        dst[i] = src[idx[r] * h + d];
    }
}

// a * b rounded to fp32 on its own: the empty asm keeps the compiler from fusing it into the add
// that follows (a fused multiply-add, v_fma_mix_f32 with the fp16 weight, rounds once)
HX_INLINE float rounded_product(float a, float b)
{
    float p = a * b;
    asm volatile("" : "+v"(p));
    return p;
}

// y[idx[r]][:] += fp32(w[r]) * src[r][:], the product and the sum each rounded once (fp32), one
// writer per element: idx holds distinct rows within a call (reference glue::scatter_add_rows,
// src/engine/glue.cu:62-82).  4 elements per thread when h % 4 == 0.
__global__ __launch_bounds__(256) void scatter_add_rows_kernel(float* y, const float* src, const int64_t* idx,
                                                               const _Float16* w, long n, int h)
{
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if ((h & 3) == 0) {
        const int hv = h >> 2;
        if (i >= n * hv) return;
        const long r = i / hv, d = i % hv;
        const float wv = (float)w[r];
        hx_f4* dst = reinterpret_cast<hx_f4*>(y) + idx[r] * hv + d;
        const hx_f4 s4 = reinterpret_cast<const hx_f4*>(src)[i];
        hx_f4 v = *dst;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = v[j] + rounded_product(wv, s4[j]);
        *dst = v;
    } else {
        if (i >= n * h) return;
        const long r = i / h, d = i % h;
        float* dst = y + idx[r] * h + d;
        *dst = *dst + rounded_product((float)w[r], src[i]);
    }
}

hipError_t launch_gather_rows(const _Float16* src, const int64_t* idx, _Float16* dst, int n, int h, hipStream_t st)
{
    if (n == 0 || h == 0) return hipSuccess;
    const long work = (long)n * ((h & 7) == 0 ? h / 8 : h);
    hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, st, src, idx, dst,
                       (long)n, h);
    return hipGetLastError();
}

hipError_t launch_scatter_add_rows(float* y, const float* src, const int64_t* idx, const _Float16* w, int n, int h,
                                   hipStream_t st)
{
    if (n == 0 || h == 0) return hipSuccess;
    const long work = (long)n * ((h & 3) == 0 ? h / 4 : h);
    hipLaunchKernelGGL(scatter_add_rows_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, st, y, src, idx,
                       w, (long)n, h);
    return hipGetLastError();
}

// ------------------------------------------------------------------ sign packing, inf / NaN count

// packed[c] bit i = sign bit of fp16 unpacked[16 c + i] (reference pack_signs_kernel,
// src/cuda/quant/pack.cu:180-204: each value is shifted in at bit 15, then right, so value i ends in
// bit i).  One lane per column: its 16 values are 32 contiguous bytes, two 16-byte loads when the
// buffer is 16-byte aligned.
template <bool VEC>
__global__ __launch_bounds__(256) void pack_signs_kernel(uint16_t* packed, const uint16_t* unpacked, int cols)
{
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= cols) return;
    uint32_t w[8];
    if constexpr (VEC) {
        const uint4* src = reinterpret_cast<const uint4*>(unpacked + (size_t)16 * c);
        const uint4 a = src[0], b = src[1];
        w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w, w[4] = b.x, w[5] = b.y, w[6] = b.z, w[7] = b.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            w[j] = (uint32_t)unpacked[(size_t)16 * c + 2 * j] | ((uint32_t)unpacked[(size_t)16 * c + 2 * j + 1] << 16);
    }
    uint32_t out = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) out |= ((w[j] >> 15) & 1u) << (2 * j) | (w[j] >> 31) << (2 * j + 1);
    packed[c] = (uint16_t)out;
}

hipError_t launch_pack_signs(uint16_t* packed, const uint16_t* unpacked, int cols, hipStream_t st)
{
    const dim3 grid((unsigned)((cols + 255) / 256));
    if (reinterpret_cast<uintptr_t>(unpacked) % 16 == 0)
        hipLaunchKernelGGL(pack_signs_kernel<true>, grid, dim3(256), 0, st, packed, unpacked, cols);
    else
        hipLaunchKernelGGL(pack_signs_kernel<false>, grid, dim3(256), 0, st, packed, unpacked, cols);
    return hipGetLastError();
}

// counts[0] += infinities, counts[1] += NaNs among numel fp16 (T = uint16_t) or fp32 (uint32_t) values
// (reference count_inf_nan_kernel, src/cuda/quant/util.cu:54-80).  An infinity has every exponent
// bit and no mantissa bit, a NaN every exponent bit and some mantissa bit.  Grid-stride over 16-byte
// chunks (element by element when the buffer is not 16-byte aligned), a wave then workgroup sum, one
// atomic add per counter per workgroup.
template <class T, bool VEC>
__global__ __launch_bounds__(256) void count_inf_nan_kernel(const T* x, unsigned long long* counts, uint64_t numel)
{
    constexpr uint32_t EXP = sizeof(T) == 2 ? 0x7c00u : 0x7f800000u, ABS = sizeof(T) == 2 ? 0x7fffu : 0x7fffffffu;
    uint32_t n_inf = 0, n_nan = 0;
    auto classify = [&](uint32_t v) {
        v &= ABS;
        n_inf += v == EXP;
        n_nan += v > EXP;
    };
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    uint64_t done = 0;
    if constexpr (VEC) {
        constexpr int PER = 16 / sizeof(T);  // values per 16-byte chunk
        const uint64_t chunks = numel / PER;
        const uint4* src = reinterpret_cast<const uint4*>(x);
        for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < chunks; i += stride) {
            const uint4 v = src[i];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (sizeof(T) == 2) {
                    classify(w[j] & 0xffffu);
                    classify(w[j] >> 16);
                } else {
                    classify(w[j]);
                }
            }
        }
        done = chunks * PER;
    }
    for (uint64_t i = done + (uint64_t)blockIdx.x * 256 + threadIdx.x; i < numel; i += stride) classify(x[i]);
    // per-thread counts stay below 2^32: numel / stride < 2^32 for every launch (grid below)
    unsigned long long a = n_inf, b = n_nan;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        a += __shfl_xor(a, o, 64);
        b += __shfl_xor(b, o, 64);
    }
    __shared__ unsigned long long part[2][4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        part[0][wave] = a;
        part[1][wave] = b;
    }
    __syncthreads();
    if (threadIdx.x < 2) {
        const unsigned long long t = part[threadIdx.x][0] + part[threadIdx.x][1] + part[threadIdx.x][2] + part[threadIdx.x][3];
        if (t) __hip_atomic_fetch_add(&counts[threadIdx.x], t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

hipError_t launch_count_inf_nan(const void* x, unsigned long long* counts, uint64_t numel, bool fp32, hipStream_t st)
{
    // enough workgroups to fill the GPU a few times over, each thread covering numel / (grid * 256)
    // values (below 2^32 for any numel below 2^51)
    const uint64_t per = 16 / (fp32 ? 4 : 2), want = (numel / per + 255) / 256;
    const unsigned grid = (unsigned)(want < 1 ? 1 : want > 4096 ? 4096 : want);
    const bool vec = reinterpret_cast<uintptr_t>(x) % 16 == 0;
    if (fp32) {
        if (vec) hipLaunchKernelGGL((count_inf_nan_kernel<uint32_t, true>), dim3(grid), dim3(256), 0, st, (const uint32_t*)x, counts, numel);
        else hipLaunchKernelGGL((count_inf_nan_kernel<uint32_t, false>), dim3(grid), dim3(256), 0, st, (const uint32_t*)x, counts, numel);
    } else {
        if (vec) hipLaunchKernelGGL((count_inf_nan_kernel<uint16_t, true>), dim3(grid), dim3(256), 0, st, (const uint16_t*)x, counts, numel);
        else hipLaunchKernelGGL((count_inf_nan_kernel<uint16_t, false>), dim3(grid), dim3(256), 0, st, (const uint16_t*)x, counts, numel);
    }
    return hipGetLastError();
}

}  // namespace hx
