// hx_device.hpp -- gfx950 device primitives for the EXL3 trellis path.
//
// Trellis format (reference src/cuda/quant/exl3_gemm.cuh:17-29, pack.cu:6-54):
//   a K x N weight is (K/16) x (N/16) tiles of 16x16; tile (tk, tn) is 8*bits little-endian
//   uint32 words at word offset (tk * (N/16) + tn) * 8 * bits.  Stream bit b of a tile is bit
//   31 - (b % 32) of word b / 32.  Position p (0..255) decodes the 16-bit window made of stream
//   bits [(p+1)*bits - 16, (p+1)*bits) (cyclic), read MSB first (exl3_dq.cuh:17-32).
//   Position p holds weight (k, n) of the tile with l = p/8, j = p%8:
//     k = 2*(l%4) + (j&1) + 8*((j>>1)&1),  n = 8*(j>>2) + l/4        (reconstruct.cu:36-81)
//   so positions p (even) and p+1 are the k-adjacent pair (k, k+1) of one column n.
//
// Everything here is written for 64-lane wavefronts.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 hx_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 hx_h4 __attribute__((ext_vector_type(4)));
typedef _Float16 hx_h8 __attribute__((ext_vector_type(8)));
typedef float hx_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t hx_u4 __attribute__((ext_vector_type(4)));
typedef float hx_f16v __attribute__((ext_vector_type(16)));

#define HX_INLINE __device__ __forceinline__
#define HX_INLINE_HD __host__ __device__ __forceinline__

#define HX_SETPRIO(p) __builtin_amdgcn_s_setprio(p)

static constexpr float HX_RSQRT128 = 0.088388347648f;

// Workgroup size in threads / waves (kernels here run 256 or 1024 threads).
HX_INLINE int hx_nthreads() { return (int)blockDim.x; }
HX_INLINE int hx_nwaves() { return (int)blockDim.x >> 6; }

// Rotated wave / thread index of a 4-wave (256-thread) workgroup: wave (blockIdx.x & 3) acts as wave
// 0.  The waves of a workgroup sit on the CU's four SIMDs in order, so serial per-workgroup work
// (routing, bookkeeping, one-row epilogues) given to wave 0 of every co-resident workgroup would
// all land on one SIMD and run there one workgroup after the other.
HX_INLINE int hx_vwave() { return (int)(((threadIdx.x >> 6) - blockIdx.x) & 3u); }
HX_INLINE int hx_vtid() { return (int)((threadIdx.x + 256u - 64u * (blockIdx.x & 3u)) & 255u); }

HX_INLINE hx_h2 u32_as_h2(uint32_t u) { return __builtin_bit_cast(hx_h2, u); }
HX_INLINE uint32_t h2_as_u32(hx_h2 h) { return __builtin_bit_cast(uint32_t, h); }
HX_INLINE _Float16 u16_as_h(uint16_t u) { return __builtin_bit_cast(_Float16, u); }
HX_INLINE uint16_t h_as_u16(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }

// ------------------------------------------------------------------ window extraction

// Window of position P from the tile's words held in registers.  P is a compile-time constant in
// every caller (fully unrolled loops), so each window folds to one v_alignbit_b32 or v_bfe_u32.
template <int BITS, int P>
HX_INLINE uint32_t hx_window(const uint32_t* w)
{
    constexpr int total = 256 * BITS;
    constexpr int nw = 8 * BITS;
    constexpr int s = (((P + 1) * BITS - 16) % total + total) % total;  // first stream bit
    constexpr int wi = s >> 5;
    constexpr int off = s & 31;
    if constexpr (off <= 16) {
        return (w[wi] >> (16 - off)) & 0xffffu;
    } else {
        // bits from the low (32-off) bits of w[wi] followed by the top bits of w[wi+1]
        return __builtin_amdgcn_alignbit(w[wi], w[(wi + 1) % nw], 48 - off) & 0xffffu;
    }
}

// ------------------------------------------------------------------ codebooks

// Two decoded weights (windows w0 -> low half, w1 -> high half) as fp16x2.
// codebook.cuh:57-124.  cb2: x = w * 0x83DCD12D; h = fp16(0x6400 + bytesum(x)) = 1024 + s exactly;
// v = fma(h, 0x1eee, 0xc931) in fp16 (v_pk_fma_f16 is one rounding of the exact value, as hfma).
// cb0/cb1: x = w*a (+b); x = (x & 0x8fff8fff) ^ 0x3b603b60; v = lo16 + hi16 in fp16.
template <int CB>
HX_INLINE hx_h2 hx_decode2(uint32_t w0, uint32_t w1)
{
    if constexpr (CB == 2) {
        uint32_t x0 = w0 * 0x83DCD12Du;
        uint32_t x1 = w1 * 0x83DCD12Du;
        uint32_t s0 = __builtin_amdgcn_udot4(x0, 0x01010101u, 0x6400u, false);
        uint32_t s1 = __builtin_amdgcn_udot4(x1, 0x01010101u, 0x6400u, false);
        hx_h2 h = u32_as_h2((s1 << 16) | s0);
        const hx_h2 c1 = u32_as_h2(0x1eee1eeeu);
        const hx_h2 c0 = u32_as_h2(0xc931c931u);
        return __builtin_elementwise_fma(h, c1, c0);
    } else {
        uint32_t x0, x1;
        if constexpr (CB == 1) {
            x0 = w0 * 0xCBAC1FEDu;
            x1 = w1 * 0xCBAC1FEDu;
        } else {
            x0 = w0 * 89226354u + 64248484u;
            x1 = w1 * 89226354u + 64248484u;
        }
        x0 = (x0 & 0x8fff8fffu) ^ 0x3b603b60u;
        x1 = (x1 & 0x8fff8fffu) ^ 0x3b603b60u;
        uint32_t lo = __builtin_amdgcn_perm(x1, x0, 0x05040100u);  // (x0.lo, x1.lo)
        uint32_t hi = __builtin_amdgcn_perm(x1, x0, 0x07060302u);  // (x0.hi, x1.hi)
        return u32_as_h2(lo) + u32_as_h2(hi);
    }
}

// ------------------------------------------------------------------ codebook 2, register level

// The 32 stream bits ending at (cyclic) stream bit E of a tile, MSB first: bit 0 is stream bit E-1.
// Its low half is the window ending at E, its high half the window ending at E - 16.
template <int BITS, int E>
HX_INLINE uint32_t hx_reg_end(const uint32_t* w)
{
    constexpr int total = 256 * BITS, nw = 8 * BITS;
    constexpr int e = ((E % total) + total) % total;
    constexpr int j = e >> 5, r = e & 31;
    if constexpr (r == 0) return w[(j - 1 + nw) % nw];
    else return __builtin_amdgcn_alignbit(w[(j - 1 + nw) % nw], w[j % nw], 32 - r);
}

// x = window * 0x83DCD12D mod 2^32 for the 16-bit window in the low (HI = false) or high half of
// r, whatever the other half holds: x = w*0xD12D + ((w*0x83DC mod 2^16) << 16), i.e. one
// v_pk_mul_lo_u16 producing (w*0x83DC) << 16 and one v_mad_u32_u16 (both full rate, where
// v_mul_lo_u32 is a quarter-rate op and would also need the window masked first).
template <bool HI>
HX_INLINE uint32_t hx_mul1_x(uint32_t r)
{
    uint32_t t, x;
    if constexpr (!HI) {
        asm("v_pk_mul_lo_u16 %0, %1, %2 op_sel_hi:[0,1]" : "=v"(t) : "v"(r), "s"(0x83dc0000u));
        asm("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(x) : "v"(r), "s"(0xd12du), "v"(t));
    } else {
        asm("v_pk_mul_lo_u16 %0, %1, %2 op_sel:[1,0] op_sel_hi:[1,1]" : "=v"(t) : "v"(r), "s"(0x83dc0000u));
        asm("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[1,0,0,0]" : "=v"(x) : "v"(r), "s"(0xd12du), "v"(t));
    }
    return x;
}

// x of position P.  When BITS divides 16, positions D = 16/BITS apart share one register (low and
// high half), so a tile needs one alignbit per two positions.
template <int BITS, int P>
HX_INLINE uint32_t hx_mul1_pos(const uint32_t* w)
{
    constexpr int D = (16 % BITS == 0) ? 16 / BITS : 0;
    if constexpr (D != 0 && (P % (2 * D)) < D) return hx_mul1_x<true>(hx_reg_end<BITS, (P + D + 1) * BITS>(w));
    else return hx_mul1_x<false>(hx_reg_end<BITS, (P + 1) * BITS>(w));
}

// Decoded fp16 pair (positions P, P+1) of codebook 2: h = fp16(0x6400 + bytesum(x)) = 1024 + s
// exactly, v = fma(h, 0x1eee, 0xc931) rounded once (codebook.cuh:77-90).
template <int BITS, int P>
HX_INLINE hx_h2 hx_mul1_pair(const uint32_t* w)
{
    const uint32_t s0 = __builtin_amdgcn_udot4(hx_mul1_pos<BITS, P>(w), 0x01010101u, 0x6400u, false);
    const uint32_t s1 = __builtin_amdgcn_udot4(hx_mul1_pos<BITS, P + 1>(w), 0x01010101u, 0x6400u, false);
    const hx_h2 h = u32_as_h2((s1 << 16) | s0);
    return __builtin_elementwise_fma(h, u32_as_h2(0x1eee1eeeu), u32_as_h2(0xc931c931u));
}

template <int CB>
HX_INLINE _Float16 hx_decode1(uint32_t w)
{
    hx_h2 v = hx_decode2<CB>(w, w);
    return v.x;
}

// Position pair (P, P+1), P even -> column n and k-pair index kp (the pair covers k = 2*kp, 2*kp+1).
template <int P> struct hx_pos {
    static constexpr int l = P >> 3, j = P & 7;
    static constexpr int k = 2 * (l & 3) + (j & 1) + 8 * ((j >> 1) & 1);
    static constexpr int n = 8 * (j >> 2) + (l >> 2);
    static constexpr int kp = k >> 1;
};

// Inverse map (k, n) -> position.
HX_INLINE int hx_kn_to_pos(int k, int n)
{
    int l = 4 * (n & 7) + ((k >> 1) & 3);
    int j = (k & 1) + 2 * (k >> 3) + 4 * (n >> 3);
    return 8 * l + j;
}

// Window p (16 stream bits ending at stream bit (p+1)*bits, cyclic over the tile) of a tile held as
// 8*bits uint32 words, with a run-time bit width (reconstruct paths).
HX_INLINE uint32_t window_rt(const uint32_t* w, int bits, int p)
{
    const int total = 256 * bits, nw = 8 * bits;
    int s = (p + 1) * bits - 16;
    if (s < 0) s += total;
    const int wi = s >> 5, off = s & 31;
    if (off <= 16) return (w[wi] >> (16 - off)) & 0xffffu;
    int wj = wi + 1;
    if (wj == nw) wj = 0;
    return __builtin_amdgcn_alignbit(w[wi], w[wj], 48 - off) & 0xffffu;
}

// ------------------------------------------------------------------ wave-level Hadamard-128

// 128-point Sylvester transform of one vector held as 2 values per lane (elements 2*lane,
// 2*lane+1) across a 64-lane wave; scaled by 1/sqrt(128).
HX_INLINE void hx_had128_wave(float& v0, float& v1)
{
    const int lane = threadIdx.x & 63;
    float a = v0 + v1, b = v0 - v1;
    v0 = a;
    v1 = b;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        float p0 = __shfl_xor(v0, m, 64);
        float p1 = __shfl_xor(v1, m, 64);
        bool upper = (lane & m) != 0;
        v0 = upper ? p0 - v0 : v0 + p0;
        v1 = upper ? p1 - v1 : v1 + p1;
    }
    v0 *= HX_RSQRT128;
    v1 *= HX_RSQRT128;
}

// 128-point Sylvester transform held as 8 consecutive values per lane in groups of 16 lanes
// (element 8 * (lane % 16) + j), four vectors per wave: H128 = H16 (across the 16 lanes) x H8 (in the
// lane), both natural-order butterflies; scaled by 1/sqrt(128).
HX_INLINE void hx_had128_x8(float (&v)[8])
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (!(j & h)) {
                const float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
        const bool upper = (lane & m) != 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float p = __shfl_xor(v[j], m, 64);
            v[j] = upper ? p - v[j] : v[j] + p;
        }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] *= HX_RSQRT128;
}

// Workgroup barrier that waits only for this wave's LDS traffic (s_waitcnt lgkmcnt(0)), so global
// loads issued before it stay in flight across the barrier.  The waitcnt immediate encodes
// vmcnt = 63, expcnt = 7, lgkmcnt = 0 (gfx9 field layout).
HX_INLINE void hx_lds_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Maximum of a u32 over the 64 lanes of a wave with DPP row shifts and row broadcasts (each step a
// VALU op with a lane-permuted operand, no LDS round trip); every lane gets the result.
HX_INLINE uint32_t hx_wave_max_u32(uint32_t v)
{
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false));  // row_shr:1
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false));  // row_shr:2
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false));  // row_shr:4
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false));  // row_shr:8
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false));  // row_bcast:15
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false));  // row_bcast:31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// ------------------------------------------------------------------ cross-agent handoff

HX_INLINE int hx_atomic_add_acqrel(int* p, int v)
{
    return __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
HX_INLINE void hx_atomic_store_relaxed(int* p, int v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// fp32 SiLU in the fp16 chain order of hadamard_inner.cuh:331-340 (exp, 1+e, rcp, mul), each
// step rounded to fp16 as the reference's half2 ops are.
HX_INLINE _Float16 hx_silu_h(_Float16 g)
{
    _Float16 e = (_Float16)__expf(-(float)g);
    _Float16 s = (_Float16)(1.0f + (float)e);
    _Float16 r = (_Float16)(1.0f / (float)s);
    return (_Float16)((float)g * (float)r);
}

// Tanh-form GELU of an fp16 value in fp32, rounded to fp16 (hadamard_inner.cuh:342-349):
// 0.5 x (1 + tanh(y)), y = sqrt(2/pi) (x + 0.044715 x^3), written as x / (1 + exp(-2y)) -- the same
// function without the cancellation of 1 + tanh(y) at large negative y.
HX_INLINE _Float16 hx_gelu_h(_Float16 g)
{
    const float x = (float)g;
    const float y = 0.797884560803f * (x + 0.044715f * x * x * x);
    return (_Float16)(x / (1.0f + __expf(-2.0f * y)));
}

// Routed-expert activations of the MoE kernels (exl3_moe_common.cuh:6-8).
enum : int { HX_ACT_SILU = 0, HX_ACT_GELU = 1, HX_ACT_RELU2_NOGATE = 2 };

// The gate lane after activation: SiLU / GELU of the transformed gate, or relu(u) for the
// non-gated relu2 (hadamard_inner.cuh:365-385); the clamps follow.
HX_INLINE _Float16 hx_gate_act(int act, _Float16 g, _Float16 u)
{
    if (act == HX_ACT_GELU) return hx_gelu_h(g);
    if (act == HX_ACT_RELU2_NOGATE) return u > (_Float16)0.0f ? u : (_Float16)0.0f;
    return hx_silu_h(g);
}
