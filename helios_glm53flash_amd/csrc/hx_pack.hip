// hx_pack.hip -- trellis bit packing and the original-basis reconstruction on gfx950.
//
//   pack / unpack   blocks of 256 K-bit symbols <-> 16*K uint16 trellis words (src/cuda/quant/pack.cu
//                   pack_trellis / unpack_trellis): symbol p occupies stream bits [p*K, (p+1)*K), most
//                   significant bit first; stream bit b is bit 31 - (b mod 32) of little-endian uint32
//                   word b / 32 of the block.  One wave per block: for packing, lane w composes output
//                   word w from the 32 stream bits it covers; for unpacking, a lane extracts 4 symbols.
//   reconstruct_had W = diag(suh) . H128 . W_hat . H128 . diag(svh) / 128 per 128 x 128 tile, fp16 out
//                   (src/cuda/quant/reconstruct.cu:150-374, reconstruct_had_slice): W_hat decoded
//                   bit-exact into LDS as fp32, column then row butterflies in fp32 on the wave, one
//                   rounding to fp16 at the end.
#include "hx_device.hpp"
#include "hx_kernels.hpp"

namespace hx {

__global__ __launch_bounds__(256) void pack_trellis_kernel(uint16_t* packed, const uint16_t* unpacked, long blocks,
                                                           int K)
{
    __shared__ uint16_t sym[4][256];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long b = (long)blockIdx.x * 4 + wave;
    if (b >= blocks) return;  // whole wave (uniform)
    const uint16_t mask = (uint16_t)((1u << K) - 1);
#pragma unroll
    for (int j = 0; j < 4; ++j) sym[wave][lane + 64 * j] = unpacked[b * 256 + lane + 64 * j] & mask;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    if (lane < 8 * K) {
        uint32_t acc = 0;
        for (int i = 0; i < 32; ++i) {
            const int s = 32 * lane + i;  // stream bit
            const int p = s / K, q = s - p * K;
            acc |= (uint32_t)((sym[wave][p] >> (K - 1 - q)) & 1u) << (31 - i);
        }
        reinterpret_cast<uint32_t*>(packed + b * 16 * K)[lane] = acc;
    }
}

__global__ __launch_bounds__(256) void unpack_trellis_kernel(uint16_t* unpacked, const uint16_t* packed, long blocks,
                                                             int K)
{
    __shared__ uint32_t words[4][64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long b = (long)blockIdx.x * 4 + wave;
    if (b >= blocks) return;
    if (lane < 8 * K) words[wave][lane] = reinterpret_cast<const uint32_t*>(packed + b * 16 * K)[lane];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int p = lane + 64 * j, s = p * K, w = s >> 5, o = s & 31;
        // the symbol's bits sit at stream offsets o .. o+K-1 of the 64-bit pair (word w, word w+1)
        const uint64_t pair = ((uint64_t)words[wave][w] << 32) | (w + 1 < 8 * K ? words[wave][w + 1] : 0u);
        unpacked[b * 256 + p] = (uint16_t)((pair >> (64 - o - K)) & ((1u << K) - 1));
    }
}

hipError_t launch_pack_trellis(uint16_t* packed, const uint16_t* unpacked, long blocks, int K, hipStream_t st)
{
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(pack_trellis_kernel, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, st, packed, unpacked,
                       blocks, K);
    return hipGetLastError();
}

hipError_t launch_unpack_trellis(uint16_t* unpacked, const uint16_t* packed, long blocks, int K, hipStream_t st)
{
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(unpack_trellis_kernel, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, st, unpacked, packed,
                       blocks, K);
    return hipGetLastError();
}

// One workgroup per 128 x 128 output tile (blockIdx.x: column group, blockIdx.y: row group).
template <int CB>
__global__ __launch_bounds__(256) void reconstruct_had_kernel(_Float16* out, const uint16_t* packed,
                                                              const _Float16* suh, const _Float16* svh,
                                                              int packed_cols, int packed_n_offset, int out_cols,
                                                              int bits)
{
    constexpr int LD = 129;  // padded fp32 row
    __shared__ float w[128 * LD];
    __shared__ uint32_t words[8][64];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int nw = 8 * bits;
    const int tn0 = packed_n_offset + blockIdx.x * 8;
    // W_hat: 8 tile rows of 8 tiles each, decoded exactly (fp16 values held in fp32)
    for (int tr = 0; tr < 8; ++tr) {
        const int tk = blockIdx.y * 8 + tr;
        const uint32_t* src = reinterpret_cast<const uint32_t*>(packed) + ((size_t)tk * packed_cols + tn0) * nw;
        __syncthreads();
        for (int i = t; i < 8 * nw; i += 256) words[i / nw][i % nw] = src[i];
        __syncthreads();
        const int k = t >> 4, c0 = (t & 15) * 8, tile = c0 >> 4, n0 = c0 & 15;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            w[(16 * tr + k) * LD + c0 + i] = (float)hx_decode1<CB>(window_rt(words[tile], bits, hx_kn_to_pos(k, n0 + i)));
    }
    __syncthreads();
    // columns: H over k (wave w takes columns 32w .. 32w+31)
    for (int c = 32 * wave; c < 32 * wave + 32; ++c) {
        float v0 = w[(2 * lane) * LD + c], v1 = w[(2 * lane + 1) * LD + c];
        hx_had128_wave(v0, v1);
        w[(2 * lane) * LD + c] = v0;
        w[(2 * lane + 1) * LD + c] = v1;
    }
    __syncthreads();
    // rows: H over n, then the scales, one rounding to fp16
    const float s0 = (float)svh[blockIdx.x * 128 + 2 * lane], s1 = (float)svh[blockIdx.x * 128 + 2 * lane + 1];
    for (int r = 32 * wave; r < 32 * wave + 32; ++r) {
        float v0 = w[r * LD + 2 * lane], v1 = w[r * LD + 2 * lane + 1];
        hx_had128_wave(v0, v1);
        const float su = (float)suh[blockIdx.y * 128 + r];
        hx_h2 o = {(_Float16)(v0 * su * s0), (_Float16)(v1 * su * s1)};
        *reinterpret_cast<hx_h2*>(out + (size_t)(blockIdx.y * 128 + r) * out_cols + blockIdx.x * 128 + 2 * lane) = o;
    }
}

hipError_t launch_reconstruct_had(_Float16* out, const uint16_t* packed, const _Float16* suh, const _Float16* svh,
                                  int packed_rows, int packed_cols, int unpacked_rows, int unpacked_cols, int bits,
                                  int cb, long n_offset, hipStream_t st)
{
    if (bits < 1 || bits > 8 || unpacked_rows % 128 || unpacked_cols % 128 || n_offset % 128 || n_offset < 0 ||
        n_offset + unpacked_cols > (long)packed_cols * 16 || unpacked_rows > packed_rows * 16)
        return hipErrorInvalidValue;
    if (unpacked_rows == 0 || unpacked_cols == 0) return hipSuccess;
    dim3 grid(unpacked_cols / 128, unpacked_rows / 128);
    const int off = (int)(n_offset / 16);
    switch (cb) {
        case 0: hipLaunchKernelGGL(reconstruct_had_kernel<0>, grid, dim3(256), 0, st, out, packed, suh, svh, packed_cols, off, unpacked_cols, bits); break;
        case 1: hipLaunchKernelGGL(reconstruct_had_kernel<1>, grid, dim3(256), 0, st, out, packed, suh, svh, packed_cols, off, unpacked_cols, bits); break;
        default: hipLaunchKernelGGL(reconstruct_had_kernel<2>, grid, dim3(256), 0, st, out, packed, suh, svh, packed_cols, off, unpacked_cols, bits); break;
    }
    return hipGetLastError();
}

}  // namespace hx
