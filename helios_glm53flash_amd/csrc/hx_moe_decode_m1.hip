// Instantiation of the few-token MoE layer kernel for up to 1 rows per expert.
#include "hx_moe_decode.hpp"
#include "hx_kernels.hpp"
#include "hx_moe.hpp"

#include <stdlib.h>


namespace hx {

// Grid = the gate/up units then the down units (decode_units).
template <class Kernel>
static hipError_t launch_k(Kernel kernel, const MoeDecodeArgs& a0, hipStream_t st)
{
    MoeDecodeArgs a = a0;
    // LDS for the input rows of the longest unit: the unit count depends on the occupancy, which
    // depends on the LDS (iterated to a fixed point); then padded to hold 4 workgroups per CU
    const void* k = reinterpret_cast<const void*>(kernel);
    size_t lds = (size_t)1 * 1024 * sizeof(_Float16);
    for (int it = 0; it < 4; ++it) {
        const size_t need = (size_t)1 * decode_units(a, decode_resident(k, DEC_THREADS, lds, 4)) * sizeof(_Float16);
        if (need == lds) break;
        lds = need;
    }
    lds = decode_lds_pad(k, lds, 4);
    hipLaunchKernelGGL(kernel, dim3(a.units_gu + a.units_d), dim3(DEC_THREADS), lds, st, a);
    return hipGetLastError();
}

template <int BITS, int CB>
static hipError_t launch_t(const MoeDecodeArgs& a, hipStream_t st)
{
    if constexpr (BITS != 0) return launch_k(moe_decode_kernel<BITS, CB, 1>, a, st);
    else return launch_k(moe_decode_mixed_kernel<CB, 1>, a, st);
}

template <int CB>
static hipError_t launch_cb(const MoeDecodeArgs& a, int bits, hipStream_t st)
{
    switch (bits) {
        case 1: return launch_t<1, CB>(a, st);
        case 2: return launch_t<2, CB>(a, st);
        case 3: return launch_t<3, CB>(a, st);
        case 4: return launch_t<4, CB>(a, st);
        case 5: return launch_t<5, CB>(a, st);
        case 6: return launch_t<6, CB>(a, st);
        case 7: return launch_t<7, CB>(a, st);
        case 8: return launch_t<8, CB>(a, st);
        default: return launch_t<0, CB>(a, st);
    }
}

hipError_t launch_moe_decode_m1(const MoeDecodeArgs& a, int cb, int bits, hipStream_t st)
{
    return cb == 1 ? launch_cb<1>(a, bits, st) : launch_cb<2>(a, bits, st);
}

}  // namespace hx
