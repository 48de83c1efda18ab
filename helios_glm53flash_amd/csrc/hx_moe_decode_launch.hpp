// Launch of the few-token MoE layer kernel (moe_decode_kernel for one bit width,
// moe_decode_mixed_kernel for several) for up to MT = 1, 4 or 8 rows per expert.
#pragma once
#include "hx_kernels.hpp"
#include "hx_moe.hpp"
#include "hx_moe_decode.hpp"

namespace hx {

// Grid = the gate/up units then the down units (decode_units).  The dynamic LDS holds MT input
// rows of the longest unit: the unit count depends on the occupancy, which depends on the LDS
// (iterated to a fixed point); then padded to hold 4 workgroups per CU.
template <int MT, class Kernel>
static hipError_t launch_k(Kernel kernel, const MoeDecodeArgs& a0, hipStream_t st)
{
    MoeDecodeArgs a = a0;
    const void* k = reinterpret_cast<const void*>(kernel);
    size_t lds = (size_t)MT * 1024 * sizeof(_Float16);
    for (int it = 0; it < 4; ++it) {
        const size_t need = (size_t)MT * decode_units(a, decode_resident(k, DEC_THREADS, lds, 4)) * sizeof(_Float16);
        if (need == lds) break;
        lds = need;
    }
    lds = decode_lds_pad(k, lds, 4);
    hipLaunchKernelGGL(kernel, dim3(a.units_gu + a.units_d), dim3(DEC_THREADS), lds, st, a);
    return hipGetLastError();
}

template <int BITS, int CB, int MT>
static hipError_t launch_t(const MoeDecodeArgs& a, hipStream_t st)
{
    if constexpr (BITS != 0) return launch_k<MT>(moe_decode_kernel<BITS, CB, MT>, a, st);
    else return launch_k<MT>(moe_decode_mixed_kernel<CB, MT>, a, st);
}

template <int CB, int MT>
static hipError_t launch_cb(const MoeDecodeArgs& a, int bits, hipStream_t st)
{
    switch (bits) {
        case 1: return launch_t<1, CB, MT>(a, st);
        case 2: return launch_t<2, CB, MT>(a, st);
        case 3: return launch_t<3, CB, MT>(a, st);
        case 4: return launch_t<4, CB, MT>(a, st);
        case 5: return launch_t<5, CB, MT>(a, st);
        case 6: return launch_t<6, CB, MT>(a, st);
        case 7: return launch_t<7, CB, MT>(a, st);
        case 8: return launch_t<8, CB, MT>(a, st);
        default: return launch_t<0, CB, MT>(a, st);
    }
}

// One instantiation per row count, each in its own compile unit (hx_moe_decode_m*.hip).
template <int MT>
hipError_t launch_moe_decode_mt(const MoeDecodeArgs& a, int cb, int bits, hipStream_t st)
{
    return cb == 1 ? launch_cb<1, MT>(a, bits, st) : launch_cb<2, MT>(a, bits, st);
}

}  // namespace hx
