// Instantiation of the few-token MoE kernels for up to 8 rows per expert.
#include "hx_moe_decode.hpp"
#include "hx_kernels.hpp"

namespace hx {

template <int BITS, int CB>
static void launch_pair(const MoeDecodeArgs& a, bool gu, hipStream_t st)
{
    const int slots = a.routed_slots + 1;
    const int kc = gu ? a.kc_gu : a.kc_d;
    const int blocks = gu ? slots * 2 * (a.inter / 128) * a.splits_gu : slots * (a.hidden / 128) * a.splits_d;
    const size_t lds = (size_t)8 * kc * sizeof(_Float16);
    if (gu) hipLaunchKernelGGL((moe_decode_gu_kernel<BITS, CB, 8>), dim3(blocks), dim3(GEMV_THREADS), lds, st, a);
    else hipLaunchKernelGGL((moe_decode_d_kernel<BITS, CB, 8>), dim3(blocks), dim3(GEMV_THREADS), lds, st, a);
}

template <int CB>
static void launch_cb(const MoeDecodeArgs& a, bool gu, int bits, hipStream_t st)
{
    switch (bits) {
        case 1: launch_pair<1, CB>(a, gu, st); break;
        case 2: launch_pair<2, CB>(a, gu, st); break;
        case 3: launch_pair<3, CB>(a, gu, st); break;
        case 4: launch_pair<4, CB>(a, gu, st); break;
        case 5: launch_pair<5, CB>(a, gu, st); break;
        case 6: launch_pair<6, CB>(a, gu, st); break;
        case 7: launch_pair<7, CB>(a, gu, st); break;
        case 8: launch_pair<8, CB>(a, gu, st); break;
        default: break;
    }
}

hipError_t launch_moe_decode_phase_m8(const MoeDecodeArgs& a, int cb, bool gu, int bits, hipStream_t st)
{
    if (cb == 1) launch_cb<1>(a, gu, bits, st);
    else launch_cb<2>(a, gu, bits, st);
    return hipGetLastError();
}

}  // namespace hx
