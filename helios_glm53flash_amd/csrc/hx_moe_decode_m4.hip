// Instantiation of the few-token MoE layer kernel for up to 4 rows per expert.
#include "hx_moe_decode.hpp"
#include "hx_kernels.hpp"
#include "hx_moe.hpp"

#include <stdlib.h>

namespace hx {

// Grid = every workgroup that fits at once; LDS = the input rows of the longest segment, i.e. one
// share of 128-k blocks (capped at K / 128), with the share sized for all slots active.
template <class Kernel>
static hipError_t launch_k(Kernel kernel, const MoeDecodeArgs& a, hipStream_t st)
{
    const long slots = a.routed_slots + 1;
    const long gg = a.inter / 128, gd = a.hidden / 128;
    const long nmax = 2 * slots * gg * gd > slots * gd * gg ? 2 * slots * gg * gd : slots * gd * gg;
    const long kbmax = gg > gd ? gg : gd;
    size_t lds = (size_t)4 * 128 * sizeof(_Float16);
    int grid = 1;
    for (int it = 0; it < 3; ++it) {
        grid = resident_blocks(reinterpret_cast<const void*>(kernel), DEC_THREADS, lds);
        if (grid < 1) grid = 1;
        if (const char* v = getenv("HX_MOE_WG_PER_CU")) {  // tuning: fewer workgroups per CU
            int cus = 0;
            (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0);
            const int cap = cus * atoi(v);
            if (cap > 0 && cap < grid) grid = cap;
        }
        long share = (nmax + grid - 1) / grid;
        if (share > kbmax) share = kbmax;
        const size_t need = (size_t)4 * share * 128 * sizeof(_Float16);
        if (need <= lds) break;
        lds = need;
    }
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(DEC_THREADS), lds, st, a);
    return hipGetLastError();
}

template <int BITS, int CB>
static hipError_t launch_t(const MoeDecodeArgs& a, hipStream_t st)
{
    if constexpr (BITS != 0) return launch_k(moe_decode_kernel<BITS, CB, 4>, a, st);
    else return launch_k(moe_decode_mixed_kernel<CB, 4>, a, st);
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

hipError_t launch_moe_decode_m4(const MoeDecodeArgs& a, int cb, int bits, hipStream_t st)
{
    return cb == 1 ? launch_cb<1>(a, bits, st) : launch_cb<2>(a, bits, st);
}

}  // namespace hx
