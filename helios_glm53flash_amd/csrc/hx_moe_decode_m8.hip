// Few-token MoE layer kernels for up to 8 row(s) per expert (one compile unit per row count).
#include "hx_moe_decode_launch.hpp"

namespace hx {
template hipError_t launch_moe_decode_mt<8>(const MoeDecodeArgs& a, int cb, int bits, hipStream_t st);
}
