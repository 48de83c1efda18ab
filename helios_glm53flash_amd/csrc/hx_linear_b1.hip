// Instantiation of the small-M linear kernels for 1-bit trellis.
#include "hx_linear_impl.hpp"

namespace hx {
template hipError_t launch_gemv_cb<1>(int, const GemvArgs&, const _Float16*, void*, bool, hipStream_t);
}  // namespace hx
