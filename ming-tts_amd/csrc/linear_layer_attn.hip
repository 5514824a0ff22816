// Instantiations of the decode-layer kernel with attention items (layer_kernel.hpp), in a
// code object of their own, so the linear-only kernels' code is unchanged by them.
#include "layer_kernel.hpp"

namespace mt {

seq_fn layer_attn_kernel_fn(int wt, uint32_t M) {
    if (wt == DT_BF16) {
        if (M == 1) return layer_kernel<DT_BF16, 1, true>;
        if (M == 2) return layer_kernel<DT_BF16, 2, true>;
        if (M == 4) return layer_kernel<DT_BF16, 4, true>;
    } else if (wt == DT_F16) {
        if (M == 1) return layer_kernel<DT_F16, 1, true>;
        if (M == 2) return layer_kernel<DT_F16, 2, true>;
        if (M == 4) return layer_kernel<DT_F16, 4, true>;
    }
    return nullptr;
}

}  // namespace mt
