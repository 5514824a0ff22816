// Instantiations of the decode-layer kernel (layer_kernel.hpp), in a code object of their own.
#include "layer_kernel.hpp"

namespace mt {

seq_fn layer_kernel_fn(int wt, uint32_t M) {
    if (wt == DT_BF16) {
        if (M == 1) return layer_kernel<DT_BF16, 1>;
        if (M == 2) return layer_kernel<DT_BF16, 2>;
        if (M == 4) return layer_kernel<DT_BF16, 4>;
    } else if (wt == DT_F16) {
        if (M == 1) return layer_kernel<DT_F16, 1>;
        if (M == 2) return layer_kernel<DT_F16, 2>;
        if (M == 4) return layer_kernel<DT_F16, 4>;
    }
    return nullptr;
}

}  // namespace mt
