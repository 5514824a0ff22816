// Instantiations of the decode-layer kernel (layer_kernel.hpp) without attention items, in a
// code object of their own; layer_kernel_fn picks among these and, for plans with attention
// items, linear_layer_attn.hip's.
#include "layer_kernel.hpp"

namespace mt {

seq_fn layer_kernel_fn(int wt, uint32_t M, bool att) {
    if (att) return layer_attn_kernel_fn(wt, M);
    if (wt == DT_BF16) {
        if (M == 1) return layer_kernel<DT_BF16, 1, false>;
        if (M == 2) return layer_kernel<DT_BF16, 2, false>;
        if (M == 4) return layer_kernel<DT_BF16, 4, false>;
    } else if (wt == DT_F16) {
        if (M == 1) return layer_kernel<DT_F16, 1, false>;
        if (M == 2) return layer_kernel<DT_F16, 2, false>;
        if (M == 4) return layer_kernel<DT_F16, 4, false>;
    }
    return nullptr;
}

}  // namespace mt
