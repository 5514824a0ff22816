// Instantiations of the DiT-block kernel (layer_kernel.hpp), in a code object of their own.
#include "layer_kernel.hpp"

namespace mt {

seq_fn dit_block_kernel_fn(int wt, uint32_t M) {
    if (M == 6) return wt == DT_BF16 ? dit_block_kernel<DT_BF16, 6> : dit_block_kernel<DT_F16, 6>;
    if (M == 2) return wt == DT_BF16 ? dit_block_kernel<DT_BF16, 2> : dit_block_kernel<DT_F16, 2>;
    return nullptr;
}

}  // namespace mt
