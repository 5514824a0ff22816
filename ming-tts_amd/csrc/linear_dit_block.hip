// Instantiations of the DiT-block kernel (layer_kernel.hpp), in a code object of their own.
#include "layer_kernel.hpp"

namespace mt {

seq_fn dit_block_kernel_fn(int wt) {
    if (wt == DT_BF16) return dit_block_kernel<DT_BF16>;
    if (wt == DT_F16) return dit_block_kernel<DT_F16>;
    return nullptr;
}

}  // namespace mt
