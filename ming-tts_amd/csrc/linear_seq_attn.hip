// The sequence kernels of plans with attention items, in a code object of their own.
#include "seq_kernel.hpp"

namespace mt {

seq_fn seq_attn_kernel(int wt, bool m2) {
    if (wt == DT_BF16) return m2 ? seq_kernel<DT_BF16, 2, true> : seq_kernel<DT_BF16, 0, true>;
    return m2 ? seq_kernel<DT_F16, 2, true> : seq_kernel<DT_F16, 0, true>;
}

}  // namespace mt
