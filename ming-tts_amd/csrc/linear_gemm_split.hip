// Pipelined MFMA GEMM of mt_linear for fp32 activations, with or without a fused RMSNorm: the
// instantiations of tiled_kernel.hpp's split path (x = hi + lo of the weights' type, two
// MFMAs per k step), which the launcher in linear_gemm_lds.hip picks by weight type, gate,
// norm and tile shape.
//
// Reference kernel replaced: gemm_kernel<32,64,32,4> (Shaders.swift:297-410), whose X is fp32.
#include "tiled_kernel.hpp"

namespace mt {

tiled::tiled_fn pick_tiled_split(int wt, bool gated, bool norm, int shape) {
    using tiled::pick_shape;
    if (wt == DT_BF16) {
        if (gated) return norm ? pick_shape<DT_BF16, true, 1, DT_F32, true>(shape) : pick_shape<DT_BF16, true, 1, DT_F32, false>(shape);
        return norm ? pick_shape<DT_BF16, false, 1, DT_F32, true>(shape) : pick_shape<DT_BF16, false, 1, DT_F32, false>(shape);
    }
    if (gated) return norm ? pick_shape<DT_F16, true, 1, DT_F32, true>(shape) : pick_shape<DT_F16, true, 1, DT_F32, false>(shape);
    return norm ? pick_shape<DT_F16, false, 1, DT_F32, true>(shape) : pick_shape<DT_F16, false, 1, DT_F32, false>(shape);
}

}  // namespace mt
