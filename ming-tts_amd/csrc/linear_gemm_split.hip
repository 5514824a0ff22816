// Pipelined MFMA GEMM of mt_linear for fp32 activations, with or without a fused RMSNorm: the
// instantiations of tiled_kernel.hpp's split path (x = hi + lo of the weights' type, two
// MFMAs per k step), which the launcher in linear_gemm_lds.hip picks by weight type, gate,
// norm and tile shape.
//
// Reference kernel replaced: gemm_kernel<32,64,32,4> (Shaders.swift:297-410), whose X is fp32.
#include "tiled_kernel.hpp"

namespace mt {

namespace {

// Tile shape 0 (128 x 128, by request only) has the loop that commits only the split's stages;
// the 64-row tiles have both loops (stages 1: that loop, 2: the branch-free one).
template <int WT, bool GATED, bool NORM>
tiled::tiled_fn pick_split(int shape, int stages) {
    using tiled::tiled_kernel;
    if (shape == 0) return tiled_kernel<WT, 128, 128, GATED, 1, 2, DT_F32, NORM>;
    if (GATED || shape == 1)
        return stages == 1 ? tiled_kernel<WT, 64, 128, GATED, 1, 2, DT_F32, NORM>
                           : tiled_kernel<WT, 64, 128, GATED, 2, 2, DT_F32, NORM>;
    return stages == 1 ? tiled_kernel<WT, 64, 64, false, 1, 2, DT_F32, NORM>
                       : tiled_kernel<WT, 64, 64, false, 2, 2, DT_F32, NORM>;
}

template <int WT>
tiled::tiled_fn pick_split_wt(bool gated, bool norm, int shape, int stages) {
    if (gated) return norm ? pick_split<WT, true, true>(shape, stages) : pick_split<WT, true, false>(shape, stages);
    return norm ? pick_split<WT, false, true>(shape, stages) : pick_split<WT, false, false>(shape, stages);
}

}  // namespace

tiled::tiled_fn pick_tiled_split(int wt, bool gated, bool norm, int shape, int stages) {
    return wt == DT_BF16 ? pick_split_wt<DT_BF16>(gated, norm, shape, stages)
                         : pick_split_wt<DT_F16>(gated, norm, shape, stages);
}

}  // namespace mt
