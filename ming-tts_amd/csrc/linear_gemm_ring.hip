// Instances of the gated ring GEMM (ring_kernel.hpp): the SiLU-gated linear with x of the
// weights' type at M large enough to fill the chip with 96-feature tiles.  Its own code object,
// so the tiled kernels' instances keep their code layout.
//
// Reference kernel replaced: gemm_kernel<32,64,32,4> (Shaders.swift:297-410).
#include "ring_kernel.hpp"

namespace mt {

ring::ring_fn pick_ring_gated(int wt) {
    return wt == DT_BF16 ? ring::ring_gated_kernel<DT_BF16> : ring::ring_gated_kernel<DT_F16>;
}

ring::ring_fn pick_ring_split(int wt, bool norm) {
    if (wt == DT_BF16) return norm ? ring::ring_split_kernel<DT_BF16, true> : ring::ring_split_kernel<DT_BF16, false>;
    return norm ? ring::ring_split_kernel<DT_F16, true> : ring::ring_split_kernel<DT_F16, false>;
}

}  // namespace mt
