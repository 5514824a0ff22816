// RMSNorm on its own: y = x * rsqrt(mean(x^2) + eps) * g over rows of fp32 activations, the
// reference's Encoder.rmsnorm (Kernels.swift:163-171; kernel rmsnorm, Shaders.swift:414-440).
// The linears fuse the norm into their prologue (mt_linear_rmsnorm); this launch is for rows
// that are read as data, such as the backbone's final norm (Qwen.swift:94), whose output
// feeds two heads and the host.
//
// Layout on gfx950: one wave per row, four rows per 256-thread workgroup.  Each lane reads
// 16-byte chunks k = 4 lane + 256 j of the row and keeps its sum of squares; the wave adds
// them on DPP; the lanes then write their chunks scaled, the gain read as 8-byte chunks.
// The row is read twice (its second read hits the cache), so y may be x itself.
#include "mt_device.hpp"
#include "mt_internal.hpp"
#include "mingtts_hip.h"

namespace mt {

namespace {

template <int WT>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *x, uint32_t ldx, uint32_t rows, uint32_t width,
                                                      const uint16_t *g, float *y, uint32_t ldy, float eps) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + static_cast<size_t>(row) * ldx;
    float ss = 0.0f;
    for (uint32_t k = 4 * lane; k < width; k += 256) {
        const float4 v = *reinterpret_cast<const float4 *>(xr + k);
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    ss = group_sum(ss, 64);
    const float scale = rsqrt_hw(ss / static_cast<float>(width) + eps);
    float *yr = y + static_cast<size_t>(row) * ldy;
    for (uint32_t k = 4 * lane; k < width; k += 256) {
        const float4 v = *reinterpret_cast<const float4 *>(xr + k);
        const uint2 w = *reinterpret_cast<const uint2 *>(g + k);
        float4 o;
        o.x = v.x * scale * dec_lo<WT>(w.x);
        o.y = v.y * scale * dec_hi<WT>(w.x);
        o.z = v.z * scale * dec_lo<WT>(w.y);
        o.w = v.w * scale * dec_hi<WT>(w.y);
        *reinterpret_cast<float4 *>(yr + k) = o;
    }
}

}  // namespace

}  // namespace mt

using namespace mt;

extern "C" {

int mt_rmsnorm(const float *x, uint32_t ldx, uint32_t rows, uint32_t width, const void *g, mt_dtype wt, float *y,
               uint32_t ldy, float eps, mt_stream_t stream) {
    if (rows == 0) return MT_OK;
    if (!x || !g || !y) return set_error(MT_EINVAL, "mt_rmsnorm: null pointer");
    if (width == 0 || width % 4) return set_error(MT_EINVAL, "mt_rmsnorm: width %u must be a positive multiple of 4", width);
    if (ldx < width || ldy < width || ldx % 4 || ldy % 4)
        return set_error(MT_EINVAL, "mt_rmsnorm: strides ldx %u / ldy %u must be multiples of 4 and >= width %u", ldx,
                         ldy, width);
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15)
        return set_error(MT_EINVAL, "mt_rmsnorm: x and y must be 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(g) & 7) return set_error(MT_EINVAL, "mt_rmsnorm: g must be 8-byte aligned");
    if (wt != MT_F16 && wt != MT_BF16) return set_error(MT_EINVAL, "mt_rmsnorm: the gain must be f16 or bf16");
    if (x != y) {
        const char *xa = reinterpret_cast<const char *>(x), *ya = reinterpret_cast<const char *>(y);
        const size_t xb = (static_cast<size_t>(rows - 1) * ldx + width) * 4, yb = (static_cast<size_t>(rows - 1) * ldy + width) * 4;
        if (xa < ya + yb && ya < xa + xb)
            return set_error(MT_EINVAL, "mt_rmsnorm: y overlaps x without being x");
    } else if (ldx != ldy) {
        return set_error(MT_EINVAL, "mt_rmsnorm: in place needs ldy == ldx");
    }
    const dim3 grid((rows + 3) / 4);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const uint16_t *gw = static_cast<const uint16_t *>(g);
    if (wt == MT_BF16) hipLaunchKernelGGL(rmsnorm_kernel<DT_BF16>, grid, dim3(256), 0, s, x, ldx, rows, width, gw, y, ldy, eps);
    else hipLaunchKernelGGL(rmsnorm_kernel<DT_F16>, grid, dim3(256), 0, s, x, ldx, rows, width, gw, y, ldy, eps);
    return check_launch("rmsnorm");
}

}  // extern "C"
