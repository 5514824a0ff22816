// Standalone decode GEMV launches of mt_linear (M up to 8 rows per row block; 3..8 rows go
// to the MFMA kernel of linear_gemv_mfma.hip unless tuned otherwise).
//
// Reference kernel replaced: gemv_kernel<MR> (Shaders.swift:47-108) and, for 3..8 rows,
// gemm8_kernel (Shaders.swift:188-283).  One wave64 holds 64 / L output features; the
// workgroup size is the one that leaves the busiest CU the fewest features.
#include "gemv_core.hpp"
#include "mt_internal.hpp"

namespace mt {

template <int MR, int WT, int XT, bool GATED, bool NORM>
__global__ __launch_bounds__(256) void gemv_kernel(LinearArgs a, int lanes_log2) {
    const int L = 1 << lanes_log2;
    const int groups = static_cast<int>(blockDim.x) >> lanes_log2;
    const int g = static_cast<int>(threadIdx.x) >> lanes_log2;
    const int j = static_cast<int>(threadIdx.x) & (L - 1);
    const uint32_t n = blockIdx.x * groups + g;
    if (n >= a.N) return;  // the whole lane group leaves together; no block barrier follows
    const uint32_t row0 = blockIdx.y * MR;
    const int rows = min(MR, static_cast<int>(a.M - row0));
    gemv_feature<MR, WT, XT, GATED, NORM, 4>(a, n, row0, rows, L, j);
}

namespace {

typedef void (*gemv_fn)(LinearArgs, int);

template <int MR, int WT, int XT>
gemv_fn pick_variant(bool gated, bool norm) {
    if (gated) return norm ? gemv_kernel<MR, WT, XT, true, true> : gemv_kernel<MR, WT, XT, true, false>;
    return norm ? gemv_kernel<MR, WT, XT, false, true> : gemv_kernel<MR, WT, XT, false, false>;
}

template <int MR, int WT>
gemv_fn pick_x(int xt, bool gated, bool norm) {
    switch (xt) {
        case DT_F32: return pick_variant<MR, WT, DT_F32>(gated, norm);
        case DT_F16: return pick_variant<MR, WT, DT_F16>(gated, norm);
        default: return pick_variant<MR, WT, DT_BF16>(gated, norm);
    }
}

template <int MR>
gemv_fn pick_w(int wt, int xt, bool gated, bool norm) {
    return wt == DT_BF16 ? pick_x<MR, DT_BF16>(xt, gated, norm) : pick_x<MR, DT_F16>(xt, gated, norm);
}

gemv_fn pick(int mr, int wt, int xt, bool gated, bool norm) {
    switch (mr) {
        case 1: return pick_w<1>(wt, xt, gated, norm);
        case 2: return pick_w<2>(wt, xt, gated, norm);
        case 4: return pick_w<4>(wt, xt, gated, norm);
        default: return pick_w<8>(wt, xt, gated, norm);
    }
}

}  // namespace

int gemv_lanes_log2(uint32_t K, int override_lanes, uint32_t M) {
    if (override_lanes >= 8 && override_lanes <= 64) {
        int l2 = 3;
        while ((1 << l2) < override_lanes) l2++;
        return l2;
    }
    // About eight 16-byte chunks per lane for one row, four for two or more (each chunk then
    // feeds every row): K = 896 -> 16 lanes at M = 1 (7 chunks each), 32 at M = 2 (3.5);
    // K = 4864 -> 64 lanes (9.5).  Measured on 4864 x 896 at M = 2: 5.2 us with 32 lanes,
    // 5.5-5.9 us with 16.
    const uint32_t kc = K / 8, target = M >= 2 ? 4u : 8u;
    int l2 = 3;
    while ((1u << l2) < 64u && (1u << l2) * target < kc) l2++;
    return l2;
}

int launch_gemv(const LinearArgs &a, int xt, int wt, hipStream_t stream, int override_lanes) {
    const bool gated = (a.flags & F_SILU_GATE) != 0;
    const bool norm = a.norm != nullptr;
    const int mr = a.M <= 1 ? 1 : a.M <= 2 ? 2 : a.M <= 4 ? 4 : 8;
    const int l2 = gemv_lanes_log2(a.K, override_lanes, a.M);
    const int L = 1 << l2;
    // The workgroup size (64..256 threads) that puts the fewest output features on the
    // busiest CU (ties: the larger size): with 4864 features of 16 lanes on 256 CUs, 128-thread
    // workgroups leave 2 or 3 (16 or 24 features) per CU, 64-thread ones 4 or 5 (at most 20).
    const int cus = device_cus() > 0 ? device_cus() : 256;
    int threads = 256;
    long best = -1;
    for (int t = 256; t >= 64; t >>= 1) {
        const long per = t / L, wgs = (static_cast<long>(a.N) + per - 1) / per;
        const long load = (wgs + cus - 1) / cus * per;
        if (best < 0 || load < best) {
            best = load;
            threads = t;
        }
    }
    const int per_group = threads / L;
    dim3 grid((a.N + per_group - 1) / per_group, (a.M + mr - 1) / mr);
    gemv_fn fn = pick(mr, wt, xt, gated, norm);
    hipLaunchKernelGGL(fn, grid, dim3(threads), 0, stream, a, l2);
    return check_launch("gemv");
}

}  // namespace mt
