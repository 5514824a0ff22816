// Pipelined MFMA GEMM of mt_linear (prefill and DiT shapes, M above the GEMV row limit): the
// instantiations for activations of the weights' own 16-bit type, the tile plan and the
// launcher.  The kernel template and its design are in tiled_kernel.hpp; fp32 activations
// (with or without a fused RMSNorm) are instantiated in linear_gemm_split.hip.
//
// Reference kernel replaced: gemm_kernel<32,64,32,4> (Shaders.swift:297-410).
#include <algorithm>

#include "ring_kernel.hpp"
#include "tiled_kernel.hpp"

namespace mt {

using tiled::tiled_fn;
using tiled::TiledArgs;
using tiled::SHAPE_BM;
using tiled::SHAPE_BN;
using tiled::SHAPE_KS;
using tiled::TBK;

namespace {

template <int WT, bool GATED>
tiled_fn pick_tiled(int shape, int stages) {
    switch (stages) {
        case 1: return tiled::pick_shape<WT, GATED, 1, WT, false>(shape);
        case 2: return tiled::pick_shape<WT, GATED, 2, WT, false>(shape);
        case 3: return tiled::pick_shape<WT, GATED, 3, WT, false>(shape);
        default: return tiled::pick_shape<WT, GATED, 4, WT, false>(shape);
    }
}

}  // namespace

// Tile shape, split count and pipeline depth of an (M, N, K) linear, from measurements on
// MI355X (256 CUs) of the backbone and DiT shapes at M = 64 .. 512:
//   - A workgroup fills LDS from L2 at about 50 GB/s, a CU at about 80-110 GB/s with two, so
//     throughput comes from having one or two workgroups on every CU, not from deeper
//     pipelines; a workgroup's fixed cost (first stage, epilogue) is about 3 us.
//   - Not gated: 64 x 64 tiles, 4 stages (64 KB of LDS: two per CU); K is split only when it
//     is long: parts of about 16 stages, or of 8 while the tiles alone fill under a third of the
//     CUs, and at most two workgroups per CU (down, 896 x 4864, graph replay: at M = 256 4 parts
//     take 12.5 us against 14.7 for 9, at M = 512 4 parts 16.0 against 16.9 for 2; at M = 64 6
//     parts 11.0 against 11.3 for 4 and 11.7 for 9).
//   - Gated: 64 x 128 tiles while they fit the CUs in one wave (gate|up up to 192 rows: at
//     M = 96 / 128 10.9 / 11.3 us against 13.6 / 13.7 on 128 x 128), else 128 x 128; with more
//     tiles than CUs the double-buffered ring (68 KB) keeps two 128 x 128 workgroups on a CU.
//   - fp32 activations (split): staged through registers into two LDS buffers.  K is split
//     into as many parts as fill the CUs once, or into parts of at most 20 stages, within two
//     workgroups per CU, parts of at least 3 stages and 8 parts, 2 parts when gated (the last
//     workgroup of a tile adds the parts); long K (32 stages and more) takes 64 x 128 tiles
//     from 384 rows.  Graph replay (fp32 x): at M = 512 rmsnorm+qkv 13.3 us unsplit against
//     14.3 in 3 parts, o 11.4 in 2 against 12.6 unsplit, down 24.0 on 64 x 128 tiles in 4
//     parts against 25.8 on 64 x 64; at M = 256 down 16.9 on 64 x 64 against 18.0 on 64 x 128;
//     at M = 64 o 8.7 in 6-7 parts against 9.5 in 3, rmsnorm+gate|up 13.6 in 2 against 14.1 in
//     3; rmsnorm+qkv and o (14 stages) at M = 24-128 0.2-1 us faster in 5 parts of 3 stages
//     than in 7 of 2.  Gated: 64 x 128 tiles below the ring kernel's rows (a 128 x 128 split tile needs 98 KB
//     of LDS, one workgroup per CU).
//   - 64 x 128 tiles (not gated) hold one workgroup a CU (96 KB of LDS at 4 stages, or the
//     branch-free fp32-x loop's registers), so their K parts stop at one workgroup per CU; they
//     take long K from 512 rows for x of the weights' type (down, graph replay: M = 512 15.2 us
//     in 4 parts against 15.7 on 64 x 64, M = 640 / 768 / 1024 16.5 / 17.4 / 20.5 in 3 / 3 / 2
//     parts against 18.1 / 18.9 / 23.0), and any K once the 64 x 64 tiles alone outnumber the
//     CUs (qkv at M = 1024: 15.5 against 18.0 us with fp32 x and the norm, 8.6 against 9.0).
//     fp32-x down at M = 640 / 768: 26.7 / 27.7 us in 3 parts against 35.6 / 35.5 in 4.
TiledPlan tiled_plan(uint32_t M, uint32_t N, uint32_t K, bool gated, int cus, int shape_override, int splitk_override,
                     bool split) {
    TiledPlan p{};
    const uint32_t KT = (K + TBK - 1) / TBK;
    const uint32_t ncu = static_cast<uint32_t>(cus > 0 ? cus : 256);
    int s = gated ? (split || M <= 64 || static_cast<uint64_t>((M + 63) / 64) * ((N + 63) / 64) <= ncu ? 1 : 0) : 2;
    if (!gated) {
        const uint64_t t64 = static_cast<uint64_t>((M + 63) / 64) * ((N + 63) / 64);
        if ((KT >= 32 && M >= (split ? 384u : 512u)) || t64 > ncu) s = 1;
    }
    if (shape_override > 0) s = shape_override - 1;
    if (gated && SHAPE_BN[s] != 128) return p;  // bm == 0: no such tile for a gated linear
    const uint32_t feats = gated ? 64u : static_cast<uint32_t>(SHAPE_BN[s]);
    p.shape = s;
    p.bm = SHAPE_BM[s];
    p.bn = SHAPE_BN[s];
    p.tiles_m = (M + p.bm - 1) / p.bm;
    p.tiles_n = (N + feats - 1) / feats;
    const uint32_t tiles = p.tiles_m * p.tiles_n;
    uint32_t S = 1;
    if (splitk_override > 0) {
        S = static_cast<uint32_t>(splitk_override);
    } else if (split) {
        const uint32_t t1 = std::max(tiles, 1u);
        const uint32_t slots = (!gated && p.bn == 128 ? 1 : 2) * ncu;  // workgroups the CUs hold at once
        S = std::min({slots / t1, std::max(ncu / t1, (KT + 19) / 20), std::max((KT + 2) / 3, 1u), 8u});
        if (gated) S = std::min(S, 2u);  // a gated part carries two partial tiles
        S = std::max(1u, S);
    } else if (!gated) {
        const uint32_t t1 = std::max(tiles, 1u);
        const uint32_t slots = (p.bn == 128 ? 1 : 2) * ncu;
        S = std::max(1u, std::min(slots / t1, std::max(KT / 16, std::min(KT / 8, ncu / (3 * t1)))));
    }
    S = std::max(1u, std::min(S, KT));
    p.kps = (KT + S - 1) / S;
    p.splits = (KT + p.kps - 1) / p.kps;
    // fp32 x: the branch-free loop (stages 2) holds more registers, one workgroup a CU at the
    // 64 x 128 tiles, so those take the other loop when their workgroups outnumber the CUs.
    if (split)
        p.stages = p.bm == 128 ? 1 : (p.bn == 64 || tiles * p.splits <= ncu) ? 2 : 1;
    else
        p.stages = (s == 0 && tiles > ncu) ? 2 : 4;
    return p;
}

size_t tiled_partial_bytes(const TiledPlan &p, bool gated, bool norm) {
    if (p.splits <= 1) return 0;
    const size_t ne = static_cast<size_t>(gated ? 2 : 1) * p.bm * (gated ? 64 : p.bn) + (norm ? p.bm : 0);
    return static_cast<size_t>(p.tiles_m) * p.tiles_n * p.splits * ne * sizeof(float);
}

// The gated ring kernel (ring_kernel.hpp, one workgroup a CU) takes a SiLU-gated linear (auto
// tile choice, x of the weights' type or fp32) when its tiles of 128 rows x 96 features fill at
// least three quarters of their last wave on the CUs.  Measured on gate|up (2 x 4864 x 896,
// graph replay, 256 CUs), ring against the best tiled plan, fp16 x / fp32 x with the norm:
//   M = 384 (153 tiles, 0.60 of a wave)   16.7 / 29.7 us against 14.4 / 26.2 (tiled)
//   M = 448-640 (204-255 tiles, 0.80-1)   17.4-19.5 / 28.9-30.8 against 19.8-21.0 / 35-36
//   M = 704-768 (306 tiles, 0.60 of two)  32.3 / 54.6 against 21.9 / 45.3 (tiled)
//   M = 1024 (408 tiles, 0.80 of two)     33.8 / 56.8 against 36.8 / 59.1
// Below 384 rows (102 tiles or fewer) the tiled plans are faster as well.
static bool ring_fills(uint32_t M, uint32_t N, int cus) {
    const uint64_t t = static_cast<uint64_t>((M + ring::BM - 1) / ring::BM) * ((N + ring::FN - 1) / ring::FN);
    const uint64_t c = static_cast<uint64_t>(cus > 0 ? cus : 256);
    const uint64_t waves = (t + c - 1) / c;
    return t > 0 && 4 * t >= 3 * waves * c;
}

int launch_gemm_tiled(const LinearArgs &a, int xt, int wt, hipStream_t stream, const FixedWs *fixed) {
    const bool gated = (a.flags & F_SILU_GATE) != 0;
    const bool split = xt == DT_F32, norm = a.norm != nullptr;
    if (!split && (xt != wt || norm)) return set_error(MT_ENOTSUP, "gemm: no pipelined kernel for this activation type");
    const int cus = device_cus();
    if (cus <= 0) return set_error(MT_EHIP, "gemm: cannot query the device");
    const int tile = tuning().gemm_tile, splitk = tuning().gemm_splitk, stages_override = tuning().gemm_stages;
    if (gated && !split && (tile == 5 || (tile == 0 && splitk == 0 && ring_fills(a.M, a.N, cus)))) {
        ring::RingArgs r{};
        r.x = static_cast<const uint16_t *>(a.x);
        r.w = a.w;
        r.w2 = a.w2;
        r.bias = a.bias;
        r.y = a.y;
        r.M = a.M; r.N = a.N; r.K = a.K; r.ldx = a.ldx; r.ldy = a.ldy; r.flags = a.flags;
        r.tiles_m = (a.M + ring::BM - 1) / ring::BM;
        r.tiles_n = (a.N + ring::FN - 1) / ring::FN;
        const uint64_t G = static_cast<uint64_t>(r.tiles_m) * r.tiles_n;
        if (G == 0 || G > 0x7FFFFFFFu) return set_error(MT_EINVAL, "gemm: %llu ring tiles", static_cast<unsigned long long>(G));
        hipLaunchKernelGGL(pick_ring_gated(wt), dim3(static_cast<uint32_t>(G)), dim3(ring::NT), 0, stream, r);
        return check_launch("gemm (ring)");
    }
    if (gated && split && (tile == 5 || (tile == 0 && splitk == 0 && ring_fills(a.M, a.N, cus)))) {
        ring::RingArgs r{};
        r.xf = static_cast<const float *>(a.x);
        r.norm = a.norm;
        r.eps = a.eps;
        r.w = a.w;
        r.w2 = a.w2;
        r.bias = a.bias;
        r.y = a.y;
        r.M = a.M; r.N = a.N; r.K = a.K; r.ldx = a.ldx; r.ldy = a.ldy; r.flags = a.flags;
        r.tiles_m = (a.M + ring::BM - 1) / ring::BM;
        r.tiles_n = (a.N + ring::FN - 1) / ring::FN;
        const uint64_t G = static_cast<uint64_t>(r.tiles_m) * r.tiles_n;
        if (G == 0 || G > 0x7FFFFFFFu) return set_error(MT_EINVAL, "gemm: %llu ring tiles", static_cast<unsigned long long>(G));
        hipLaunchKernelGGL(pick_ring_split(wt, norm), dim3(static_cast<uint32_t>(G)), dim3(ring::NT), 0, stream, r);
        return check_launch("gemm (ring, fp32 x)");
    }
    if (tile == 5) return set_error(MT_EINVAL, "gemm: tile 5 (the gated ring kernel) takes a SiLU-gated linear");
    TiledPlan p = tiled_plan(a.M, a.N, a.K, gated, cus, tile, splitk, split);
    if (stages_override >= 1) p.stages = !split ? stages_override : (p.bm == 128 || stages_override == 1) ? 1 : 2;
    if (p.bm == 0) return set_error(MT_EINVAL, "gemm: tile shape %d does not apply to this linear", tile);
    TiledArgs t;
    t.x = a.x;
    t.w = a.w;
    t.w2 = a.w2;
    t.bias = a.bias;
    t.norm = a.norm;
    t.eps = a.eps;
    t.y = a.y;
    t.M = a.M; t.N = a.N; t.K = a.K; t.ldx = a.ldx; t.ldy = a.ldy; t.flags = a.flags;
    t.tiles_m = p.tiles_m; t.tiles_n = p.tiles_n; t.splits = p.splits; t.kps = p.kps;
    t.part = nullptr;
    t.part_bytes = 0;
    t.cnt = nullptr;
    if (p.splits > 1) {
        const uint32_t tiles = p.tiles_m * p.tiles_n;
        void *part = nullptr;
        uint32_t *cnt = nullptr;
        const size_t pb = tiled_partial_bytes(p, gated, norm);
        if (pb > 0x7FFFFFF0u) return set_error(MT_ENOTSUP, "gemm: split-K partials of %zu bytes exceed 2 GiB", pb);
        const int rc = split_workspace(fixed, stream, pb, tiles, &part, &cnt, "gemm");
        if (rc) return rc;
        t.part = static_cast<float *>(part);
        t.part_bytes = static_cast<uint32_t>(pb);
        t.cnt = cnt;
    }
    const int stages = p.stages;
    tiled_fn fn = split ? pick_tiled_split(wt, gated, norm, p.shape, stages)
                  : wt == DT_BF16
                      ? (gated ? pick_tiled<DT_BF16, true>(p.shape, stages) : pick_tiled<DT_BF16, false>(p.shape, stages))
                      : (gated ? pick_tiled<DT_F16, true>(p.shape, stages) : pick_tiled<DT_F16, false>(p.shape, stages));
    const uint32_t G = p.tiles_m * p.tiles_n * p.splits;
    hipLaunchKernelGGL(fn, dim3(G), dim3(256 * SHAPE_KS[p.shape]), 0, stream, t);
    return check_launch("gemm");
}

}  // namespace mt
