// Decode GEMV core for gfx950: y[m, n] = x[m, :] . w[n, :] (+ epilogue) for up to MR rows.
//
// Layout of the work (one output feature n per lane group):
//   - a group of L lanes (L = 8..64, a power of two, always inside one wave64) owns one
//     output feature n and strides its weight row in 16-byte chunks (8 weights): lane j
//     reads chunks j, j + L, j + 2L, ... so every load instruction of a wave covers
//     (64 / L) rows x (L * 16) contiguous bytes;
//   - U chunk loads per lane are issued back to back before any is consumed, so each
//     lane keeps U * 16 bytes (x2 with the gate partner) of weights in flight;
//   - the MR activation rows reuse every weight load (the CFG pair at MR = 2);
//   - the group's partial sums meet by butterfly shuffles; lane 0 of the group runs the
//     epilogue and stores MR floats.
// Fused RMSNorm prologue (NORM): the reference normalises x in its own dispatch
// (Shaders.swift:414-441: x * rsqrt(mean(x^2) + eps) * g) before qkv and gate|up
// (Qwen.swift:84-90).  Here the group that streams row n already reads every x chunk, so it
// also sums x^2 over the row, multiplies x by the gain g on the fly, and applies the
// per-row scale rsqrt(mean(x^2) + eps) to the finished dot products -- no extra pass over x
// and no extra launch.
// Rows of x past M are never read.  The reduction order is fixed, so results are
// bit-identical from run to run.
#pragma once

#include "mt_device.hpp"

namespace mt {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Eight activations of row `row` at element offset k (k % 8 == 0) as fp32.
template <int XT>
__device__ __forceinline__ void load_x8(const void *X, size_t off, float *o) {
    if constexpr (XT == DT_F32) {
        const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(X) + off);
        const float4 a = p[0], b = p[1];
        o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
        o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
    } else {
        const uint4 v = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(X) + off);
        unpack8<XT>(v, o);
    }
}

__device__ __forceinline__ uint4 as_uint4(u32x4 v) { return make_uint4(v.x, v.y, v.z, v.w); }

// Computes output feature n for rows row0 .. row0 + rows - 1 (rows <= MR) with the calling
// group of L lanes; j is the lane's index in the group.  Lane j == 0 stores.
template <int MR, int WT, int XT, bool GATED, bool NORM, int U>
__device__ __forceinline__ void gemv_feature(const LinearArgs &a, uint32_t n, uint32_t row0, int rows,
                                             int L, int j) {
    const int KC = static_cast<int>(a.K >> 3);
    const u32x4 *wr = reinterpret_cast<const u32x4 *>(a.w + static_cast<size_t>(n) * a.K);
    const u32x4 *gr = reinterpret_cast<const u32x4 *>((GATED ? a.w2 : a.w) + static_cast<size_t>(n) * a.K);
    const u32x4 *nr = reinterpret_cast<const u32x4 *>(NORM ? a.norm : a.w);
    float acc[MR], acc2[MR], ss[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) { acc[m] = 0.0f; acc2[m] = 0.0f; ss[m] = 0.0f; }
    // The epilogue's bias and old y (lane 0 of the group uses them), requested now so the
    // epilogue does not wait for them; rows past `rows` read row row0.
    const float bias = (a.flags & F_BIAS) ? dec1<WT>(a.bias[n]) : 0.0f;
    float yold[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) yold[m] = 0.0f;
    if (a.flags & F_ACCUM) {
#pragma unroll
        for (int m = 0; m < MR; m++) yold[m] = a.y[static_cast<size_t>(row0 + (m < rows ? m : 0)) * a.ldy + n];
    }
    // With at most two rows, a lane's x chunks (and gain chunks) of an iteration are requested
    // with its weights, before any is used; more rows load them at the point of use.
    constexpr bool XPRE = MR <= 2;
    constexpr int XW = XT == DT_F32 ? 2 : 1;  // 16-byte loads per 8 activations
    typedef __attribute__((address_space(1))) const u32x4 *gx_cp;

    for (int c0 = j; c0 < KC; c0 += U * L) {
        u32x4 wv[U], gv[U], xr[XPRE ? U : 1][MR][XW], nv[XPRE && NORM ? U : 1];
#pragma unroll
        for (int u = 0; u < U; u++) {
            // Chunks past the row end load the row's last chunk (in bounds) and are skipped.
            const int c = min(c0 + u * L, KC - 1);
            wv[u] = __builtin_nontemporal_load(wr + c);
            if constexpr (GATED) gv[u] = __builtin_nontemporal_load(gr + c);
            if constexpr (XPRE) {
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    const size_t off = (static_cast<size_t>(row0 + (m < rows ? m : 0)) * a.ldx + static_cast<size_t>(c) * 8) *
                                       (XT == DT_F32 ? 4 : 2);
                    const gx_cp p = reinterpret_cast<gx_cp>(reinterpret_cast<uintptr_t>(static_cast<const char *>(a.x) + off));
#pragma unroll
                    for (int h = 0; h < XW; h++) xr[u][m][h] = p[h];
                }
                if constexpr (NORM) nv[u] = *reinterpret_cast<gx_cp>(reinterpret_cast<uintptr_t>(nr + c));
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = c0 + u * L;
            if (c < KC) {
                float wf[8], gf[8], nf[8];
                unpack8<WT>(as_uint4(wv[u]), wf);
                if constexpr (GATED) unpack8<WT>(as_uint4(gv[u]), gf);
                if constexpr (NORM) unpack8<WT>(as_uint4(XPRE ? nv[XPRE ? u : 0] : nr[c]), nf);
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    if (m < rows) {
                        float xf[8];
                        if constexpr (XPRE) {
                            if constexpr (XT == DT_F32) {
#pragma unroll
                                for (int h = 0; h < 2; h++) {
                                    const u32x4 v = xr[XPRE ? u : 0][m][h];
                                    xf[4 * h] = __uint_as_float(v.x);
                                    xf[4 * h + 1] = __uint_as_float(v.y);
                                    xf[4 * h + 2] = __uint_as_float(v.z);
                                    xf[4 * h + 3] = __uint_as_float(v.w);
                                }
                            } else {
                                unpack8<XT>(as_uint4(xr[XPRE ? u : 0][m][0]), xf);
                            }
                        } else {
                            load_x8<XT>(a.x, static_cast<size_t>(row0 + m) * a.ldx + static_cast<size_t>(c) * 8, xf);
                        }
                        if constexpr (NORM) {
                            float q = ss[m];
#pragma unroll
                            for (int e = 0; e < 8; e++) q = fmaf(xf[e], xf[e], q);
                            ss[m] = q;
#pragma unroll
                            for (int e = 0; e < 8; e++) xf[e] *= nf[e];
                        }
                        float s = acc[m];
#pragma unroll
                        for (int e = 0; e < 8; e++) s = fmaf(xf[e], wf[e], s);
                        acc[m] = s;
                        if constexpr (GATED) {
                            float s2 = acc2[m];
#pragma unroll
                            for (int e = 0; e < 8; e++) s2 = fmaf(xf[e], gf[e], s2);
                            acc2[m] = s2;
                        }
                    }
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; m++) {
        acc[m] = group_sum(acc[m], L);
        if constexpr (GATED) acc2[m] = group_sum(acc2[m], L);
        if constexpr (NORM) {
            const float scale = rsqrt_hw(group_sum(ss[m], L) / static_cast<float>(a.K) + a.eps);
            acc[m] *= scale;
            acc2[m] *= scale;
        }
    }
    if (j == 0) {
#pragma unroll
        for (int m = 0; m < MR; m++) {
            if (m < rows) {
                float v = epilogue(acc[m], acc2[m], bias, a.flags);
                if (a.flags & F_ACCUM) v += yold[m];
                a.y[static_cast<size_t>(row0 + m) * a.ldy + n] = v;
            }
        }
    }
}

}  // namespace mt
