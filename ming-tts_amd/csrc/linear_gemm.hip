// Register-staged MFMA GEMM of mt_linear for prefill and DiT shapes (M above the GEMV row
// limit) whose activations need converting: fp32 x, 16-bit x of the other type, or a fused
// RMSNorm.  Activations of the weights' own type go to the pipelined kernel of
// linear_gemm_lds.hip instead.
//
// Reference kernel replaced: gemm_kernel<32,64,32,4> (Shaders.swift:297-410), which stages
// X (fp32) and W (bf16 -> fp32) through threadgroup memory and multiplies 8x8 fp32 tiles.
//
// Here: a 64 (x rows) x 64 (weight rows) output tile per 256-thread workgroup, K in
// 64-wide slices staged through LDS as 16-bit values, four waves each owning a 32 x 32
// block computed with v_mfma_f32_32x32x16_{f16,bf16} (fp32 accumulate).  The next slice
// is fetched into registers while the current one is multiplied.
//   - Weights enter the MFMA unchanged (fp16 or bf16).
//   - Activations of the weights' type enter unchanged.  Any other activation type (fp32,
//     or the other 16-bit type) is split into hi = round16(x) and lo = round16(x - hi):
//     two MFMAs per step, and x is represented to 2^-22 (fp16) / 2^-17 (bf16) relative,
//     so the result keeps the reference's fp32-activation accuracy.
//   - SiLU-gate accumulates W and W2 tiles against the same activation fragments.
//   - Fused RMSNorm prologue (NORM): x is multiplied by the gain while it is staged (then
//     always split, so x * g is never rounded to 16 bits alone), each row's sum of squares
//     is accumulated from the same loads, and the epilogue scales by rsqrt(mean(x^2) + eps).
//   - Rows past M, weight rows past N and k past K are zero-filled in LDS, never read.
// MFMA 32x32x16 operand layout (wave64): lane l holds A[l % 32][8 (l / 32) .. + 7] and
// B[8 (l / 32) .. + 7][l % 32]; the 16 accumulators of lane l are
// D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32], r = 0..15.  Any other layout would scramble
// the output, which the GEMM parity tests would catch on every shape.
#include "mt_device.hpp"
#include "mt_internal.hpp"

namespace mt {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4g __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2g __attribute__((ext_vector_type(2)));

namespace {

constexpr int BM = 64, BN = 64, BK = 64;
constexpr int LDK = BK + 8;  // LDS row stride in 16-bit elements: 144 B, conflict-free b128 reads
constexpr int NT = 256;

template <int T>
__device__ __forceinline__ f32x16 mfma32(u32x4g a, u32x4g b, f32x16 c) {
    if constexpr (T == DT_BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <int T>
__device__ __forceinline__ uint32_t round16(float x) {
    if constexpr (T == DT_BF16) return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
    else return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

// hi/lo split of two fp32 values into packed 16-bit pairs of type T.
template <int T>
__device__ __forceinline__ void split2(float x0, float x1, uint32_t &hi, uint32_t &lo) {
    const uint32_t h0 = round16<T>(x0), h1 = round16<T>(x1);
    const float r0 = x0 - dec1<T>(static_cast<uint16_t>(h0));
    const float r1 = x1 - dec1<T>(static_cast<uint16_t>(h1));
    hi = h0 | (h1 << 16);
    lo = round16<T>(r0) | (round16<T>(r1) << 16);
}

template <int WT, int XT, bool GATED, bool NORM>
__global__ __launch_bounds__(NT) void gemm_kernel(LinearArgs a) {
    constexpr bool SPLIT = (XT != WT) || NORM;
    constexpr int XP = SPLIT ? 2 : 1;
    constexpr int WP = GATED ? 2 : 1;
    constexpr bool XF32 = (XT == DT_F32);
    constexpr int XCH = XF32 ? 4 : 2;          // 16-byte x chunks per thread per slice
    constexpr int XROW = XF32 ? 16 : 8;        // threads sharing one x row in a slice
    __shared__ __attribute__((aligned(16))) uint16_t xs[XP][BM * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t ws[WP][BN * LDK];
    __shared__ float row_scale[NORM ? BM : 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    // The epilogue's bias of the lane's feature, requested now so the epilogue does not wait
    // for it (lanes past N read element 0).
    const uint32_t bn = n0 + 32 * wn + (lane & 31);
    const float bv = (a.flags & F_BIAS) ? dec1<WT>(a.bias[bn < a.N ? bn : 0u]) : 0.0f;
    const uint32_t M = a.M, N = a.N, K = a.K;

    f32x16 acc, acc2;
#pragma unroll
    for (int r = 0; r < 16; r++) { acc[r] = 0.0f; acc2[r] = 0.0f; }
    float ss[XCH];
#pragma unroll
    for (int i = 0; i < XCH; i++) ss[i] = 0.0f;

    u32x4g wreg[2], w2reg[2], xreg[XCH], greg[XCH];

    auto fetch = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int q = tid + i * NT, r = q >> 3, kc = q & 7;
            const uint32_t n = n0 + r, k = k0 + kc * 8;
            u32x4g v = {0u, 0u, 0u, 0u}, v2 = {0u, 0u, 0u, 0u};
            if (n < N && k < K) {
                v = __builtin_nontemporal_load(reinterpret_cast<const u32x4g *>(a.w + static_cast<size_t>(n) * K + k));
                if constexpr (GATED)
                    v2 = __builtin_nontemporal_load(reinterpret_cast<const u32x4g *>(a.w2 + static_cast<size_t>(n) * K + k));
            }
            wreg[i] = v;
            if constexpr (GATED) w2reg[i] = v2;
        }
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int q = tid + i * NT;
            u32x4g v = {0u, 0u, 0u, 0u}, g = {0u, 0u, 0u, 0u};
            if constexpr (XF32) {
                const int r = q >> 4, c4 = q & 15;
                const uint32_t m = m0 + r, k = k0 + c4 * 4;
                if (m < M && k < K) {
                    v = *reinterpret_cast<const u32x4g *>(static_cast<const float *>(a.x) + static_cast<size_t>(m) * a.ldx + k);
                    if constexpr (NORM) {
                        const u32x2g g2 = *reinterpret_cast<const u32x2g *>(a.norm + k);
                        g.x = g2.x;
                        g.y = g2.y;
                    }
                }
            } else {
                const int r = q >> 3, kc = q & 7;
                const uint32_t m = m0 + r, k = k0 + kc * 8;
                if (m < M && k < K) {
                    v = *reinterpret_cast<const u32x4g *>(static_cast<const uint16_t *>(a.x) + static_cast<size_t>(m) * a.ldx + k);
                    if constexpr (NORM) g = *reinterpret_cast<const u32x4g *>(a.norm + k);
                }
            }
            xreg[i] = v;
            if constexpr (NORM) greg[i] = g;
        }
    };

    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int q = tid + i * NT, r = q >> 3, kc = q & 7;
            *reinterpret_cast<u32x4g *>(&ws[0][r * LDK + kc * 8]) = wreg[i];
            if constexpr (GATED) *reinterpret_cast<u32x4g *>(&ws[WP - 1][r * LDK + kc * 8]) = w2reg[i];
        }
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int q = tid + i * NT;
            const u32x4g v = xreg[i];
            if constexpr (XF32) {
                const int r = q >> 4, c4 = q & 15;
                float xf[4] = {__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w)};
                if constexpr (NORM) {
                    const u32x4g g = greg[i];
                    const float gf[4] = {dec_lo<WT>(g.x), dec_hi<WT>(g.x), dec_lo<WT>(g.y), dec_hi<WT>(g.y)};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        ss[i] = fmaf(xf[e], xf[e], ss[i]);
                        xf[e] *= gf[e];
                    }
                }
                uint32_t h0, l0, h1, l1;
                split2<WT>(xf[0], xf[1], h0, l0);
                split2<WT>(xf[2], xf[3], h1, l1);
                const u32x2g hi = {h0, h1}, lo = {l0, l1};
                *reinterpret_cast<u32x2g *>(&xs[0][r * LDK + c4 * 4]) = hi;
                *reinterpret_cast<u32x2g *>(&xs[XP - 1][r * LDK + c4 * 4]) = lo;
            } else if constexpr (!SPLIT) {
                const int r = q >> 3, kc = q & 7;
                *reinterpret_cast<u32x4g *>(&xs[0][r * LDK + kc * 8]) = v;
            } else {
                // 16-bit activations of the other type, or normalised: widen, then split.
                const int r = q >> 3, kc = q & 7;
                u32x4g hi, lo;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float x0 = dec_lo<XT>(v[e]), x1 = dec_hi<XT>(v[e]);
                    if constexpr (NORM) {
                        ss[i] = fmaf(x0, x0, ss[i]);
                        ss[i] = fmaf(x1, x1, ss[i]);
                        x0 *= dec_lo<WT>(greg[i][e]);
                        x1 *= dec_hi<WT>(greg[i][e]);
                    }
                    uint32_t h, l;
                    split2<WT>(x0, x1, h, l);
                    hi[e] = h;
                    lo[e] = l;
                }
                *reinterpret_cast<u32x4g *>(&xs[0][r * LDK + kc * 8]) = hi;
                *reinterpret_cast<u32x4g *>(&xs[XP - 1][r * LDK + kc * 8]) = lo;
            }
        }
    };

    fetch(0);
    for (uint32_t k0 = 0; k0 < K; k0 += BK) {
        __syncthreads();  // every wave is done reading the previous slice
        stage();
        __syncthreads();
        if (k0 + BK < K) fetch(k0 + BK);  // in flight while this slice is multiplied
        const int arow = (32 * wm + (lane & 31)) * LDK + (lane >> 5) * 8;
        const int brow = (32 * wn + (lane & 31)) * LDK + (lane >> 5) * 8;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            const u32x4g ah = *reinterpret_cast<const u32x4g *>(&xs[0][arow + kk]);
            const u32x4g b = *reinterpret_cast<const u32x4g *>(&ws[0][brow + kk]);
            acc = mfma32<WT>(ah, b, acc);
            u32x4g al;
            if constexpr (SPLIT) {
                al = *reinterpret_cast<const u32x4g *>(&xs[XP - 1][arow + kk]);
                acc = mfma32<WT>(al, b, acc);
            }
            if constexpr (GATED) {
                const u32x4g b2 = *reinterpret_cast<const u32x4g *>(&ws[WP - 1][brow + kk]);
                acc2 = mfma32<WT>(ah, b2, acc2);
                if constexpr (SPLIT) acc2 = mfma32<WT>(al, b2, acc2);
            }
        }
    }

    if constexpr (NORM) {
        // Row sums of squares: the XROW threads sharing a row are adjacent lanes of one wave.
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            float s = ss[i];
            for (int off = XROW >> 1; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
            const int r = (tid + i * NT) / XROW;
            if ((tid & (XROW - 1)) == 0) row_scale[r] = rsqrt_hw(s / static_cast<float>(K) + a.eps);
        }
        __syncthreads();
    }

    const uint32_t n = n0 + 32 * wn + (lane & 31);
    if (n >= N) return;
    // The old y of the lane's 16 rows, requested before the first is used (rows past M
    // read y[0]).
    float yo[16];
    if (a.flags & F_ACCUM) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const uint32_t m = m0 + 32 * wm + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            yo[r] = a.y[m < M ? static_cast<size_t>(m) * a.ldy + n : 0u];
        }
    }
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int ml = 32 * wm + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const uint32_t m = m0 + ml;
        if (m < M) {
            float c = acc[r], c2 = acc2[r];
            if constexpr (NORM) {
                c *= row_scale[ml];
                c2 *= row_scale[ml];
            }
            float v = epilogue(c, c2, bv, a.flags);
            if (a.flags & F_ACCUM) v += yo[r];
            a.y[static_cast<size_t>(m) * a.ldy + n] = v;
        }
    }
}

typedef void (*gemm_fn)(LinearArgs);

template <int WT, int XT>
gemm_fn pick_v(bool gated, bool norm) {
    if (gated) return norm ? gemm_kernel<WT, XT, true, true> : gemm_kernel<WT, XT, true, false>;
    return norm ? gemm_kernel<WT, XT, false, true> : gemm_kernel<WT, XT, false, false>;
}

template <int WT>
gemm_fn pick_x(int xt, bool gated, bool norm) {
    switch (xt) {
        case DT_F32: return pick_v<WT, DT_F32>(gated, norm);
        case DT_F16: return pick_v<WT, DT_F16>(gated, norm);
        default: return pick_v<WT, DT_BF16>(gated, norm);
    }
}

}  // namespace

int launch_gemm(const LinearArgs &a, int xt, int wt, hipStream_t stream, const FixedWs *fixed) {
    if (((xt == wt && a.norm == nullptr) || xt == DT_F32) && tuning().gemm_tile != 4)
        return launch_gemm_tiled(a, xt, wt, stream, fixed);
    const bool gated = (a.flags & F_SILU_GATE) != 0;
    const bool norm = a.norm != nullptr;
    gemm_fn fn = wt == DT_BF16 ? pick_x<DT_BF16>(xt, gated, norm) : pick_x<DT_F16>(xt, gated, norm);
    dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM);
    hipLaunchKernelGGL(fn, grid, dim3(NT), 0, stream, a);
    return check_launch("gemm");
}

}  // namespace mt
