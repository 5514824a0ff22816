// Device helpers shared by the gfx950 kernels: 16-bit decode, the linear epilogue,
// wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mt {

enum : uint32_t { F_BIAS = 1, F_ACCUM = 2, F_GELU = 4, F_SILU_GATE = 8, F_SILU = 16 };
enum : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

struct LinearArgs {
    const void *x;
    const uint16_t *w;
    const uint16_t *w2;
    const uint16_t *bias;
    float *y;
    uint32_t M, N, K, ldx, ldy, flags;
    const uint16_t *norm;  // RMSNorm gain [K] (type of w) applied to x first, or null
    float eps;             // RMSNorm epsilon
};

// bf16 is the top half of an fp32 (Shaders.swift:12).
__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }
__device__ __forceinline__ float f16_lo(uint32_t v) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFFu));
}
__device__ __forceinline__ float f16_hi(uint32_t v) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}

template <int T>
__device__ __forceinline__ float dec_lo(uint32_t v) {
    if constexpr (T == DT_BF16) return bf16_lo(v); else return f16_lo(v);
}
template <int T>
__device__ __forceinline__ float dec_hi(uint32_t v) {
    if constexpr (T == DT_BF16) return bf16_hi(v); else return f16_hi(v);
}

// Eight 16-bit values of type T, packed little-endian in a uint4, to fp32.
template <int T>
__device__ __forceinline__ void unpack8(const uint4 v, float *o) {
    o[0] = dec_lo<T>(v.x); o[1] = dec_hi<T>(v.x);
    o[2] = dec_lo<T>(v.y); o[3] = dec_hi<T>(v.y);
    o[4] = dec_lo<T>(v.z); o[5] = dec_hi<T>(v.z);
    o[6] = dec_lo<T>(v.w); o[7] = dec_hi<T>(v.w);
}

template <int T>
__device__ __forceinline__ float dec1(uint16_t v) {
    if constexpr (T == DT_BF16) return __uint_as_float((uint32_t)v << 16);
    else return (float)__builtin_bit_cast(_Float16, v);
}

// Clamped tanh-GELU and SiLU, the reference's epilogue activations (Shaders.swift:21-29), on
// the hardware exp2 and reciprocal (each within 1 ulp): silu(v) = v / (1 + 2^(-v log2 e)),
// tanh(u) = 1 - 2 / (1 + 2^(2 u log2 e)).  A wave issues about one instruction every four
// cycles, and these sit on the critical path of every persistent op's outputs: they take a few
// instructions where expf, tanhf and IEEE division take tens (decode step 378 -> 371 us, flow
// stage 2249 -> 2082 us).  They differ from expf / tanhf and a correctly rounded division by a
// few ulp.  tanh(15) is already 1 in fp32, so the clamp changes no representable result.
__device__ __forceinline__ float silu_hw(float v) {
    return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v * -1.4426950408889634f));
}
__device__ __forceinline__ float gelu_hw(float x) {
    const float k = 0.7978845608028654f;
    float u = k * (x + 0.044715f * x * x * x);
    u = fminf(fmaxf(u, -15.0f), 15.0f);
    const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(u * 2.8853900817779268f));
    return 0.5f * x * (1.0f + t);
}
__device__ __forceinline__ float gelu_tanh(float x) { return gelu_hw(x); }
__device__ __forceinline__ float silu(float x) { return silu_hw(x); }
// e^x on the hardware exp2 (softmax weights, x <= 0).
__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
// 1 / sqrt(x) on the hardware reciprocal square root (the RMSNorm scale; within 1 ulp).
__device__ __forceinline__ float rsqrt_hw(float x) { return __builtin_amdgcn_rsqf(x); }

// The epilogue in the reference order (Shaders.swift:92-103): bias, SiLU-gate, GELU, SiLU,
// then accumulate into the old output.  yp is the output element's address.
__device__ __forceinline__ float epilogue(float acc, float acc2, float b, uint32_t flags) {
    float v = acc + b;
    if (flags & F_SILU_GATE) v = silu(v) * acc2;
    if (flags & F_GELU) v = gelu_tanh(v);
    if (flags & F_SILU) v = silu(v);
    return v;
}

// The epilogue with its flag set FL fixed at compile time, for kernels that branch on the flags
// once rather than per output (the same arithmetic as epilogue()).
template <uint32_t FL>
__device__ __forceinline__ float epilogue_fixed(float acc, float acc2, float b) {
    float v = acc;
    if constexpr ((FL & F_BIAS) != 0) v += b;
    if constexpr ((FL & F_SILU_GATE) != 0) v = silu_hw(v) * acc2;
    if constexpr ((FL & F_GELU) != 0) v = gelu_hw(v);
    if constexpr ((FL & F_SILU) != 0) v = silu_hw(v);
    return v;
}

// The flag sets the GEMM kernels specialise (every combination of bias, accumulate and the SiLU
// gate, and bias with GELU); any other set takes the out-of-line epilogue.
constexpr uint32_t EPI_OTHER = 0x80000000u;
template <uint32_t V>
struct FlagSet {
    static constexpr uint32_t value = V;
};
template <typename F>
__device__ __forceinline__ void with_flag_set(uint32_t flags, F &&f) {
    switch (flags) {
        case 0: f(FlagSet<0>{}); break;
        case F_BIAS: f(FlagSet<F_BIAS>{}); break;
        case F_ACCUM: f(FlagSet<F_ACCUM>{}); break;
        case F_BIAS | F_ACCUM: f(FlagSet<F_BIAS | F_ACCUM>{}); break;
        case F_SILU_GATE: f(FlagSet<F_SILU_GATE>{}); break;
        case F_SILU_GATE | F_BIAS: f(FlagSet<F_SILU_GATE | F_BIAS>{}); break;
        case F_SILU_GATE | F_ACCUM: f(FlagSet<F_SILU_GATE | F_ACCUM>{}); break;
        case F_GELU | F_BIAS: f(FlagSet<F_GELU | F_BIAS>{}); break;
        default: f(FlagSet<EPI_OTHER>{}); break;
    }
}
__device__ __attribute__((noinline)) inline float epilogue_out_of_line(float acc, float acc2, float b, uint32_t flags) {
    return epilogue(acc, acc2, b, flags);
}
// Epilogue of flag set FL (EPI_OTHER: the runtime flags, out of line), without the accumulate.
template <uint32_t FL>
__device__ __forceinline__ float epilogue_set(float acc, float acc2, float b, uint32_t flags) {
    if constexpr (FL == EPI_OTHER) return epilogue_out_of_line(acc, acc2, b, flags & ~F_ACCUM);
    else return epilogue_fixed<FL>(acc, acc2, b);
}
template <uint32_t FL>
__device__ __forceinline__ bool accumulates(uint32_t flags) {
    if constexpr (FL == EPI_OTHER) return (flags & F_ACCUM) != 0;
    else return (FL & F_ACCUM) != 0;
}

// One DPP lane move (quad permutes, row shifts and mirrors) of a float.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned octets of lanes, the same bits in all eight: two quad swaps, then the
// half-row mirror (lane i and 7 - i), all on DPP.
__device__ __forceinline__ float octet_sum(float v) {
    v += dpp_mov<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    return v + dpp_mov<0x141>(v);  // row_half_mirror
}

// octet_sum of n values at once, value by value the same steps, so the n sums' DPP steps
// overlap.
template <int N>
__device__ __forceinline__ void octet_sums(float *v) {
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_mov<0xB1>(v[i]);  // quad_perm [1, 0, 3, 2]
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_mov<0x4E>(v[i]);  // quad_perm [2, 3, 0, 1]
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_mov<0x141>(v[i]);  // row_half_mirror
}

// NeoX rotation of the pair (x0, x1) by the angle whose cosine and sine are c and s: r0 =
// x0 c - x1 s, r1 = x1 c + x0 s, with the contraction written out (the product x0 c or x1 c
// rounded, then one fused multiply-add), so every kernel that rotates a pair gets its bits.
__device__ __forceinline__ void rope_rotate(float x0, float x1, float c, float s, float &r0, float &r1) {
    r0 = fmaf(-x1, s, x0 * c);
    r1 = fmaf(x0, s, x1 * c);
}

// Sum over aligned groups of `width` lanes (8, 16, 32 or 64), the same bits in every lane of
// a group: quad swaps and the half-row mirror on DPP (8), the row mirror (16), then
// exchanges between rows.
__device__ __forceinline__ float group_sum(float v, int width) {
    v += dpp_mov<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v += dpp_mov<0x141>(v);  // row_half_mirror
    if (width >= 16) v += dpp_mov<0x140>(v);  // row_mirror
    if (width >= 32) v += __shfl_xor(v, 16, 64);
    if (width >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

}  // namespace mt
