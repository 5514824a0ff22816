// One item of the DiT's full attention with interleaved RoPE (Shaders.swift:598-648):
// query row i of one sequence of S rows, one head, computed by a half wave.  Lane p of the
// half wave owns dims 2p, 2p + 1 (one interleaved-RoPE pair, frequency inv_freq[p]); the q.k
// dot is a 5-step reduction over the half wave's 32 lanes; fp32 scores, scaled after the
// dot, max-subtracted softmax, fp32 p.v.  Shared by dit_attention_kernel and the out-projection
// linear that computes its own x from qkv, so both produce the same bits.  An item is
// requested (dit_item_load) apart from its arithmetic (dit_item_attend), so a kernel can put
// the loads of several items in flight before it waits for any.
#pragma once

#include "mt_device.hpp"

namespace mt {

constexpr int DIT_MAXS = 8;  // rows per DiT sequence

// cos and sin of position j's angle j * freq for the lane's pair, j < S (the rest unused).
__device__ __forceinline__ void dit_rope_table(float freq, uint32_t S, float (&c)[DIT_MAXS], float (&s)[DIT_MAXS]) {
#pragma unroll
    for (uint32_t j = 0; j < DIT_MAXS; j++) {
        c[j] = 1.0f;
        s[j] = 0.0f;
        if (j < S) {
            const float angle = static_cast<float>(j) * freq;
            c[j] = cosf(angle);
            s[j] = sinf(angle);
        }
    }
}

// x_transformers interleaved rotary pair: (x, y) -> (x c - y s, y c + x s).
__device__ __forceinline__ float2 dit_rope_pair(float2 v, float c, float s) {
    // The contraction written out, as rope_rotate does, so both kernels that inline this get
    // the same bits.
    return make_float2(fmaf(-v.y, s, v.x * c), fmaf(v.x, s, v.y * c));
}

// The lane's operands of one item: its q pair and the k and v pairs of the S keys.
struct DitItem {
    float2 q, k[DIT_MAXS], v[DIT_MAXS];
};

// rows: the sequence's first qkv row, offset by h * 64 + 2p (q of head h; its k sits D floats
// on, its v 2 D); ld: the qkv row stride; D: heads * 64.
__device__ __forceinline__ void dit_item_load(const float *rows, uint32_t ld, uint32_t D, uint32_t i, uint32_t S,
                                              DitItem &it) {
    it.q = *reinterpret_cast<const float2 *>(rows + static_cast<size_t>(i) * ld);
#pragma unroll
    for (uint32_t j = 0; j < DIT_MAXS; j++) {
        it.k[j] = it.v[j] = make_float2(0.0f, 0.0f);
        if (j < S) {
            it.k[j] = *reinterpret_cast<const float2 *>(rows + static_cast<size_t>(j) * ld + D);
            it.v[j] = *reinterpret_cast<const float2 *>(rows + static_cast<size_t>(j) * ld + 2 * D);
        }
    }
}

// Output dims 2p, 2p + 1 of query row i.  Every lane of the half wave must take part (the
// dot is a butterfly).
__device__ __forceinline__ float2 dit_item_attend(const DitItem &it, uint32_t i, uint32_t S, const float (&c)[DIT_MAXS],
                                                  const float (&s)[DIT_MAXS], float scale) {
    float ci = c[0], si = s[0];
#pragma unroll
    for (uint32_t j = 1; j < DIT_MAXS; j++) {
        ci = j == i ? c[j] : ci;
        si = j == i ? s[j] : si;
    }
    const float2 q = dit_rope_pair(it.q, ci, si);
    float sc[DIT_MAXS];
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t j = 0; j < DIT_MAXS; j++) {
        if (j < S) {
            const float2 k = dit_rope_pair(it.k[j], c[j], s[j]);
            sc[j] = group_sum(q.x * k.x + q.y * k.y, 32) * scale;
            mx = fmaxf(mx, sc[j]);
        }
    }
    float sum = 0.0f;
    float2 acc = make_float2(0.0f, 0.0f);
#pragma unroll
    for (uint32_t j = 0; j < DIT_MAXS; j++) {
        if (j < S) {
            const float e = exp_hw(sc[j] - mx);
            sum += e;
            acc.x = fmaf(e, it.v[j].x, acc.x);
            acc.y = fmaf(e, it.v[j].y, acc.y);
        }
    }
    return make_float2(acc.x / sum, acc.y / sum);
}

}  // namespace mt
