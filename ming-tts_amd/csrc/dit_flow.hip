// The DiT flow step around its linears: full attention with interleaved RoPE over the
// short DiT sequences, the flow input assembly with its inline x-embedder, and the CFG
// Euler update of the sampler.
//
// Reference kernels replaced: dit_attention (Shaders.swift:598-648), flow_assemble
// (Shaders.swift:650-676) and flow_euler (Shaders.swift:678-693), dispatched by
// Encoder.ditAttention / flowAssemble / flowEuler (Kernels.swift:208-246) inside the flow
// loop of MingEngine.encodeStep (Engine.swift:395-402).  Same arithmetic: fp32 scores,
// scale after the q.k dot, max-subtracted softmax, fp32 p.v; fp32 embedder dots over the
// latent dims in order; y += (c + (c - u) cfg) dt.
//
// Layout on gfx950:
//   - dit_attention: one (sequence, query row, head) item per half wave (32 lanes), lane p
//     owning dims 2p, 2p + 1 (one interleaved-RoPE pair, one cos/sin per position); the
//     q.k dot is a 5-step butterfly inside the half wave, so a wave runs two items and a
//     256-thread workgroup eight.  The S <= 8 scores stay in registers;
//   - flow_assemble: one thread per output element; an embedder row (latent_dim 16-bit
//     weights) is read in 16-byte loads;
//   - flow_euler: one thread per latent dim.
#include "mt_device.hpp"
#include "mt_internal.hpp"
#include "mingtts_hip.h"

namespace mt {

namespace {

constexpr int DIT_MAXS = 8;
constexpr int DIT_ITEMS = 8;  // items per 256-thread workgroup

// Sum over the 32 lanes of a half wave (xor distances below 32 stay inside it).
__device__ __forceinline__ float half_sum(float v) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// x_transformers interleaved rotary pair: (x, y) -> (x c - y s, y c + x s).
__device__ __forceinline__ float2 rope_pair(float2 v, float angle) {
    const float c = cosf(angle), s = sinf(angle);
    return make_float2(v.x * c - v.y * s, v.y * c + v.x * s);
}

__global__ __launch_bounds__(256) void dit_attention_kernel(const float *qkv, uint32_t ld, uint32_t B, uint32_t S,
                                                            uint32_t H, const float *inv_freq, float *out, uint32_t ldo,
                                                            float scale) {
    const uint32_t item = blockIdx.x * DIT_ITEMS + (threadIdx.x >> 5);
    const uint32_t p = threadIdx.x & 31;
    if (item >= B * S * H) return;  // a whole half wave leaves together
    const uint32_t h = item % H, i = (item / H) % S, b = item / (H * S);
    const uint32_t D = H * 64;
    const float freq = inv_freq[p];
    const float *rows = qkv + static_cast<size_t>(b) * S * ld + h * 64 + 2 * p;
    const float2 q = rope_pair(*reinterpret_cast<const float2 *>(rows + static_cast<size_t>(i) * ld),
                               static_cast<float>(i) * freq);
    float sc[DIT_MAXS];
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t j = 0; j < DIT_MAXS; j++) {
        if (j < S) {
            const float2 k = rope_pair(*reinterpret_cast<const float2 *>(rows + static_cast<size_t>(j) * ld + D),
                                       static_cast<float>(j) * freq);
            sc[j] = half_sum(q.x * k.x + q.y * k.y) * scale;
            mx = fmaxf(mx, sc[j]);
        }
    }
    float sum = 0.0f;
    float2 acc = make_float2(0.0f, 0.0f);
#pragma unroll
    for (uint32_t j = 0; j < DIT_MAXS; j++) {
        if (j < S) {
            const float e = expf(sc[j] - mx);
            const float2 v = *reinterpret_cast<const float2 *>(rows + static_cast<size_t>(j) * ld + 2 * D);
            sum += e;
            acc.x = fmaf(e, v.x, acc.x);
            acc.y = fmaf(e, v.y, acc.y);
        }
    }
    *reinterpret_cast<float2 *>(out + static_cast<size_t>(b * S + i) * ldo + h * 64 + 2 * p) =
        make_float2(acc.x / sum, acc.y / sum);
}

// Row r of the flow input (rows 0-2 the conditional batch, 3-5 the unconditional one):
// slot r % 3 = 0: t + c (cemb, or the cond embedder's bias for the unconditional rows);
// 1: emb(history); 2: emb(y), emb(v) = x_b + x_w v.
template <int WT>
__global__ __launch_bounds__(256) void flow_assemble_kernel(const float *y, const float *history, const float *cemb,
                                                            const uint16_t *cbias, const float *temb,
                                                            const uint16_t *xw, const uint16_t *xb, float *x,
                                                            uint32_t ldx, uint32_t hidden, uint32_t latent) {
    const uint32_t c = blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
    if (c >= hidden) return;
    const uint32_t s = r % 3;
    float v;
    if (s == 0) {
        v = temb[c] + (r < 3 ? cemb[c] : dec1<WT>(cbias[c]));
    } else {
        const float *src = s == 1 ? history : y;
        const uint16_t *w = xw + static_cast<size_t>(c) * latent;
        v = dec1<WT>(xb[c]);
        for (uint32_t d = 0; d < latent; d += 8) {
            const uint4 wv = *reinterpret_cast<const uint4 *>(w + d);
            float wf[8];
            unpack8<WT>(wv, wf);
#pragma unroll
            for (int e = 0; e < 8; e++) v = fmaf(wf[e], src[d + e], v);
        }
    }
    x[static_cast<size_t>(r) * ldx + c] = v;
}

__global__ __launch_bounds__(256) void flow_euler_kernel(float *y, const float *pred, uint32_t ldp, uint32_t pred_row,
                                                         uint32_t null_row, float *capture, uint32_t latent, float cfg,
                                                         float dt) {
    const uint32_t d = blockIdx.x * 256 + threadIdx.x;
    if (d >= latent) return;
    const float c = pred[static_cast<size_t>(pred_row) * ldp + d];
    const float u = pred[static_cast<size_t>(null_row) * ldp + d];
    if (capture) {
        capture[d] = c;
        capture[latent + d] = u;
    }
    y[d] += (c + (c - u) * cfg) * dt;
}

}  // namespace

int launch_dit_attention(const float *qkv, uint32_t ld, uint32_t B, uint32_t S, uint32_t H, const float *inv_freq,
                         float *out, uint32_t ldo, float scale, hipStream_t stream) {
    const uint32_t items = B * S * H;
    hipLaunchKernelGGL(dit_attention_kernel, dim3((items + DIT_ITEMS - 1) / DIT_ITEMS), dim3(256), 0, stream, qkv, ld,
                       B, S, H, inv_freq, out, ldo, scale);
    return check_launch("dit_attention");
}

int launch_flow_assemble(const float *y, const float *history, const float *cemb, const void *cbias, const float *temb,
                         const void *xw, const void *xb, int wt, float *x, uint32_t ldx, uint32_t hidden,
                         uint32_t latent, hipStream_t stream) {
    const dim3 grid((hidden + 255) / 256, 6);
    const uint16_t *cb = static_cast<const uint16_t *>(cbias), *w = static_cast<const uint16_t *>(xw),
                   *b = static_cast<const uint16_t *>(xb);
    if (wt == DT_BF16)
        hipLaunchKernelGGL(flow_assemble_kernel<DT_BF16>, grid, dim3(256), 0, stream, y, history, cemb, cb, temb, w, b,
                           x, ldx, hidden, latent);
    else
        hipLaunchKernelGGL(flow_assemble_kernel<DT_F16>, grid, dim3(256), 0, stream, y, history, cemb, cb, temb, w, b,
                           x, ldx, hidden, latent);
    return check_launch("flow_assemble");
}

int launch_flow_euler(float *y, const float *pred, uint32_t ldp, uint32_t pred_row, uint32_t null_row, float *capture,
                      uint32_t latent, float cfg, float dt, hipStream_t stream) {
    hipLaunchKernelGGL(flow_euler_kernel, dim3((latent + 255) / 256), dim3(256), 0, stream, y, pred, ldp, pred_row,
                       null_row, capture, latent, cfg, dt);
    return check_launch("flow_euler");
}

}  // namespace mt
