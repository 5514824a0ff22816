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
//     256-thread workgroup eight.  The S <= 8 scores stay in registers.  The item's
//     arithmetic (dit_attend.hpp) is shared with the out projection that computes its x
//     from qkv itself (mt_dit_attention_linear);
//   - flow_assemble: one thread per output element; an embedder row (latent_dim 16-bit
//     weights) is read in 16-byte loads;
//   - flow_euler: one thread per latent dim.
#include "dit_attend.hpp"
#include "mt_device.hpp"
#include "mt_internal.hpp"
#include "mingtts_hip.h"

namespace mt {

namespace {

constexpr int DIT_ITEMS = 8;  // items per 256-thread workgroup

__global__ __launch_bounds__(256) void dit_attention_kernel(const float *qkv, uint32_t ld, uint32_t B, uint32_t S,
                                                            uint32_t H, const float *inv_freq, float *out, uint32_t ldo,
                                                            float scale) {
    const uint32_t item = blockIdx.x * DIT_ITEMS + (threadIdx.x >> 5);
    const uint32_t p = threadIdx.x & 31;
    if (item >= B * S * H) return;  // a whole half wave leaves together
    const uint32_t h = item % H, i = (item / H) % S, b = item / (H * S);
    DitItem it;
    dit_item_load(qkv + static_cast<size_t>(b) * S * ld + h * 64 + 2 * p, ld, H * 64, i, S, it);
    float c[DIT_MAXS], s[DIT_MAXS];
    dit_rope_table(inv_freq[p], S, c, s);
    *reinterpret_cast<float2 *>(out + static_cast<size_t>(b * S + i) * ldo + h * 64 + 2 * p) =
        dit_item_attend(it, i, S, c, s, scale);
}

// y + (c + (c - u) cfg) dt with the multiply-adds written out, so the separate and the fused
// Euler kernels round alike.
__device__ __forceinline__ float euler_step(float y, float c, float u, float cfg, float dt) {
    return fmaf(fmaf(c - u, cfg, c), dt, y);
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
    y[d] = euler_step(y[d], c, u, cfg, dt);
}

// flow_euler of ODE step k then flow_assemble of step k + 1 in one workgroup: the Euler update
// of the latent in place (kept in LDS), then the six flow-input rows, thread c taking column
// c; rows 1 and 4 (x_b + x_w history) and rows 2 and 5 (x_b + x_w y) are the same sums, so
// each is computed once and stored twice.  Same arithmetic as the two kernels.
constexpr uint32_t FLOW_LATENT_MAX = 2048;
template <int WT>
__global__ __launch_bounds__(1024) void flow_euler_assemble_kernel(float *y, const float *pred, uint32_t ldp,
                                                                  uint32_t pred_row, uint32_t null_row, float *capture,
                                                                  float cfg, float dt, const float *history,
                                                                  const float *cemb, const uint16_t *cbias,
                                                                  const float *temb, const uint16_t *xw,
                                                                  const uint16_t *xb, float *x, uint32_t ldx,
                                                                  uint32_t hidden, uint32_t latent) {
    __shared__ float ys[FLOW_LATENT_MAX], hs[FLOW_LATENT_MAX];
    for (uint32_t d = threadIdx.x; d < latent; d += blockDim.x) {
        const float c = pred[static_cast<size_t>(pred_row) * ldp + d];
        const float u = pred[static_cast<size_t>(null_row) * ldp + d];
        if (capture) {
            capture[d] = c;
            capture[latent + d] = u;
        }
        const float v = euler_step(y[d], c, u, cfg, dt);
        y[d] = v;
        ys[d] = v;
        hs[d] = history[d];
    }
    __syncthreads();
    for (uint32_t c = threadIdx.x; c < hidden; c += blockDim.x) {
        x[c] = temb[c] + cemb[c];
        x[3 * static_cast<size_t>(ldx) + c] = temb[c] + dec1<WT>(cbias[c]);
        const uint16_t *w = xw + static_cast<size_t>(c) * latent;
        const float b = dec1<WT>(xb[c]);
        float vh = b, vy = b;
        for (uint32_t d = 0; d < latent; d += 8) {
            const uint4 wv = *reinterpret_cast<const uint4 *>(w + d);
            float wf[8];
            unpack8<WT>(wv, wf);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                vh = fmaf(wf[e], hs[d + e], vh);
                vy = fmaf(wf[e], ys[d + e], vy);
            }
        }
        x[static_cast<size_t>(ldx) + c] = vh;
        x[2 * static_cast<size_t>(ldx) + c] = vy;
        x[4 * static_cast<size_t>(ldx) + c] = vh;
        x[5 * static_cast<size_t>(ldx) + c] = vy;
    }
}

}  // namespace

int launch_flow_euler_assemble(float *y, const float *pred, uint32_t ldp, uint32_t pred_row, uint32_t null_row,
                               float *capture, float cfg, float dt, const float *history, const float *cemb,
                               const void *cbias, const float *temb, const void *xw, const void *xb, int wt, float *x,
                               uint32_t ldx, uint32_t hidden, uint32_t latent, hipStream_t stream) {
    const uint16_t *cb = static_cast<const uint16_t *>(cbias), *w = static_cast<const uint16_t *>(xw),
                   *b = static_cast<const uint16_t *>(xb);
    if (wt == DT_BF16)
        hipLaunchKernelGGL(flow_euler_assemble_kernel<DT_BF16>, dim3(1), dim3(1024), 0, stream, y, pred, ldp, pred_row,
                           null_row, capture, cfg, dt, history, cemb, cb, temb, w, b, x, ldx, hidden, latent);
    else
        hipLaunchKernelGGL(flow_euler_assemble_kernel<DT_F16>, dim3(1), dim3(1024), 0, stream, y, pred, ldp, pred_row,
                           null_row, capture, cfg, dt, history, cemb, cb, temb, w, b, x, ldx, hidden, latent);
    return check_launch("flow_euler_assemble");
}

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
