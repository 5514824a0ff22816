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
// An embedder row's 16-byte chunks d0 / 8 .. d0 / 8 + EMB_CHUNKS - 1, all requested before the
// first is used (one load round trip for a latent of up to 64); chunks past the row repeat its
// last one, so every load stays inside the row and none is conditional.
constexpr uint32_t EMB_CHUNKS = 8;
__device__ __forceinline__ void emb_chunks(const uint16_t *w, uint32_t d0, uint32_t latent, uint4 *wv) {
#pragma unroll
    for (uint32_t i = 0; i < EMB_CHUNKS; i++)
        wv[i] = *reinterpret_cast<const uint4 *>(w + min(d0 + 8 * i, latent - 8));
}

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
        const auto dot = [&](uint4 wv, uint32_t d) {
            float wf[8];
            unpack8<WT>(wv, wf);
#pragma unroll
            for (int e = 0; e < 8; e++) v = fmaf(wf[e], src[d + e], v);
        };
        for (uint32_t d0 = 0; d0 < latent; d0 += 8 * EMB_CHUNKS) {
            uint4 wv[EMB_CHUNKS];
            emb_chunks(w, d0, latent, wv);
            if (d0 + 8 * EMB_CHUNKS <= latent) {
#pragma unroll
                for (uint32_t i = 0; i < EMB_CHUNKS; i++) dot(wv[i], d0 + 8 * i);
            } else {
#pragma unroll
                for (uint32_t i = 0; i < EMB_CHUNKS; i++)
                    if (d0 + 8 * i < latent) dot(wv[i], d0 + 8 * i);
            }
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
    // The inputs of this thread's first column (clamped into the matrix: hidden >= 1) are
    // requested before the Euler update, so their round trip overlaps the update's.
    uint32_t c = min(threadIdx.x, hidden - 1);
    uint4 wv[EMB_CHUNKS];
    emb_chunks(xw + static_cast<size_t>(c) * latent, 0, latent, wv);
    float te = temb[c], ce = cemb[c];
    uint16_t cb = cbias[c], bb = xb[c];
    for (uint32_t d = threadIdx.x; d < latent; d += blockDim.x) {
        const float cv = pred[static_cast<size_t>(pred_row) * ldp + d];
        const float u = pred[static_cast<size_t>(null_row) * ldp + d];
        if (capture) {
            capture[d] = cv;
            capture[latent + d] = u;
        }
        const float v = euler_step(y[d], cv, u, cfg, dt);
        y[d] = v;
        ys[d] = v;
        hs[d] = history[d];
    }
    __syncthreads();
    // Column c's six rows, the first batch of its embedder row's chunks in w0.
    const auto column = [&](uint32_t c, const uint4 (&w0)[EMB_CHUNKS], float te, float ce, uint16_t cb, uint16_t bb,
                            uint32_t z) {
        x[c] = te + ce;
        x[3 * static_cast<size_t>(ldx) + c] = te + dec1<WT>(cb);
        const uint16_t *w = xw + static_cast<size_t>(c) * latent;
        const float b = dec1<WT>(bb);
        float vh = b, vy = b;
        const auto batch = [&](const uint4 (&wb)[EMB_CHUNKS], uint32_t d0) {
#pragma unroll
            for (uint32_t i = 0; i < EMB_CHUNKS; i++) {
                const uint32_t d = d0 + 8 * i;
                if (d0 + 8 * EMB_CHUNKS > latent && d >= latent) break;
                float wf[8];
                unpack8<WT>(wb[i], wf);
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    vh = fmaf(wf[e], hs[z + d + e], vh);
                    vy = fmaf(wf[e], ys[z + d + e], vy);
                }
            }
        };
        batch(w0, 0);
        for (uint32_t d0 = 8 * EMB_CHUNKS; d0 < latent; d0 += 8 * EMB_CHUNKS) {
            uint4 wb[EMB_CHUNKS];
            emb_chunks(w, d0, latent, wb);
            batch(wb, d0);
        }
        x[static_cast<size_t>(ldx) + c] = vh;
        x[2 * static_cast<size_t>(ldx) + c] = vy;
        x[4 * static_cast<size_t>(ldx) + c] = vh;
        x[5 * static_cast<size_t>(ldx) + c] = vy;
    };
    if (threadIdx.x < hidden) column(threadIdx.x, wv, te, ce, cb, bb, 0);
    // Columns past the first blockDim.x (hidden above 1024): z is 0 but opaque to the compiler,
    // which would otherwise keep every LDS value of the first batch in registers across the loop.
    for (c = threadIdx.x + blockDim.x; c < hidden; c += blockDim.x) {
        uint32_t z = 0;
        asm volatile("" : "+v"(z));
        uint4 w0[EMB_CHUNKS];
        emb_chunks(xw + static_cast<size_t>(c) * latent, 0, latent, w0);
        column(c, w0, temb[c], cemb[c], cbias[c], xb[c], z);
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
