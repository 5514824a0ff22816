// The audio VAE decoder's tail around its linears: the x4 linear upsample of fc1 outputs, the
// ISTFT frame synthesis and the overlap-add emission.
//
// Reference kernels replaced: upsample4, istft_frames and istft_emit (Shaders.swift:697-790),
// dispatched by Encoder.upsample4 / istftFrames / istftEmit (Kernels.swift:247-283) from
// VAEDecoder.decodeDispatches (VAEDecoder.swift:81-107).  Same arithmetic: torch's linear
// upsample weights (0.625 / 0.375, 0.875 / 0.125, neighbours clamped when absent); frame f
// = irfft(min(e^logmag, 100) e^{i phase}) / N * window with the DFT summed directly from a
// cos table; out = sum of overlapping frames / sum of their window^2.
//
// Layout on gfx950:
//   - upsample4: one thread per feature, writing its four frame rows;
//   - istft_frames: one 512-thread workgroup per (frame, 32 samples t and their mirrors N - t):
//     the frame's bins (re, im) and the cos table sit in LDS; a lane computes samples t and
//     N - t in one pass over the bins, since cos(2 pi k (N - t) / N) = cos(2 pi k t / N) and the
//     sine terms only change sign, which halves the table reads and multiply-adds of the
//     reference loop; the 16 half-waves take 16 ranges of the bins, and the bins and the table
//     sit in LDS as (re, im) and (cos, sin) pairs, one 8-byte read each per bin (the reference
//     walks all bins in one dependent chain: 28 workgroups of such chains took 78 us for a
//     latent's 4 frames);
//   - istft_emit: one thread per output sample.
#include "mt_device.hpp"
#include "mt_internal.hpp"
#include "mingtts_hip.h"

namespace mt {

namespace {

constexpr int ISTFT_NMAX = 4096;   // nfft limit of the LDS tables

// One thread per feature writes all four frame rows from one read of prev, cur and next.
__global__ __launch_bounds__(256) void upsample4_kernel(const float *prev, const float *cur, const float *next,
                                                        float *frames, uint32_t ldf, uint32_t hidden, uint32_t has_prev,
                                                        uint32_t has_next) {
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;
    if (c >= hidden) return;
    const float h = cur[c];
    const float p = has_prev ? prev[c] : h, n = has_next ? next[c] : h;
    frames[c] = has_prev ? 0.625f * h + 0.375f * p : h;
    frames[static_cast<size_t>(ldf) + c] = has_prev ? 0.875f * h + 0.125f * p : h;
    frames[2 * static_cast<size_t>(ldf) + c] = has_next ? 0.875f * h + 0.125f * n : h;
    frames[3 * static_cast<size_t>(ldf) + c] = has_next ? 0.625f * h + 0.375f * n : h;
}

// Samples t and N - t of frame blockIdx.y for the 32 t = blockIdx.x * 32 + (tid % 32) (t <=
// N / 2): the 16 half-waves r = tid / 32 each sum the bins of range r of 1 .. N/2 - 1 (the
// index k t mod N advanced by t per bin, so no division and no chain through the table
// reads), and the 16 partial sums meet in LDS in range order.  The bins sit in LDS as (re, im)
// pairs and the table as (cos a, sin a) pairs, so a bin costs one uniform and one gathered
// 8-byte read.
constexpr int ISTFT_T = 32;     // samples (and their mirrors) per workgroup
constexpr int ISTFT_R = 16;     // bin ranges: one per half-wave
__global__ __launch_bounds__(ISTFT_T * ISTFT_R) void istft_frames_kernel(const float *spec, uint32_t ld_spec,
                                                                        const float *cos_table, const float *window,
                                                                        float *ring_frames, uint32_t nfft, uint32_t frame0,
                                                                        uint32_t ring) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    __shared__ f2 bin[ISTFT_NMAX / 2 + 1];   // (re, im)
    __shared__ f2 cs[ISTFT_NMAX];            // (cos 2 pi i / N, sin 2 pi i / N)
    __shared__ float part[ISTFT_R][2][ISTFT_T];
    constexpr uint32_t NT = ISTFT_T * ISTFT_R;
    const uint32_t N = nfft, bins = N / 2 + 1, f = blockIdx.y, tid = threadIdx.x;
    const float *row = spec + static_cast<size_t>(f) * ld_spec;
    for (uint32_t k = tid; k < bins; k += NT) {
        const float mag = fminf(expf(row[k]), 100.0f);
        const float ph = row[bins + k];
        bin[k] = f2{mag * cosf(ph), mag * sinf(ph)};
    }
    // The sine is read from the cos table a quarter turn on: sin(a) = cos(a + 3 pi / 2).
    const uint32_t quarter3 = 3 * (N / 4);
    for (uint32_t i = tid; i < N; i += NT) {
        const uint32_t j = i + quarter3;
        cs[i] = f2{cos_table[i], cos_table[j >= N ? j - N : j]};
    }
    __syncthreads();
    const uint32_t tq = tid % ISTFT_T, r = tid / ISTFT_T;
    const uint32_t t = blockIdx.x * ISTFT_T + tq;
    const uint32_t tt = t <= N / 2 ? t : 0u;  // lanes past N / 2 sum for t = 0 and store nothing
    const uint32_t nk = N / 2 - 1, k0 = 1 + r * nk / ISTFT_R, k1 = 1 + (r + 1) * nk / ISTFT_R;
    uint32_t idx = ((k0 - 1) * tt) % N;
    float sc = 0.0f, ss = 0.0f;
#pragma unroll 4
    for (uint32_t k = k0; k < k1; k++) {
        idx += tt;
        if (idx >= N) idx -= N;
        const f2 b = bin[k], c = cs[idx];
        sc = fmaf(b.x, c.x, sc);
        ss = fmaf(b.y, c.y, ss);
    }
    part[r][0][tq] = sc;
    part[r][1][tq] = ss;
    __syncthreads();
    if (r != 0 || t > N / 2) return;
    sc = part[0][0][tq];
    ss = part[0][1][tq];
#pragma unroll
    for (uint32_t q = 1; q < ISTFT_R; q++) {
        sc += part[q][0][tq];
        ss += part[q][1][tq];
    }
    const f2 b0 = bin[0], bh = bin[N / 2];
    const float base = b0.x + ((t & 1) ? -bh.x : bh.x);  // N even: t and N - t share parity
    const float scale = 1.0f / static_cast<float>(N);
    float *out = ring_frames + static_cast<size_t>((frame0 + f) % ring) * N;
    out[t] = (base + 2.0f * (sc - ss)) * scale * window[t];
    if (t > 0 && t < N / 2) out[N - t] = (base + 2.0f * (sc + ss)) * scale * window[N - t];
}

__global__ __launch_bounds__(256) void istft_emit_kernel(const float *ring_frames, const float *window, float *out,
                                                         uint32_t nfft, uint32_t hop, uint32_t pad, uint32_t s0,
                                                         uint32_t count, uint32_t last_frame, uint32_t ring) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= count) return;
    const uint32_t s = s0 + i + pad;
    const uint32_t fhi = min(s / hop, last_frame);
    const uint32_t flo = s >= nfft ? (s - nfft) / hop + 1 : 0u;
    float acc = 0.0f, env = 0.0f;
    for (uint32_t f = flo; f <= fhi; f++) {
        const uint32_t t = s - f * hop;
        if (t >= nfft) continue;
        const float w = window[t];
        acc += ring_frames[static_cast<size_t>(f % ring) * nfft + t];
        env = fmaf(w, w, env);
    }
    out[i] = acc / env;
}

}  // namespace

}  // namespace mt

using namespace mt;

extern "C" {

int mt_upsample4(const float *prev, const float *cur, const float *next, float *frames, uint32_t ldf, uint32_t hidden,
                 mt_stream_t stream) {
    if (hidden == 0) return MT_OK;
    if (!cur || !frames) return set_error(MT_EINVAL, "mt_upsample4: null pointer");
    if (ldf < hidden) return set_error(MT_EINVAL, "mt_upsample4: ldf %u < hidden %u", ldf, hidden);
    hipLaunchKernelGGL(upsample4_kernel, dim3((hidden + 255) / 256), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), prev ? prev : cur, cur, next ? next : cur, frames, ldf,
                       hidden, prev ? 1u : 0u, next ? 1u : 0u);
    return check_launch("upsample4");
}

int mt_istft_frames(const float *spec, uint32_t ld_spec, uint32_t count, uint32_t nfft, const float *cos_table,
                    const float *window, float *ring_frames, uint32_t frame0, uint32_t ring, mt_stream_t stream) {
    if (count == 0) return MT_OK;
    if (!spec || !cos_table || !window || !ring_frames) return set_error(MT_EINVAL, "mt_istft_frames: null pointer");
    if (nfft < 8 || nfft % 4 || nfft > static_cast<uint32_t>(ISTFT_NMAX))
        return set_error(MT_EINVAL, "mt_istft_frames: nfft %u must be a multiple of 4 in 8..%d", nfft, ISTFT_NMAX);
    if (ld_spec < nfft + 2) return set_error(MT_EINVAL, "mt_istft_frames: ld_spec %u < nfft + 2", ld_spec);
    if (ring == 0 || count > ring) return set_error(MT_EINVAL, "mt_istft_frames: %u frames for a ring of %u", count, ring);
    const dim3 grid((nfft / 2 + 1 + ISTFT_T - 1) / ISTFT_T, count);
    hipLaunchKernelGGL(istft_frames_kernel, grid, dim3(ISTFT_T * ISTFT_R), 0, reinterpret_cast<hipStream_t>(stream), spec, ld_spec,
                       cos_table, window, ring_frames, nfft, frame0, ring);
    return check_launch("istft_frames");
}

int mt_istft_emit(const float *ring_frames, const float *window, uint32_t nfft, uint32_t hop, uint32_t s0,
                  uint32_t count, uint32_t last_frame, uint32_t ring, float *out, mt_stream_t stream) {
    if (count == 0) return MT_OK;
    if (!ring_frames || !window || !out) return set_error(MT_EINVAL, "mt_istft_emit: null pointer");
    if (hop == 0 || hop > nfft || ring == 0) return set_error(MT_EINVAL, "mt_istft_emit: hop %u, nfft %u, ring %u", hop, nfft, ring);
    hipLaunchKernelGGL(istft_emit_kernel, dim3((count + 255) / 256), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       ring_frames, window, out, nfft, hop, (nfft - hop) / 2, s0, count, last_frame, ring);
    return check_launch("istft_emit");
}

}  // extern "C"
