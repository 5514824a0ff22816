// Persistent execution of a linear sequence (mt_seq_*): the decode step's chain of
// dependent GEMVs as ONE launch of one workgroup per CU, synchronised by dataflow instead
// of barriers.
//
// Reference counterpart: QwenForward.dispatches encoded on one serial compute encoder
// (Qwen.swift:72-97); every dispatch sees the writes of the ones before it.
//
// Why dataflow: on MI355X a device-wide barrier among 256 resident workgroups costs
// 2.5-4 us (a counter) and agent-scope fences (L2 write-back + invalidate on every XCD)
// cost more still, against 0.2-2.9 us of weight streaming per decode linear.  So:
//   - every op writes its outputs to a plan-owned tagged buffer: one fp32 word per
//     element whose lowest mantissa bit is replaced by the run's parity (epoch & 1),
//     stored device-coherently.  A consumer that reads a word with the current parity has
//     the current value (a 32-bit access is single-copy atomic): readiness and data arrive
//     in one memory round trip, with no barrier, fence or counter.  The consumer clears the
//     tag bit before use, so results do not depend on the parity;
//   - the run epoch lives in the plan's sync area; the last workgroup out increments it,
//     so re-running the plan needs no memset;
//   - user buffers: an op reads a user buffer only where nothing earlier in the sequence
//     wrote it, and writes a user buffer only if it is the last op writing that region
//     (the host plan compiler resolves both), so every user element is written once per run.
// Work of one op in a workgroup (the tiling is in seq_tiles.hpp): its share of the weight
// rows is cut into v_mfma_f32_16x16x32 tiles, each wave owning a contiguous range of
// tiles.  Per op a wave
//   1. has the op's weight chunks (the MFMA A operands) in registers already, requested
//      during the previous op;
//   2. requests the activations its tiles need (the B operands: SM = S * M columns of 32 k
//      per tile) straight from the producer's tagged buffer, spread over all 64 lanes in
//      16-byte chunks, and re-polls only the chunks whose tags are stale;
//   3. per chunk: clears the tag bits, adds x^2 to the RMSNorm sum, multiplies by the
//      gain (staged in LDS one op ahead), splits each fp32 value into a hi + lo pair of the
//      weights' 16-bit type (fp32-grade inputs on the 16-bit MFMA) and writes both to the
//      wave's LDS staging area in the B-fragment layout;
//   4. runs two MFMAs per tile (hi and lo), writing a finished row tile's partial sums to
//      LDS, requests the next op's weight chunks, and meets the other waves at one LDS-only
//      barrier (global loads stay in flight across it);
// then one lane per output sums the waves' partials in a fixed order, applies the norm
// scale and the epilogue and stores the tagged word (and the user output when final).
// Partials alternate between two LDS buffers by op parity, so one barrier per op suffices.
// Every wait is bounded: past SPIN_LIMIT polls a lane gives up, sets the plan's timeout
// flag (read by mt_seq_check) and stops waiting for the rest of the run.  An fp16 weight
// sequence also flags activations beyond the fp16 range (the hi part would overflow).
#include <stdlib.h>
#include <string.h>

#include "gemv_core.hpp"
#include "mt_internal.hpp"
#include "mingtts_hip.h"
#include "seq_tiles.hpp"

namespace mt {

enum : int { SYNC_EPOCH = 0, SYNC_EXIT = 32, SYNC_TIMEOUT = 64, SYNC_RANGE = 80, SYNC_WORDS = 96 };
constexpr int SEQ_THREADS = SEQ_THREADS_N;
constexpr int NW = SEQ_THREADS / 64;
constexpr int TMAX = SEQ_TMAX;
constexpr int PARTW = SEQ_PARTW;
constexpr int XCH = SEQ_XCH;
constexpr int XW = SEQ_XW;
constexpr int GCH = SEQ_GMAX / 8 / SEQ_THREADS;
constexpr uint32_t SPIN_LIMIT = 1u << 20;
constexpr uint32_t BUF_DWORD3 = 0x00020000u;  // raw 32-bit buffer resource word 3 for gfx9
constexpr int SC1 = 16;                         // buffer cache policy: device-coherent

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(1))) const uint32_t *g32_cp;
typedef __attribute__((address_space(1))) uint32_t *g32_p;
typedef __attribute__((address_space(1))) const u32x4 *gw_cp;

__device__ __forceinline__ uint32_t ld32(const uint32_t *p) {
    return __hip_atomic_load((g32_cp)(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Tagged word: the fp32 value with its lowest mantissa bit replaced by the run parity.
__device__ __forceinline__ void st_tag(uint32_t *p, float v, uint32_t parity) {
    __hip_atomic_store((g32_p)(p), (__float_as_uint(v) & ~1u) | parity, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void raise_flag(uint32_t *sync, int which) {
    __hip_atomic_store(sync + which, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The value a tagged word carries: its lowest mantissa bit cleared.
__device__ __forceinline__ float untag(uint32_t v) { return __uint_as_float(v & ~1u); }

// Four tagged words at byte offset off of the plan's tag buffer, device-coherently.
__device__ __forceinline__ u32x4 ldtag4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, SC1);
}
// Do all four words carry the parity?
__device__ __forceinline__ bool tagged4(const u32x4 a, uint32_t parity) {
    const uint32_t all = a.x & a.y & a.z & a.w, any = a.x | a.y | a.z | a.w;
    return parity ? (all & 1u) != 0 : (any & 1u) == 0;
}

template <int T>
__device__ __forceinline__ f32x4 mfma16(const u32x4 a, const u32x4 b, const f32x4 c) {
    if constexpr (T == DT_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
}
template <int T>
__device__ __forceinline__ uint32_t round16(float x) {
    if constexpr (T == DT_BF16) return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
    else return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}
// x = hi + lo in type T, packed in pairs.
template <int T>
__device__ __forceinline__ void split4(const float (&x)[4], u32x2 &hi, u32x2 &lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        h[e] = round16<T>(x[e]);
        l[e] = round16<T>(x[e] - dec1<T>(static_cast<uint16_t>(h[e])));
    }
    hi = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    lo = u32x2{l[0] | (l[1] << 16), l[2] | (l[3] << 16)};
}

// The tiles of op o owned by wave w of workgroup g.
struct WaveTiles {
    SeqTiles s;
    uint32_t t0, n;    // first tile, tile count
    uint32_t rt0, j0;  // row tile and block step of t0
};
__device__ __forceinline__ WaveTiles wave_tiles(const SeqOp &o, uint32_t g, uint32_t G, uint32_t w) {
    WaveTiles wt;
    wt.s = seq_tiles(o.N, o.K, o.M, (o.flags & F_SILU_GATE) != 0, g, G);
    wt.t0 = seq_tile_begin(wt.s.T, w, NW);
    wt.n = seq_tile_begin(wt.s.T, w + 1, NW) - wt.t0;
    wt.rt0 = wt.s.KBs ? wt.t0 / wt.s.KBs : 0;
    wt.j0 = wt.t0 - wt.rt0 * wt.s.KBs;
    return wt;
}

// This lane's A chunk of every tile of the wave into wr[u] (zero outside the share):
// A row a = lane % 16 (virtual row, or segment x virtual row when packed), k group
// q = lane / 16 (8 k at 32-k block offset 8 q).
__device__ __forceinline__ void load_w(const SeqOp &o, const WaveTiles &wt, u32x4 (&wr)[TMAX]) {
    const SeqTiles &s = wt.s;
    // Both row bases up front (uniform): the per-lane choice is then a register select.
    const uint16_t *const w1 = o.w, *const w2 = o.w2;
    const uint32_t lane = threadIdx.x & 63, a = lane & 15, q = lane >> 4;
    const uint32_t sa = s.S > 1 ? a / s.V : 0;
    const uint32_t va = s.S > 1 ? a - sa * s.V : a;
    uint32_t rt = wt.rt0, j = wt.j0;
#pragma unroll
    for (int u = 0; u < TMAX; u++) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (static_cast<uint32_t>(u) < wt.n) {
            const uint32_t vrow = s.S > 1 ? va : rt * 16 + a;
            const uint32_t kb = sa * s.KBs + j, k0 = kb * 32 + q * 8;
            if (sa < s.S && vrow < s.V && kb < s.KB && k0 < o.K) {
                const bool up = vrow >= s.nr;
                const uint16_t *row = (up ? w2 : w1) + static_cast<size_t>(s.r0 + (up ? vrow - s.nr : vrow)) * o.K;
                v = __builtin_nontemporal_load((gw_cp)(row + k0));
            }
            if (++j == s.KBs) {
                j = 0;
                rt++;
            }
        }
        wr[u] = v;
    }
}

// Partial sums of a finished row tile from the MFMA accumulator into this wave's LDS
// slice: pw[(v * M + m) * S + s] for virtual row v, x row m, segment s.
__device__ __forceinline__ void flush(const f32x4 acc, const SeqTiles &s, uint32_t M, uint32_t rt, float *pw) {
    const uint32_t lane = threadIdx.x & 63, c = lane & 15, qd = lane >> 4;
    const uint32_t sc = c / M, m = c - sc * M;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t a = qd * 4 + i;
        if (s.S > 1) {
            const uint32_t sa = a / s.V, v = a - sa * s.V;
            if (sa < s.S && sa == sc) pw[(v * M + m) * s.S + sa] = acc[i];
        } else {
            const uint32_t v = rt * 16 + a;
            if (v < s.V && c < M) pw[v * M + c] = acc[i];
        }
    }
}

// The RMSNorm gain of op o into LDS gb (16-bit, K elements): requested before a wait,
// stored after it.
__device__ __forceinline__ void gain_request(const SeqOp &o, u32x4 (&gr)[GCH]) {
    if (!o.norm) return;
#pragma unroll
    for (int r = 0; r < GCH; r++) {
        const uint32_t ch = threadIdx.x + r * SEQ_THREADS;
        if (ch * 8 < o.K) gr[r] = *reinterpret_cast<const u32x4 *>(o.norm + ch * 8);
    }
}
__device__ __forceinline__ void gain_store(const SeqOp &o, const u32x4 (&gr)[GCH], uint16_t *gb) {
    if (!o.norm) return;
#pragma unroll
    for (int r = 0; r < GCH; r++) {
        const uint32_t ch = threadIdx.x + r * SEQ_THREADS;
        if (ch * 8 < o.K) *reinterpret_cast<u32x4 *>(gb + ch * 8) = gr[r];
    }
}

// LDS-only workgroup barrier: global loads in flight stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// One 512-thread workgroup per CU runs every op of the sequence in order (see the top of
// the file).  tags / tag_bytes: the plan's tagged activation buffer, read through a buffer
// resource with device-coherent loads.
template <int WT>
__global__ __launch_bounds__(SEQ_THREADS) void seq_kernel(const SeqOp *__restrict__ ops, uint32_t n_ops,
                                                         uint32_t *sync, const uint32_t *tags, uint32_t tag_bytes) {
    __shared__ __attribute__((aligned(16))) float part[2][NW * PARTW];
    __shared__ __attribute__((aligned(16))) uint16_t gbuf[2][SEQ_GMAX];
    __shared__ __attribute__((aligned(16))) uint16_t xst[NW][2][XW * 32];  // [wave][hi, lo][(u SMP + c) 32 + k]
    __shared__ float ssw[2][NW * 16];
    const uint32_t G = gridDim.x, g = blockIdx.x;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t epoch = __hip_atomic_load(sync + SYNC_EPOCH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t parity = epoch & 1u;
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t *>(tags), 0, static_cast<int>(tag_bytes), BUF_DWORD3);
    bool gave_up = false;
    u32x4 wr[TMAX];
    u32x4 gr[GCH];

    if (n_ops > 0) {
        const SeqOp o0 = ops[0];
        load_w(o0, wave_tiles(o0, g, G, w), wr);
        gain_request(o0, gr);
        gain_store(o0, gr, gbuf[0]);
        lds_barrier();
    }
    for (uint32_t i = 0; i < n_ops; i++) {
        const SeqOp o = ops[i];
        const int b = i & 1;
        const WaveTiles wt = wave_tiles(o, g, G, w);
        const SeqTiles &s = wt.s;
        const uint32_t M = o.M;
        const bool norm = o.norm != nullptr;

        // Output lanes: bias and old y of output (feature r0 + v, row m), requested first.
        const uint32_t nout = s.nr * M;
        const uint32_t ov = tid / M, om = tid - ov * M;
        float bias = 0.0f, yold = 0.0f;
        uint32_t yw = 0;
        const uint32_t *yp = nullptr;
        if (tid < nout) {
            if (o.flags & F_BIAS) bias = dec1<WT>(o.bias[s.r0 + ov]);
            if (o.flags & F_ACCUM) {
                if (o.ysrc >= 0) {
                    yp = tags + o.yoff + static_cast<size_t>(om) * o.yld + s.r0 + ov;
                    yw = ld32(yp);
                } else {
                    yold = o.y[static_cast<size_t>(om) * o.ldy + s.r0 + ov];
                }
            }
        }
        // The next op's RMSNorm gain, stored to LDS after this op's wait.
        const bool next = i + 1 < n_ops;
        const SeqOp on = ops[next ? i + 1 : i];
        if (next) gain_request(on, gr);

        // Activation chunks of the wave's tiles: chunk e = lane + 64 r is tile u, B column
        // c (x row m of segment sc), 4 k at 4 h into the tile's 32-k block.  Columns are
        // padded to SMP, a power of two.
        const uint32_t SM = s.S * M;
        const uint32_t lsm = SM <= 1 ? 0u : SM <= 2 ? 1u : SM <= 4 ? 2u : SM <= 8 ? 3u : 4u;
        const uint32_t SMP = 1u << lsm, nch = wt.n << (lsm + 3);
        const uint32_t magic = (256u + M - 1) / M;  // c * magic >> 8 == c / M for c < 16
        const bool ext = o.xsrc < 0;
        u32x4 xv[XCH];
        uint32_t live = 0;  // chunks this lane holds
        auto chunk = [&](int r, uint32_t &u, uint32_t &c, uint32_t &m, uint32_t &k, uint32_t &rt) {
            const uint32_t e = lane + 64u * r;
            u = e >> (lsm + 3);
            c = (e >> 3) & (SMP - 1);
            const uint32_t sc = (c * magic) >> 8;
            m = c - sc * M;
            uint32_t j = wt.j0 + u;
            rt = wt.rt0;
            if (j >= s.KBs) {
                j -= s.KBs;
                rt++;
            }
            const uint32_t kb = sc * s.KBs + j;
            k = kb * 32 + (e & 7) * 4;
            return e < nch && c < SM && kb < s.KB && k < o.K;
        };
#pragma unroll
        for (int r = 0; r < XCH; r++) {
            uint32_t u, c, m, k, rt;
            xv[r] = u32x4{0u, 0u, 0u, 0u};
            if (chunk(r, u, c, m, k, rt)) {
                live |= 1u << r;
                if (!ext) {
                    xv[r] = ldtag4(rsrc, (o.xoff + m * o.xld + k) * 4u);
                } else if (o.xt == DT_F32) {
                    const float *p = static_cast<const float *>(o.x) + static_cast<size_t>(m) * o.ldx + k;
                    xv[r] = u32x4{__float_as_uint(p[0]), __float_as_uint(p[1]), __float_as_uint(p[2]),
                                  __float_as_uint(p[3])};
                } else {
                    const uint16_t *p = static_cast<const uint16_t *>(o.x) + static_cast<size_t>(m) * o.ldx + k;
                    float f[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) f[e] = o.xt == DT_BF16 ? dec1<DT_BF16>(p[e]) : dec1<DT_F16>(p[e]);
                    xv[r] = u32x4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                                  __float_as_uint(f[3])};
                }
            }
        }
        // Wait for the tagged chunks: every round re-requests all stale ones at once.
        if (!ext) {
            uint32_t spins = 0;
            while (!gave_up) {
                uint32_t stale = 0;
#pragma unroll
                for (int r = 0; r < XCH; r++)
                    if (((live >> r) & 1u) && !tagged4(xv[r], parity)) stale |= 1u << r;
                if (!stale) break;
                if (++spins > SPIN_LIMIT) {
                    gave_up = true;
                    raise_flag(sync, SYNC_TIMEOUT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
#pragma unroll
                for (int r = 0; r < XCH; r++) {
                    if ((stale >> r) & 1u) {
                        uint32_t u, c, m, k, rt;
                        chunk(r, u, c, m, k, rt);
                        xv[r] = ldtag4(rsrc, (o.xoff + m * o.xld + k) * 4u);
                    }
                }
            }
        }
        // Convert the chunks into the wave's B staging area (zeros past K).
        uint16_t *xh = xst[w][0], *xl = xst[w][1];
        const uint16_t *gb = gbuf[b];
        float ss0 = 0.0f, ss1 = 0.0f;
        bool range_ok = true;
#pragma unroll
        for (int r = 0; r < XCH; r++) {
            uint32_t u, c, m, k, rt;
            const bool ok = chunk(r, u, c, m, k, rt);
            const uint32_t e = lane + 64u * r;
            if (e < nch && c < SM) {
                float x[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                if (ok) {
                    const uint32_t clear = ext ? ~0u : ~1u;  // tagged words: drop the tag bit
                    x[0] = __uint_as_float(xv[r].x & clear);
                    x[1] = __uint_as_float(xv[r].y & clear);
                    x[2] = __uint_as_float(xv[r].z & clear);
                    x[3] = __uint_as_float(xv[r].w & clear);
                    if (norm) {
                        if (rt == 0) {  // each x element once per workgroup
                            float t = x[0] * x[0];
                            t = fmaf(x[1], x[1], t);
                            t = fmaf(x[2], x[2], t);
                            t = fmaf(x[3], x[3], t);
                            if (r & 1) ss1 += t; else ss0 += t;
                        }
                        const u32x2 gg = *reinterpret_cast<const u32x2 *>(gb + k);
                        x[0] *= dec_lo<WT>(gg.x);
                        x[1] *= dec_hi<WT>(gg.x);
                        x[2] *= dec_lo<WT>(gg.y);
                        x[3] *= dec_hi<WT>(gg.y);
                    }
                    if constexpr (WT == DT_F16)
                        range_ok = range_ok && fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3]))) <= 65504.0f;
                }
                u32x2 hi, lo;
                split4<WT>(x, hi, lo);
                const uint32_t at = ((u << lsm) + c) * 32 + (e & 7) * 4;
                *reinterpret_cast<u32x2 *>(xh + at) = hi;
                *reinterpret_cast<u32x2 *>(xl + at) = lo;
            }
        }
        if (!range_ok) raise_flag(sync, SYNC_RANGE);

        // MFMAs over the wave's tiles (hi and lo in two accumulators); a finished row tile
        // goes to LDS.  Lane (c, q) reads its B fragment, 8 k of column c, from the staging.
        float *pw = part[b] + w * PARTW;
        {
            const uint32_t c = lane & 15, q = lane >> 4;
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, acc2 = acc;
            uint32_t rt = wt.rt0, j = wt.j0;
#pragma unroll
            for (int u = 0; u < TMAX; u++) {
                if (static_cast<uint32_t>(u) < wt.n) {
                    u32x4 bh = {0u, 0u, 0u, 0u}, bl = bh;
                    if (c < SM) {
                        const uint32_t at = ((static_cast<uint32_t>(u) << lsm) + c) * 32 + q * 8;
                        bh = *reinterpret_cast<const u32x4 *>(xh + at);
                        bl = *reinterpret_cast<const u32x4 *>(xl + at);
                    }
                    acc = mfma16<WT>(wr[u], bh, acc);
                    acc2 = mfma16<WT>(wr[u], bl, acc2);
                    if (++j == s.KBs || static_cast<uint32_t>(u) + 1 == wt.n) {
                        flush(acc + acc2, s, M, rt, pw);
                        acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                        acc2 = acc;
                    }
                    if (j == s.KBs) {
                        j = 0;
                        rt++;
                    }
                }
            }
        }
        if (norm) {  // the wave's sum of x^2 per B column
            float t0 = ss0 + (SMP < 16 ? ss1 : 0.0f), t1 = SMP < 16 ? 0.0f : ss1;
            t0 += __shfl_xor(t0, 1, 64);
            t0 += __shfl_xor(t0, 2, 64);
            t0 += __shfl_xor(t0, 4, 64);
            t1 += __shfl_xor(t1, 1, 64);
            t1 += __shfl_xor(t1, 2, 64);
            t1 += __shfl_xor(t1, 4, 64);
            for (uint32_t bit = 8u * SMP; bit < 64u; bit <<= 1) t0 += __shfl_xor(t0, static_cast<int>(bit), 64);
            if ((lane & 7) == 0) {
                const uint32_t c0 = lane >> 3;
                if (c0 < SMP) ssw[b][w * 16 + c0] = t0;
                if (SMP == 16) ssw[b][w * 16 + c0 + 8] = t1;
            }
        }
        if (next) {
            load_w(on, wave_tiles(on, g, G, w), wr);
            gain_store(on, gr, gbuf[b ^ 1]);
        }
        lds_barrier();

        if (tid < nout) {
            if (yp) {
                uint32_t spins = 0;
                while ((yw & 1u) != parity && !gave_up) {
                    if (++spins > SPIN_LIMIT) {
                        gave_up = true;
                        raise_flag(sync, SYNC_TIMEOUT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                    yw = ld32(yp);
                }
                yold = untag(yw);
            }
            // Sum of the waves' partials for virtual row vr: the waves whose tile range
            // meets vr's row tile, by segment, then by wave (fixed order).
            auto total = [&](uint32_t vr) {
                const uint32_t rt = s.S > 1 ? 0 : vr / 16;
                const uint32_t lo_t = rt * s.KBs, hi_t = lo_t + s.KBs;
                bool take[NW];
#pragma unroll
                for (int ww = 0; ww < NW; ww++) {
                    const uint32_t b0 = seq_tile_begin(s.T, ww, NW), b1 = seq_tile_begin(s.T, ww + 1, NW);
                    take[ww] = b0 < b1 && b0 < hi_t && b1 > lo_t;
                }
                const float *p = part[b] + (vr * M + om) * s.S;
                float a = 0.0f;
                for (uint32_t sg = 0; sg < s.S; sg++) {
                    float v[NW];
#pragma unroll
                    for (int ww = 0; ww < NW; ww++) v[ww] = p[ww * PARTW + sg];
#pragma unroll
                    for (int ww = 0; ww < NW; ww++) a += take[ww] ? v[ww] : 0.0f;
                }
                return a;
            };
            float scale = 1.0f;
            if (norm) {
                float t = 0.0f;
                for (uint32_t sg = 0; sg < s.S; sg++) {
                    float v[NW];
#pragma unroll
                    for (int ww = 0; ww < NW; ww++) v[ww] = ssw[b][ww * 16 + sg * M + om];
#pragma unroll
                    for (int ww = 0; ww < NW; ww++) t += v[ww];
                }
                scale = 1.0f / sqrtf(t / static_cast<float>(o.K) + o.eps);
            }
            const float a1 = total(ov);
            const float a2 = (o.flags & F_SILU_GATE) ? total(ov + s.nr) : 0.0f;
            float v = epilogue(a1 * scale, a2 * scale, bias, o.flags);
            if (o.flags & F_ACCUM) v += yold;
            const uint32_t n = s.r0 + ov;
            st_tag(o.tag + static_cast<size_t>(om) * o.N + n, v, parity);
            if (o.final_out) o.y[static_cast<size_t>(om) * o.ldy + n] = v;
        }
    }
    // The last workgroup out advances the epoch for the next run.
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(sync + SYNC_EXIT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == G - 1) {
            __hip_atomic_store(sync + SYNC_EXIT, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(sync + SYNC_EPOCH, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

typedef void (*seq_fn)(const SeqOp *, uint32_t, uint32_t *, const uint32_t *, uint32_t);

struct SeqPlan {
    SeqOp *d_ops = nullptr;
    uint32_t *d_sync = nullptr;
    uint32_t *d_tags = nullptr;
    uint32_t tag_bytes = 0;
    uint32_t n_ops = 0;
    int groups = 0;
    int device = 0;
    seq_fn fn = nullptr;
};

int seq_limits(int *groups_out) {
    int dev = 0, cus = 0, per_cu = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(seq_kernel<DT_F16>),
                                                         SEQ_THREADS, 0);
    if (e != hipSuccess || cus <= 0 || per_cu <= 0)
        return set_error(MT_EHIP, "mt_seq_create: occupancy query failed (%s, cus %d, per_cu %d)", hipGetErrorString(e),
                         cus, per_cu);
    const int want = tuning().seq_groups;
    const int resident = cus * per_cu;
    // Default: one 512-thread workgroup per CU.
    *groups_out = want > 0 ? (want < resident ? want : resident) : cus;
    return MT_OK;
}

int seq_create(SeqOp *ops, uint32_t n_ops, int wt, int groups, SeqPlan **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(MT_EHIP, "mt_seq_create: hipGetDevice: %s", hipGetErrorString(e));
    // Each op's tagged output starts 16-byte aligned.
    size_t tag_words = 0;
    for (uint32_t i = 0; i < n_ops; i++) tag_words += (static_cast<size_t>(ops[i].M) * ops[i].N + 3) & ~size_t(3);
    if (tag_words * 4 > 0x7FFFFFF0u) return set_error(MT_ENOTSUP, "mt_seq_create: the ops' outputs exceed 2 GiB");
    SeqPlan *p = new SeqPlan();
    p->n_ops = n_ops;
    p->device = dev;
    p->fn = wt == DT_BF16 ? seq_kernel<DT_BF16> : seq_kernel<DT_F16>;
    p->groups = groups;
    p->tag_bytes = static_cast<uint32_t>((tag_words ? tag_words : 1) * 4);
    e = hipMalloc(&p->d_ops, sizeof(SeqOp) * (n_ops ? n_ops : 1));
    if (e == hipSuccess) e = hipMalloc(&p->d_sync, SYNC_WORDS * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&p->d_tags, p->tag_bytes);
    if (e == hipSuccess) {
        size_t off = 0;
        for (uint32_t i = 0; i < n_ops; i++) {
            ops[i].tag = p->d_tags + off;
            off += (static_cast<size_t>(ops[i].M) * ops[i].N + 3) & ~size_t(3);
        }
        // Tagged sources as offsets into the tag buffer (no dependent lookups on the device).
        for (uint32_t i = 0; i < n_ops; i++) {
            if (ops[i].xsrc >= 0) {
                const SeqOp &src = ops[ops[i].xsrc];
                ops[i].xoff = static_cast<uint32_t>(src.tag - p->d_tags) + ops[i].xcol;
                ops[i].xld = src.N;
            }
            if (ops[i].ysrc >= 0) {
                const SeqOp &src = ops[ops[i].ysrc];
                ops[i].yoff = static_cast<uint32_t>(src.tag - p->d_tags) + ops[i].ycol;
                ops[i].yld = src.N;
            }
        }
        e = hipMemcpy(p->d_ops, ops, sizeof(SeqOp) * n_ops, hipMemcpyHostToDevice);
    }
    // Tagged words start with parity 0 and the first run uses epoch 1 (parity 1), so no
    // stale word can pass for a current one.
    if (e == hipSuccess) e = hipMemset(p->d_tags, 0, p->tag_bytes);
    if (e == hipSuccess) e = hipMemset(p->d_sync, 0, SYNC_WORDS * sizeof(uint32_t));
    const uint32_t one = 1;
    if (e == hipSuccess) e = hipMemcpy(p->d_sync + SYNC_EPOCH, &one, sizeof(one), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(p->d_ops);
        (void)hipFree(p->d_sync);
        (void)hipFree(p->d_tags);
        delete p;
        return set_error(MT_EHIP, "mt_seq_create: %s", hipGetErrorString(e));
    }
    *out = p;
    return MT_OK;
}

int seq_run(SeqPlan *p, hipStream_t stream) {
    if (p->n_ops == 0) return MT_OK;
    void *args[] = {&p->d_ops, &p->n_ops, &p->d_sync, &p->d_tags, &p->tag_bytes};
    hipError_t e;
    if (tuning().seq_launch == 1) {
        // Ordinary launch: the workgroups are co-resident only while nothing else occupies
        // the CUs; the bounded waits turn a shortfall into the timeout flag.
        e = hipLaunchKernel(reinterpret_cast<const void *>(p->fn), dim3(p->groups), dim3(SEQ_THREADS), args, 0, stream);
    } else {
        e = hipLaunchCooperativeKernel(reinterpret_cast<const void *>(p->fn), dim3(p->groups), dim3(SEQ_THREADS), args,
                                       0, stream);
    }
    if (e != hipSuccess) return set_error(MT_EHIP, "mt_seq_run: launch: %s", hipGetErrorString(e));
    return MT_OK;
}

int seq_check(SeqPlan *p) {
    uint32_t flags[SYNC_WORDS];
    hipError_t e = hipMemcpy(flags, p->d_sync, sizeof(flags), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return set_error(MT_EHIP, "mt_seq_check: %s", hipGetErrorString(e));
    if (flags[SYNC_TIMEOUT]) return set_error(MT_EHIP, "mt_seq_check: a dataflow wait exceeded its spin bound");
    if (flags[SYNC_RANGE])
        return set_error(MT_ERANGE, "mt_seq_check: an activation exceeded the fp16 range of the weights' type "
                                    "(|x| > 65504); the results of that run are not valid");
    return MT_OK;
}

int seq_groups(const SeqPlan *p) { return p->groups; }

void seq_destroy(SeqPlan *p) {
    if (!p) return;
    (void)hipFree(p->d_ops);
    (void)hipFree(p->d_sync);
    (void)hipFree(p->d_tags);
    delete p;
}

}  // namespace mt
