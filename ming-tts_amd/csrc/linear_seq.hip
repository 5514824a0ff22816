// Persistent execution of a linear sequence (mt_seq_*): the decode step's chain of
// dependent GEMVs as ONE cooperative launch, synchronised by dataflow instead of barriers.
//
// Reference counterpart: QwenForward.dispatches encoded on one serial compute encoder
// (Qwen.swift:72-97); every dispatch sees the writes of the ones before it.
//
// Why dataflow: on MI355X a device-wide barrier among 256 resident workgroups costs
// 2.5-4 us (a counter) and agent-scope fences (L2 write-back + invalidate on every XCD)
// cost more still, against 0.2-2.9 us of weight streaming per decode linear.  So:
//   - every op writes its outputs to a plan-owned tagged buffer: one 64-bit word per
//     element, {fp32 value, run epoch}, stored with an agent-scope (device-coherent) store.
//     A 64-bit access is single-copy atomic, so a consumer that reads a word with the
//     current epoch has the value; readiness and data arrive in one memory round trip,
//     with no barrier, no fence and no counter;
//   - a workgroup stages the activations of an op into LDS (fp32) by polling the
//     producer's tagged words, then every lane group reads them from LDS;
//   - the next op's weights are loaded into registers before the workgroup waits for that
//     op's activations, so weight streaming overlaps the dependency wait;
//   - user buffers: an op reads a user buffer only where nothing earlier in the sequence
//     wrote it, and writes a user buffer only if it is the last op writing that region
//     (the host plan compiler resolves both), so every user element is written once per run;
//   - the run epoch lives in the plan's sync area; the last workgroup out increments it,
//     so re-running (or capturing) the plan needs no memset.
// Work split of one op: output features r0..r1 of workgroup g (an even split over the G
// workgroups); a group of L lanes owns one feature and holds up to CHMAX 16-byte chunks of
// its weight row (and of the gate partner) in registers.
// Every wait is bounded: past SPIN_LIMIT polls a lane gives up, sets the plan's timeout
// flag (read by mt_seq_check) and stops waiting for the rest of the run.
#include <stdlib.h>
#include <string.h>

#include "gemv_core.hpp"
#include "mt_internal.hpp"
#include "mingtts_hip.h"

namespace mt {

enum : int { SYNC_EPOCH = 0, SYNC_EXIT = 32, SYNC_TIMEOUT = 64, SYNC_WORDS = 96 };
constexpr int SEQ_THREADS = SEQ_THREADS_N;
constexpr int NWAVE = SEQ_THREADS / 64;
constexpr int CHMAX = SEQ_CHMAX;
constexpr int XLDS = SEQ_XLDS;
constexpr int PART = SEQ_PART;
constexpr int RMAX = SEQ_RMAX;
constexpr int XBATCH = 16;         // activation pairs in flight per thread while staging
constexpr uint32_t SPIN_LIMIT = 1u << 20;

typedef __attribute__((address_space(1))) const uint32_t *g32_cp;
typedef __attribute__((address_space(1))) uint32_t *g32_p;
typedef __attribute__((address_space(1))) const uint64_t *g64_cp;
typedef __attribute__((address_space(1))) const u32x4 *gw_cp;

__device__ __forceinline__ uint32_t ld32(const uint32_t *p) {
    return __hip_atomic_load((g32_cp)(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld64(const uint32_t *p) {
    return __hip_atomic_load((g64_cp)(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Tagged word: the fp32 value with its lowest mantissa bit replaced by the run parity.
__device__ __forceinline__ void st_tag(uint32_t *p, float v, uint32_t parity) {
    __hip_atomic_store((g32_p)(p), (__float_as_uint(v) & ~1u) | parity, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void give_up(uint32_t *sync, bool &gave_up) {
    gave_up = true;
    __hip_atomic_store(sync + SYNC_TIMEOUT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The value a tagged word carries: its lowest mantissa bit cleared, so what a consumer
// computes with does not depend on the run's parity (runs stay bit-identical).
__device__ __forceinline__ float untag(uint32_t v) { return __uint_as_float(v & ~1u); }

// Re-polls a tagged word (bounded) until it carries the run's parity; returns its value.
__device__ __forceinline__ float settle32(const uint32_t *p, uint32_t v, uint32_t parity, uint32_t *sync, bool &gave_up) {
    uint32_t spins = 0;
    while ((v & 1u) != parity && !gave_up) {
        if (++spins > SPIN_LIMIT) { give_up(sync, gave_up); break; }
        __builtin_amdgcn_s_sleep(1);
        v = ld32(p);
    }
    return untag(v);
}
__device__ __forceinline__ uint64_t settle64(const uint32_t *p, uint64_t v, uint32_t parity, uint32_t *sync, bool &gave_up) {
    const uint64_t both = (static_cast<uint64_t>(parity) << 32) | parity;
    uint32_t spins = 0;
    while ((v & 0x100000001ull) != both && !gave_up) {
        if (++spins > SPIN_LIMIT) { give_up(sync, gave_up); break; }
        __builtin_amdgcn_s_sleep(1);
        v = ld64(p);
    }
    return v;
}

template <int WT>
__device__ __forceinline__ float dec(uint16_t h) { return dec1<WT>(h); }

__device__ __forceinline__ float load_ext(const void *x, int xt, size_t off) {
    if (xt == DT_F32) return static_cast<const float *>(x)[off];
    const uint16_t h = static_cast<const uint16_t *>(x)[off];
    return xt == DT_BF16 ? dec1<DT_BF16>(h) : dec1<DT_F16>(h);
}

// One op's share of this workgroup: features r0 .. r0 + nr - 1, and as chunks (16-byte
// weight pieces) the virtual rows 0 .. nr - 1 (w) and, gated, nr .. 2 nr - 1 (w2), KC each.
struct Share {
    uint32_t r0, nr, kc, chunks;
};
__device__ __forceinline__ Share share_of(const SeqOp &o, uint32_t g, uint32_t G) {
    Share s;
    s.r0 = static_cast<uint32_t>(static_cast<uint64_t>(g) * o.N / G);
    s.nr = static_cast<uint32_t>(static_cast<uint64_t>(g + 1) * o.N / G) - s.r0;
    s.kc = o.K >> 3;
    s.chunks = s.nr * s.kc * ((o.flags & F_SILU_GATE) ? 2u : 1u);
    return s;
}

// Chunk f = threadIdx.x + u * 512 of the share into wr[u]: consecutive threads read
// consecutive 16-byte pieces of a weight row.
__device__ __forceinline__ void load_w(const SeqOp &o, const Share &s, u32x4 (&wr)[CHMAX]) {
#pragma unroll
    for (int u = 0; u < CHMAX; u++) {
        const uint32_t f = threadIdx.x + u * SEQ_THREADS;
        if (f < s.chunks) {
            const uint32_t v = f / s.kc, c = f - v * s.kc;
            const bool up = v >= s.nr;
            const uint16_t *w = (up ? o.w2 : o.w) + static_cast<size_t>(s.r0 + (up ? v - s.nr : v)) * o.K;
            wr[u] = __builtin_nontemporal_load((gw_cp)(w) + c);
        }
    }
}

// Staging of op o (whole workgroup): x (times the RMSNorm gain) into xs, the per-wave sums
// of x^2 into ssw, the share's bias into rb and old y (accumulate) into ry -- every global
// read of the op besides its weights, issued as one batch.
template <int MR, int WT>
__device__ __forceinline__ void stage(const SeqOp &o, const SeqOp *__restrict__ ops, const Share &s, float *xs,
                                      float *rb, float *ry, float *ssw, uint32_t parity, uint32_t *sync,
                                      bool &gave_up) {
    const uint32_t K = o.K, M = o.M, tid = threadIdx.x;
    const bool norm = o.norm != nullptr;
    // old y and bias of the share: at most RMAX * MR + RMAX items, one or two per thread
    const bool accum = (o.flags & F_ACCUM) != 0;
    const uint32_t nyo = accum ? s.nr * M : 0;
    uint32_t yw = 0;
    const uint32_t *yp = nullptr;
    if (tid < nyo) {
        const uint32_t r = tid / M, m = tid - r * M;
        if (o.ysrc >= 0) {
            yp = ops[o.ysrc].tag + static_cast<size_t>(m) * ops[o.ysrc].N + o.ycol + s.r0 + r;
            yw = ld32(yp);
        } else {
            ry[r * MR + m] = o.y[static_cast<size_t>(m) * o.ldy + s.r0 + r];
        }
    }
    if (tid < s.nr) rb[tid] = (o.flags & F_BIAS) ? dec<WT>(o.bias[s.r0 + tid]) : 0.0f;

    float ssl[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) ssl[m] = 0.0f;
    auto put = [&](uint32_t e, float x0, float x1) {  // elements e, e + 1 of row e / K
        const uint32_t m = e / K, k = e - m * K;
        if (norm) {
            const uint32_t g2 = *reinterpret_cast<const uint32_t *>(o.norm + k);
#pragma unroll
            for (int mm = 0; mm < MR; mm++)
                if (mm == static_cast<int>(m)) ssl[mm] = fmaf(x1, x1, fmaf(x0, x0, ssl[mm]));
            x0 *= dec_lo<WT>(g2);
            x1 *= dec_hi<WT>(g2);
        }
        *reinterpret_cast<float2 *>(xs + e) = make_float2(x0, x1);
    };
    const uint32_t pairs = M * K / 2;
    if (o.xsrc >= 0) {
        const uint32_t *src = ops[o.xsrc].tag;
        const uint32_t srcN = ops[o.xsrc].N;
        const bool aligned = ((srcN | o.xcol) & 1u) == 0;
        for (uint32_t p0 = tid; p0 < pairs; p0 += XBATCH * SEQ_THREADS) {
            uint64_t v[XBATCH];
#pragma unroll
            for (int b = 0; b < XBATCH; b++) {
                const uint32_t p = p0 + b * SEQ_THREADS;
                if (p < pairs) {
                    const uint32_t e = 2 * p, m = e / K, k = e - m * K;
                    const uint32_t *a = src + static_cast<size_t>(m) * srcN + o.xcol + k;
                    v[b] = aligned ? ld64(a) : (static_cast<uint64_t>(ld32(a + 1)) << 32) | ld32(a);
                }
            }
#pragma unroll
            for (int b = 0; b < XBATCH; b++) {
                const uint32_t p = p0 + b * SEQ_THREADS;
                if (p < pairs) {
                    const uint32_t e = 2 * p, m = e / K, k = e - m * K;
                    const uint32_t *a = src + static_cast<size_t>(m) * srcN + o.xcol + k;
                    uint64_t w = v[b];
                    if (aligned) {
                        w = settle64(a, w, parity, sync, gave_up);
                    } else {
                        const float lo = settle32(a, static_cast<uint32_t>(w), parity, sync, gave_up);
                        const float hi = settle32(a + 1, static_cast<uint32_t>(w >> 32), parity, sync, gave_up);
                        w = (static_cast<uint64_t>(__float_as_uint(hi)) << 32) | __float_as_uint(lo);
                    }
                    put(e, untag(static_cast<uint32_t>(w)), untag(static_cast<uint32_t>(w >> 32)));
                }
            }
        }
    } else {
        for (uint32_t p = tid; p < pairs; p += SEQ_THREADS) {
            const uint32_t e = 2 * p, m = e / K, k = e - m * K;
            const size_t off = static_cast<size_t>(m) * o.ldx + k;
            put(e, load_ext(o.x, o.xt, off), load_ext(o.x, o.xt, off + 1));
        }
    }
    if (yp) ry[(tid / M) * MR + (tid - (tid / M) * M)] = settle32(yp, yw, parity, sync, gave_up);
    if (norm) {
        const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
        for (int m = 0; m < MR; m++) {
            float v = ssl[m];
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
            if (lane == 0) ssw[wave * MR + m] = v;
        }
    }
}

// The chunks' partial dot products into part[m * chunks + f].
template <int MR, int WT>
__device__ __forceinline__ void partials(const SeqOp &o, const Share &s, const float *xs, const u32x4 (&wr)[CHMAX],
                                         float *part) {
    const int M = static_cast<int>(o.M);
#pragma unroll
    for (int u = 0; u < CHMAX; u++) {
        const uint32_t f = threadIdx.x + u * SEQ_THREADS;
        if (f < s.chunks) {
            const uint32_t v = f / s.kc, c = f - v * s.kc;
            float wf[8];
            unpack8<WT>(as_uint4(wr[u]), wf);
#pragma unroll
            for (int m = 0; m < MR; m++) {
                if (m < M) {
                    const float4 *xp = reinterpret_cast<const float4 *>(xs + m * o.K + c * 8);
                    const float4 a = xp[0], b = xp[1];
                    float d = a.x * wf[0];
                    d = fmaf(a.y, wf[1], d);
                    d = fmaf(a.z, wf[2], d);
                    d = fmaf(a.w, wf[3], d);
                    d = fmaf(b.x, wf[4], d);
                    d = fmaf(b.y, wf[5], d);
                    d = fmaf(b.z, wf[6], d);
                    d = fmaf(b.w, wf[7], d);
                    part[m * s.chunks + f] = d;
                }
            }
        }
    }
}

// DPP lane moves (no LDS round trip): v from another lane of the same 16-lane row.
template <int CTRL, bool BOUND_ZERO>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF,
                                                                 BOUND_ZERO));
}

// Sum over aligned groups of 2^lg lanes (lg 3..6).  lg == 3: the group's lanes 4..7 hold
// the total; lg >= 4: every lane of the group does.  The order is fixed.
__device__ __forceinline__ float group_total(float v, int lg) {
    v += dpp<0xB1, false>(v);  // quad_perm [1,0,3,2]
    v += dpp<0x4E, false>(v);  // quad_perm [2,3,0,1]: every lane holds its quad's sum
    if (lg == 3) return v + dpp<0x114, true>(v);  // row_shr:4 -> lanes 4..7 of each 8
    v += dpp<0x124, false>(v);                    // row_ror:4
    v += dpp<0x128, false>(v);                    // row_ror:8 -> the 16-lane row's sum
    if (lg >= 5) v += __shfl_xor(v, 16, 64);
    if (lg >= 6) v += __shfl_xor(v, 32, 64);
    return v;
}

// Feature sums and the epilogue, all of the share's features at once: 2^lg lanes per
// feature (as many as fit in the workgroup, 8..64) add its chunks' partials in a fixed
// lane-strided order, then a fixed group reduction; the group's last lane stores the
// tagged output (and the user output when this op writes its region last).
template <int MR, int WT>
__device__ __forceinline__ void finish(const SeqOp &o, const Share &s, const float *part, const float *rb,
                                       const float *ry, const float *ssw, uint32_t parity) {
    const int M = static_cast<int>(o.M);
    const bool gated = (o.flags & F_SILU_GATE) != 0;
    int lg = 3;
    while (lg < 6 && (s.nr << (lg + 1)) <= static_cast<uint32_t>(SEQ_THREADS)) lg++;
    const uint32_t r = threadIdx.x >> lg;
    const uint32_t q = threadIdx.x & ((1u << lg) - 1);
    const bool live = r < s.nr;
    float a[MR], a2[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) {
        a[m] = 0.0f;
        a2[m] = 0.0f;
        if (live && m < M) {
            const float *p = part + m * s.chunks + r * s.kc;
            const float *p2 = p + s.nr * s.kc;
            for (uint32_t c = q; c < s.kc; c += (1u << lg)) {
                a[m] += p[c];
                if (gated) a2[m] += p2[c];
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; m++) {
        if (m < M) {  // M is uniform: every lane of the wave takes part in the lane moves
            a[m] = group_total(a[m], lg);
            if (gated) a2[m] = group_total(a2[m], lg);
        }
    }
    if (live && q == (1u << lg) - 1) {
        const uint32_t n = s.r0 + r;
#pragma unroll
        for (int m = 0; m < MR; m++) {
            if (m < M) {
                float scale = 1.0f;
                if (o.norm) {
                    float t = 0.0f;
#pragma unroll
                    for (int w = 0; w < NWAVE; w++) t += ssw[w * MR + m];
                    scale = 1.0f / sqrtf(t / static_cast<float>(o.K) + o.eps);
                }
                float v = epilogue(a[m] * scale, a2[m] * scale, rb[r], o.flags);
                if (o.flags & F_ACCUM) v += ry[r * MR + m];
                st_tag(o.tag + static_cast<size_t>(m) * o.N + n, v, parity);
                if (o.final_out) o.y[static_cast<size_t>(m) * o.ldy + n] = v;
            }
        }
    }
}

// One 512-thread workgroup per CU.  Per op: stage (one batch of global reads), barrier,
// partial dots from the prefetched weight chunks, barrier, feature sums and stores, then
// the next op's weight chunks are requested before its staging waits.  Activations,
// bias, old y and sums of squares alternate between two LDS buffers by op parity: a wave
// past op i's first barrier has finished op i - 1, so staging op i + 1 never overwrites
// what a slower wave still reads; the partials buffer is written only after op i + 1's
// first barrier.
template <int MR, int WT>
__global__ __launch_bounds__(SEQ_THREADS) void seq_kernel(const SeqOp *__restrict__ ops, uint32_t n_ops,
                                                         uint32_t *sync) {
    __shared__ __attribute__((aligned(16))) float xs[2][XLDS];
    __shared__ __attribute__((aligned(16))) float part[PART];
    __shared__ float rb[2][RMAX];
    __shared__ float ry[2][RMAX * MR];
    __shared__ float ssw[2][NWAVE * MR];
    const uint32_t G = gridDim.x, g = blockIdx.x;
    const uint32_t epoch = __hip_atomic_load(sync + SYNC_EPOCH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t parity = epoch & 1u;
    bool gave_up = false;
    u32x4 wr[CHMAX];

    if (n_ops > 0) {
        const SeqOp o = ops[0];
        load_w(o, share_of(o, g, G), wr);
    }
    for (uint32_t i = 0; i < n_ops; i++) {
        const SeqOp o = ops[i];
        const Share s = share_of(o, g, G);
        const int b = i & 1;
        stage<MR, WT>(o, ops, s, xs[b], rb[b], ry[b], ssw[b], parity, sync, gave_up);
        __syncthreads();
        partials<MR, WT>(o, s, xs[b], wr, part);
        __syncthreads();
        finish<MR, WT>(o, s, part, rb[b], ry[b], ssw[b], parity);
        if (i + 1 < n_ops) {
            const SeqOp on = ops[i + 1];
            load_w(on, share_of(on, g, G), wr);
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

typedef void (*seq_fn)(const SeqOp *, uint32_t, uint32_t *);

namespace {

template <int MR>
seq_fn pick_w(int wt) { return wt == DT_BF16 ? seq_kernel<MR, DT_BF16> : seq_kernel<MR, DT_F16>; }

seq_fn pick(int mr, int wt) {
    switch (mr) {
        case 1: return pick_w<1>(wt);
        case 2: return pick_w<2>(wt);
        case 4: return pick_w<4>(wt);
        default: return pick_w<8>(wt);
    }
}

}  // namespace

struct SeqPlan {
    SeqOp *d_ops = nullptr;
    uint32_t *d_sync = nullptr;
    uint32_t *d_tags = nullptr;
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
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(seq_kernel<8, DT_F16>),
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

int seq_create(SeqOp *ops, uint32_t n_ops, int mr, int wt, int groups, SeqPlan **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(MT_EHIP, "mt_seq_create: hipGetDevice: %s", hipGetErrorString(e));
    SeqPlan *p = new SeqPlan();
    p->n_ops = n_ops;
    p->device = dev;
    p->fn = pick(mr, wt);
    p->groups = groups;
    // Each op's tagged output starts 16-byte aligned (pairs of words are read as one).
    size_t tag_words = 0;
    for (uint32_t i = 0; i < n_ops; i++) tag_words += (static_cast<size_t>(ops[i].M) * ops[i].N + 3) & ~size_t(3);
    e = hipMalloc(&p->d_ops, sizeof(SeqOp) * (n_ops ? n_ops : 1));
    if (e == hipSuccess) e = hipMalloc(&p->d_sync, SYNC_WORDS * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&p->d_tags, sizeof(uint32_t) * (tag_words ? tag_words : 1));
    if (e == hipSuccess) {
        size_t off = 0;
        for (uint32_t i = 0; i < n_ops; i++) {
            ops[i].tag = p->d_tags + off;
            off += (static_cast<size_t>(ops[i].M) * ops[i].N + 3) & ~size_t(3);
        }
        e = hipMemcpy(p->d_ops, ops, sizeof(SeqOp) * n_ops, hipMemcpyHostToDevice);
    }
    // Tagged words start with parity 0 and the first run uses epoch 1 (parity 1), so no
    // stale word can pass for a current one.
    if (e == hipSuccess) e = hipMemset(p->d_tags, 0, sizeof(uint32_t) * (tag_words ? tag_words : 1));
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
    void *args[] = {&p->d_ops, &p->n_ops, &p->d_sync};
    hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void *>(p->fn), dim3(p->groups),
                                              dim3(SEQ_THREADS), args, 0, stream);
    if (e != hipSuccess) return set_error(MT_EHIP, "mt_seq_run: cooperative launch: %s", hipGetErrorString(e));
    return MT_OK;
}

int seq_check(SeqPlan *p) {
    uint32_t flag = 0;
    hipError_t e = hipMemcpy(&flag, p->d_sync + SYNC_TIMEOUT, sizeof(flag), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return set_error(MT_EHIP, "mt_seq_check: %s", hipGetErrorString(e));
    if (flag) return set_error(MT_EHIP, "mt_seq_check: a dataflow wait exceeded its spin bound");
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
