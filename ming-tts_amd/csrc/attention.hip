// NeoX RoPE + KV-cache append, and causal GQA attention over the cache.
//
// Reference kernels replaced: rope_cache (Shaders.swift:451-486) and attention_cache<SPLIT>
// (Shaders.swift:490-596).  Same arithmetic (fp32 scores, scale after the q.k dot,
// max-subtracted softmax, fp32 p.v), caches of fp32 (reference) or fp16 (decode config).
//
// Attention layout on gfx950: one 256-thread workgroup per (query row, head) item.
//   - scores: groups of 8 lanes own one key (lane r of a group reads dims 8r..8r+7, so a
//     wave reads 8 whole key rows per load instruction), 32 keys per pass, sixteen passes'
//     keys requested before any is used (a decode step's keys, up to 512, in one round trip),
//     the 8 partial dots meet on DPP; scores land in LDS (at most 4096 keys);
//   - softmax: block max and block sum through LDS;
//   - p.v: 16 lanes cover the 64 dims of one V row (4 dims each, one coalesced row per
//     16 lanes), 16 key phases per workgroup, 32 rows per lane requested at a time,
//     partial sums meet in LDS in a fixed order.
// Batched decode (mt_attention_decode) is the same kernel with a per-row cache base and
// the row's query position read from a device array.
#include "mt_device.hpp"
#include "mt_internal.hpp"
#include "mingtts_hip.h"

namespace mt {

namespace {

constexpr int ATT_THREADS = 256;
constexpr int ATT_MAXKEYS = 4096;

template <int CT>
__device__ __forceinline__ float4 load4(const void *base, size_t off) {
    if constexpr (CT == DT_F32) {
        return *reinterpret_cast<const float4 *>(static_cast<const float *>(base) + off);
    } else {
        const uint2 v = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(base) + off);
        return make_float4(dec_lo<CT>(v.x), dec_hi<CT>(v.x), dec_lo<CT>(v.y), dec_hi<CT>(v.y));
    }
}

template <int CT>
__device__ __forceinline__ void store1(void *base, size_t off, float v) {
    if constexpr (CT == DT_F32) static_cast<float *>(base)[off] = v;
    else static_cast<_Float16 *>(base)[off] = static_cast<_Float16>(v);
}

// One 256-thread workgroup per row: lane t & 31 is the rotation pair i, and the eight groups
// of 32 lanes take the row's head slots (hq query heads, hkv key heads, hkv value heads) in
// turn, so a lane forms cos and sin of its pair's angle (pos * inv_freq[i]) once for all the
// heads it rotates, and each group reads and writes a head's 64 words in two coalesced
// 128-byte halves.
template <int CT>
__global__ __launch_bounds__(256) void rope_cache_kernel(float *qkv, uint32_t ldq, uint32_t hq, uint32_t hkv,
                                                         uint32_t pos0, const uint32_t *pos_arr, void *kc,
                                                         void *vc, uint32_t cache_len, uint64_t cache_stride,
                                                         const float *inv_freq) {
    const uint32_t i = threadIdx.x & 31, grp = threadIdx.x >> 5;
    const uint32_t m = blockIdx.x;
    const uint32_t pos = pos_arr ? pos_arr[m] : pos0 + m;
    const uint64_t cbase = pos_arr ? static_cast<uint64_t>(m) * cache_stride : 0;
    // A device-side position past the cache (only possible through pos_arr, which the host
    // cannot see) appends nothing; the query heads are still rotated.
    const bool append = pos < cache_len;
    float *row = qkv + static_cast<size_t>(m) * ldq;
    // The group's first RC_SLOTS slots are requested together (clamped to the row's last slot,
    // so every load stays in the row) before the angle's cosine and sine are computed, then
    // rotated and stored: one load round trip, overlapping the trigonometry, for the 18 slots
    // of a Qwen2-0.5B row instead of one per slot.
    constexpr uint32_t RC_SLOTS = 3;
    const uint32_t nslot = hq + 2 * hkv;
    float x0s[RC_SLOTS], x1s[RC_SLOTS];
#pragma unroll
    for (uint32_t u = 0; u < RC_SLOTS; u++) {
        const uint32_t sl = min(grp + 8 * u, nslot - 1);
        x0s[u] = row[sl * 64 + i];
        x1s[u] = row[sl * 64 + i + 32];
    }
    const float angle = static_cast<float>(pos) * inv_freq[i];
    const float c = cosf(angle), s = sinf(angle);
    for (uint32_t slot = grp, u = 0; slot < nslot; slot += 8, u++) {
        const float x0 = u < RC_SLOTS ? x0s[u] : row[slot * 64 + i];
        const float x1 = u < RC_SLOTS ? x1s[u] : row[slot * 64 + i + 32];
        float r0, r1;
        rope_rotate(x0, x1, c, s, r0, r1);
        if (slot < hq) {
            row[slot * 64 + i] = r0;
            row[slot * 64 + i + 32] = r1;
        } else if (!append) {
            continue;
        } else if (slot < hq + hkv) {
            const size_t dst = cbase + (static_cast<size_t>(slot - hq) * cache_len + pos) * 64;
            store1<CT>(kc, dst + i, r0);
            store1<CT>(kc, dst + i + 32, r1);
        } else {
            const size_t dst = cbase + (static_cast<size_t>(slot - hq - hkv) * cache_len + pos) * 64;
            store1<CT>(vc, dst + i, x0);
            store1<CT>(vc, dst + i + 32, x1);
        }
    }
}

// Max / sum over the 64 lanes, the same bits in every lane: quad swaps and the half-row and
// row mirrors on DPP (rows of 16), then two exchanges between rows.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    v = fmaxf(v, dpp_mov<0x140>(v));
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    return fmaxf(v, __shfl_xor(v, 32, 64));
}
__device__ __forceinline__ float wave_sum(float v) { return group_sum(v, 64); }

// The 16-byte raw loads of eight cached values (one of fp16, two of fp32) and their decode.
template <int CT>
struct Raw8 {
    uint4 a, b;
};
template <int CT>
__device__ __forceinline__ Raw8<CT> load8_raw(const void *base, size_t off) {
    Raw8<CT> r;
    if constexpr (CT == DT_F32) {
        const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const float *>(base) + off);
        r.a = p[0];
        r.b = p[1];
    } else {
        r.a = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(base) + off);
        r.b = make_uint4(0u, 0u, 0u, 0u);
    }
    return r;
}
template <int CT>
__device__ __forceinline__ void decode8(const Raw8<CT> &r, float *o) {
    if constexpr (CT == DT_F32) {
        o[0] = __uint_as_float(r.a.x); o[1] = __uint_as_float(r.a.y); o[2] = __uint_as_float(r.a.z); o[3] = __uint_as_float(r.a.w);
        o[4] = __uint_as_float(r.b.x); o[5] = __uint_as_float(r.b.y); o[6] = __uint_as_float(r.b.z); o[7] = __uint_as_float(r.b.w);
    } else {
        unpack8<CT>(r.a, o);
    }
}

template <int CT>
__global__ __launch_bounds__(ATT_THREADS) void attention_kernel(const float *q, uint32_t ldq, uint32_t hq,
                                                                uint32_t hkv, uint32_t pos0, const uint32_t *lens,
                                                                uint32_t window, const void *kc, const void *vc,
                                                                uint32_t cache_len, uint64_t cache_stride,
                                                                float *out, uint32_t ldo, float scale) {
    __shared__ float sc[ATT_MAXKEYS];
    __shared__ float red[ATT_THREADS / 64];
    __shared__ float4 part[16][16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t m = blockIdx.x / hq, h = blockIdx.x % hq;
    const uint32_t kvh = h / (hq / hkv);
    // Device-side lengths are clamped to the cache; a zero length attends to nothing and
    // writes zeros.
    const uint32_t len = lens ? min(lens[m], cache_len) : pos0 + m + 1;
    const uint64_t cbase = lens ? static_cast<uint64_t>(m) * cache_stride : 0;
    const uint32_t jEnd = len;
    const uint32_t jStart = (window > 0 && jEnd > window) ? jEnd - window : 0;
    const int nk = static_cast<int>(jEnd - jStart);
    const size_t kvbase = cbase + (static_cast<size_t>(kvh) * cache_len + jStart) * 64;

    // Scores.
    const int r = tid & 7;
    float qf[8];
    {
        const float4 *qp = reinterpret_cast<const float4 *>(q + static_cast<size_t>(m) * ldq + h * 64 + 8 * r);
        const float4 a = qp[0], b = qp[1];
        qf[0] = a.x; qf[1] = a.y; qf[2] = a.z; qf[3] = a.w;
        qf[4] = b.x; qf[5] = b.y; qf[6] = b.z; qf[7] = b.w;
    }
    // Sixteen passes of 32 keys per round, all requested before any is used (keys past the
    // end re-read the last key and are skipped).
    float mx = -INFINITY;
    constexpr int KP = ATT_THREADS / 8, KU = 16;
    for (int t0 = tid >> 3; t0 < nk; t0 += KU * KP) {
        Raw8<CT> kr[KU];
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int t = min(t0 + u * KP, nk - 1);
            kr[u] = load8_raw<CT>(kc, kvbase + static_cast<size_t>(t) * 64 + 8 * r);
        }
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int t = t0 + u * KP;
            if (t < nk) {  // the 8 lanes of a key agree
                float kf[8];
                decode8<CT>(kr[u], kf);
                float s = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) s = fmaf(qf[e], kf[e], s);
                s = octet_sum(s);
                s *= scale;
                if (r == 0) sc[t] = s;
                mx = fmaxf(mx, s);
            }
        }
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();

    // Softmax numerators and their sum.
    float sum = 0.0f;
    for (int t = tid; t < nk; t += ATT_THREADS) {
        const float e = exp_hw(sc[t] - mx);
        sc[t] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    sum = (red[0] + red[1]) + (red[2] + red[3]);

    // p . v: 16 lanes per V row (4 dims each), 16 key phases, keys t = ks, ks + 16, ... in
    // order; 32 rows per round requested before any is used (rows past the end re-read
    // the last row and are skipped).
    const int d4 = tid & 15, ks = tid >> 4;
    constexpr int VU = 32;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int t0 = ks; t0 < nk; t0 += 16 * VU) {
        float4 v[VU];
#pragma unroll
        for (int u = 0; u < VU; u++)
            v[u] = load4<CT>(vc, kvbase + static_cast<size_t>(min(t0 + 16 * u, nk - 1)) * 64 + 4 * d4);
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const int t = t0 + 16 * u;
            if (t < nk) {
                const float p = sc[t];
                acc.x = fmaf(p, v[u].x, acc.x);
                acc.y = fmaf(p, v[u].y, acc.y);
                acc.z = fmaf(p, v[u].z, acc.z);
                acc.w = fmaf(p, v[u].w, acc.w);
            }
        }
    }
    part[ks][d4] = acc;
    __syncthreads();
    if (tid < 16) {
        float4 o = part[0][tid];
        for (int k = 1; k < 16; k++) {
            const float4 pp = part[k][tid];
            o.x += pp.x; o.y += pp.y; o.z += pp.z; o.w += pp.w;
        }
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        float4 res = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
        *reinterpret_cast<float4 *>(out + static_cast<size_t>(m) * ldo + h * 64 + 4 * tid) = res;
    }
}

// attention_kernel's arithmetic for R consecutive rows of one sequence at a time, for rows whose
// keys all start at position 0 (no window, or a window longer than every row's span): one
// 256-thread workgroup per (head, block of R rows), so a block's keys and values are read
// once for R rows, and the values' first loads are in flight during the softmax.  Every
// value is the row kernel's, bit for bit:
//   - scores: lane r8 of an octet holds dims 8 r8 .. 8 r8 + 7 of all R queries, the octet one
//     key; the same eight chains and octet_sum per (row, key), then the scale;
//   - sum: thread t holds keys t, t + 256, ... of each row in order, then the 64-lane tree
//     and the (w0 + w1) + (w2 + w3) join of the four waves, as the row kernel's 256 threads;
//   - p.v: thread (ks, d4) folds keys ks, ks + 16, ... of each row in order, and the 16
//     phases meet in phase order.
// A block's scores live in LDS as sc[key][row]; the phases' partial sums reuse that space.
constexpr int AR_ROWS = 4;
constexpr int AR_MAXKEYS = 1024;  // pos0 + rows the row-block kernel takes
constexpr uint32_t AR_MIN_ROWS = 8;  // fewer rows go row by row

// The raw load of four cached values (16 bytes of fp32, 8 of fp16) and their decode.
template <int CT>
struct Raw4 {
    uint4 a;  // fp16: a.x, a.y
};
template <int CT>
__device__ __forceinline__ Raw4<CT> load4_raw(const void *base, size_t off) {
    Raw4<CT> r;
    if constexpr (CT == DT_F32) {
        r.a = *reinterpret_cast<const uint4 *>(static_cast<const float *>(base) + off);
    } else {
        const uint2 v = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(base) + off);
        r.a = make_uint4(v.x, v.y, 0u, 0u);
    }
    return r;
}
template <int CT>
__device__ __forceinline__ float4 decode4(const Raw4<CT> &r) {
    if constexpr (CT == DT_F32)
        return make_float4(__uint_as_float(r.a.x), __uint_as_float(r.a.y), __uint_as_float(r.a.z),
                           __uint_as_float(r.a.w));
    else
        return make_float4(dec_lo<CT>(r.a.x), dec_hi<CT>(r.a.x), dec_lo<CT>(r.a.y), dec_hi<CT>(r.a.y));
}

template <int CT, int R>
__global__ __launch_bounds__(ATT_THREADS) void attention_rows_kernel(const float *q, uint32_t ldq, uint32_t hq,
                                                                     uint32_t hkv, uint32_t pos0, uint32_t rows,
                                                                     const void *kc, const void *vc,
                                                                     uint32_t cache_len, float *out, uint32_t ldo,
                                                                     float scale) {
    static_assert(R == 2 || R == 4 || R == 8, "a key's R scores move as whole 8- or 16-byte words");
    __shared__ __attribute__((aligned(16))) float sc[AR_MAXKEYS * R];  // sc[key * R + row]
    __shared__ float red[R][ATT_THREADS / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t h = blockIdx.x, kvh = h / (hq / hkv);
    const uint32_t m0 = (gridDim.y - 1 - blockIdx.y) * R;  // the longest rows first
    const int rn = min(R, static_cast<int>(rows - m0));
    const int p0 = static_cast<int>(pos0 + m0);  // row r attends keys 0 .. p0 + r
    const int nk = p0 + rn;
    const size_t kvbase = static_cast<size_t>(kvh) * cache_len * 64;

    // The R queries' dims 8 r8 .. 8 r8 + 7 in registers (rows past the end repeat the last
    // row and are never stored).
    const int r8 = tid & 7;
    float qf[R][8];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float4 *qp = reinterpret_cast<const float4 *>(q + static_cast<size_t>(m0 + min(r, rn - 1)) * ldq +
                                                            h * 64 + 8 * r8);
        const float4 a = qp[0], b = qp[1];
        qf[r][0] = a.x; qf[r][1] = a.y; qf[r][2] = a.z; qf[r][3] = a.w;
        qf[r][4] = b.x; qf[r][5] = b.y; qf[r][6] = b.z; qf[r][7] = b.w;
    }

    // Scores: 32 keys per pass, eight passes' keys requested before any is used.  A key up to
    // p0 belongs to every row; keys p0 + 1 .. nk - 1 only to the rows they precede.
    float mx[R];
#pragma unroll
    for (int r = 0; r < R; r++) mx[r] = -INFINITY;
    constexpr int KP = ATT_THREADS / 8, KU = 8;
    for (int t0 = tid >> 3; t0 < nk; t0 += KU * KP) {
        Raw8<CT> kr[KU];
#pragma unroll
        for (int u = 0; u < KU; u++)
            kr[u] = load8_raw<CT>(kc, kvbase + static_cast<size_t>(min(t0 + u * KP, nk - 1)) * 64 + 8 * r8);
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int t = t0 + u * KP;
            if (t < nk) {  // the 8 lanes of a key agree
                float kf[8];
                decode8<CT>(kr[u], kf);
                float s[R];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    float a = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; e++) a = fmaf(qf[r][e], kf[e], a);
                    s[r] = a;
                }
                octet_sums<R>(s);
#pragma unroll
                for (int r = 0; r < R; r++) s[r] *= scale;
                if (r8 == 0) {
#pragma unroll
                    for (int r = 0; r < R; r++) sc[t * R + r] = s[r];
                }
                if (t <= p0) {
#pragma unroll
                    for (int r = 0; r < R; r++) mx[r] = fmaxf(mx[r], s[r]);
                } else {
#pragma unroll
                    for (int r = 0; r < R; r++)
                        if (t <= p0 + r) mx[r] = fmaxf(mx[r], s[r]);
                }
            }
        }
        // Every key load of this round done (a skipped pass leaves its load outstanding), so
        // the next round's address arithmetic waits for nothing.
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    // p . v's first VU keys of this thread's phase, requested now (after the keys, so no
    // score waits for them), used after the softmax (keys past the end re-read the last key).
    // Few at a time: requested before the scores, or 8-16 at a time, they made the kernel
    // slower (16 ahead of the keys: 7.9 against 7.0 us at 174 rows).
    const int d4 = tid & 15, ks = tid >> 4;
    constexpr int VU = 4;
    Raw4<CT> vr[VU];
#pragma unroll
    for (int u = 0; u < VU; u++)
        vr[u] = load4_raw<CT>(vc, kvbase + static_cast<size_t>(min(ks + 16 * u, nk - 1)) * 64 + 4 * d4);
#pragma unroll
    for (int r = 0; r < R; r++) mx[r] = wave_max(mx[r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; r++) red[r][wave] = mx[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; r++) mx[r] = fmaxf(fmaxf(red[r][0], red[r][1]), fmaxf(red[r][2], red[r][3]));
    __syncthreads();

    // Softmax numerators (a row's keys past its end hold 0) and the rows' sums.
    float sum[R];
#pragma unroll
    for (int r = 0; r < R; r++) sum[r] = 0.0f;
    for (int t = tid; t < nk; t += ATT_THREADS) {
        float s[R];
#pragma unroll
        for (int r = 0; r < R; r++) s[r] = sc[t * R + r];
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (t <= p0 + r) {
                s[r] = exp_hw(s[r] - mx[r]);
                sum[r] += s[r];
            } else {
                s[r] = 0.0f;
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) sc[t * R + r] = s[r];
    }
#pragma unroll
    for (int r = 0; r < R; r++) sum[r] = wave_sum(sum[r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; r++) red[r][wave] = sum[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; r++) sum[r] = (red[r][0] + red[r][1]) + (red[r][2] + red[r][3]);

    // p . v: 16 lanes per V row (4 dims each), 16 key phases.
    float4 acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int t0 = ks; t0 < nk; t0 += 16 * VU) {
        if (t0 != ks) {
#pragma unroll
            for (int u = 0; u < VU; u++)
                vr[u] = load4_raw<CT>(vc, kvbase + static_cast<size_t>(min(t0 + 16 * u, nk - 1)) * 64 + 4 * d4);
        }
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const int t = t0 + 16 * u;
            if (t < nk) {
                const float4 v = decode4<CT>(vr[u]);
                float p[R];
#pragma unroll
                for (int r = 0; r < R; r++) p[r] = sc[t * R + r];
                if (t <= p0) {
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        acc[r].x = fmaf(p[r], v.x, acc[r].x);
                        acc[r].y = fmaf(p[r], v.y, acc[r].y);
                        acc[r].z = fmaf(p[r], v.z, acc[r].z);
                        acc[r].w = fmaf(p[r], v.w, acc[r].w);
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        if (t <= p0 + r) {
                            acc[r].x = fmaf(p[r], v.x, acc[r].x);
                            acc[r].y = fmaf(p[r], v.y, acc[r].y);
                            acc[r].z = fmaf(p[r], v.z, acc[r].z);
                            acc[r].w = fmaf(p[r], v.w, acc[r].w);
                        }
                    }
                }
            }
        }
    }
    __syncthreads();  // every probability read; the phases' sums take sc's space
    float4 *part = reinterpret_cast<float4 *>(sc);  // part[(ks * 16 + d4) * R + r]
#pragma unroll
    for (int r = 0; r < R; r++) part[(ks * 16 + d4) * R + r] = acc[r];
    __syncthreads();
    if (tid < 16 * R) {
        const int dd = tid & 15, r = tid >> 4;
        if (r < rn) {
            float s = sum[0];
#pragma unroll
            for (int rr = 1; rr < R; rr++)
                if (r == rr) s = sum[rr];
            float4 o = part[dd * R + r];
            for (int k = 1; k < 16; k++) {
                const float4 pp = part[(k * 16 + dd) * R + r];
                o.x += pp.x; o.y += pp.y; o.z += pp.z; o.w += pp.w;
            }
            const float inv = s > 0.0f ? 1.0f / s : 0.0f;
            const float4 res = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
            *reinterpret_cast<float4 *>(out + static_cast<size_t>(m0 + r) * ldo + h * 64 + 4 * dd) = res;
        }
    }
}

// rope_cache then attention over one sequence's M new rows (positions pos0 .. pos0 + M - 1),
// in one launch: workgroup (row m, head h) rotates its q (and writes it back to qkv), appends
// row m's rotated k and raw v of kv head h / (hq / hkv) to the caches when h is the first head
// of its group, and attends over keys [max(0, pos0 + m + 1 - window), pos0 + m].  Keys before
// pos0 come from the cache; the chunk's own rows (pos0 ..) are rebuilt from qkv in LDS,
// rounded to the cache type as the cache holds them, so no workgroup reads a cache row that
// another is writing.  Every value, and every summation order, is attention_kernel's.
constexpr int RA_MAXROWS = 64;
template <int CT>
__global__ __launch_bounds__(ATT_THREADS) void rope_attention_kernel(float *qkv, uint32_t ldq, uint32_t hq, uint32_t hkv,
                                                                     uint32_t pos0, uint32_t window, void *kc, void *vc,
                                                                     uint32_t cache_len, const float *inv_freq, float *out,
                                                                     uint32_t ldo, float scale) {
    __shared__ float sc[ATT_MAXKEYS];
    __shared__ float red[ATT_THREADS / 64];
    __shared__ float4 part[16][16];
    __shared__ __attribute__((aligned(16))) float qs[64];
    __shared__ __attribute__((aligned(16))) float ck[RA_MAXROWS][64];
    __shared__ __attribute__((aligned(16))) float cv[RA_MAXROWS][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t m = blockIdx.x / hq, h = blockIdx.x % hq;
    const uint32_t group = hq / hkv, kvh = h / group;
    const uint32_t jEnd = pos0 + m + 1;
    const uint32_t jStart = (window > 0 && jEnd > window) ? jEnd - window : 0;
    const int nk = static_cast<int>(jEnd - jStart);
    const uint32_t c0 = jStart > pos0 ? jStart - pos0 : 0u;  // first chunk row attended
    const int nc = jStart < pos0 ? static_cast<int>(pos0 - jStart) : 0;  // keys from the cache
    const size_t kvbase = (static_cast<size_t>(kvh) * cache_len + jStart) * 64;

    // The rotations (rope_cache_kernel's arithmetic): q of (m, h), and k, v of kv head kvh
    // for chunk rows c0 .. m; row m's k and v also go to the caches (first head of the group).
    if (tid < 32) {
        const uint32_t i = tid;
        const float angle = static_cast<float>(pos0 + m) * inv_freq[i];
        const float c = cosf(angle), sn = sinf(angle);
        float *row = qkv + static_cast<size_t>(m) * ldq + static_cast<size_t>(h) * 64;
        const float x0 = row[i], x1 = row[i + 32];
        float r0, r1;
        rope_rotate(x0, x1, c, sn, r0, r1);
        row[i] = r0;
        row[i + 32] = r1;
        qs[i] = r0;
        qs[i + 32] = r1;
    }
    for (uint32_t e = tid; e < (m + 1 - c0) * 32; e += ATT_THREADS) {
        const uint32_t rr = c0 + e / 32, i = e % 32, pos = pos0 + rr;
        const float *row = qkv + static_cast<size_t>(rr) * ldq + static_cast<size_t>(hq + kvh) * 64;
        const float angle = static_cast<float>(pos) * inv_freq[i];
        const float c = cosf(angle), sn = sinf(angle);
        const float x0 = row[i], x1 = row[i + 32];
        float r0, r1;
        rope_rotate(x0, x1, c, sn, r0, r1);
        const float *vrow = row + static_cast<size_t>(hkv) * 64;
        float k0 = r0, k1 = r1, v0 = vrow[i], v1 = vrow[i + 32];
        if constexpr (CT == DT_F16) {  // as the fp16 cache holds them
            k0 = static_cast<float>(static_cast<_Float16>(k0));
            k1 = static_cast<float>(static_cast<_Float16>(k1));
            v0 = static_cast<float>(static_cast<_Float16>(v0));
            v1 = static_cast<float>(static_cast<_Float16>(v1));
        }
        ck[rr][i] = k0;
        ck[rr][i + 32] = k1;
        cv[rr][i] = v0;
        cv[rr][i + 32] = v1;
        if (rr == m && h % group == 0) {
            const size_t dst = (static_cast<size_t>(kvh) * cache_len + pos) * 64;
            store1<CT>(kc, dst + i, r0);
            store1<CT>(kc, dst + i + 32, r1);
            store1<CT>(vc, dst + i, vrow[i]);
            store1<CT>(vc, dst + i + 32, vrow[i + 32]);
        }
    }
    __syncthreads();

    // Scores: the cache's keys in rounds of sixteen passes, then the chunk's keys from LDS.
    const int r = tid & 7;
    float qf[8];
#pragma unroll
    for (int e = 0; e < 8; e++) qf[e] = qs[8 * r + e];
    float mx = -INFINITY;
    constexpr int KP = ATT_THREADS / 8, KU = 16;
    for (int t0 = tid >> 3; t0 < nc; t0 += KU * KP) {
        Raw8<CT> kr[KU];
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int t = min(t0 + u * KP, nc - 1);
            kr[u] = load8_raw<CT>(kc, kvbase + static_cast<size_t>(t) * 64 + 8 * r);
        }
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int t = t0 + u * KP;
            if (t < nc) {
                float kf[8];
                decode8<CT>(kr[u], kf);
                float s = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) s = fmaf(qf[e], kf[e], s);
                s = octet_sum(s);
                s *= scale;
                if (r == 0) sc[t] = s;
                mx = fmaxf(mx, s);
            }
        }
    }
    for (int t = nc + (((tid >> 3) - nc) % KP + KP) % KP; t < nk; t += KP) {
        const float *kf = &ck[c0 + (t - nc)][8 * r];
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) s = fmaf(qf[e], kf[e], s);
        s = octet_sum(s);
        s *= scale;
        if (r == 0) sc[t] = s;
        mx = fmaxf(mx, s);
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();

    float sum = 0.0f;
    for (int t = tid; t < nk; t += ATT_THREADS) {
        const float e = exp_hw(sc[t] - mx);
        sc[t] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    sum = (red[0] + red[1]) + (red[2] + red[3]);

    // p . v in attention_kernel's order (keys ks, ks + 16, ... of each phase).
    const int d4 = tid & 15, ks = tid >> 4;
    constexpr int VU = 32;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int t0 = ks; t0 < nk; t0 += 16 * VU) {
        float4 v[VU];
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const int t = t0 + 16 * u;
            v[u] = t < nc ? load4<CT>(vc, kvbase + static_cast<size_t>(t) * 64 + 4 * d4)
                          : *reinterpret_cast<const float4 *>(&cv[c0 + (t < nk ? t - nc : 0)][4 * d4]);
        }
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const int t = t0 + 16 * u;
            if (t < nk) {
                const float p = sc[t];
                acc.x = fmaf(p, v[u].x, acc.x);
                acc.y = fmaf(p, v[u].y, acc.y);
                acc.z = fmaf(p, v[u].z, acc.z);
                acc.w = fmaf(p, v[u].w, acc.w);
            }
        }
    }
    part[ks][d4] = acc;
    __syncthreads();
    if (tid < 16) {
        float4 o = part[0][tid];
        for (int k = 1; k < 16; k++) {
            const float4 pp = part[k][tid];
            o.x += pp.x; o.y += pp.y; o.z += pp.z; o.w += pp.w;
        }
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        float4 res = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
        *reinterpret_cast<float4 *>(out + static_cast<size_t>(m) * ldo + h * 64 + 4 * tid) = res;
    }
}

}  // namespace

int launch_rope_attention(float *qkv, uint32_t ldq, uint32_t rows, uint32_t hq, uint32_t hkv, uint32_t pos0,
                          uint32_t window, void *kc, void *vc, int ct, uint32_t cache_len, const float *inv_freq,
                          float *out, uint32_t ldo, float scale, hipStream_t stream) {
    dim3 grid(rows * hq);
    if (ct == DT_F32)
        hipLaunchKernelGGL(rope_attention_kernel<DT_F32>, grid, dim3(ATT_THREADS), 0, stream, qkv, ldq, hq, hkv, pos0,
                           window, kc, vc, cache_len, inv_freq, out, ldo, scale);
    else
        hipLaunchKernelGGL(rope_attention_kernel<DT_F16>, grid, dim3(ATT_THREADS), 0, stream, qkv, ldq, hq, hkv, pos0,
                           window, kc, vc, cache_len, inv_freq, out, ldo, scale);
    return check_launch("rope_attention");
}

int launch_rope_cache(float *qkv, uint32_t ldq, uint32_t rows, uint32_t hq, uint32_t hkv, uint32_t pos0,
                      const uint32_t *pos_arr, void *kc, void *vc, int ct, uint32_t cache_len,
                      uint64_t cache_stride, const float *inv_freq, hipStream_t stream) {
    const dim3 grid(rows);
    if (ct == DT_F32)
        hipLaunchKernelGGL(rope_cache_kernel<DT_F32>, grid, dim3(256), 0, stream, qkv, ldq, hq, hkv, pos0, pos_arr,
                           kc, vc, cache_len, cache_stride, inv_freq);
    else
        hipLaunchKernelGGL(rope_cache_kernel<DT_F16>, grid, dim3(256), 0, stream, qkv, ldq, hq, hkv, pos0, pos_arr,
                           kc, vc, cache_len, cache_stride, inv_freq);
    return check_launch("rope_cache");
}

int launch_attention(const float *q, uint32_t ldq, uint32_t rows, uint32_t hq, uint32_t hkv, uint32_t pos0,
                     const uint32_t *lens, uint32_t window, const void *kc, const void *vc, int ct,
                     uint32_t cache_len, uint64_t cache_stride, float *out, uint32_t ldo, float scale,
                     hipStream_t stream) {
    // Rows of one sequence whose keys all start at position 0 go by blocks of AR_ROWS rows.
    if (!lens && rows >= AR_MIN_ROWS && pos0 + rows <= static_cast<uint32_t>(AR_MAXKEYS) &&
        (window == 0 || pos0 + rows <= window)) {
        const dim3 g(hq, (rows + AR_ROWS - 1) / AR_ROWS);
        if (ct == DT_F32)
            hipLaunchKernelGGL((attention_rows_kernel<DT_F32, AR_ROWS>), g, dim3(ATT_THREADS), 0, stream, q, ldq, hq,
                               hkv, pos0, rows, kc, vc, cache_len, out, ldo, scale);
        else
            hipLaunchKernelGGL((attention_rows_kernel<DT_F16, AR_ROWS>), g, dim3(ATT_THREADS), 0, stream, q, ldq, hq,
                               hkv, pos0, rows, kc, vc, cache_len, out, ldo, scale);
        return check_launch("attention");
    }
    dim3 grid(rows * hq);
    if (ct == DT_F32)
        hipLaunchKernelGGL(attention_kernel<DT_F32>, grid, dim3(ATT_THREADS), 0, stream, q, ldq, hq, hkv, pos0, lens,
                           window, kc, vc, cache_len, cache_stride, out, ldo, scale);
    else
        hipLaunchKernelGGL(attention_kernel<DT_F16>, grid, dim3(ATT_THREADS), 0, stream, q, ldq, hq, hkv, pos0, lens,
                           window, kc, vc, cache_len, cache_stride, out, ldo, scale);
    return check_launch("attention");
}

}  // namespace mt
