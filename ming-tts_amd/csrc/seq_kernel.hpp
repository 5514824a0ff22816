// Persistent execution of a linear sequence (mt_seq_*): the decode step's chain of
// dependent GEMVs as ONE launch of at most one workgroup per CU, synchronised by dataflow instead
// of barriers.
//
// Reference counterpart: QwenForward.dispatches encoded on one serial compute encoder
// (Qwen.swift:72-97); every dispatch sees the writes of the ones before it.
//
// Dataflow between workgroups:
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
// Inside a workgroup (512 threads, at most one per CU) every wave computes.  A wave owns a
// contiguous range of each op's MFMA tiles (16 weight rows x 32 k, one 16-byte chunk per
// lane, as seq_tiles.hpp cuts them) and keeps them in registers, loaded one op ahead:
//   - a wave's vector loads retire in order, so per op it issues its activation loads
//     first and the next op's weight tiles right after them; waiting for the activations
//     then never waits for the weight stream, which lands while the op computes;
//   - per op a wave polls the activation chunks it stages (16-byte device-coherent loads
//     of tagged words, re-requesting only stale ones) and converts each element once (tag
//     clear, x^2 for the RMSNorm sum, gain, fp32 -> hi + lo pair of the weights' 16-bit
//     type) into the workgroup's LDS B staging; after a workgroup barrier it runs two
//     MFMAs per tile (hi and lo) and writes finished row tiles' partial sums to LDS; after
//     a second barrier one lane per output sums the partials in a fixed order, applies the
//     norm scale and the epilogue and stores the tagged word (and the user output when
//     final).
// LDS partial sums, sums of squares and gains alternate between two buffers by op parity.
// Every wait is bounded: past SPIN_LIMIT polls a lane gives up, sets the plan's timeout
// flag (read by mt_seq_check) and stops waiting for the rest of the run.  An fp16 weight
// sequence also flags activations beyond the fp16 range (the hi part would overflow).
//
// This header holds the kernel; linear_seq.hip instantiates the linear-only kernels and holds
// the host side, linear_seq_attn.hip instantiates the kernels of plans with attention items
// (a code object of their own, so their size does not move the linear-only kernels).
#pragma once

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
constexpr int PARTW = SEQ_PARTW;
constexpr int XCH = (SEQ_XLDS / 4 + SEQ_CW * 64 - 1) / (SEQ_CW * 64);  // 16-byte x chunks per compute lane
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

// Plain loads through global-address-space pointers (global_load, counted on vmcnt alone;
// a generic pointer would make a flat load that also occupies lgkmcnt).
template <class T>
__device__ __forceinline__ T gld(const T *p) {
    return *reinterpret_cast<const __attribute__((address_space(1))) T *>(reinterpret_cast<uintptr_t>(p));
}
// One tagged word at byte offset off of the plan's tag buffer, device-coherently (a plain
// load: no ordering against the loads in flight before it).
__device__ __forceinline__ uint32_t ldtag1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, SC1);
}
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

constexpr int CW = SEQ_CW;             // waves (all compute)
constexpr int CTHREADS = CW * 64;
constexpr int TA = SEQ_TA;              // weight tiles a wave holds per op
constexpr int CGCH = SEQ_GMAX / 8 / CTHREADS + ((SEQ_GMAX / 8) % CTHREADS ? 1 : 0);
constexpr int OUTR = (SEQ_RMAX * 8 + CTHREADS - 1) / CTHREADS;  // outputs per thread
static_assert(CW == NW, "every wave computes");
constexpr int XPAD = 256;  // LDS staging padding past M K: the largest B over-read is 32 S + 8 elements

// Loaded in place of a weight chunk outside the op's share (padding rows, K tails).
static __device__ __attribute__((aligned(16))) uint32_t g_zero_chunk[4];  // one per code object

typedef __attribute__((address_space(3))) void *lds_vp;

// x = hi + lo in type T, packed in pairs; both parts rounded toward zero (fp16) or to
// nearest (bf16) with one packed conversion per pair.
template <int T>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (T == DT_BF16) {
        typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
        typedef float f2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, bf2));
    } else {
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
    }
}
template <int T>
__device__ __forceinline__ void split4p(const float (&x)[4], u32x2 &hi, u32x2 &lo) {
    const uint32_t h0 = pack2<T>(x[0], x[1]), h1 = pack2<T>(x[2], x[3]);
    hi = u32x2{h0, h1};
    lo = u32x2{pack2<T>(x[0] - dec_lo<T>(h0), x[1] - dec_hi<T>(h0)), pack2<T>(x[2] - dec_lo<T>(h1), x[3] - dec_hi<T>(h1))};
}

// A wave's tiles of an op: the contiguous range [t0, t0 + n) of the workgroup's tiles,
// starting at row tile rt0, block step j0 (staged in LDS for every op at kernel start).
struct WaveTiles {
    uint16_t t0, n, rt0, j0;
};
__device__ __forceinline__ WaveTiles wave_tiles(const SeqTiles &st, uint32_t w) {
    WaveTiles wt;
    const uint32_t t0 = seq_tile_begin(st.T, w, CW);
    wt.t0 = static_cast<uint16_t>(t0);
    wt.n = static_cast<uint16_t>(seq_tile_begin(st.T, w + 1, CW) - t0);
    const uint32_t rt0 = st.KBs ? t0 / st.KBs : 0;
    wt.rt0 = static_cast<uint16_t>(rt0);
    wt.j0 = static_cast<uint16_t>(t0 - rt0 * st.KBs);
    return wt;
}

// LDS word access that the compiler neither reorders nor caches.
__device__ __forceinline__ uint32_t lds_ld(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// A wave's weight tiles of op o into registers (nontemporal 16-byte loads: the stream does
// not displace L2 lines), exactly NL loads whatever the wave's tile count, so that the
// number of loads in flight behind the activations is known where they are awaited;
// chunks outside the share (padding rows, K tails, tiles past the wave's count) read the
// zero chunk.
template <int NL>
__device__ __forceinline__ void tile_loads(const SeqOp &o, const SeqTiles &s, const WaveTiles &wt, u32x4 (&A)[TA]) {
    const uint32_t lane = threadIdx.x & 63, a = lane & 15, q = lane >> 4;
    const uint32_t sa = a & (s.S - 1), va = a >> s.ls;
    const uint32_t kbase = sa * s.KBs * 32 + q * 8;  // k of the lane's chunk at block step 0
    // The lane's chunks are real for block steps j < jlim (its segment's blocks, k < K).
    const uint32_t jseg = s.KB > sa * s.KBs ? s.KB - sa * s.KBs : 0u;
    const uint32_t jk = o.K > kbase ? (o.K - kbase + 31) / 32 : 0u;
    const uint32_t jlim = jseg < jk ? jseg : jk;
    // The lane's weight row in row tile rt (a wave's tiles span at most two row tiles).
    auto row_of = [&](uint32_t rt, bool &ok) {
        const uint32_t vrow = s.S > 1 ? va : rt * 16 + a;
        const bool up = vrow >= s.nr;
        ok = vrow < s.V;
        return (up ? o.w2 : o.w) + static_cast<size_t>(s.r0 + (up ? vrow - s.nr : vrow)) * o.K + kbase;
    };
    bool rok;
    const uint16_t *p = row_of(wt.rt0, rok) + wt.j0 * 32u;
    uint32_t j = wt.j0;
    const u32x4 *zero = reinterpret_cast<const u32x4 *>(g_zero_chunk);
#pragma unroll
    for (int k = 0; k < NL; k++) {  // exactly NL loads: tiles past the wave's n read the zero chunk
        const bool ok = static_cast<uint32_t>(k) < wt.n && rok && j < jlim;
        const u32x4 *src = ok ? reinterpret_cast<const u32x4 *>(p) : zero;
        A[k] = __builtin_nontemporal_load(reinterpret_cast<gw_cp>(reinterpret_cast<uintptr_t>(src)));
        p += 32;
        if (++j == s.KBs) {
            j = 0;
            p = row_of(wt.rt0 + 1u, rok);
        }
    }
    // Every register of A is written, so A carries no value of an earlier op and keeps one
    // register assignment across the op loop (no copy, no wait for the loads at its end).
#pragma unroll
    for (int k = NL; k < TA; k++) A[k] = u32x4{0u, 0u, 0u, 0u};
}

// Sum over aligned lane pairs / quads of a wave (fixed order).
__device__ __forceinline__ float dpp_pair(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_quad(float v) {
    v = dpp_pair(v);  // quad_perm [1,0,3,2]
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
}

// Sum over aligned lane octets (quads, then the half-row mirror): fixed order.
__device__ __forceinline__ float dpp_oct(float v) {
    v = dpp_quad(v);
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
}

// Partial sums of a finished row tile from the MFMA accumulator into this wave's LDS
// slice, pw[v * M + m] for virtual row v and x row m.  B column c carries x row m over
// segment s, half h (hi or lo): c = 2 (m S + s) + h.  Lane (row group qd, column c) holds
// D[4 qd + i][c]; the entry of (virtual row, x row) over segment s sits in the columns
// with that segment and the rows (4 qd + i) with (4 qd + i) % S == s, so the 2 S
// neighbouring lanes of x row m add the segments and both halves.
__device__ __forceinline__ void flush(const f32x4 acc, const SeqTiles &s, uint32_t M, uint32_t rt, float *pw) {
    const uint32_t lane = threadIdx.x & 63, c = lane & 15, qd = lane >> 4;
    if (s.S == 1) {  // rows 4 qd + i: virtual row rt 16 + 4 qd + i; columns 2 m + h
        const uint32_t m = c >> 1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float e = dpp_pair(acc[i]);
            const uint32_t v = rt * 16 + qd * 4 + i;
            if ((c & 1) == 0 && v < s.V && m < M) pw[v * M + m] = e;
        }
    } else if (s.S == 2) {  // rows 4 qd + i: virtual row 2 qd + i / 2, segment i % 2
        const uint32_t sc = (c >> 1) & 1, m = c >> 2;
        const float e0 = dpp_quad(sc ? acc[1] : acc[0]);
        const float e1 = dpp_quad(sc ? acc[3] : acc[2]);
        if ((c & 3) == 0 && m < M) {
            if (2 * qd < s.V) pw[(2 * qd) * M + m] = e0;
            if (2 * qd + 1 < s.V) pw[(2 * qd + 1) * M + m] = e1;
        }
    } else {  // S == 4: rows 4 qd + i: virtual row qd, segment i
        const uint32_t sc = (c >> 1) & 3, m = c >> 3;
        const float e = dpp_oct(sc == 0 ? acc[0] : sc == 1 ? acc[1] : sc == 2 ? acc[2] : acc[3]);
        if ((c & 7) == 0 && m < M && qd < s.V) pw[qd * M + m] = e;
    }
}

// The RMSNorm gain of op o into LDS gb (16-bit, K elements) by the compute threads:
// requested before a wait, stored after it.
__device__ __forceinline__ void gain_request(const SeqOp &o, bool live, u32x4 (&gr)[CGCH]) {
    // Issued whether or not the op has a gain (then it reads the first chunks of w), so the
    // number of loads in flight behind the activations does not depend on the op.
    const bool use = live && o.norm != nullptr;
    const uint16_t *src = use ? o.norm : o.w;
#pragma unroll
    for (int r = 0; r < CGCH; r++) {  // no lane-divergent branch around the loads
        const uint32_t ch = threadIdx.x + r * CTHREADS;
        gr[r] = gld(reinterpret_cast<const u32x4 *>(src + (use && ch * 8 < o.K ? ch * 8 : 0u)));
    }
}
__device__ __forceinline__ void gain_store(const SeqOp &o, const u32x4 (&gr)[CGCH], uint16_t *gb) {
    if (!o.norm) return;
#pragma unroll
    for (int r = 0; r < CGCH; r++) {
        const uint32_t ch = threadIdx.x + r * CTHREADS;
        if (ch * 8 < o.K) *reinterpret_cast<u32x4 *>(gb + ch * 8) = gr[r];
    }
}

// Sum over the 64 lanes of a wave in a fixed order: DPP within rows of 16 (quad swaps,
// then half-row and row mirrors), then the four rows' sums.
__device__ __forceinline__ float wave_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    const int iv = __builtin_bit_cast(int, v);
    return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16))) +
           (__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48)));
}

// Cache element access of the attention items: 8 or 4 consecutive elements as fp32, and
// the value a cache slot of type CT holds for v.
template <int CT>
__device__ __forceinline__ void cache_load8(const void *base, size_t off, float (&o)[8]) {
    if constexpr (CT == DT_F32) {
        const f32x4 a = gld(reinterpret_cast<const f32x4 *>(static_cast<const float *>(base) + off));
        const f32x4 b = gld(reinterpret_cast<const f32x4 *>(static_cast<const float *>(base) + off + 4));
        o[0] = a[0]; o[1] = a[1]; o[2] = a[2]; o[3] = a[3];
        o[4] = b[0]; o[5] = b[1]; o[6] = b[2]; o[7] = b[3];
    } else {
        const u32x4 v = gld(reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(base) + off));
        o[0] = dec_lo<DT_F16>(v.x); o[1] = dec_hi<DT_F16>(v.x);
        o[2] = dec_lo<DT_F16>(v.y); o[3] = dec_hi<DT_F16>(v.y);
        o[4] = dec_lo<DT_F16>(v.z); o[5] = dec_hi<DT_F16>(v.z);
        o[6] = dec_lo<DT_F16>(v.w); o[7] = dec_hi<DT_F16>(v.w);
    }
}
template <int CT>
__device__ __forceinline__ f32x4 cache_load4(const void *base, size_t off) {
    if constexpr (CT == DT_F32) {
        return gld(reinterpret_cast<const f32x4 *>(static_cast<const float *>(base) + off));
    } else {
        const u32x2 v = gld(reinterpret_cast<const u32x2 *>(static_cast<const uint16_t *>(base) + off));
        return f32x4{dec_lo<DT_F16>(v.x), dec_hi<DT_F16>(v.x), dec_lo<DT_F16>(v.y), dec_hi<DT_F16>(v.y)};
    }
}
template <int CT>
__device__ __forceinline__ float cache_round(float v) {
    if constexpr (CT == DT_F32) return v;
    else return static_cast<float>(static_cast<_Float16>(v));
}
template <int CT>
__device__ __forceinline__ void cache_store(void *base, size_t off, float v) {
    typedef __attribute__((address_space(1))) float gf;
    typedef __attribute__((address_space(1))) _Float16 gh;
    if constexpr (CT == DT_F32) *reinterpret_cast<gf *>(reinterpret_cast<uintptr_t>(static_cast<float *>(base) + off)) = v;
    else *reinterpret_cast<gh *>(reinterpret_cast<uintptr_t>(static_cast<_Float16 *>(base) + off)) = static_cast<_Float16>(v);
}
// Max / sum over the 64 lanes, the same bits in every lane (DPP within rows of 16, then two
// exchanges between rows).
__device__ __forceinline__ float wave_max_bfly(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    v = fmaxf(v, dpp_mov<0x140>(v));
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    return fmaxf(v, __shfl_xor(v, 32, 64));
}
__device__ __forceinline__ float wave_sum_bfly(float v) { return group_sum(v, 64); }

// Decode attention of query row b, head h of an attention item (Shaders.swift:451-596 as
// rope_cache then attention_cache).
//   - Thread (key group kq = tid / 8, lane r = tid % 8) owns keys t = kq + 64 u (u < KU) of
//     each chunk of 64 KU keys, dims 8 r .. 8 r + 7 of their k and v rows.  The first
//     chunk's k and v are requested before the qkv activations are polled (they do not
//     depend on them), so the wait for the activations also covers the cache reads.
//   - The row's q head and its kv head's k and v are polled from the qkv activations; q and
//     k are rotated (NeoX pairs i, i + 32, angle = pos * inv_freq[i]); k and v, rounded to
//     the cache type, are appended at pos by the first head of each kv group and used for
//     key pos from LDS by every head, so no workgroup waits for another's cache write.
//   - Rows of one sequence (a shared cache: cache_stride 0 with more than one row, at
//     positions pos[0] + b, as mt_rope_attention's rows): row b also takes the keys at
//     pos[0] .. pos - 1 from rows 0 .. b - 1 of the activations (rotated and rounded the same
//     way), since those rows' items append them concurrently; older keys come from the cache.
//   - Scores: the 8 lanes of a key group sum their dims by shuffles; each thread keeps a
//     running maximum, the sum of exp(score - max) and the p-weighted v sum of its keys
//     (rescaled when the maximum grows).  At the end the workgroup maximum rescales every
//     thread's part, and the parts meet in LDS in a fixed order.
// The head's output row is stored as tagged words (and to the user buffer when final).
// NW: the workgroup's waves (8 key groups each).  Uses lds (floats) as scratch: 7168 words.
template <int CT, int NW = CW>
__device__ __forceinline__ void attend_item(const SeqOp &o, uint32_t b, uint32_t h, __amdgpu_buffer_rsrc_t rsrc,
                                            uint32_t parity, float *lds, bool &gave_up, uint32_t *sync,
                                            const uint32_t *pos_pre = nullptr) {
    static_assert(NW == 7 || NW == 8, "the final sums are written out for 7 or 8 waves");
    constexpr int KG = 8 * NW;  // key groups of 8 lanes
    // The thread index is made opaque here, so nothing derived from it is hoisted out of
    // the sequence's op loop (where it would hold registers through every linear op).
    uint32_t tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const uint32_t lane = tid & 63, w = tid >> 6;
    constexpr int KU = CT == DT_F32 ? 4 : 8;  // keys per thread per chunk
    constexpr int CH = KG * KU;                // keys per chunk
    constexpr int WV = CT == DT_F32 ? 2 : 1;   // 16-byte loads per 8 elements
    const uint32_t hq = o.heads & 0xFFFFu, hkv = o.heads >> 16;
    const uint32_t kvh = h / (hq / hkv);
    float *sraw = lds;          // [64] q of the row, as read
    float *sq = lds + 192;      // [64] rotated q
    float *red = lds + 384;     // [16] wave maxima, then wave sums of the softmax denominators
    float *part = lds + 512;    // [64][64] p.v parts of the key groups
    float *part2 = lds + 4608;  // [8][64] sums of eight key groups
    float *kvraw = lds + 5120;  // [8][128] k | v of the rows whose keys come from the activations
    float *skv = lds + 6144;    // [8][128] those keys: k rotated | v, rounded to the cache type
    float *trig = lds + 512;    // [1 + nnew][cos 32 | sin 32] of the rotation angles (in part's
                                // space, which the scores' end first writes)

    // pos_pre: the row's position and pos[0], loaded by the caller ahead of the item.
    const uint32_t pos = pos_pre ? pos_pre[0] : gld(o.pos + b);
    // Keys at positions pos0 .. pos come from rows 0 .. nnew - 1 of the activations: the row
    // itself, or with a shared cache rows 0 .. b of the sequence.
    const bool shared = o.cache_stride == 0 && o.M > 1;
    const uint32_t pos0 = shared ? (pos_pre ? pos_pre[1] : gld(o.pos)) : pos;
    const uint32_t nnew = shared ? b + 1 : 1u;
    const bool append = pos < o.cache_len;
    // Keys [j0, len): len = pos + 1 (the new key at pos comes from LDS), or the whole cache
    // when pos is past it.
    const uint32_t len = append ? pos + 1 : o.cache_len;
    const uint32_t j0 = (o.window > 0 && len > o.window) ? len - o.window : 0u;
    const int nk = static_cast<int>(len - j0);
    const uint64_t cbase = static_cast<uint64_t>(b) * o.cache_stride;
    const size_t kvbase = cbase + (static_cast<size_t>(kvh) * o.cache_len + j0) * 64;
    const int kq = static_cast<int>(tid >> 3), r = static_cast<int>(tid & 7);
    u32x4 kraw[KU][WV], vraw[KU][WV];
    auto chunk_loads = [&](int c0) {
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int t = min(c0 + kq + KG * u, nk - 1);  // past the keys: a valid row, unused
            const size_t e = kvbase + static_cast<size_t>(t) * 64 + 8 * r;
#pragma unroll
            for (int q = 0; q < WV; q++) {
                if constexpr (CT == DT_F32) {
                    kraw[u][q] = gld(reinterpret_cast<const u32x4 *>(reinterpret_cast<const float *>(o.w) + e + 4 * q));
                    vraw[u][q] = gld(reinterpret_cast<const u32x4 *>(reinterpret_cast<const float *>(o.w2) + e + 4 * q));
                } else {
                    kraw[u][q] = gld(reinterpret_cast<const u32x4 *>(o.w + e));
                    vraw[u][q] = gld(reinterpret_cast<const u32x4 *>(o.w2 + e));
                }
            }
        }
    };
    auto unpack = [&](const u32x4 (&raw)[WV], float (&f)[8]) {
        if constexpr (CT == DT_F32) {
#pragma unroll
            for (int q = 0; q < 2; q++) {
                f[4 * q + 0] = __uint_as_float(raw[q].x);
                f[4 * q + 1] = __uint_as_float(raw[q].y);
                f[4 * q + 2] = __uint_as_float(raw[q].z);
                f[4 * q + 3] = __uint_as_float(raw[q].w);
            }
        } else {
            f[0] = dec_lo<DT_F16>(raw[0].x); f[1] = dec_hi<DT_F16>(raw[0].x);
            f[2] = dec_lo<DT_F16>(raw[0].y); f[3] = dec_hi<DT_F16>(raw[0].y);
            f[4] = dec_lo<DT_F16>(raw[0].z); f[5] = dec_hi<DT_F16>(raw[0].z);
            f[6] = dec_lo<DT_F16>(raw[0].w); f[7] = dec_hi<DT_F16>(raw[0].w);
        }
    };
    // The last wave (which polls nothing below) requests the inverse frequencies ahead of its
    // key chunks, so forming the rotation angles' cosines and sines waits for them alone.
    const bool trig_wave = w == NW - 1 && lane < 32;
    float invf = 0.0f;
    if (trig_wave) invf = gld(o.inv_freq + lane);
    chunk_loads(0);
    // The angles depend on positions only: their cosines and sines are formed while the
    // other waves poll the activations (q at pos, the activations' keys at pos0 .. pos0 +
    // nnew - 1).
    if (trig_wave) {
        const float aq = static_cast<float>(pos) * invf;
        trig[lane] = cosf(aq);
        trig[32 + lane] = sinf(aq);
        for (uint32_t rr = 0; rr < nnew; rr++) {
            const float ar = static_cast<float>(pos0 + rr) * invf;
            trig[64 * (rr + 1) + lane] = cosf(ar);
            trig[64 * (rr + 1) + 32 + lane] = sinf(ar);
        }
    }

    // q head h of row b (16 chunks of 4 words), then k and v heads kvh of each row the keys
    // pos0 .. pos come from (32 chunks a row).
    if (tid < 16 + 32 * nnew) {
        uint32_t row = b, col;
        float *dst;
        if (tid < 16) {
            col = h * 64 + 4 * tid;
            dst = sraw + 4 * tid;
        } else {
            const uint32_t u = tid - 16, rr = u >> 5, pt = (u >> 4) & 1u, c4 = 4 * (u & 15);
            row = shared ? rr : b;
            col = (pt == 0 ? (hq + kvh) * 64 : (hq + hkv + kvh) * 64) + c4;
            dst = kvraw + rr * 128 + pt * 64 + c4;
        }
        u32x4 v;
        if (o.xsrc >= 0) {
            const uint32_t off = (o.xoff + row * o.xld + col) * 4u;
            v = ldtag4(rsrc, off);
            uint32_t spins = 0;
            while (!tagged4(v, parity) && !gave_up) {
                if (++spins > SPIN_LIMIT) {
                    gave_up = true;
                    raise_flag(sync, SYNC_TIMEOUT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                v = ldtag4(rsrc, off);
            }
            v &= ~1u;
        } else {
            v = gld(reinterpret_cast<const u32x4 *>(static_cast<const float *>(o.x) + static_cast<size_t>(row) * o.ldx + col));
        }
        *reinterpret_cast<u32x4 *>(dst) = v;
    }
    __syncthreads();
    if (tid < 32) {
        const uint32_t i = tid;
        const float q0 = sraw[i], q1 = sraw[i + 32];
        rope_rotate(q0, q1, trig[i], trig[32 + i], sq[i], sq[i + 32]);
        for (uint32_t rr = 0; rr < nnew; rr++) {
            const float cr = trig[64 * (rr + 1) + i], sr = trig[64 * (rr + 1) + 32 + i];
            const float *kr = kvraw + rr * 128;
            const float k0 = kr[i], k1 = kr[32 + i];
            float *d = skv + rr * 128;
            float r0, r1;
            rope_rotate(k0, k1, cr, sr, r0, r1);
            d[i] = cache_round<CT>(r0);
            d[i + 32] = cache_round<CT>(r1);
            d[64 + i] = cache_round<CT>(kr[64 + i]);
            d[96 + i] = cache_round<CT>(kr[96 + i]);
        }
        if (append && h % (hq / hkv) == 0) {
            const float *d = skv + (nnew - 1) * 128;  // the row's own key
            const size_t dst = cbase + (static_cast<size_t>(kvh) * o.cache_len + pos) * 64;
            cache_store<CT>(const_cast<uint16_t *>(o.w), dst + i, d[i]);
            cache_store<CT>(const_cast<uint16_t *>(o.w), dst + i + 32, d[i + 32]);
            cache_store<CT>(const_cast<uint16_t *>(o.w2), dst + i, d[64 + i]);
            cache_store<CT>(const_cast<uint16_t *>(o.w2), dst + i + 32, d[96 + i]);
        }
    }
    __syncthreads();

    float qf[8];
#pragma unroll
    for (int e = 0; e < 8; e++) qf[e] = sq[8 * r + e];
    float m = -INFINITY, l = 0.0f, acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] = 0.0f;
    for (int c0 = 0; c0 < nk; c0 += CH) {
        if (c0 > 0) chunk_loads(c0);
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int t = c0 + kq + KG * u;
            if (t < nk) {  // the 8 lanes of a key group agree
                float kf[8], vf[8];
                const uint32_t p = j0 + static_cast<uint32_t>(t);
                if (p >= pos0) {  // a key from the activations
                    const uint32_t rr = min(p - pos0, nnew - 1);
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        kf[e] = skv[rr * 128 + 8 * r + e];
                        vf[e] = skv[rr * 128 + 64 + 8 * r + e];
                    }
                } else {
                    unpack(kraw[u], kf);
                    unpack(vraw[u], vf);
                }
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) d = fmaf(qf[e], kf[e], d);
                d = octet_sum(d);
                d *= o.eps;
                const float mn = fmaxf(m, d);
                const float a = exp_hw(m - mn), pb = exp_hw(d - mn);
                l = fmaf(l, a, pb);
#pragma unroll
                for (int e = 0; e < 8; e++) acc[e] = fmaf(acc[e], a, pb * vf[e]);
                m = mn;
            }
        }
    }
    // Workgroup maximum; every thread's part rescaled to it.
    // A wave without keys has m = -inf.  Its slot holds -1e30 instead: this scratch is the
    // next linear's activation staging, and past that op's M K its stale words are over-read
    // (against zero weights) as 16-bit halves, where -inf or -FLT_MAX would be a NaN that
    // survives the multiply by zero.  -1e30 is below any score and finite in fp16 and bf16.
    float mx = wave_max_bfly(m);
    if (lane == 0) red[w] = fmaxf(mx, -1.0e30f);
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int ww = 1; ww < NW; ww++) mx = fmaxf(mx, red[ww]);
    const float f = exp_hw(m - mx);  // 0 for a thread without keys (m = -inf)
    const float ls = wave_sum_bfly(r == 0 ? l * f : 0.0f);
    if (lane == 0) red[8 + w] = ls;
#pragma unroll
    for (int e = 0; e < 8; e++) part[kq * 64 + 8 * r + e] = acc[e] * f;
    __syncthreads();
    {  // eight key groups per sum, then the eight sums, in order
        const uint32_t d = tid & 63, gi = tid >> 6;
        float a = part[(8 * gi) * 64 + d];
#pragma unroll
        for (int k = 1; k < 8; k++) a += part[(8 * gi + k) * 64 + d];
        part2[gi * 64 + d] = a;
    }
    __syncthreads();
    if (tid < 64) {
        float a = part2[tid];
#pragma unroll
        for (int k = 1; k < NW; k++) a += part2[k * 64 + tid];
        const float sum = NW == 8 ? ((red[8] + red[9]) + (red[10] + red[11])) + ((red[12] + red[13]) + (red[14] + red[15]))
                                  : ((red[8] + red[9]) + (red[10] + red[11])) + ((red[12] + red[13]) + red[14]);
        const float v = sum > 0.0f ? a / sum : 0.0f;
        const uint32_t n = h * 64 + tid;
        st_tag(o.tag + static_cast<size_t>(b) * o.N + n, v, parity);
        if (o.final_out)
            *reinterpret_cast<__attribute__((address_space(1))) float *>(
                reinterpret_cast<uintptr_t>(o.y + static_cast<size_t>(b) * o.ldy + n)) = v;
    }
    __syncthreads();  // the scratch is free again
}

// Each 512-thread workgroup (at most one per CU) runs every op of the sequence in order (see the top of
// the file).  tags / tag_bytes: the plan's tagged activation buffer, read through a buffer
// resource with device-coherent loads.  MS: the rows M of every op when the plan has one
// common M the kernel is specialised for (1 or 2), else 0 (M read per op).  ATTN: the plan
// holds attention items (a linear-only plan runs a kernel without their code).
template <int WT, int MS, bool ATTN>
__global__ __launch_bounds__(SEQ_THREADS) void seq_kernel(const SeqOp *__restrict__ ops, uint32_t n_ops,
                                                         uint32_t *sync, const uint32_t *tags, uint32_t tag_bytes) {
    // The op's x as [hi, lo][M][K]; MFMA B reads past M K (K tails) land in the padding,
    // which holds zeros or earlier ops' finite values.
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][SEQ_XLDS + XPAD];
    __shared__ __attribute__((aligned(16))) float part[2][CW * PARTW];
    __shared__ __attribute__((aligned(16))) uint16_t gbuf[2][SEQ_GMAX];
    __shared__ float ssw[2][CW * 8];
    __shared__ __attribute__((aligned(16))) SeqOp sdesc[SEQ_OPS_MAX];
    __shared__ SeqTiles stile[SEQ_OPS_MAX];
    __shared__ WaveTiles swt[SEQ_OPS_MAX][CW];
    const uint32_t G = gridDim.x, g = blockIdx.x;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);

    // The op descriptors and this workgroup's tiling of every op, staged in LDS once (no
    // op then waits for a descriptor load).
    for (uint32_t e = tid; e < n_ops * (sizeof(SeqOp) / 16); e += SEQ_THREADS)
        reinterpret_cast<u32x4 *>(sdesc)[e] = gld(reinterpret_cast<const u32x4 *>(ops) + e);
    for (uint32_t e = tid; e < 2 * (SEQ_XLDS + XPAD) / 8; e += SEQ_THREADS)
        reinterpret_cast<u32x4 *>(&xs[0][0])[e] = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();
    for (uint32_t t = tid; t < n_ops; t += SEQ_THREADS) {
        const SeqOp &o = sdesc[t];
        stile[t] = seq_tiles(o.kind == SEQ_ATTN ? 0u : o.N, o.K, o.M, (o.flags & F_SILU_GATE) != 0, g, G);
    }
    __syncthreads();
    for (uint32_t e = tid; e < n_ops * CW; e += SEQ_THREADS) swt[e / CW][e % CW] = wave_tiles(stile[e / CW], e % CW);
    __syncthreads();

    const uint32_t epoch = __hip_atomic_load(sync + SYNC_EPOCH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t parity = epoch & 1u;
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t *>(tags), 0, static_cast<int>(tag_bytes), BUF_DWORD3);
    bool gave_up = false;
    u32x4 gr[CGCH];
    // Weight tiles of two consecutive ops: even ops multiply P0 while P1 receives the next
    // op's tiles, odd ops the other way round.  The loop runs two ops per iteration, so no
    // register copy (which would wait for the next op's tiles to land) ends an op.
    u32x4 P0[TA], P1[TA];

    if (n_ops > 0) {
        gain_request(sdesc[0], true, gr);
        tile_loads<TA>(sdesc[0], stile[0], swt[0][w], P0);
        gain_store(sdesc[0], gr, gbuf[0]);
        __syncthreads();
    }
    // One op: A holds its weight tiles; An receives the next op's.
    auto run_op = [&](uint32_t i, const u32x4 (&A)[TA], u32x4 (&An)[TA]) __attribute__((always_inline)) {
        const int b = i & 1;
        const SeqOp o = sdesc[i];  // by value: read once, kept in registers
        const SeqTiles s = stile[i];
        const WaveTiles wt = swt[i][w];
        if (ATTN && o.kind == SEQ_ATTN) {
            // Decode attention: items (row, head) go to workgroups g, g + G, ...; then every
            // workgroup requests the next op's gain and weight tiles as a linear would.
            const uint32_t hq = o.heads & 0xFFFFu, items = o.M * hq;
            float *scratch = reinterpret_cast<float *>(&xs[0][0]);
            for (uint32_t it = g; it < items; it += G) {
                if (o.cache_t == DT_F32) attend_item<DT_F32>(o, it / hq, it % hq, rsrc, parity, scratch, gave_up, sync);
                else attend_item<DT_F16>(o, it / hq, it % hq, rsrc, parity, scratch, gave_up, sync);
            }
            const bool next = i + 1 < n_ops;
            const SeqOp on = sdesc[next ? i + 1 : i];
            const SeqTiles sn = stile[next ? i + 1 : i];
            const WaveTiles wtn = swt[next ? i + 1 : i][w];
            // The items' scratch is the next linear's staging: the 256 elements past its M K in
            // each half, which its MFMAs read against zero weights when K is not a multiple of
            // their blocks, are cleared (a scratch word's halves may read as a NaN).
            if (g < items && next && on.kind == SEQ_LINEAR && tid < 64) {
                const uint32_t e0 = on.M * on.K + 8 * (tid & 31);
                *reinterpret_cast<u32x4 *>(&xs[tid >> 5][e0]) = u32x4{0u, 0u, 0u, 0u};
            }
            gain_request(on, next, gr);
            if (wtn.n <= 2) tile_loads<2>(on, sn, wtn, An);
            else if (wtn.n <= 6) tile_loads<6>(on, sn, wtn, An);
            else tile_loads<TA>(on, sn, wtn, An);
            if (next) gain_store(on, gr, gbuf[b ^ 1]);
            __syncthreads();
        } else {
            const uint32_t M = MS ? static_cast<uint32_t>(MS) : o.M;
            const bool norm = o.norm != nullptr;

            // The op's activations x [M][K] are staged once per workgroup: chunk e = tid + 384 r
            // is 4 k of one row of the row-major x; every compute lane polls its chunks, then
            // converts them into LDS as hi + lo halves (xs[0], xs[1], row-major [M][K]).
            const uint32_t K = o.K, K4 = K >> 2, nchunk = M * K4;
            const uint32_t rows_used = (nchunk + CTHREADS - 1) / CTHREADS;  // chunk rounds (uniform)
            const uint32_t k4magic = 0xFFFFFFFFu / K4 + 1u;                 // e / K4 = umulhi(e, k4magic)
            const bool ext = o.xsrc < 0;
            // Loads are issued without branches around them (lanes past the op read past the end
            // of the tag buffer, which returns zeros): a load under a lane-divergent branch makes
            // the compiler wait for every load in flight where the branch rejoins.
            u32x4 xv[XCH];
            if (!ext) {
                // Tagged chunks (lanes past the op read past the end of the tag buffer, which
                // returns zeros).
#pragma unroll
                for (int r = 0; r < XCH; r++) {
                    xv[r] = u32x4{0u, 0u, 0u, 0u};
                    if (static_cast<uint32_t>(r) < rows_used) {  // uniform; the tiles requested after these are not
                        const uint32_t e = tid + CTHREADS * r;
                        const uint32_t m = __umulhi(e, k4magic), k = (e - m * K4) * 4;
                        const bool ok = e < nchunk;
                        xv[r] = ldtag4(rsrc, ok ? (o.xoff + m * o.xld + k) * 4u : 0xFFFFFFF0u);
                    }
                }
            } else {
#pragma unroll
                for (int r = 0; r < XCH; r++) {
                    xv[r] = u32x4{0u, 0u, 0u, 0u};
                    const uint32_t e = tid + CTHREADS * r;
                    if (static_cast<uint32_t>(r) < rows_used && e < nchunk) {
                        const uint32_t m = __umulhi(e, k4magic), k = (e - m * K4) * 4;
                        if (o.xt == DT_F32) {
                            const float *p = static_cast<const float *>(o.x) + static_cast<size_t>(m) * o.ldx + k;
                            xv[r] = u32x4{__float_as_uint(gld(p)), __float_as_uint(gld(p + 1)), __float_as_uint(gld(p + 2)),
                                          __float_as_uint(gld(p + 3))};
                        } else {
                            const uint16_t *p = static_cast<const uint16_t *>(o.x) + static_cast<size_t>(m) * o.ldx + k;
                            float f[4];
#pragma unroll
                            for (int ee = 0; ee < 4; ee++)
                                f[ee] = o.xt == DT_BF16 ? dec1<DT_BF16>(gld(p + ee)) : dec1<DT_F16>(gld(p + ee));
                            xv[r] = u32x4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                                          __float_as_uint(f[3])};
                        }
                    }
                }
            }
            // Output lanes: bias and old y of outputs (feature r0 + v, row m), requested after
            // the activations (which the wave waits for first).
            const uint32_t nout = s.nr * M;
            uint32_t yw[OUTR], braw[OUTR];  // old y (tagged word or user fp32 bits), raw 16-bit bias
#pragma unroll
            for (int r = 0; r < OUTR; r++) {
                const uint32_t idx = tid + r * CTHREADS;
                const uint32_t ov = idx / M, om = idx - ov * M;
                const bool live_out = idx < nout;
                braw[r] = 0;
                yw[r] = 0;
                // Uniform branches only; lanes past the outputs read element 0.
                if (o.flags & F_BIAS) braw[r] = gld(o.bias + (live_out ? s.r0 + ov : 0u));
                if (o.flags & F_ACCUM) {
                    if (o.ysrc >= 0)
                        yw[r] = ldtag1(rsrc, live_out ? (o.yoff + om * o.yld + s.r0 + ov) * 4u : 0xFFFFFFF0u);
                    else
                        yw[r] = gld(reinterpret_cast<const uint32_t *>(o.y) +
                                    (live_out ? static_cast<size_t>(om) * o.ldy + s.r0 + ov : 0u));
                }
            }
            // The next op's RMSNorm gain (stored to LDS after this op's MFMAs) and weight tiles,
            // requested behind the activations.
            const bool next = i + 1 < n_ops;
            const SeqOp on = sdesc[next ? i + 1 : i];
            const SeqTiles sn = stile[next ? i + 1 : i];
            const WaveTiles wtn = swt[next ? i + 1 : i][w];
            gain_request(on, next, gr);

            // The next op's weight tiles, requested right behind the activations: a wave's loads
            // return in order, so they land after the activations, while this op computes.  The
            // count issued is 2, 6 or TA (the wave's tiles of the next op rounded up), each with
            // its own first check of the activations, so that check waits for the activations
            // alone and not for the tiles behind them.
            auto stale_mask = [&]() {
                uint32_t st = 0;
                if (!ext) {
#pragma unroll
                    for (int r = 0; r < XCH; r++)
                        if (static_cast<uint32_t>(r) < rows_used && tid + CTHREADS * r < nchunk && !tagged4(xv[r], parity))
                            st |= 1u << r;
                }
                return st;
            };
            uint32_t stale;
            if (wtn.n <= 2) {
                tile_loads<2>(on, sn, wtn, An);
                stale = stale_mask();
            } else if (wtn.n <= 6) {
                tile_loads<6>(on, sn, wtn, An);
                stale = stale_mask();
            } else {
                tile_loads<TA>(on, sn, wtn, An);
                stale = stale_mask();
            }
            // Stale chunks: every round re-requests all of them at once.
            {
                uint32_t spins = 0;
                while (stale && !gave_up) {
                    if (++spins > SPIN_LIMIT) {
                        gave_up = true;
                        raise_flag(sync, SYNC_TIMEOUT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
#pragma unroll
                    for (int r = 0; r < XCH; r++) {
                        if ((stale >> r) & 1u) {
                            const uint32_t e = tid + CTHREADS * r;
                            const uint32_t m = __umulhi(e, k4magic), k = (e - m * K4) * 4;
                            xv[r] = ldtag4(rsrc, (o.xoff + m * o.xld + k) * 4u);
                        }
                    }
                    stale = stale_mask();
                }
            }
            // Convert: hi = x rounded toward zero to the weights' 16-bit type (to nearest for
            // bf16), lo = the rest, rounded the same way; x^2 summed per row for the RMSNorm.
            const uint16_t *gb = gbuf[b];
            float ssr[8];
#pragma unroll
            for (int mm = 0; mm < 8; mm++) ssr[mm] = 0.0f;
            bool range_ok = true;
            const uint32_t clear = ext ? ~0u : ~1u;  // tagged words: drop the tag bit
#pragma unroll
            for (int r = 0; r < XCH; r++) {
                const uint32_t e = tid + CTHREADS * r;
                if (static_cast<uint32_t>(r) < rows_used && e < nchunk) {
                    const uint32_t m = __umulhi(e, k4magic), k = (e - m * K4) * 4;
                    float x[4];
                    x[0] = __uint_as_float(xv[r].x & clear);
                    x[1] = __uint_as_float(xv[r].y & clear);
                    x[2] = __uint_as_float(xv[r].z & clear);
                    x[3] = __uint_as_float(xv[r].w & clear);
                    if (norm) {
                        float t = x[0] * x[0];
                        t = fmaf(x[1], x[1], t);
                        t = fmaf(x[2], x[2], t);
                        t = fmaf(x[3], x[3], t);
#pragma unroll
                        for (int mm = 0; mm < 8; mm++)
                            if (static_cast<uint32_t>(mm) < M) ssr[mm] += m == static_cast<uint32_t>(mm) ? t : 0.0f;
                        const u32x2 gg = *reinterpret_cast<const u32x2 *>(gb + k);
                        x[0] *= dec_lo<WT>(gg.x);
                        x[1] *= dec_hi<WT>(gg.x);
                        x[2] *= dec_lo<WT>(gg.y);
                        x[3] *= dec_hi<WT>(gg.y);
                    }
                    if constexpr (WT == DT_F16)
                        range_ok = range_ok && fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3]))) <= 65504.0f;
                    u32x2 hi, lo;
                    split4p<WT>(x, hi, lo);
                    *reinterpret_cast<u32x2 *>(&xs[0][m * K + k]) = hi;
                    *reinterpret_cast<u32x2 *>(&xs[1][m * K + k]) = lo;
                }
            }
            if (!range_ok) raise_flag(sync, SYNC_RANGE);
            if (norm) {  // the wave's sum of x^2 per row
#pragma unroll
                for (int mm = 0; mm < 8; mm++) {
                    if (static_cast<uint32_t>(mm) < M) {
                        const float t = wave_sum(ssr[mm]);
                        if (lane == 0) ssw[b][w * 8 + mm] = t;
                    }
                }
            }
            __syncthreads();  // the op's x is staged

            // MFMAs over the wave's tiles, A in registers, B from the staging: lane (bc, q) reads
            // column bc = 2 (m S + s) + h, 8 k of x row m over segment s from half h (hi or lo),
            // so one MFMA covers both halves (2 S M <= 16 columns).  The wave's tiles span at
            // most two row tiles (the plan checks it): tiles [0, ks) are in row tile rt0 and the
            // rest in rt0 + 1, each with its own accumulator, flushed to LDS at the end.  B
            // chunks past K meet zero A chunks (and hold finite values).
            float *pw = part[b] + w * PARTW;
            {
                const uint32_t bc = lane & 15, q = lane >> 4;
                const uint32_t col = bc >> 1, h = bc & 1;
                const uint32_t bkb = (col & (s.S - 1)) * s.KBs;  // segment's first block
                const uint32_t boff = h * (SEQ_XLDS + XPAD) + (col >> s.ls) * K + bkb * 32 + q * 8;
                const bool bcol = col < s.S * M;
                const uint16_t *xsb = &xs[0][0];
                const uint32_t n = wt.n;
                const uint32_t ks = min(n, s.KBs - wt.j0);
                f32x4 a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0;
                uint32_t bo = boff + wt.j0 * 32u;
#pragma unroll
                for (int k = 0; k < TA; k++) {
                    if (static_cast<uint32_t>(k) < n) {
                        if (static_cast<uint32_t>(k) == ks) bo = boff;
                        u32x4 bv = {0u, 0u, 0u, 0u};
                        if (bcol) bv = *reinterpret_cast<const u32x4 *>(xsb + bo);
                        if (static_cast<uint32_t>(k) < ks) a0 = mfma16<WT>(A[k], bv, a0);
                        else a1 = mfma16<WT>(A[k], bv, a1);
                        bo += 32;
                    }
                }
                if (n > 0) flush(a0, s, M, wt.rt0, pw);
                if (n > ks) flush(a1, s, M, wt.rt0 + 1u, pw);
            }
            if (next) gain_store(on, gr, gbuf[b ^ 1]);
            __syncthreads();  // every wave's partial sums are in LDS

            // Outputs: sums of the waves' partials in wave order.
#pragma unroll
            for (int r = 0; r < OUTR; r++) {
                const uint32_t idx = tid + r * CTHREADS;
                if (idx >= nout) continue;
                const uint32_t ov = idx / M, om = idx - ov * M;
                float yold = 0.0f;
                if (o.flags & F_ACCUM && o.ysrc < 0) yold = __uint_as_float(yw[r]);
                if (o.flags & F_ACCUM && o.ysrc >= 0) {
                    const uint32_t yoff = (o.yoff + om * o.yld + s.r0 + ov) * 4u;
                    uint32_t v = yw[r], spins = 0;
                    while ((v & 1u) != parity && !gave_up) {
                        if (++spins > SPIN_LIMIT) {
                            gave_up = true;
                            raise_flag(sync, SYNC_TIMEOUT);
                            break;
                        }
                        __builtin_amdgcn_s_sleep(1);
                        v = ldtag1(rsrc, yoff);
                    }
                    yold = untag(v);
                }
                auto total = [&](uint32_t vr) {
                    const uint32_t rt = s.S > 1 ? 0 : vr / 16;
                    const uint32_t lo_t = rt * s.KBs, hi_t = lo_t + s.KBs;
                    const float *p = part[b] + vr * M + om;
                    float v[CW];
#pragma unroll
                    for (int ww = 0; ww < CW; ww++) v[ww] = p[ww * PARTW];
                    float a = 0.0f;
#pragma unroll
                    for (int ww = 0; ww < CW; ww++) {
                        const uint32_t b0 = seq_tile_begin(s.T, ww, CW), b1 = seq_tile_begin(s.T, ww + 1, CW);
                        a += (b0 < b1 && b0 < hi_t && b1 > lo_t) ? v[ww] : 0.0f;
                    }
                    return a;
                };
                float scale = 1.0f;
                if (norm) {
                    float v[CW];
#pragma unroll
                    for (int ww = 0; ww < CW; ww++) v[ww] = ssw[b][ww * 8 + om];
                    float t = 0.0f;
#pragma unroll
                    for (int ww = 0; ww < CW; ww++) t += v[ww];
                    scale = rsqrt_hw(t / static_cast<float>(o.K) + o.eps);
                }
                const float a1 = total(ov);
                const float a2 = (o.flags & F_SILU_GATE) ? total(ov + s.nr) : 0.0f;
                // (the empty asm keeps the decode here, after the wait, rather than next to the load)
                asm volatile("" : "+v"(braw[r]));
                const float bias = (o.flags & F_BIAS) ? dec1<WT>(static_cast<uint16_t>(braw[r])) : 0.0f;
                float v = epilogue(a1 * scale, a2 * scale, bias, o.flags);
                if (o.flags & F_ACCUM) v += yold;
                const uint32_t n = s.r0 + ov;
                st_tag(o.tag + static_cast<size_t>(om) * o.N + n, v, parity);
                if (o.final_out)
                    *reinterpret_cast<__attribute__((address_space(1))) float *>(
                        reinterpret_cast<uintptr_t>(o.y + static_cast<size_t>(om) * o.ldy + n)) = v;
            }
        }
    };
    for (uint32_t i = 0; i < n_ops; i += 2) {
        run_op(i, P0, P1);
        if (i + 1 < n_ops) run_op(i + 1, P1, P0);
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

// The kernel of a plan with attention items (linear_seq_attn.hip): weights wt, specialised
// for two rows when m2.
seq_fn seq_attn_kernel(int wt, bool m2);
// The decode-layer kernel (linear_layer.hip) for weights wt at M rows (1, 2 or 4), or null.
seq_fn layer_kernel_fn(int wt, uint32_t M, bool att);
seq_fn layer_attn_kernel_fn(int wt, uint32_t M);
seq_fn dit_block_kernel_fn(int wt, uint32_t M);

}  // namespace mt
