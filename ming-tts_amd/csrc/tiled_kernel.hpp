// Pipelined MFMA GEMM of mt_linear (prefill and DiT shapes, M above the GEMV row limit):
// the kernel template, instantiated for activations of the weights' own 16-bit type in
// linear_gemm_lds.hip and for fp32 activations (with or without a fused RMSNorm) in
// linear_gemm_split.hip.
//
// Reference kernel replaced: gemm_kernel<32,64,32,4> (Shaders.swift:297-410).
//
// y[m][n] = epilogue(sum_k x[m][k] w[n][k]) on a 512-thread workgroup per BM x BN tile
// (BM x rows, BN weight rows; SiLU-gate: 64 features, whose W and W2 rows make the 128
// weight rows of the tile), with v_mfma_f32_32x32x16_{f16,bf16}.
//   - Weights travel global -> LDS with global_load_lds_dwordx4 (no register staging) into a
//     ring of P stages of 64 k each; stage s + 1 .. s + P - 1 are in flight while stage s is
//     multiplied.  Within a 128-byte row of a stage, 16-byte chunk c sits in slot c ^ g(row),
//     g(r) = (r & 7) ^ ((r >> 3) & 1): the MFMA operand reads (32 rows of one chunk per
//     half-wave) then hit 8 different slots in every 8 consecutive rows, and 16 different
//     (row parity, slot) bank groups in every 16, so they are conflict-free whether LDS
//     serves 8 lanes over 32 banks or 16 lanes over 64 banks per cycle.
//   - Activations of the weights' type take the same direct path: a stage holds the tile's
//     BM x rows, then its BN weight rows.
//   - fp32 activations (SPLIT) are staged through registers two stages ahead, together with
//     the weights (two LDS buffers, as P == 1 below): each thread loads 8 k of one or two x
//     rows, multiplies them by the RMSNorm gain (NORM) while summing the row's x^2 from the
//     same loads, and writes x = hi + lo as two planes of the weights' type (hi = round(x),
//     lo = round(x - hi): x to 2^-22 relative with fp16, 2^-17 with bf16, so the product
//     keeps the reference's fp32-activation accuracy).  A stage then holds BM hi rows, BM lo
//     rows and the BN weight rows; each k step takes two MFMAs (hi and lo against the same
//     weight fragment).  The epilogue scales row m by 1 / sqrt(mean(x_m^2) + eps) (NORM); with
//     split-K each split's partial tile carries its rows' partial sums of x^2, which the
//     last workgroup adds in split order with the tiles.
//   - Waves 0-3 and 4-7 form two 2 x 2 grids over the tile, each wave (BM / 2) x (BN / 2);
//     the first grid multiplies k 0-31 of every stage, the second k 32-63.  Two waves per
//     SIMD hide each other's LDS reads, and each stage is read from LDS only twice.  The two
//     grids swap halves of their sums through LDS (added first + second, a fixed order), and
//     every wave runs the epilogue from its registers; each store covers two 128-byte row
//     segments.
//   - Split-K: when the output tiles alone cannot fill the chip, S workgroups share a tile's
//     K range.  Each writes its partial sums in register order (1 KB per store) to a
//     per-stream workspace with device-coherent stores, waits for them, and counts itself in
//     at the tile's counter; the workgroup that arrives last reads the other partials
//     device-coherently (a batch of splits in flight at once) and adds the S parts in split
//     order 0 .. S-1, so the result does not depend on arrival order.  It then runs the
//     epilogue and re-arms the counter.
//   - Workgroup -> tile order is XCD-aware: consecutive workgroup ids go to different XCDs, so
//     the id is remapped to give each XCD a contiguous run of tiles (the x-row tiles of one
//     weight tile first), which then share that XCD's L2.
//   - Rows past M or N and k past K are loaded from a zero block, never from outside the
//     operands; rows past M or N are not stored.
// MFMA 32x32x16 operand layout (wave64): lane l holds A[l % 32][8 (l / 32) .. + 7] and
// B[8 (l / 32) .. + 7][l % 32]; accumulator r of lane l is D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
#pragma once

#include "mt_device.hpp"
#include "mt_internal.hpp"

#include <type_traits>

namespace mt {
namespace tiled {

typedef _Float16 f16x8t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8t __attribute__((ext_vector_type(8)));
typedef float f32x16t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4t __attribute__((ext_vector_type(4)));
typedef float f32x4t __attribute__((ext_vector_type(4)));

constexpr int TBK = 64;   // k per stage
constexpr int SC1 = 16;   // buffer cache policy: device-coherent

// Loaded in place of any 16-byte chunk outside the operands (one per code object).
static __device__ __attribute__((aligned(16))) uint32_t g_zero_chunk[4];

struct TiledArgs {
    const void *x;                          // type WT, or fp32 (SPLIT)
    const uint16_t *w, *w2, *bias;
    const uint16_t *norm;                   // RMSNorm gain [K] (NORM)
    float *y;
    uint32_t M, N, K, ldx, ldy, flags;
    float eps;
    uint32_t tiles_m, tiles_n, splits, kps;  // kps: 64-k steps per split
    float *part;                            // split partial tiles, or null when splits == 1
    uint32_t part_bytes;
    uint32_t *cnt;                          // per-tile arrival counters (zero between launches)
};

template <int T>
__device__ __forceinline__ f32x16t mfma32x(u32x4t a, u32x4t b, f32x16t c) {
    if constexpr (T == DT_BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8t, a), __builtin_bit_cast(bf16x8t, b),
                                                       c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8t, a), __builtin_bit_cast(f16x8t, b), c,
                                                      0, 0, 0);
}

// One wave-wide direct load: lane l's 16 bytes at gaddr land at LDS byte lds + 16 l (lds
// wave-uniform; the compiler sets m0 from it).
__device__ __forceinline__ void dma16(uint32_t lds, const void *gaddr) {
    __builtin_amdgcn_global_load_lds(
        reinterpret_cast<const __attribute__((address_space(1))) void *>(reinterpret_cast<uintptr_t>(gaddr)),
        reinterpret_cast<__attribute__((address_space(3))) void *>(lds), 16, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier that waits only for this wave's LDS reads (lgkmcnt), not for its loads in
// flight: __syncthreads adds a fence that the compiler may turn into vmcnt(0).
__device__ __forceinline__ void tiled_bar() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Workgroup id -> tile order with a contiguous run of ids per XCD (ids are dealt to the
// 8 XCDs round-robin).
__device__ __forceinline__ uint32_t xcd_order(uint32_t b, uint32_t G) {
    const uint32_t x = b & 7u, i = b >> 3, q = G >> 3, r = G & 7u;
    return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + i;
}

// hi = round(x), lo = round(x - hi) in type T (round to nearest even), for 8 values packed in
// pairs.  x - hi is exact in fp32, so with fp16 halves each lo is one mixed-precision fma
// (fp32 x minus the fp16 hi, rounded to fp16 into the pair's low or high half) after one
// packed conversion for the pair's hi: 3 instructions a pair.  bf16 has no mixed fma: the
// pair's hi is widened back and subtracted.
typedef float f32x2t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2t __attribute__((ext_vector_type(2)));
template <int T>
__device__ __forceinline__ void split2(float x0, float x1, uint32_t &hi, uint32_t &lo) {
    if constexpr (T == DT_BF16) {
        const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2t{x0, x1}, bf16x2t));
        hi = h;
        lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2t{x0 - bf16_lo(h), x1 - bf16_hi(h)}, bf16x2t));
    } else {
        const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2t{x0, x1}, f16x2t));
        uint32_t l;
        asm("v_fma_mixlo_f16 %0, %1, 1.0, -%2 op_sel_hi:[0,0,1]" : "=v"(l) : "v"(x0), "v"(h));
        asm("v_fma_mixhi_f16 %0, %1, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "+v"(l) : "v"(x1), "v"(h));
        hi = h;
        lo = l;
    }
}
template <int T>
__device__ __forceinline__ void split8(const float (&x)[8], u32x4t &hi, u32x4t &lo) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
        uint32_t h, l;
        split2<T>(x[2 * e], x[2 * e + 1], h, l);
        hi[e] = h;
        lo[e] = l;
    }
}

template <int BM, int BN, bool GATED, int KS, bool SPLIT>
struct TileShape {
    static constexpr int NW = 4 * KS;                 // waves: KS grids of 2 x 2 over the tile
    static constexpr int NT = 64 * NW;                // threads
    static constexpr int WMT = BM / 64;               // 32-row A tiles per wave
    static constexpr int WNT = BN / 64;               // 32-row B tiles per wave (gated: W and W2)
    static constexpr int KKW = 4 / KS;                // 16-k MFMA steps per wave per stage
    static constexpr int NACC = WMT * WNT == 1 ? 2 : 1;  // accumulator sets: a lone tile alternates two
    static constexpr int XP = SPLIT ? 2 : 1;          // activation planes (hi, lo)
    static constexpr int AR = XP * BM;                // activation rows of a stage
    static constexpr int SB = (AR + BN) * 128;        // bytes per stage
    // 1 KB direct loads per wave per stage: x and weight rows, or only the weight rows (SPLIT).
    static constexpr int LPW = (SPLIT ? BN : BM + BN) / (8 * NW);
    static constexpr int IA = BM * 8 / NT;            // SPLIT: 8-k activation items per thread per stage
    static constexpr int FN = GATED ? 64 : BN;        // output features per tile
    static constexpr int NE = (GATED ? 2 : 1) * BM * FN;  // partial-tile elements (gated: W and W2 sums)
};
// Floats of one split's partial tile in the workspace: the tile, then (normed) its rows'
// partial sums of x^2.
template <int BM, int BN, bool GATED, bool NORM>
constexpr int partial_floats() {
    return (GATED ? 2 : 1) * BM * (GATED ? 64 : BN) + (NORM ? BM : 0);
}

template <int WT, int BM, int BN, bool GATED, int P, int KS, int XT, bool NORM>
__global__ __launch_bounds__(256 * KS) void tiled_kernel(TiledArgs a) {
    constexpr bool SPLIT = XT != WT;
    static_assert(!SPLIT || XT == DT_F32, "split activations are fp32");
    static_assert(!NORM || SPLIT, "a fused RMSNorm takes fp32 activations");
    typedef TileShape<BM, BN, GATED, KS, SPLIT> TS;
    constexpr int NT = TS::NT, NW = TS::NW, WMT = TS::WMT, WNT = TS::WNT, KKW = TS::KKW, NACC = TS::NACC;
    constexpr int AR = TS::AR, SB = TS::SB, LPW = TS::LPW, IA = TS::IA, FN = TS::FN, NE = TS::NE;
    constexpr int XBYTES = 8 * WMT * WNT * 2 * 64 * 16;  // the k grids' hand-over: [4][2][blocks][2] float4 a lane
    constexpr int NBUF = P == 1 ? 2 : P;  // LDS stages (P == 1: register-staged loads, two LDS buffers)
    constexpr int LBYTES = NBUF * SB > XBYTES ? NBUF * SB : XBYTES;
    static_assert(!GATED || BN == 128, "a gated tile is 64 features of W and W2");
    static_assert(LPW * 8 * NW == (SPLIT ? BN : BM + BN) && P >= 1 && P <= 4 && LBYTES <= 160 * 1024, "tile shape");
    static_assert(!SPLIT || ((P == 1 || P == 2) && IA * NT == BM * 8), "split staging: two register-staged LDS buffers");
    static_assert(NE % (4 * NT) == 0, "partial tiles move as float4 per thread");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[LBYTES];
    __shared__ uint32_t last_flag;
    __shared__ __attribute__((aligned(16))) float row_ss[NORM ? BM : 4];  // rows' sums of x^2, then scales (NORM)

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kh = wave >> 2, wm = wave & 1, wn = (wave >> 1) & 1;

    const uint32_t G = gridDim.x;
    const uint32_t t = xcd_order(blockIdx.x, G);
    const uint32_t tm = t % a.tiles_m, rest = t / a.tiles_m;
    const uint32_t split = rest % a.splits, tn = rest / a.splits;
    const uint32_t tile = tn * a.tiles_m + tm;
    const uint32_t m0 = tm * BM;
    const uint32_t n0 = tn * FN;  // first output feature
    const uint32_t M = a.M, N = a.N, K = a.K;
    // The bias of the lane's output columns (see the epilogue), requested now so the epilogue
    // does not wait for it: block column j covers features n0 + 32 (wn WNT + j) + lane % 32
    // (gated: one column, n0 + 32 wn + lane % 32).
    float bv[WNT];
#pragma unroll
    for (int j = 0; j < WNT; j++) {
        const uint32_t n = n0 + (GATED ? 32 * wn : 32 * (wn * WNT + j)) + (lane & 31);
        bv[j] = (a.flags & F_BIAS) && n < N ? dec1<WT>(a.bias[n]) : 0.0f;
    }
    const uint32_t KT = (K + TBK - 1) / TBK;
    const uint32_t ks0 = split * a.kps;
    const uint32_t nsteps = min(ks0 + a.kps, KT) - ks0;

    // Direct-load sources of this lane: row block b = wave + NW i holds stage rows 8 b .. 8 b
    // + 7 (SPLIT: weight rows 8 b .. 8 b + 7, staged after the AR activation rows); the lane
    // fills slot lane & 7 of row 8 b + lane / 8, so it fetches chunk c_i = (lane & 7) ^ g(row) =
    // (lane & 7) ^ (lane >> 3) ^ (b & 1) (AR is a multiple of 16, so g is the same either way).
    uint32_t ci[LPW];
    const char *src[LPW];
    bool rowok[LPW];
    const uint32_t lds0 =
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void *)(lds)));
    constexpr int XROWS = SPLIT ? 0 : BM;  // x rows among the direct-load rows
#pragma unroll
    for (int i = 0; i < LPW; i++) {
        const int b = wave + NW * i;
        const int r = 8 * b + (lane >> 3);
        ci[i] = (lane & 7) ^ (lane >> 3) ^ (b & 1);
        const uint16_t *base;
        uint32_t row, lim;
        size_t ld;
        if (r < XROWS) {
            base = static_cast<const uint16_t *>(a.x); row = m0 + r; lim = M; ld = a.ldx;
        } else if (!GATED) {
            base = a.w; row = n0 + (r - XROWS); lim = N; ld = K;
        } else {
            const int j = r - XROWS;
            base = j < 64 ? a.w : a.w2; row = n0 + (j & 63); lim = N; ld = K;
        }
        rowok[i] = row < lim;
        src[i] = reinterpret_cast<const char *>(base + static_cast<size_t>(rowok[i] ? row : 0) * ld + 8 * ci[i]);
    }
    const char *zero = reinterpret_cast<const char *>(g_zero_chunk);

    auto issue = [&](uint32_t buf, uint32_t kstep) {
        const uint32_t k = kstep * TBK;
#pragma unroll
        for (int i = 0; i < LPW; i++) {
            const char *g = (rowok[i] && k + 8 * ci[i] < K) ? src[i] + 2 * static_cast<size_t>(k) : zero;
            dma16(__builtin_amdgcn_readfirstlane(lds0 + buf * SB + (wave + NW * i) * 1024), g);
        }
    };
    // Wait until at most n (0, 1 or 2) of this wave's stages are still in flight.
    auto wait_pending = [&](uint32_t n) {
        if (n >= 2) wait_vm<2 * LPW>();
        else if (n == 1) wait_vm<LPW>();
        else wait_vm<0>();
    };

    // MFMA operand reads: row (l & 31) of each 32-row tile (g(row) = g(l & 31), the tiles
    // start at multiples of 16 rows), chunk 2 kk + l / 32 of the stage, kk = KKW kh .. KKW kh
    // + KKW - 1 for this wave's part of the stage.
    uint32_t swz[KKW];
#pragma unroll
    for (int q = 0; q < KKW; q++) swz[q] = (((2 * (KKW * kh + q) + (lane >> 5)) ^ (lane & 7) ^ ((lane >> 3) & 1)) << 4);
    const uint32_t arow = (32 * wm * WMT + (lane & 31)) * 128;
    uint32_t brow[WNT];
#pragma unroll
    for (int j = 0; j < WNT; j++)
        brow[j] = (AR + (GATED ? 64 * j + 32 * wn : 32 * (wn * WNT + j)) + (lane & 31)) * 128;

    struct Frags {
        u32x4t a[KKW][WMT], b[KKW][WNT];
        u32x4t al[SPLIT ? KKW : 1][SPLIT ? WMT : 1];  // SPLIT: the lo plane
    };
    auto load = [&](Frags &f, uint32_t buf) {
        const uint8_t *st = lds + buf * SB;
#pragma unroll
        for (int q = 0; q < KKW; q++) {
#pragma unroll
            for (int i = 0; i < WMT; i++) {
                f.a[q][i] = *reinterpret_cast<const u32x4t *>(st + arow + i * 32 * 128 + swz[q]);
                if constexpr (SPLIT) f.al[q][i] = *reinterpret_cast<const u32x4t *>(st + BM * 128 + arow + i * 32 * 128 + swz[q]);
            }
#pragma unroll
            for (int j = 0; j < WNT; j++) f.b[q][j] = *reinterpret_cast<const u32x4t *>(st + brow[j] + swz[q]);
        }
    };
    f32x16t acc[NACC][WMT][WNT];
#pragma unroll
    for (int h = 0; h < NACC; h++)
#pragma unroll
        for (int i = 0; i < WMT; i++)
#pragma unroll
            for (int j = 0; j < WNT; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[h][i][j][r] = 0.0f;
    auto mma = [&](const Frags &f) {
#pragma unroll
        for (int q = 0; q < KKW; q++) {
            if constexpr (!SPLIT) {
#pragma unroll
                for (int i = 0; i < WMT; i++)
#pragma unroll
                    for (int j = 0; j < WNT; j++)
                        acc[q % NACC][i][j] = mfma32x<WT>(f.a[q][i], f.b[q][j], acc[q % NACC][i][j]);
            } else {
                // hi then lo against each weight fragment; a lone tile keeps them in two sets.
#pragma unroll
                for (int i = 0; i < WMT; i++)
#pragma unroll
                    for (int j = 0; j < WNT; j++) acc[0][i][j] = mfma32x<WT>(f.a[q][i], f.b[q][j], acc[0][i][j]);
#pragma unroll
                for (int i = 0; i < WMT; i++)
#pragma unroll
                    for (int j = 0; j < WNT; j++)
                        acc[NACC - 1][i][j] = mfma32x<WT>(f.al[q][i], f.b[q][j], acc[NACC - 1][i][j]);
            }
        }
    };

    // SPLIT row sums of x^2 (item j of this thread: row (tid + NT j) / 8, k 8 (tid % 8) of every
    // stage).
    float ss[SPLIT ? IA : 1];
#pragma unroll
    for (int j = 0; j < (SPLIT ? IA : 1); j++) ss[j] = 0.0f;

    if constexpr (SPLIT) {
        // Register staging of both operands, stages s + 1 and s + 2 in flight while stage s is
        // multiplied (the P == 1 scheme below): the weight rows' chunks as the direct loads
        // would fetch them, and activation items of 8 k (two 16-byte loads of fp32) of row
        // r_j = (tid + NT j) / 8 at k 8 (tid % 8) of the stage, with the gain's 8 values (one
        // load, the same k for every item of the thread).  The commit writes the weight chunks
        // and the items' hi and lo halves into the stage's swizzled layout.  Loads past the K
        // range read the zero chunk.
        const uint32_t kc = tid & 7;
        const float *xrow[IA];
        bool xok[IA];
        uint32_t aoff[IA];  // LDS byte offset of the item's hi chunk in a stage
#pragma unroll
        for (int j = 0; j < IA; j++) {
            const uint32_t r = (tid + NT * j) >> 3, m = m0 + r;
            xok[j] = m < M;
            xrow[j] = static_cast<const float *>(a.x) + static_cast<size_t>(xok[j] ? m : 0u) * a.ldx + 8 * kc;
            aoff[j] = r * 128 + ((kc ^ (r & 7) ^ ((r >> 3) & 1)) << 4);
        }
        typedef const __attribute__((address_space(1))) u32x4t *gp;
        auto ld16 = [](const void *p) { return *reinterpret_cast<gp>(reinterpret_cast<uintptr_t>(p)); };
        struct Stage {
            u32x4t b[LPW], x[IA][2], g;
        };
        auto gload = [&](Stage &r, uint32_t kstep) {
            const uint32_t k = kstep * TBK;
#pragma unroll
            for (int i = 0; i < LPW; i++) {
                const char *g = (rowok[i] && kstep < KT && k + 8 * ci[i] < K) ? src[i] + 2 * static_cast<size_t>(k) : zero;
                r.b[i] = __builtin_nontemporal_load(reinterpret_cast<gp>(reinterpret_cast<uintptr_t>(g)));
            }
            const uint32_t kx = k + 8 * kc;
            const bool kok = kx < K;
#pragma unroll
            for (int j = 0; j < IA; j++) {
                const bool ok = kok && xok[j];
                r.x[j][0] = ld16(ok ? static_cast<const void *>(xrow[j] + k) : zero);
                r.x[j][1] = ld16(ok ? static_cast<const void *>(xrow[j] + k + 4) : zero);
            }
            if constexpr (NORM) r.g = ld16(kok ? static_cast<const void *>(a.norm + kx) : zero);
        };
        // in_range: the stage is one of this split's (a stage past them is staged but never
        // multiplied, and its x^2 is not summed).
        auto commit = [&](const Stage &r, uint32_t buf, bool in_range) {
            uint8_t *st = lds + buf * SB;
#pragma unroll
            for (int i = 0; i < LPW; i++) *reinterpret_cast<u32x4t *>(st + (AR / 8 + wave + NW * i) * 1024 + lane * 16) = r.b[i];
#pragma unroll
            for (int j = 0; j < IA; j++) {
                float x[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    x[e] = __uint_as_float(r.x[j][0][e]);
                    x[4 + e] = __uint_as_float(r.x[j][1][e]);
                }
                if constexpr (NORM) {
                    float t = ss[j];
#pragma unroll
                    for (int e = 0; e < 8; e++) t = fmaf(x[e], x[e], t);
                    ss[j] = in_range ? t : ss[j];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        if constexpr (WT == DT_F16) {  // x times the fp16 gain in one mixed fma each
                            float p0, p1;
                            asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "=v"(p0) : "v"(x[2 * e]), "v"(r.g[e]));
                            asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
                                : "=v"(p1) : "v"(x[2 * e + 1]), "v"(r.g[e]));
                            x[2 * e] = p0;
                            x[2 * e + 1] = p1;
                        } else {
                            x[2 * e] *= dec_lo<WT>(r.g[e]);
                            x[2 * e + 1] *= dec_hi<WT>(r.g[e]);
                        }
                    }
                }
                u32x4t hi, lo;
                split8<WT>(x, hi, lo);
                *reinterpret_cast<u32x4t *>(st + aoff[j]) = hi;
                *reinterpret_cast<u32x4t *>(st + BM * 128 + aoff[j]) = lo;
            }
        };
        Stage r0, r1;
        gload(r0, ks0);
        gload(r1, ks0 + 1);
        commit(r0, 0, true);
        gload(r0, ks0 + 2);
        __syncthreads();
        if constexpr (P == 2) {
            // The steady loop has no branch: every step commits the next stage and requests the
            // one two on (a stage past the split is staged, never multiplied; its loads read the
            // zero chunk or the next split's rows), so the compiler sees the same loads in flight
            // on every path and waits for exactly the stage it commits, with the following
            // stage's loads still in flight.  A scheduling fence after each barrier keeps a
            // step's conversions in that step: hoisted into the step before, they wait for loads
            // issued only a step earlier.  An odd last stage runs after the loop.  It holds more
            // registers than the loop below (one workgroup a CU at the 64 x 128 tiles).
            uint32_t s = 0;
            for (; s + 2 <= nsteps; s += 2) {
                {  // stage s in buffer 0; r1 holds s + 1, r0 is bound for s + 2
                    Frags f;
                    load(f, 0);
                    mma(f);
                    commit(r1, 1, true);
                    gload(r1, ks0 + s + 3);
                    __syncthreads();
                    __builtin_amdgcn_sched_barrier(0);
                }
                {  // stage s + 1 in buffer 1; r0 holds s + 2
                    Frags f;
                    load(f, 1);
                    mma(f);
                    commit(r0, 0, s + 2 < nsteps);
                    gload(r0, ks0 + s + 4);
                    __syncthreads();
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            if (s < nsteps) {  // the odd last stage, in buffer 0
                Frags f;
                load(f, 0);
                mma(f);
            }
        } else {
            // Commits and requests only within the split: fewer registers, but the compiler's
            // waits then cover the following stage's loads too.
            for (uint32_t s = 0; s < nsteps; s += 2) {
                {  // stage s in buffer 0; r1 holds s + 1, r0 is bound for s + 2
                    Frags f;
                    load(f, 0);
                    mma(f);
                    if (s + 1 < nsteps) {
                        commit(r1, 1, true);
                        gload(r1, ks0 + s + 3);
                    }
                    __syncthreads();
                }
                if (s + 1 < nsteps) {  // stage s + 1 in buffer 1; r0 holds s + 2
                    Frags f;
                    load(f, 1);
                    mma(f);
                    if (s + 2 < nsteps) {
                        commit(r0, 0, true);
                        gload(r0, ks0 + s + 4);
                    }
                    __syncthreads();
                }
            }
        }
        if constexpr (NORM) {
            // Row sums over the 8 threads of a row (an aligned lane octet): this split's part,
            // or with K whole the row's scale.
#pragma unroll
            for (int j = 0; j < IA; j++) {
                const float t = octet_sum(ss[j]);
                if (kc == 0) row_ss[(tid + NT * j) >> 3] = a.splits > 1 ? t : rsqrt_hw(t / static_cast<float>(K) + a.eps);
            }
        }
    } else if constexpr (P == 1) {
        // Register staging: stages s + 1 and s + 2 travel global -> registers while stage s is
        // multiplied; stage s + 1 is then written to the other LDS buffer (same swizzled
        // layout as the direct loads).  Loads past the K range read the zero chunk, so every
        // step issues the same loads and the waits stay exact.
        u32x4t rg0[LPW], rg1[LPW];
        auto gload = [&](u32x4t (&rg)[LPW], uint32_t kstep) {
            const uint32_t k = kstep * TBK;
#pragma unroll
            for (int i = 0; i < LPW; i++) {
                const char *g = (rowok[i] && kstep < KT && k + 8 * ci[i] < K) ? src[i] + 2 * static_cast<size_t>(k) : zero;
                rg[i] = __builtin_nontemporal_load(
                    reinterpret_cast<const __attribute__((address_space(1))) u32x4t *>(reinterpret_cast<uintptr_t>(g)));
            }
        };
        auto commit = [&](const u32x4t (&rg)[LPW], uint32_t buf) {
#pragma unroll
            for (int i = 0; i < LPW; i++)
                *reinterpret_cast<u32x4t *>(lds + buf * SB + (wave + NW * i) * 1024 + lane * 16) = rg[i];
        };
        gload(rg0, ks0);
        gload(rg1, ks0 + 1);
        commit(rg0, 0);
        gload(rg0, ks0 + 2);
        __syncthreads();
        for (uint32_t s = 0; s < nsteps; s += 2) {
            {  // stage s in buffer 0; rg1 holds s + 1, rg0 is bound for s + 2
                Frags f;
                load(f, 0);
                mma(f);
                if (s + 1 < nsteps) {
                    commit(rg1, 1);
                    gload(rg1, ks0 + s + 3);
                }
                __syncthreads();
            }
            if (s + 1 < nsteps) {  // stage s + 1 in buffer 1; rg0 holds s + 2
                Frags f;
                load(f, 1);
                mma(f);
                if (s + 2 < nsteps) {
                    commit(rg0, 0);
                    gload(rg0, ks0 + s + 4);
                }
                __syncthreads();
            }
        }
    } else if constexpr (P == 2) {
        // Double buffer: stage s + 1 is in flight while stage s is read from LDS and multiplied.
        issue(0, ks0);
        uint32_t buf = 0;
        for (uint32_t s = 0; s < nsteps; s++) {
            wait_vm<0>();
            __syncthreads();  // stage s is in; every wave is done reading stage s - 1
            if (s + 1 < nsteps) issue(buf ^ 1u, ks0 + s + 1);
            Frags f;
            load(f, buf);
            mma(f);
            buf ^= 1u;
        }
    } else {
        // Stages s + 1 .. s + P - 2 are in flight (or landed) while stage s is multiplied from
        // registers; stage s + 1's fragments are read from LDS meanwhile.  A wave issues about
        // one instruction every four cycles and a branch costs more, so the steady state (every
        // iteration issues a stage) runs without conditions: exact waits, direct-load addresses
        // that step by a fixed stride (rows past M or N step by 0 on the zero block; only a K
        // tail takes the checked issue), and the two fragment sets alternating by unrolling
        // instead of being copied.
        const char *gp[LPW];
        uint32_t gstride[LPW];
#pragma unroll
        for (int i = 0; i < LPW; i++) {
            gp[i] = rowok[i] ? src[i] : zero;
            gstride[i] = rowok[i] ? 2u * TBK : 0u;
        }
        const uint32_t ldsw = __builtin_amdgcn_readfirstlane(lds0 + wave * 1024);
        const bool ktail = (K % TBK) != 0;
        auto issue_step = [&](uint32_t buf, uint32_t kstep) {
            if (ktail && kstep + 1 == KT) {
                issue(buf, kstep);
                return;
            }
#pragma unroll
            for (int i = 0; i < LPW; i++) dma16(ldsw + buf * SB + NW * i * 1024, gp[i] + static_cast<size_t>(gstride[i]) * kstep);
        };
#pragma unroll
        for (int i = 0; i < P - 1; i++)
            if (static_cast<uint32_t>(i) < nsteps) issue_step(i, ks0 + i);
        wait_pending(min(static_cast<uint32_t>(P - 2), nsteps - 1));
        __syncthreads();
        Frags fa, fb;
        load(fa, 0);
        // Iteration s: stage s + 1 is in once at most P - 3 later stages are in flight; the barrier
        // also tells that every wave is done reading stage s - 1's buffer, which takes stage
        // s + P - 1.
        uint32_t s = 0, bs = 0;  // bs: buffer of stage s
        auto steady = [&](Frags &cur, Frags &nxt) {
            const uint32_t b1 = bs + 1 == P ? 0 : bs + 1, bi = bs == 0 ? P - 1 : bs - 1;
            wait_vm<(P - 3) * LPW>();
            tiled_bar();
            issue_step(bi, ks0 + s + P - 1);
            load(nxt, b1);
            mma(cur);
            bs = b1;
            s++;
        };
        while (s + P < nsteps) {  // two steady iterations
            steady(fa, fb);
            steady(fb, fa);
        }
        if (s + P - 1 < nsteps) {
            steady(fa, fb);
            fa = fb;
        }
        // The last P - 1 stages: nothing left to issue.
        for (; s < nsteps; s++) {
            const uint32_t b1 = bs + 1 == P ? 0 : bs + 1;
            if (s + 1 < nsteps) {
                wait_pending(nsteps - 1 - (s + 1));
                tiled_bar();
                load(fb, b1);
            }
            mma(fa);
            fa = fb;
            bs = b1;
        }
    }
    if constexpr (NACC == 2) {
#pragma unroll
        for (int i = 0; i < WMT; i++)
#pragma unroll
            for (int j = 0; j < WNT; j++) acc[0][i][j] += acc[1][i][j];
    }

    // The two k grids' sums meet through LDS, each wave finishing half of its accumulator
    // registers: the wave of grid kh keeps registers 8 kh .. 8 kh + 7 of every block (rows
    // 16 kh .. 16 kh + 15 of each 32-row block) and hands the other half to its partner in the
    // other grid; the sums are first grid + second, a fixed order.  Every wave then runs the
    // epilogue (or the split-K hand-over) from registers, with no fp32 tile in LDS: lane l
    // holds rows 8 (r / 4) + 4 (l / 32) + r % 4 of column l % 32, so a store covers two
    // 128-byte row segments.  kh becomes a compile-time constant through the two
    // instantiations of `finish`, so every register index stays a constant.
    constexpr int NB = WMT * WNT;  // 32 x 32 blocks of a wave
    __syncthreads();  // the ring is no longer read; the hand-over area overlays it
    float *xch = reinterpret_cast<float *>(lds);
    const int pos = wave & 3;  // the wave's place in its 2 x 2 grid
    auto finish = [&](auto khc) {
        constexpr int KH = decltype(khc)::value;
        constexpr int GIVE = 8 * (1 - KH), KEEP = 8 * KH;
        auto slot = [&](int giver, int b, int q) { return xch + ((((pos * 2 + giver) * NB + b) * 2 + q) * 64 + lane) * 4; };
#pragma unroll
        for (int i = 0; i < WMT; i++)
#pragma unroll
            for (int j = 0; j < WNT; j++)
#pragma unroll
                for (int q = 0; q < 2; q++)
                    *reinterpret_cast<f32x4t *>(slot(KH, i * WNT + j, q)) =
                        f32x4t{acc[0][i][j][GIVE + 4 * q], acc[0][i][j][GIVE + 4 * q + 1], acc[0][i][j][GIVE + 4 * q + 2],
                               acc[0][i][j][GIVE + 4 * q + 3]};
        __syncthreads();
        float sm[NB][8];
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const f32x4t v = *reinterpret_cast<const f32x4t *>(slot(1 - KH, b, q));
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float own = acc[0][b / WNT][b % WNT][KEEP + 4 * q + e];
                    sm[b][4 * q + e] = KH == 0 ? own + v[e] : v[e] + own;
                }
            }
        // Row of register rr of block row i, and column of block column j (gated: j = 0 the W
        // sums, j = 1 the W2 sums of the same feature).
        const int fr = lane & 31, fh = lane >> 5;
        auto row_of = [&](int i, int rr) { return 32 * (wm * WMT + i) + 16 * KH + 8 * (rr >> 2) + 4 * fh + (rr & 3); };
        auto col_of = [&](int j) { return GATED ? 32 * wn + fr : 32 * (wn * WNT + j) + fr; };

        if (a.splits > 1) {
            // Partial tile in register order: float4 q of register half (b, q) of wave w at
            // ((w NB + b) 2 + q) 64 + lane; a normed tile's BM row sums of x^2 follow (NEP
            // floats per split).  Each store moves 1 KB of consecutive floats.
            constexpr int NEP = partial_floats<BM, BN, GATED, NORM>();
            static_assert(NEP == NE + (NORM ? BM : 0) && NE == NW * NB * 8 * 64, "partial layout");
            const __amdgpu_buffer_rsrc_t rsrc =
                __builtin_amdgcn_make_buffer_rsrc(a.part, 0, static_cast<int>(a.part_bytes), 0x00020000);
            const uint32_t tile_base = tile * a.splits * static_cast<uint32_t>(NEP) * 4u;
            auto pidx = [&](int b, int q) { return static_cast<uint32_t>((((wave * NB + b) * 2 + q) * 64 + lane) * 4); };
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int q = 0; q < 2; q++)
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(u32x4t, f32x4t{sm[b][4 * q], sm[b][4 * q + 1], sm[b][4 * q + 2], sm[b][4 * q + 3]}),
                        rsrc, tile_base + (split * NEP + pidx(b, q)) * 4u, 0, SC1);
            if constexpr (NORM) {
                if (tid < BM / 4)
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(u32x4t, *reinterpret_cast<const f32x4t *>(row_ss + 4 * tid)), rsrc,
                        tile_base + (split * NEP + NE + 4 * tid) * 4u, 0, SC1);
            }
            wait_vm<0>();
            __syncthreads();
            if (tid == 0) {
                const uint32_t old = __hip_atomic_fetch_add(a.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                last_flag = old == a.splits - 1;
            }
            __syncthreads();
            if (!last_flag) return false;
            if (tid == 0) __hip_atomic_store(a.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // Sum the S partial tiles in split order, the other splits' halves requested a batch
            // of splits at a time.
            constexpr int D = 16 / (2 * NB) > 0 ? 16 / (2 * NB) : 1;  // splits per batch
            float tot[NB][8];
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int e = 0; e < 8; e++) tot[b][e] = 0.0f;
            for (uint32_t s0 = 0; s0 < a.splits; s0 += D) {
                f32x4t v[D][NB][2];
#pragma unroll
                for (int d = 0; d < D; d++)
#pragma unroll
                    for (int b = 0; b < NB; b++)
#pragma unroll
                        for (int q = 0; q < 2; q++) {
                            const uint32_t sp = s0 + d;
                            const uint32_t off =
                                (sp < a.splits && sp != split) ? tile_base + (sp * NEP + pidx(b, q)) * 4u : 0xFFFFFFF0u;
                            v[d][b][q] = __builtin_bit_cast(f32x4t, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, SC1));
                        }
#pragma unroll
                for (int d = 0; d < D; d++) {
                    const uint32_t sp = s0 + d;
                    if (sp < a.splits) {
#pragma unroll
                        for (int b = 0; b < NB; b++)
#pragma unroll
                            for (int e = 0; e < 8; e++) tot[b][e] += sp == split ? sm[b][e] : v[d][b][e >> 2][e & 3];
                    }
                }
            }
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int e = 0; e < 8; e++) sm[b][e] = tot[b][e];
            if constexpr (NORM) {
                // The rows' sums of x^2 in split order, by the first BM / 4 threads, then their
                // scales.
                f32x4t rsum = f32x4t{0.f, 0.f, 0.f, 0.f};
                if (tid < BM / 4) {
                    for (uint32_t sp = 0; sp < a.splits; sp++)
                        rsum += sp == split ? *reinterpret_cast<const f32x4t *>(row_ss + 4 * tid)
                                            : __builtin_bit_cast(f32x4t, __builtin_amdgcn_raw_buffer_load_b128(
                                                                             rsrc, tile_base + (sp * NEP + NE + 4 * tid) * 4u, 0, SC1));
                }
                __syncthreads();  // every thread has read its own row sums
                if (tid < BM / 4) {
#pragma unroll
                    for (int e = 0; e < 4; e++) rsum[e] = rsqrt_hw(rsum[e] / static_cast<float>(K) + a.eps);
                    *reinterpret_cast<f32x4t *>(row_ss + 4 * tid) = rsum;  // the rows' scales
                }
                __syncthreads();
            }
        }

        // Epilogue: the flags are branched on once (with_flag_set), and a tile inside M x N
        // stores without per-row checks (a wave issues about one instruction every four
        // cycles, so per-output branches cost microseconds).
        const bool full = m0 + BM <= M && n0 + FN <= N;
        const uint32_t flags = a.flags;
        with_flag_set(flags, [&](auto set) {
            constexpr uint32_t FL = decltype(set)::value;
            constexpr int NO = GATED ? WMT : NB;  // output blocks (gated: a W and a W2 block each)
            const bool accum = accumulates<FL>(flags);
            float v[NO][8];
#pragma unroll
            for (int o = 0; o < NO; o++) {
                const int i = GATED ? o : o / WNT, j = GATED ? 0 : o % WNT;
                const uint32_t gn = n0 + col_of(j);
#pragma unroll
                for (int rr = 0; rr < 8; rr++) {
                    const uint32_t gm = m0 + row_of(i, rr);
                    v[o][rr] = accum ? a.y[full || (gm < M && gn < N) ? static_cast<size_t>(gm) * a.ldy + gn : 0u] : 0.0f;
                }
            }
#pragma unroll
            for (int o = 0; o < NO; o++) {
                const int i = GATED ? o : o / WNT, j = GATED ? 0 : o % WNT;
#pragma unroll
                for (int rr = 0; rr < 8; rr++) {
                    float c = GATED ? sm[i * WNT][rr] : sm[o][rr];
                    float c2 = GATED ? sm[i * WNT + 1][rr] : 0.0f;
                    if constexpr (NORM) {
                        const float sc = row_ss[row_of(i, rr)];  // the row's scale by now
                        c *= sc;
                        c2 *= sc;
                    }
                    v[o][rr] += epilogue_set<FL>(c, c2, bv[j], flags);
                }
            }
#pragma unroll
            for (int o = 0; o < NO; o++) {
                const int i = GATED ? o : o / WNT, j = GATED ? 0 : o % WNT;
                const uint32_t gn = n0 + col_of(j);
                float *yc = a.y + static_cast<size_t>(m0 + row_of(i, 0)) * a.ldy + gn;
#pragma unroll
                for (int rr = 0; rr < 8; rr++) {
                    const uint32_t dr = 8 * (rr >> 2) + (rr & 3);
                    if (full || (m0 + row_of(i, rr) < M && gn < N)) yc[static_cast<size_t>(dr) * a.ldy] = v[o][rr];
                }
            }
        });
        return true;
    };
    if (kh == 0)
        finish(std::integral_constant<int, 0>{});
    else
        finish(std::integral_constant<int, 1>{});
}

typedef void (*tiled_fn)(TiledArgs);

// Tile shapes: (BM, BN) = (128, 128), (64, 128), (64, 64); gated always has BN = 128.  The
// waves of every tile split each stage's k between two 2 x 2 grids (512 threads).
constexpr int SHAPE_KS[3] = {2, 2, 2};
constexpr int SHAPE_BM[3] = {128, 64, 64};
constexpr int SHAPE_BN[3] = {128, 128, 64};

template <int WT, bool GATED, int P, int XT, bool NORM>
tiled_fn pick_shape(int shape) {
    if constexpr (GATED) {
        return shape == 0 ? tiled_kernel<WT, 128, 128, true, P, 2, XT, NORM> : tiled_kernel<WT, 64, 128, true, P, 2, XT, NORM>;
    } else {
        switch (shape) {
            case 0: return tiled_kernel<WT, 128, 128, false, P, 2, XT, NORM>;
            case 1: return tiled_kernel<WT, 64, 128, false, P, 2, XT, NORM>;
            default: return tiled_kernel<WT, 64, 64, false, P, 2, XT, NORM>;
        }
    }
}

}  // namespace tiled

// The kernel of an fp32-activation linear (linear_gemm_split.hip): weight type wt, gated,
// normed, tile shape, loop (stages 1: commits only the split's stages; 2: branch-free).
tiled::tiled_fn pick_tiled_split(int wt, bool gated, bool norm, int shape, int stages);

}  // namespace mt
