// Ring GEMM for the SiLU-gated prefill linear (gate|up) with x of the weights' 16-bit type, at
// M large enough that its output tiles fill the chip (mt_linear routes a gated linear here when
// its tiles fill at least three quarters of their last wave: gate|up at 448-640 rows, 1024).
//
// Reference kernel replaced: gemm_kernel<32,64,32,4> with the SiLU-gate epilogue
// (Shaders.swift:297-410), as QwenForward.dispatches calls it for gate|up (Qwen.swift:90).
//
// y[m][n] = epilogue(sum_k x[m][k] w[n][k], sum_k x[m][k] w2[n][k]) on one 512-thread workgroup
// per tile of 128 x rows and 96 features (192 weight rows: 32-row blocks of W and W2 for the
// same 32 features, alternating), so 2 x 4864 features at M = 512 make 204 tiles, one wave of
// workgroups on 256 CUs, where 64-feature tiles (304) would need two.
//   - One workgroup per CU (120 KB of LDS): a ring of three 64-k stages (40 KB each: the
//     tile's 128 x rows, then its 192 weight rows, 128 bytes a row) filled with direct-to-LDS
//     loads (global_load_lds_dwordx4).  The prologue fills all three; iteration s waits for
//     stage s + 1 with an exact vmcnt, meets at a bare s_barrier and refills stage s's slot
//     with stage s + 3.  __syncthreads would add the compiler's workgroup fence, which waits
//     for every load in flight (vmcnt(0)) and so drains the ring at each stage.
//   - Chunk c of row r of a stage sits in slot c ^ (r & 7) ^ ((r >> 3) & 1): the operand reads
//     (32 rows of one chunk per half-wave) are free of bank conflicts.
//   - Eight waves, two per SIMD: waves 0-3 multiply the 16-k steps 0-1 of every stage, waves
//     4-7 steps 2-3 (the other wave of a SIMD hides a wave's LDS reads).  Wave w owns x rows
//     32 (w & 3) .. + 31 against all 192 weight rows: six 32 x 32 accumulators on
//     v_mfma_f32_32x32x16, the gate and up sums of a feature in the same lane.  After the loop
//     the two groups swap halves of their sums through LDS (added in a fixed order: first group
//     + second), so all eight waves run the epilogue.
//   - The epilogue runs from registers: lane l holds D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32]
//     of each block, so each store writes two 128-byte row segments.  The old y (accumulate) is
//     requested while the groups' sums meet.  A wave issues about one instruction every four
//     cycles, so the epilogue's instruction count is its time: the flags are branched on once,
//     not per output, and SiLU takes the hardware exp2 and reciprocal (8.1 -> 2.2 us of a 24 us
//     launch at M = 512).
//   - Rows past M or N and k past K are loaded from a zero block; rows past M or N are not
//     stored.  The workgroup -> tile order gives each XCD a contiguous run of tiles (the x-row
//     tiles of one weight tile first), which share weight rows in that XCD's L2.
#pragma once

#include "tiled_kernel.hpp"

namespace mt {
namespace ring {

using tiled::f32x16t;
using tiled::u32x4t;
using tiled::f32x4t;

constexpr int BM = 128, BN = 192, FN = 96;  // x rows, weight rows, features per tile
constexpr int NS = 3;                        // LDS stages of 64 k
constexpr int NT = 512, NW = 8;              // threads, waves
constexpr int R = BM + BN;                   // rows of a stage
constexpr int SB = R * 128;                  // bytes of a stage
constexpr int LPW = R / (8 * NW);            // direct loads per wave per stage
constexpr int WNT = BN / 32;                 // 32-row weight blocks: g0 u0 g1 u1 g2 u2
constexpr int RED = 4 * WNT * 4096;          // the k groups' hand-over (bytes)
constexpr int LDS_BYTES = NS * SB > RED ? NS * SB : RED;
static_assert(LPW * 8 * NW == R && LDS_BYTES <= 160 * 1024 && (NS - 1) * LPW <= 63, "ring shape");

// Loaded in place of any 16-byte chunk outside the operands (one per code object).
static __device__ __attribute__((aligned(16))) uint32_t g_zero_ring[4];

struct RingArgs {
    const uint16_t *x, *w, *w2, *bias;
    float *y;
    uint32_t M, N, K, ldx, ldy, flags;
    uint32_t tiles_m, tiles_n;
    const float *xf;        // ring_split_kernel: fp32 x (x unused)
    const uint16_t *norm;   // ring_split_kernel: RMSNorm gain [K] (NORM)
    float eps;
};

__device__ __forceinline__ void bar() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The second half of the kernel for k group KH (see the call site): the hand-over through LDS,
// the epilogue and the stores.  Rows past M or features past N are neither read nor stored.
// NORM: each output is scaled by its row's RMSNorm scale rs[row of the tile] before the bias.
template <int WT, int KH, bool NORM = false>
__device__ __forceinline__ void finish(const RingArgs &a, const f32x16t (&acc)[WNT], uint8_t *lds, int wm, int lane,
                                       uint32_t m0, uint32_t n0, const float (&bv)[WNT / 2], const float *rs = nullptr) {
    const int fr = lane & 31, fh = lane >> 5;
    const uint32_t M = a.M, N = a.N, flags = a.flags;
    // Accumulator register r of this group's half is x row mb + 8 (r / 4) + r % 4.
    const uint32_t mb = m0 + 32 * wm + 16 * KH + 4 * fh;
    // The old y of this half's outputs (accumulate), requested before the hand-over.
    float yo[8][WNT / 2];
#pragma unroll
    for (int r = 0; r < 8; r++)
#pragma unroll
        for (int p = 0; p < WNT / 2; p++) yo[r][p] = 0.0f;
    if (flags & F_ACCUM) {
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const uint32_t m = mb + 8 * (r >> 2) + (r & 3);
#pragma unroll
            for (int p = 0; p < WNT / 2; p++) {
                const uint32_t n = n0 + 32 * p + fr;
                if (m < M && n < N) yo[r][p] = a.y[static_cast<size_t>(m) * a.ldy + n];
            }
        }
    }
    // Hand-over area: [wave & 3][giving group][block][register quad of the half][lane] float4.
    float *red = reinterpret_cast<float *>(lds);
    auto slot = [&](int giver, int j, int q) { return red + ((((wm * 2 + giver) * WNT + j) * 2 + q) * 64 + lane) * 4; };
    bar();  // every wave is done with the ring
    constexpr int GIVE = 8 * (1 - KH), KEEP = 8 * KH;
#pragma unroll
    for (int j = 0; j < WNT; j++)
#pragma unroll
        for (int q = 0; q < 2; q++)
            *reinterpret_cast<f32x4t *>(slot(KH, j, q)) = f32x4t{acc[j][GIVE + 4 * q], acc[j][GIVE + 4 * q + 1],
                                                                 acc[j][GIVE + 4 * q + 2], acc[j][GIVE + 4 * q + 3]};
    bar();
    // The sums in a fixed order, group 0's part first.
    float sm[WNT][8];
#pragma unroll
    for (int j = 0; j < WNT; j++)
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const f32x4t v = *reinterpret_cast<const f32x4t *>(slot(1 - KH, j, q));
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float own = acc[j][KEEP + 4 * q + e];
                sm[j][4 * q + e] = KH == 0 ? own + v[e] : v[e] + own;
            }
        }
    if constexpr (NORM) {
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const float sc = rs[32 * wm + 16 * KH + 4 * fh + 8 * (r >> 2) + (r & 3)];
#pragma unroll
            for (int j = 0; j < WNT; j++) sm[j][r] *= sc;
        }
    }
    float out[8][WNT / 2];
    if ((flags & (F_GELU | F_SILU)) == 0) {
#pragma unroll
        for (int r = 0; r < 8; r++)
#pragma unroll
            for (int p = 0; p < WNT / 2; p++) out[r][p] = silu_hw(sm[2 * p][r] + bv[p]) * sm[2 * p + 1][r] + yo[r][p];
    } else {
#pragma unroll
        for (int r = 0; r < 8; r++)
#pragma unroll
            for (int p = 0; p < WNT / 2; p++)
                out[r][p] = epilogue_out_of_line(sm[2 * p][r], sm[2 * p + 1][r], bv[p], flags) + yo[r][p];
    }
    if (m0 + BM <= M && n0 + FN <= N) {
#pragma unroll
        for (int r = 0; r < 8; r++) {
            float *yr = a.y + static_cast<size_t>(mb + 8 * (r >> 2) + (r & 3)) * a.ldy + n0 + fr;
#pragma unroll
            for (int p = 0; p < WNT / 2; p++) yr[32 * p] = out[r][p];
        }
    } else {
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const uint32_t m = mb + 8 * (r >> 2) + (r & 3);
            float *yr = a.y + static_cast<size_t>(m) * a.ldy;
#pragma unroll
            for (int p = 0; p < WNT / 2; p++) {
                const uint32_t n = n0 + 32 * p + fr;
                if (m < M && n < N) yr[n] = out[r][p];
            }
        }
    }
}

template <int WT>
__global__ __launch_bounds__(NT) void ring_gated_kernel(RingArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kh = wave >> 2, wm = wave & 3;

    const uint32_t t = tiled::xcd_order(blockIdx.x, gridDim.x);
    const uint32_t tm = t % a.tiles_m, tn = t / a.tiles_m;
    const uint32_t m0 = tm * BM, n0 = tn * FN;
    const uint32_t M = a.M, N = a.N, K = a.K;
    const uint32_t nsteps = (K + 63) / 64;

    // Direct loads: instruction i of this wave fills stage rows 8 (wave + NW i) .. + 7, the lane
    // slot lane & 7 of row 8 (wave + NW i) + lane / 8 with chunk (lane & 7) ^ g(row).
    const char *src[LPW];
    bool rowok[LPW];
    uint32_t ci[LPW];
    const uint32_t lds0 =
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void *)(lds)));
#pragma unroll
    for (int i = 0; i < LPW; i++) {
        const int r = 8 * (wave + NW * i) + (lane >> 3);
        ci[i] = (lane & 7) ^ (r & 7) ^ ((r >> 3) & 1);
        const uint16_t *base;
        uint32_t row, lim;
        size_t ld;
        if (r < BM) {
            base = a.x; row = m0 + r; lim = M; ld = a.ldx;
        } else {
            const int j = r - BM, b = j >> 5;
            base = (b & 1) ? a.w2 : a.w;
            row = n0 + 32 * (b >> 1) + (j & 31);
            lim = N; ld = K;
        }
        rowok[i] = row < lim;
        src[i] = reinterpret_cast<const char *>(base + static_cast<size_t>(rowok[i] ? row : 0) * ld + 8 * ci[i]);
    }
    const char *zero = reinterpret_cast<const char *>(g_zero_ring);
    auto issue = [&](uint32_t s) {
        const uint32_t k = s * 64;
#pragma unroll
        for (int i = 0; i < LPW; i++) {
            const char *g = (rowok[i] && k + 8 * ci[i] < K) ? src[i] + 2 * static_cast<size_t>(k) : zero;
            tiled::dma16(__builtin_amdgcn_readfirstlane(lds0 + (s % NS) * SB + (wave + NW * i) * 1024), g);
        }
    };
    // This wave's part of a stage has landed once at most `ahead` later stages are in flight.
    auto wait_ahead = [&](uint32_t ahead) {
        if (ahead >= 2) tiled::wait_vm<2 * LPW>();
        else if (ahead == 1) tiled::wait_vm<LPW>();
        else tiled::wait_vm<0>();
    };

    // Operand reads: row (l & 31) of a 32-row block, chunk 2 q + (l >> 5) of the stage (q = this
    // group's 16-k step), slot chunk ^ g(l & 31).
    const int fr = lane & 31, fh = lane >> 5;
    const uint32_t gsw = (fr & 7) ^ ((fr >> 3) & 1);
    const uint32_t cofs0 = ((2 * (2 * kh) + fh) ^ gsw) << 4, cofs1 = ((2 * (2 * kh + 1) + fh) ^ gsw) << 4;
    const uint32_t aoff = (32 * wm + fr) * 128;
    uint32_t boff[WNT];
#pragma unroll
    for (int j = 0; j < WNT; j++) boff[j] = (BM + 32 * j + fr) * 128;

    f32x16t acc[WNT];
#pragma unroll
    for (int j = 0; j < WNT; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[j][r] = 0.0f;
    struct Fr {
        u32x4t a[2], b[2][WNT];
    };
    auto rd = [&](Fr &f, uint32_t slot) {
        const uint8_t *st = lds + slot * SB;
        f.a[0] = *reinterpret_cast<const u32x4t *>(st + aoff + cofs0);
        f.a[1] = *reinterpret_cast<const u32x4t *>(st + aoff + cofs1);
#pragma unroll
        for (int j = 0; j < WNT; j++) {
            f.b[0][j] = *reinterpret_cast<const u32x4t *>(st + boff[j] + cofs0);
            f.b[1][j] = *reinterpret_cast<const u32x4t *>(st + boff[j] + cofs1);
        }
    };
    auto mma = [&](const Fr &f) {
#pragma unroll
        for (int q = 0; q < 2; q++)
#pragma unroll
            for (int j = 0; j < WNT; j++) acc[j] = tiled::mfma32x<WT>(f.a[q], f.b[q][j], acc[j]);
    };

    const uint32_t flags = a.flags;
    float bv[WNT / 2];
#pragma unroll
    for (int p = 0; p < WNT / 2; p++) {
        const uint32_t n = n0 + 32 * p + fr;
        bv[p] = (flags & F_BIAS) && n < N ? dec1<WT>(a.bias[n]) : 0.0f;
    }

    if (nsteps > 0) {
        // Direct loads step by 128 bytes a stage from each lane's source row; a row past M or N
        // reads row 0 instead of the zero block (its outputs are never stored), so only a K
        // tail takes the checked issue, and an iteration costs a few uniform branches instead
        // of per-load selects (a wave issues about one instruction every four cycles).
        const uint32_t ldsw = __builtin_amdgcn_readfirstlane(lds0 + wave * 1024);
        const bool ktail = (K % 64) != 0;
        auto issue_fast = [&](uint32_t s, uint32_t slot) {
#pragma unroll
            for (int i = 0; i < LPW; i++) tiled::dma16(ldsw + slot * SB + NW * i * 1024, src[i] + 128 * static_cast<size_t>(s));
        };
        // Stages below `fast_end` take the unchecked issue.
        const uint32_t fast_end = ktail ? nsteps - 1 : nsteps;
#pragma unroll
        for (int s = 0; s < NS; s++)
            if (static_cast<uint32_t>(s) < nsteps) {
                if (static_cast<uint32_t>(s) < fast_end) issue_fast(s, s);
                else issue(s);
            }
        wait_ahead(min(static_cast<uint32_t>(NS - 1), nsteps - 1));
        bar();
        Fr f;
        rd(f, 0);
        // Iteration s: stage s + 1 is in once the stages after it are the only ones in flight;
        // the barrier also tells that every wave has read stage s, whose slot takes stage s + NS.
        // One call site of the MFMAs: with a second one (a peeled tail loop) the compiler gave
        // the accumulators a second register set and spilled.
        uint32_t slot = 0;  // slot of stage s
        for (uint32_t s = 0; s < nsteps; s++) {
            const uint32_t next = slot + 1 == NS ? 0 : slot + 1;
            mma(f);
            if (s + NS < nsteps) {
                tiled::wait_vm<(NS - 2) * LPW>();
                bar();
                if (s + NS < fast_end) issue_fast(s + NS, slot);
                else issue(s + NS);
                rd(f, next);
            } else if (s + 1 < nsteps) {
                wait_ahead(nsteps - 1 - (s + 1));
                bar();
                rd(f, next);
            }
            slot = next;
        }
    }

    // The two k groups' sums meet through LDS, each group finishing half of the accumulator
    // registers: group kh keeps registers 8 kh .. 8 kh + 7 of every block (x rows 16 kh .. +15
    // of its 32-row block) and hands the other half to its partner wave.  Both groups then run
    // the epilogue, 24 outputs a lane.  kh becomes a compile-time constant through the two
    // instantiations of `finish`, so every register index stays a constant (a kh-dependent index
    // turns into select chains over all 16 registers).
    if (kh == 0)
        finish<WT, 0>(a, acc, lds, wm, lane, m0, n0, bv);
    else
        finish<WT, 1>(a, acc, lds, wm, lane, m0, n0, bv);
}

// The same tiles for x in fp32 (the reference's activation type), with or without the fused
// RMSNorm (RingArgs::xf, ::norm, ::eps): x travels through registers, is multiplied by the norm
// gain, and is staged as hi + lo halves of the weights' type (hi = round(x), lo = round(x - hi):
// 2^-22 relative with fp16), so each 16-k step takes two MFMAs per weight fragment.  A stage
// holds the tile's 128 hi rows, its 128 lo rows and its 192 weight rows (56 KB); two stages
// alternate in LDS, and the next stage's loads travel in registers while a stage multiplies
// (the compiler sees every load and places exact waits).  The rows' sums of x^2 are summed by
// the eight threads of a row (a lane octet) and turned into scales before the epilogue.
constexpr int SX = 2 * BM + BN;          // rows of a split stage (hi, lo, weights)
constexpr int SSB = SX * 128;            // bytes of a split stage
constexpr int SIA = BM * 8 / NT;         // 8-k activation items per thread per stage
constexpr int SWL = BN * 8 / NT;         // 16-byte weight chunks per thread per stage
static_assert(SIA * NT == BM * 8 && SWL * NT == BN * 8 && 2 * SSB >= RED && 2 * SSB <= 160 * 1024, "split ring shape");

template <int WT, bool NORM>
__global__ __launch_bounds__(NT) void ring_split_kernel(RingArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * SSB];
    __shared__ __attribute__((aligned(16))) float rs[BM];  // rows' scales (NORM)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kh = wave >> 2, wm = wave & 3;
    const uint32_t t = tiled::xcd_order(blockIdx.x, gridDim.x);
    const uint32_t tm = t % a.tiles_m, tn = t / a.tiles_m;
    const uint32_t m0 = tm * BM, n0 = tn * FN;
    const uint32_t M = a.M, N = a.N, K = a.K;
    const uint32_t nsteps = (K + 63) / 64;
    const char *zero = reinterpret_cast<const char *>(g_zero_ring);
    typedef const __attribute__((address_space(1))) u32x4t *gp;
    auto ld16 = [](const void *p) { return *reinterpret_cast<gp>(reinterpret_cast<uintptr_t>(p)); };

    // Activation item j of this thread: row (tid + NT j) / 8, k 8 (tid % 8) of every stage.
    const uint32_t kc = tid & 7;
    const float *xrow[SIA];
    bool xok[SIA];
    uint32_t xoff[SIA];  // LDS byte offset of the item's hi chunk in a stage
#pragma unroll
    for (int j = 0; j < SIA; j++) {
        const uint32_t r = (tid + NT * j) >> 3, m = m0 + r;
        xok[j] = m < M;
        xrow[j] = a.xf + static_cast<size_t>(xok[j] ? m : 0u) * a.ldx + 8 * kc;
        xoff[j] = r * 128 + ((kc ^ (r & 7) ^ ((r >> 3) & 1)) << 4);
    }
    // Weight chunk i of this thread: stage weight row c / 8 (32-row blocks g0 u0 g1 u1 g2 u2),
    // slot c % 8, holding chunk (c % 8) ^ g(row) of the row.
    const char *wsrc[SWL];
    bool wok[SWL];
    uint32_t wci[SWL], woff[SWL];
#pragma unroll
    for (int i = 0; i < SWL; i++) {
        const uint32_t c = tid + NT * i, j = c >> 3, b = j >> 5, r = 2 * BM + j;
        wci[i] = (c & 7) ^ (r & 7) ^ ((r >> 3) & 1);
        const uint32_t n = n0 + 32 * (b >> 1) + (j & 31);
        wok[i] = n < N;
        wsrc[i] = reinterpret_cast<const char *>(((b & 1) ? a.w2 : a.w) + static_cast<size_t>(wok[i] ? n : 0u) * K + 8 * wci[i]);
        woff[i] = r * 128 + (c & 7) * 16;
    }
    struct Stage {
        u32x4t x[SIA][2], w[SWL], g;
    };
    auto gload = [&](Stage &st, uint32_t s) {
        const uint32_t k = s * 64;
#pragma unroll
        for (int i = 0; i < SWL; i++)
            st.w[i] = __builtin_nontemporal_load(reinterpret_cast<gp>(reinterpret_cast<uintptr_t>(
                wok[i] && k + 8 * wci[i] < K ? wsrc[i] + 2 * static_cast<size_t>(k) : zero)));
        const uint32_t kx = k + 8 * kc;
        const bool kok = kx < K;
#pragma unroll
        for (int j = 0; j < SIA; j++) {
            const bool ok = kok && xok[j];
            st.x[j][0] = ld16(ok ? static_cast<const void *>(xrow[j] + k) : zero);
            st.x[j][1] = ld16(ok ? static_cast<const void *>(xrow[j] + k + 4) : zero);
        }
        if constexpr (NORM) st.g = ld16(kok ? static_cast<const void *>(a.norm + kx) : zero);
    };
    float ss[SIA];
#pragma unroll
    for (int j = 0; j < SIA; j++) ss[j] = 0.0f;
    auto commit = [&](const Stage &st, uint32_t buf) {
        uint8_t *sb = lds + buf * SSB;
#pragma unroll
        for (int i = 0; i < SWL; i++) *reinterpret_cast<u32x4t *>(sb + woff[i]) = st.w[i];
#pragma unroll
        for (int j = 0; j < SIA; j++) {
            float x[8];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                x[e] = __uint_as_float(st.x[j][0][e]);
                x[4 + e] = __uint_as_float(st.x[j][1][e]);
            }
            if constexpr (NORM) {
#pragma unroll
                for (int e = 0; e < 8; e++) ss[j] = fmaf(x[e], x[e], ss[j]);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    x[2 * e] *= dec_lo<WT>(st.g[e]);
                    x[2 * e + 1] *= dec_hi<WT>(st.g[e]);
                }
            }
            u32x4t hi, lo;
            tiled::split8<WT>(x, hi, lo);
            *reinterpret_cast<u32x4t *>(sb + xoff[j]) = hi;
            *reinterpret_cast<u32x4t *>(sb + BM * 128 + xoff[j]) = lo;
        }
    };

    // Operand reads: row fr of a 32-row block, chunk 2 q + fh of the stage (q: this group's 16-k
    // step), slot chunk ^ g(fr).
    const int fr = lane & 31, fh = lane >> 5;
    const uint32_t gsw = (fr & 7) ^ ((fr >> 3) & 1);
    const uint32_t cofs0 = ((2 * (2 * kh) + fh) ^ gsw) << 4, cofs1 = ((2 * (2 * kh + 1) + fh) ^ gsw) << 4;
    const uint32_t aoff = (32 * wm + fr) * 128;
    f32x16t acc[WNT];
#pragma unroll
    for (int j = 0; j < WNT; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[j][r] = 0.0f;
    struct Fr {
        u32x4t a[2][2], b[2][WNT];  // [16-k step][hi, lo], [16-k step][block]
    };
    auto rd = [&](Fr &f, uint32_t buf) {
        const uint8_t *st = lds + buf * SSB;
        f.a[0][0] = *reinterpret_cast<const u32x4t *>(st + aoff + cofs0);
        f.a[0][1] = *reinterpret_cast<const u32x4t *>(st + BM * 128 + aoff + cofs0);
        f.a[1][0] = *reinterpret_cast<const u32x4t *>(st + aoff + cofs1);
        f.a[1][1] = *reinterpret_cast<const u32x4t *>(st + BM * 128 + aoff + cofs1);
#pragma unroll
        for (int j = 0; j < WNT; j++) {
            const uint32_t bo = (2 * BM + 32 * j + fr) * 128;
            f.b[0][j] = *reinterpret_cast<const u32x4t *>(st + bo + cofs0);
            f.b[1][j] = *reinterpret_cast<const u32x4t *>(st + bo + cofs1);
        }
    };
    auto mma = [&](const Fr &f) {
#pragma unroll
        for (int q = 0; q < 2; q++) {  // hi then lo on each block; the blocks' MFMAs interleave
#pragma unroll
            for (int j = 0; j < WNT; j++) acc[j] = tiled::mfma32x<WT>(f.a[q][0], f.b[q][j], acc[j]);
#pragma unroll
            for (int j = 0; j < WNT; j++) acc[j] = tiled::mfma32x<WT>(f.a[q][1], f.b[q][j], acc[j]);
        }
    };

    const uint32_t flags = a.flags;
    float bv[WNT / 2];
#pragma unroll
    for (int p = 0; p < WNT / 2; p++) {
        const uint32_t n = n0 + 32 * p + fr;
        bv[p] = (flags & F_BIAS) && n < N ? dec1<WT>(a.bias[n]) : 0.0f;
    }

    if (nsteps > 0) {
        // Stage s in buffer s % 2; the registers hold stage s + 1 while stage s multiplies.  The
        // barrier after a commit tells that the stage is in and that every wave has read the
        // other buffer's fragments (read before its MFMAs), which the next commit overwrites.
        Stage st;
        gload(st, 0);
        commit(st, 0);
        if (nsteps > 1) gload(st, 1);
        __syncthreads();
        Fr f;
        rd(f, 0);
        for (uint32_t s = 0; s < nsteps; s++) {
            mma(f);
            if (s + 1 < nsteps) {
                commit(st, (s + 1) & 1);
                if (s + 2 < nsteps) gload(st, s + 2);
                __syncthreads();
                rd(f, (s + 1) & 1);
            }
        }
    }
    if constexpr (NORM) {
        // A row's eight threads are an aligned lane octet.
#pragma unroll
        for (int j = 0; j < SIA; j++) {
            const float tsum = octet_sum(ss[j]);
            if (kc == 0) rs[(tid + NT * j) >> 3] = rsqrt_hw(tsum / static_cast<float>(K) + a.eps);
        }
    }
    // finish's first barrier also publishes the row scales.
    if (kh == 0)
        finish<WT, 0, NORM>(a, acc, lds, wm, lane, m0, n0, bv, rs);
    else
        finish<WT, 1, NORM>(a, acc, lds, wm, lane, m0, n0, bv, rs);
}

typedef void (*ring_fn)(RingArgs);

}  // namespace ring

// The gated ring kernel for weights (and x) of type wt.
ring::ring_fn pick_ring_gated(int wt);
// The gated ring kernel for fp32 x, weights of type wt, with or without the fused RMSNorm.
ring::ring_fn pick_ring_split(int wt, bool norm);

}  // namespace mt
