// Persistent decode step of a Qwen2-0.5B-shaped layer stack: mt_seq_* plans whose linears
// repeat the layer of QwenForward.dispatches (Qwen.swift:84-91) at the backbone's shapes
// (Weights.swift:81-92):
//     qkv     1152 x 896, bias, RMSNorm fused        (Qwen.swift:85)
//     o        896 x 896, += residual                (Qwen.swift:88)
//     gate|up 2 x 4864 x 896, SiLU-gate, RMSNorm     (Qwen.swift:90)
//     down     896 x 4864, += residual               (Qwen.swift:91)
// at M = 1, 2 or 4 rows, optionally with the layer's decode attention (rope_cache + attention,
// Qwen.swift:86-87) as an item between qkv and o (ATT: then 5 ops per layer).  It runs the dataflow of seq_kernel (tagged activation words, one
// workgroup per CU, every wave computing a share of every op, two workgroup barriers per op)
// with every op's shape known at compile time, on 7 waves (448 threads):
//   - each op class has a fixed tiling (below); a wave's tile range, its lanes' weight and
//     activation addresses are computed once at kernel start, so per op a wave adds one
//     64-bit base to a lane offset and issues its weight tiles with immediate offsets;
//   - every wave loads exactly TA tiles of an op (a wave with fewer tiles loads its
//     neighbours' blocks and skips their MFMAs), so the number of loads in flight behind
//     the activations is the same on every path and the wait for the activations waits
//     for nothing issued after them;
//   - the epilogue flags are constants; no lane-divergent branch surrounds a load;
//   - the weight tiles of later ops are requested in batches spread over the layer's four
//     ops (the kernel's schedule), each issued where it delays the fewest activation polls
//     and output stores (see lay_step).
// Tiling (v_mfma_f32_16x16x32: A = 16 weight rows x 32 k, one 16-byte chunk per lane; B =
// 32 k x 16 columns of activations as hi + lo halves of the weights' 16-bit type; see
// seq_tiles.hpp for the segment interleave):
//   qkv     S = 2 K-segments per row tile, 8 features, its 14 block steps 2 per wave;
//   o       S = 4, 4 features (a workgroup's whole share), block steps split over the 7
//           waves; at M = 4 the B operand's 16 columns hold rows 0-1 and a second MFMA on
//           the same weight tile takes rows 2-3 (two column groups);
//   gate|up S = 1, three row tiles of 8 gate rows and the same features' 8 up rows; the
//           84 block steps of the three row tiles in runs of 12 per wave;
//   down    split over K between the two workgroups of a pair: S = 2 over the workgroup's
//           half of K (2432), 8 features (the pair's share), its 76 block steps split over
//           the 7 waves; it stages and reads only its half of x.  Its output is two tagged
//           planes, the first half's sums plus the residual and the second half's sums, added
//           in that order by the next qkv (its x) and o (its old y); the second half writes a
//           final user output once the first half's word is current.
// A wave's partial sums go to its own slot of the op class's LDS area; one lane per output
// adds the 8 slots in slot order (slots no wave writes stay zero), so results are the same
// on every run.  A workgroup owns features [g N / G, (g + 1) N / G) of every op (down: pair
// g / 2 of G / 2), which the tiling holds for even 224 <= G <= 256 (the host checks it).
#pragma once

#include "dit_attend.hpp"
#include "seq_kernel.hpp"

namespace mt {

// Op classes: the Qwen2-0.5B decode layer's four, and the four linears of a DiT block (the
// DiT-block kernel below).  A kernel runs one set of four; SLOT indexes its per-class state.
enum : int { LC_QKV = 0, LC_O = 1, LC_GU = 2, LC_DOWN = 3, LC_DQKV = 4, LC_DO = 5, LC_FF1 = 6, LC_FF2 = 7 };

// Compile-time shape and tiling of op class C at M rows.
template <int C, int M>
struct LCls {
    static constexpr bool DIT = C >= LC_DQKV;
    static constexpr int SLOT = C & 3;
    static constexpr uint32_t N = C == LC_QKV ? LAY_QKV : C == LC_GU ? LAY_I : C == LC_DQKV ? DIT_QKV
                                : C == LC_FF1 ? DIT_FF : DIT ? DIT_H : LAY_H;
    static constexpr uint32_t K = C == LC_DOWN ? LAY_I : C == LC_FF2 ? DIT_FF : DIT ? DIT_H : LAY_H;
    static constexpr bool GATED = C == LC_GU;
    static constexpr bool NORM = C == LC_QKV || C == LC_GU || C == LC_DQKV || C == LC_FF1;
    static constexpr bool BIAS = C == LC_QKV || DIT;
    static constexpr bool ACC = C == LC_O || C == LC_DOWN || C == LC_DO || C == LC_FF2;
    static constexpr bool GELU = C == LC_FF1;
    // x is the DiT attention of the block's qkv, computed by the workgroup while staging.
    static constexpr bool ATTX = C == LC_DO;
    static constexpr uint32_t FLAGS =
        (BIAS ? F_BIAS : 0u) | (ACC ? F_ACCUM : 0u) | (GATED ? F_SILU_GATE : 0u) | (GELU ? F_GELU : 0u);
    // down is split over K between the two workgroups of a pair (g, g ^ 1): each owns the
    // pair's features over its half of K, and reads only that half of x.  Its outputs are
    // two tagged planes (the residual plus the first half's sums; the second half's sums),
    // which the next qkv (x, X2) and o (old y, Y2) add as they read them.
    // The DiT block's ff2 (4096 k) is split the same way; the next block's qkv and out add its
    // two planes.
    static constexpr uint32_t KSPLIT = C == LC_DOWN || C == LC_FF2 ? 2u : 1u;
    static constexpr uint32_t KX = K / KSPLIT;              // k a workgroup stages and sums
    static constexpr bool X2 = C == LC_QKV || C == LC_DQKV, Y2 = C == LC_O || C == LC_DO;  // may read two planes
    static constexpr uint32_t PL = M * (DIT ? DIT_H : LAY_H);  // words between a split op's two planes
    static constexpr uint32_t S = GATED || C == LC_DQKV || C == LC_FF1 ? 1u
                                : C == LC_QKV || C == LC_DOWN || C == LC_FF2 ? 2u : 4u;
    static constexpr uint32_t LS = S == 4 ? 2u : S == 2 ? 1u : 0u;
    static constexpr uint32_t CG = (2 * S * M + 15) / 16;  // B column groups (MFMAs per weight tile)
    static constexpr uint32_t RPG = M / CG;                 // x rows per column group
    static constexpr uint32_t KB = KX / 32, KBS = KB / S;
    static constexpr uint32_t FPT = GATED ? 8u : 16u / S;  // features per row tile
    static constexpr uint32_t RT = GATED ? 3u : 1u;         // row tiles
    static constexpr uint32_t NMAX = FPT * RT;              // features a workgroup can own
    // Tiles a compute wave loads: gate|up's RT KBS tiles split evenly over the 7 compute waves;
    // otherwise the most block steps any wave has.
    static constexpr uint32_t TA = GATED ? RT * KBS / 7 : (KBS + 6) / 7;
    static constexpr uint32_t K4 = KX / 4, NCH = M * K4;    // 16-byte x chunks of the op
    static constexpr uint32_t XR = (NCH + 447) / 448;       // x chunks per compute thread
    // LDS partial sums: [row tile][x row][virtual row][slot]
    static constexpr uint32_t VR = GATED ? 16u : FPT;
    static constexpr uint32_t PART = RT * M * VR * 8;
    // Column groups after the first start RPG rows further on; a group's 16 columns hold RPG rows
    // (the columns past 2 S RPG read row 0 and are not flushed).
    static_assert(KB % S == 0 && 2 * S * RPG <= 16 && (CG == 1 || 2 * S * RPG > 8) && RPG * CG == M && CG <= 3, "tiling");
    static_assert((!GATED || RT * KBS % 7 == 0) && (CG == 1 || !GATED), "tiling");
};

constexpr int LAY_CW = 7;  // waves of a workgroup (the block steps of qkv and o split evenly)
constexpr int LAY_THREADS = LAY_CW * 64;


// The fields of one op the kernel reads, packed for one scalar load (built by the plan
// compiler next to the op descriptors).  Tagged positions are word offsets into the plan's
// tag buffer.
// LAY_X2 / LAY_Y2: x / the old y is down's output, two tagged planes M LAY_H words apart.
enum : uint32_t { LAY_XEXT = 1, LAY_YEXT = 2, LAY_FINAL = 4, LAY_X2 = 8, LAY_Y2 = 16 };
struct LayOp {
    const uint16_t *w;     // weights (gate|up: the gate rows)
    const uint16_t *p2;    // gate|up: W2 (the up rows); qkv: the bias
    const uint16_t *norm;  // RMSNorm gain [K], or null
    float *y;              // user output (final op) and user old y (LAY_YEXT)
    uint32_t xoff, xld;    // tagged x, unless LAY_XEXT (then the op descriptor's x)
    uint32_t yoff, yld;    // tagged old y of an accumulate, unless LAY_YEXT
    uint32_t ldy;
    uint32_t tag;          // this op's tagged output [M][N]
    float eps;
    uint32_t flags;
};
static_assert(sizeof(LayOp) == 64, "one 64-byte scalar load");

// Compute wave w's share of an op class.  It loads TA tiles: block steps js .. of row tile
// rt, the first ks of them; gate|up's remaining TA - ks continue at block 0 of row tile
// rt + 1.  It multiplies loaded tiles [kb, ke) (a wave with fewer block steps than TA loads
// its neighbour's first ones and skips them), and its partial sums go to slot w.
struct LRange {
    uint32_t js, kb, ke, ks, rt;
};
template <int C, int M>
__host__ __device__ constexpr LRange lay_range(uint32_t w) {
    typedef LCls<C, M> L;
    if (L::GATED) {  // tiles [TA w, TA (w + 1)) of the RT KBS, row tile by row tile
        const uint32_t t0 = L::TA * w, rt = t0 / L::KBS, js = t0 - rt * L::KBS;
        const uint32_t ks = L::KBS - js < L::TA ? L::KBS - js : L::TA;
        return LRange{js, 0, L::TA, ks, rt};
    }
    const uint32_t j0 = w * L::KBS / LAY_CW, j1 = (w + 1) * L::KBS / LAY_CW;
    const uint32_t js = j0 < L::KBS - L::TA ? j0 : L::KBS - L::TA;
    return LRange{js, j0 - js, j1 - js, L::TA, 0};
}

// Per-lane constants of an op class: byte offsets of the lane's weight chunk at its first
// block step (woff: row tile rt; woff2: block 0 of row tile rt + 1, gate|up) and of its
// first B chunk in the staging.
struct LLane {
    uint32_t woff, woff2, boff;
};
template <int C, int M>
__device__ __forceinline__ uint32_t lay_row(uint32_t nr, uint32_t lane, uint32_t rt) {
    typedef LCls<C, M> L;
    const uint32_t a = lane & 15;
    // gate|up: rows 0-7 of a row tile are the gate rows of features 8 rt + a, rows 8-15 the
    // same features' up rows; otherwise row a is feature a / S over segment a % S.
    const uint32_t f = L::GATED ? rt * 8 + (a & 7) : a >> L::LS;
    return f < nr ? f : nr - 1;  // padding rows repeat the last feature (their sums are not used)
}
template <int C, int M>
__device__ __forceinline__ LLane lay_lane(uint32_t r0, uint32_t nr, uint32_t lane, const LRange &r, uint32_t plane,
                                          uint32_t kh = 0) {
    typedef LCls<C, M> L;
    const uint32_t a = lane & 15, q = lane >> 4;
    const uint32_t k = kh + (L::GATED ? 0u : (a & (L::S - 1)) * L::KBS * 32) + q * 8;
    LLane ll;
    ll.woff = ((r0 + lay_row<C, M>(nr, lane, r.rt)) * L::K + k + r.js * 32) * 2;
    ll.woff2 = L::GATED ? ((r0 + lay_row<C, M>(nr, lane, r.rt + 1 < L::RT ? r.rt + 1 : r.rt)) * L::K + k) * 2 : ll.woff;
    // B column c: x row m, segment s, half h (c = 2 (m S + s) + h) of column group 0 (rows
    // RPG .. 2 RPG - 1 of group 1 sit RPG rows further on); columns past RPG S read row 0.
    const uint32_t c = lane & 15, cc = c >> 1, h = c & 1, s = cc & (L::S - 1);
    uint32_t m = cc >> L::LS;
    m = m < L::RPG ? m : 0u;
    ll.boff = (h * plane + m * L::KX + s * L::KBS * 32 + q * 8 + r.js * 32) * 2;
    return ll;
}

// Workgroup state shared by the op steps.
template <int WT, int M>
struct LayCtx {
    // hi / lo planes of the x staging (elements): down's x; M = 6 runs only the DiT-block
    // kernel, whose widest staged x is ff2's half of K.
    static constexpr uint32_t PLANE = M * (M > 4 ? DIT_FF / 2 : LAY_I) + 64;
    uint16_t *xs;    // [2][PLANE] staged x of the current op
    float *qs;       // DiT-block kernel: the block's qkv [M][DIT_QKV] for its attention
    float *part[4];  // per class slot: [row tile][x row][virtual row][8 slots]
    float *ssw[4];   // per norm class slot: [M][8 slots] sums of x^2
    LLane ln[4];
    uint32_t r0[4], nr[4];
    uint32_t tid, lane, w, parity, g;
    uint32_t kh, half;  // down: this workgroup's half of K (its first k, and 0 / 1)
    // DiT-block kernel: the attention's RoPE table [cos, sin][pair p < 32][position j < S] and
    // its score scale.
    const float *rope;
    float ascale;
    bool up;         // gate|up: the lane's tile rows are W2's
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t *tags;
    uint32_t *sync;
    bool gave_up;
};

// Weight tiles [K0, K1) of an op of class C (weights w, and w2 for gate|up's up rows) for wave
// W into An.
template <int WT, int M, int C, int W, uint32_t K0, uint32_t K1, int NN>
__device__ __forceinline__ void lay_tiles_w(const LayCtx<WT, M> &cx, const uint16_t *w, const uint16_t *w2,
                                            u32x4 (&An)[NN]) {
    typedef LCls<C, M> L;
    static_assert(K1 <= L::TA && L::TA <= NN, "tile registers");
    constexpr LRange r = lay_range<C, M>(W);
    const uint16_t *base = (L::GATED && cx.up) ? w2 : w;
    const char *p = reinterpret_cast<const char *>(base) + cx.ln[L::SLOT].woff;
    const char *p2 = reinterpret_cast<const char *>(base) + cx.ln[L::SLOT].woff2;
    // The decode layers stream their weights (719 MB a step at M = 2) nontemporal.  The DiT
    // blocks' weights (about 200 MB for the 8 blocks of the flow head) are read again at every
    // ODE step and fit MI355X's 256 MB memory-side cache, so they are loaded with the default
    // policy, which lets them stay there (flow stage 2.65 -> 2.42 ms, aggregator 177 -> 162 us).
#pragma unroll
    for (uint32_t k = K0; k < K1; k++) {
        const char *a = k < r.ks ? p + k * 64 : p2 + (k - r.ks) * 64;
        if constexpr (L::DIT)
            An[k] = *reinterpret_cast<gw_cp>(reinterpret_cast<uintptr_t>(a));
        else
            An[k] = __builtin_nontemporal_load(reinterpret_cast<gw_cp>(reinterpret_cast<uintptr_t>(a)));
    }
}
// Tiles [K0, K1) of the op with packed descriptor d, for the calling wave.
template <int WT, int M, int C, uint32_t K0, uint32_t K1, int NN>
__device__ __forceinline__ void lay_tiles(const LayCtx<WT, M> &cx, const LayOp &d, u32x4 (&An)[NN]) {
    if constexpr (K0 >= K1) {
        return;
    } else if constexpr (!LCls<C, M>::GATED) {
        lay_tiles_w<WT, M, C, 0, K0, K1>(cx, d.w, d.p2, An);  // one row tile: the lane offsets carry the range
    } else {
        switch (cx.w) {
            case 0: lay_tiles_w<WT, M, C, 0, K0, K1>(cx, d.w, d.p2, An); break;
            case 1: lay_tiles_w<WT, M, C, 1, K0, K1>(cx, d.w, d.p2, An); break;
            case 2: lay_tiles_w<WT, M, C, 2, K0, K1>(cx, d.w, d.p2, An); break;
            case 3: lay_tiles_w<WT, M, C, 3, K0, K1>(cx, d.w, d.p2, An); break;
            case 4: lay_tiles_w<WT, M, C, 4, K0, K1>(cx, d.w, d.p2, An); break;
            case 5: lay_tiles_w<WT, M, C, 5, K0, K1>(cx, d.w, d.p2, An); break;
            default: lay_tiles_w<WT, M, C, 6, K0, K1>(cx, d.w, d.p2, An); break;
        }
    }
}

// Flush of one row tile's accumulator into slot `slot`: part[rt][m][v][slot], x rows m0 + ...
// (m0: the column group's first row).
template <int M, int C>
__device__ __forceinline__ void lay_flush(const f32x4 acc, float *part, uint32_t rt, uint32_t slot, uint32_t lane,
                                          uint32_t m0 = 0) {
    typedef LCls<C, M> L;
    float *pp = part + rt * (M * L::VR * 8) + slot;
    const uint32_t c = lane & 15, qd = lane >> 4;
    if constexpr (L::S == 1) {  // rows 4 qd + i, columns 2 m + h
        const uint32_t m = c >> 1;
        const float e0 = dpp_pair(acc[0]), e1 = dpp_pair(acc[1]), e2 = dpp_pair(acc[2]), e3 = dpp_pair(acc[3]);
        if ((c & 1) == 0 && m < static_cast<uint32_t>(M)) {
            float *q = pp + (m * L::VR + qd * 4) * 8;
            q[0] = e0;
            q[8] = e1;
            q[16] = e2;
            q[24] = e3;
        }
    } else if constexpr (L::S == 2) {  // rows 4 qd + i: virtual row 2 qd + i / 2, segment i % 2
        const uint32_t sc = (c >> 1) & 1, mg = c >> 2, m = m0 + mg;
        const float e0 = dpp_quad(sc ? acc[1] : acc[0]);
        const float e1 = dpp_quad(sc ? acc[3] : acc[2]);
        if ((c & 3) == 0 && mg < L::RPG && m < static_cast<uint32_t>(M)) {
            float *q = pp + (m * L::VR + 2 * qd) * 8;
            q[0] = e0;
            q[8] = e1;
        }
    } else {  // S == 4: rows 4 qd + i: virtual row qd, segment i
        const uint32_t sc = (c >> 1) & 3, m = m0 + (c >> 3);
        const float e = dpp_oct(sc == 0 ? acc[0] : sc == 1 ? acc[1] : sc == 2 ? acc[2] : acc[3]);
        if ((c & 7) == 0 && m < static_cast<uint32_t>(M)) pp[(m * L::VR + qd) * 8] = e;
    }
}

// Compute wave W's MFMAs of an op of class C (loaded tiles [kb, ke) of A, B from the
// staging) and the flush of its partial sums into slot W of its row tile(s).
template <int WT, int M, int C, int W, int NA>
__device__ __forceinline__ void lay_mma(const LayCtx<WT, M> &cx, const u32x4 (&A)[NA]) {
    typedef LCls<C, M> L;
    constexpr LRange r = lay_range<C, M>(W);
    const char *bp = reinterpret_cast<const char *>(cx.xs) + cx.ln[L::SLOT].boff;
    constexpr uint32_t GOFF = L::RPG * L::KX * 2;  // bytes from one column group's rows to the next's
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, acc2 = acc, accg = acc, accg2 = acc;
#pragma unroll
    for (uint32_t k = r.kb; k < r.ke; k++) {  // block js + k of row tile rt, or k - ks of rt + 1
        const char *b = k < r.ks ? bp + k * 64 : bp + (static_cast<int>(k - r.ks) - static_cast<int>(r.js)) * 64;
        const u32x4 bv = *reinterpret_cast<const u32x4 *>(b);
        if (k < r.ks) acc = mfma16<WT>(A[k], bv, acc);
        else acc2 = mfma16<WT>(A[k], bv, acc2);
        if constexpr (L::CG >= 2) accg = mfma16<WT>(A[k], *reinterpret_cast<const u32x4 *>(b + GOFF), accg);
        if constexpr (L::CG >= 3) accg2 = mfma16<WT>(A[k], *reinterpret_cast<const u32x4 *>(b + 2 * GOFF), accg2);
    }
    float *part = cx.part[L::SLOT];
    lay_flush<M, C>(acc, part, r.rt, W, cx.lane);
    if constexpr (r.ks < L::TA) lay_flush<M, C>(acc2, part, r.rt + 1, W, cx.lane);
    if constexpr (L::CG >= 2) lay_flush<M, C>(accg, part, r.rt, W, cx.lane, L::RPG);
    if constexpr (L::CG >= 3) lay_flush<M, C>(accg2, part, r.rt, W, cx.lane, 2 * L::RPG);
}

// The DiT attention that a DiT block's out projection stages as its x (DiT-block kernel; the
// attention of dit_attend.hpp: interleaved RoPE, fp32 scores scaled after the dot, max-subtracted
// softmax, fp32 p.v, with each dot summed in its own order), for B sequences of S rows at M = B S:
// (2, 3) in the flow loop, (1, 2) in the aggregator.  Each workgroup reads the block's whole
// tagged qkv (M rows of 3 H 64 words) in 16-byte chunks, chunk e = tid + 448 r, as the other ops
// read their x, and stages it in LDS (cx.qs); then each octet of lanes takes a (sequence, head)
// group, read from the staging.  So the attention adds no exchange between workgroups, and a
// lane holds 16-byte chunks (11 at M = 6) rather than every pair of its groups in registers.
template <int M>
struct DitAtt {
    static constexpr uint32_t S = M == 6 ? 3u : 2u, B = M / S;
    static constexpr uint32_t GROUPS = B * DIT_HEADS;
    static constexpr uint32_t W = DIT_QKV;                   // words of a qkv row
    static constexpr uint32_t NCH = M * W / 4;               // 16-byte chunks of the qkv
    static constexpr uint32_t XA = (NCH + LAY_THREADS - 1) / LAY_THREADS;  // chunks a thread reads
};

// Byte offset in the tag buffer of qkv chunk e (d.xoff / d.xld locate the block's qkv output);
// past the chunks an offset outside the buffer, which reads 0.
template <int M>
__device__ __forceinline__ uint32_t dit_att_off(const LayOp &d, uint32_t e) {
    typedef DitAtt<M> D;
    const uint32_t m = e / (D::W / 4), k = (e - m * (D::W / 4)) * 4;
    return e < D::NCH ? (d.xoff + m * d.xld + k) * 4u : 0xFFFFFFF0u;
}
template <int WT, int M>
__device__ __forceinline__ void dit_att_request(const LayCtx<WT, M> &cx, const LayOp &d, u32x4 (&a)[DitAtt<M>::XA]) {
    static_assert(DitAtt<M>::B * DitAtt<M>::S == M && DitAtt<M>::XA <= 16, "DiT attention shape; one stale bit per chunk");
#pragma unroll
    for (uint32_t r = 0; r < DitAtt<M>::XA; r++) a[r] = ldtag4(cx.rsrc, dit_att_off<M>(d, cx.tid + LAY_THREADS * r));
}
// Stages each requested chunk in LDS as soon as it is current (a round requests the whole array
// again, chunks already staged at an offset outside the buffer), then computes each group's S
// query rows and stages them (hi + lo) as x of the out projection (K = H 64); `item` is the
// attention item, whose user output workgroup 0 writes when it is the region's last write.
template <int WT, int M, uint32_t K>
__device__ __forceinline__ void dit_att_stage(LayCtx<WT, M> &cx, const LayOp &d, const SeqOp &item,
                                              u32x4 (&a)[DitAtt<M>::XA]) {
    typedef DitAtt<M> D;
    const uint32_t tid = cx.tid;
    uint32_t pend = 0;
#pragma unroll
    for (uint32_t r = 0; r < D::XA; r++)
        if (tid + LAY_THREADS * r < D::NCH) pend |= 1u << r;
    uint32_t spins = 0;
    while (true) {
#pragma unroll
        for (uint32_t r = 0; r < D::XA; r++) {
            if (((pend >> r) & 1u) && tagged4(a[r], cx.parity)) {
                *reinterpret_cast<f32x4 *>(cx.qs + 4 * (tid + LAY_THREADS * r)) =
                    f32x4{untag(a[r].x), untag(a[r].y), untag(a[r].z), untag(a[r].w)};
                pend &= ~(1u << r);
            }
        }
        if (!pend || cx.gave_up) break;
        if (++spins > SPIN_LIMIT) {
            cx.gave_up = true;
            raise_flag(cx.sync, SYNC_TIMEOUT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (uint32_t r = 0; r < D::XA; r++)
            a[r] = ldtag4(cx.rsrc, (pend >> r) & 1u ? dit_att_off<M>(d, tid + LAY_THREADS * r) : 0xFFFFFFF0u);
    }
    __syncthreads();  // the qkv staged
    // Octet j of wave w < 4 takes group w + 4 j (the groups spread over the four SIMDs, one
    // round); lane l of it the RoPE pairs 4l .. 4l + 3 (dims 8l .. 8l + 7) of the group's q, k
    // and v rows.  The S x S scores are summed over the octet together, so their DPP steps
    // overlap; each query row takes one reciprocal of its softmax sum.
    static_assert(D::GROUPS <= 32, "one group per octet of waves 0-3");
    const uint32_t l = cx.lane & 7, gi = cx.w + 4 * (cx.lane >> 3);
    const bool write_out = item.final_out != 0 && cx.g == 0;
    bool range_ok = true;
    if (cx.w < 4 && gi < D::GROUPS) {
        const uint32_t b = gi / DIT_HEADS, h = gi % DIT_HEADS;
        // the lane's 8 dims of row j of part u (0 q, 1 k, 2 v)
        auto dims = [&](uint32_t u, uint32_t j, float (&v)[8]) {
            const float *p = cx.qs + (b * D::S + j) * D::W + u * (DIT_HEADS * 64) + h * 64 + 8 * l;
            const f32x4 a0 = *reinterpret_cast<const f32x4 *>(p), a1 = *reinterpret_cast<const f32x4 *>(p + 4);
            v[0] = a0[0]; v[1] = a0[1]; v[2] = a0[2]; v[3] = a0[3];
            v[4] = a1[0]; v[5] = a1[1]; v[6] = a1[2]; v[7] = a1[3];
        };
        auto rotate = [&](float (&v)[8], uint32_t j) {  // position j
#pragma unroll
            for (uint32_t pi = 0; pi < 4; pi++) {
                const uint32_t pp = 4 * l + pi;
                const float2 r = dit_rope_pair(make_float2(v[2 * pi], v[2 * pi + 1]), cx.rope[pp * D::S + j],
                                               cx.rope[(32 + pp) * D::S + j]);
                v[2 * pi] = r.x;
                v[2 * pi + 1] = r.y;
            }
        };
        float q[D::S][8], k[D::S][8];
#pragma unroll
        for (uint32_t j = 0; j < D::S; j++) {
            dims(0, j, q[j]);
            dims(1, j, k[j]);
            rotate(q[j], j);
            rotate(k[j], j);
        }
        float sc[D::S][D::S];
#pragma unroll
        for (uint32_t i = 0; i < D::S; i++)
#pragma unroll
            for (uint32_t j = 0; j < D::S; j++) {
                float v = q[i][0] * k[j][0];
#pragma unroll
                for (uint32_t e = 1; e < 8; e++) v = fmaf(q[i][e], k[j][e], v);
                sc[i][j] = v;
            }
        octet_sums<D::S * D::S>(&sc[0][0]);
        float vv[D::S][8];
#pragma unroll
        for (uint32_t j = 0; j < D::S; j++) dims(2, j, vv[j]);
#pragma unroll
        for (uint32_t i = 0; i < D::S; i++) {
            float mx = -INFINITY;
#pragma unroll
            for (uint32_t j = 0; j < D::S; j++) {
                sc[i][j] *= cx.ascale;
                mx = fmaxf(mx, sc[i][j]);
            }
            float sum = 0.0f, acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t j = 0; j < D::S; j++) {
                const float e = exp_hw(sc[i][j] - mx);
                sum += e;
#pragma unroll
                for (uint32_t d2 = 0; d2 < 8; d2++) acc[d2] = fmaf(e, vv[j][d2], acc[d2]);
            }
            const float inv = 1.0f / sum;
            const uint32_t row = b * D::S + i, col = h * 64 + 8 * l;
            float o[8];
            uint32_t hv[4], lv[4];
#pragma unroll
            for (uint32_t d2 = 0; d2 < 8; d2++) o[d2] = acc[d2] * inv;
#pragma unroll
            for (uint32_t pi = 0; pi < 4; pi++) {
                hv[pi] = pack2<WT>(o[2 * pi], o[2 * pi + 1]);
                lv[pi] = pack2<WT>(o[2 * pi] - dec_lo<WT>(hv[pi]), o[2 * pi + 1] - dec_hi<WT>(hv[pi]));
                if constexpr (WT == DT_F16) range_ok = range_ok && fmaxf(fabsf(o[2 * pi]), fabsf(o[2 * pi + 1])) <= 65504.0f;
            }
            *reinterpret_cast<u32x4 *>(cx.xs + row * K + col) = u32x4{hv[0], hv[1], hv[2], hv[3]};
            *reinterpret_cast<u32x4 *>(cx.xs + LayCtx<WT, M>::PLANE + row * K + col) = u32x4{lv[0], lv[1], lv[2], lv[3]};
            if (write_out) {  // the user's row stride may be any number of floats
                float *y = item.y + static_cast<size_t>(row) * item.ldy + col;
#pragma unroll
                for (uint32_t d2 = 0; d2 < 8; d2++) y[d2] = o[d2];
            }
        }
    }
    if (!range_ok) raise_flag(cx.sync, SYNC_RANGE);
}

// One op of class C (descriptor d; ops[i] holds its full descriptor for an external x): A
// holds its weight tiles.  `issue` requests this op's share of later ops' weight tiles (NB
// loads per wave).  A CU's vector-memory requests are served in order, so a batch holds up
// whatever is requested after it until it has drained: issued after the output stores, it
// holds up the next op's activation polls; issued as soon as the activations are current, it
// holds up this op's stores unless it drains during the conversion and the MFMAs.  The
// normed ops (qkv, gate|up) at M <= 2 issue theirs early: the norm's reductions give them
// the longest window (decode step at M = 2: 421 -> 395.5 us; M = 1: 389 -> 341 us, A/B on
// one box).  down, split over K, does too in plans without attention items (ATTK false; M =
// 2: 370 -> 367 us), and with them at M = 1 (the whole layer 410.6 -> 401.5 us; at M = 2
// 439.4 -> 440.4, so not there).  At M = 4 the normed ops and down all go early (linear-only
// step 486.4 -> 462.8 us, the VAE latent's stack with attention items 580.0 -> 543.1 us; the
// normed ops alone 551.9, down alone 578.4).  Early batches from o measured slower (+27 us at
// M = 2 linear-only, +35 with attention), so o's stay behind the stores.
template <int WT, int M, int C, uint32_t NB, bool ATTK = false, int NA, class ISSUE>
__device__ __forceinline__ void lay_step(LayCtx<WT, M> &cx, const SeqOp *__restrict__ ops, uint32_t i, const LayOp &d,
                                         const u32x4 (&A)[NA], ISSUE &&issue) {
    typedef LCls<C, M> L;
    static_assert(M * L::KX <= LayCtx<WT, M>::PLANE, "x staging");
    constexpr bool EARLY = ((L::NORM || (C == LC_DOWN && (!ATTK || M == 1))) && M <= 2) ||
                           ((L::NORM || C == LC_DOWN) && M == 4);
    static_assert(NB < 16, "a batch fits the explicit wait below");
    const uint32_t tid = cx.tid, lane = cx.lane;
    const uint32_t r0 = cx.r0[L::SLOT], nr = cx.nr[L::SLOT];
    const bool xext = (d.flags & LAY_XEXT) != 0;
    // down reads its half of K; x from down's two planes is read from both.
    const uint32_t kx0 = L::KSPLIT > 1 ? cx.half * L::KX : 0u;
    const bool x2 = L::X2 && (d.flags & LAY_X2) != 0;
    constexpr uint32_t PL = L::PL;  // words between a split op's planes

    // Activations: chunk e = tid + 448 r is 4 k of x row e / K4 (or the DiT attention's qkv).
    u32x4 xv[L::XR], xv2[L::X2 ? L::XR : 1];
    u32x2 gv[L::XR];
    u32x4 att[L::ATTX ? DitAtt<M>::XA : 1];
    if constexpr (L::ATTX) dit_att_request(cx, d, att);
#pragma unroll
    for (uint32_t r = 0; r < (L::ATTX ? 0u : L::XR); r++) {
        const uint32_t e = tid + 448 * r;
        const uint32_t m = e / L::K4, k = (e - m * L::K4) * 4;
        const bool ok = e < L::NCH;
        if (!xext) {
            xv[r] = ldtag4(cx.rsrc, ok ? (d.xoff + m * d.xld + kx0 + k) * 4u : 0xFFFFFFF0u);
            if constexpr (L::X2)
                if (x2) xv2[r] = ldtag4(cx.rsrc, ok ? (d.xoff + PL + m * d.xld + k) * 4u : 0xFFFFFFF0u);
        } else {  // x from the user buffer (the sequence's first op)
            const SeqOp &o = ops[i];
            xv[r] = u32x4{0u, 0u, 0u, 0u};
            if (ok) {
                const size_t off = static_cast<size_t>(m) * o.ldx + kx0 + k;
                if (o.xt == DT_F32) {
                    xv[r] = gld(reinterpret_cast<const u32x4 *>(static_cast<const float *>(o.x) + off));
                } else {
                    const u32x2 h = gld(reinterpret_cast<const u32x2 *>(static_cast<const uint16_t *>(o.x) + off));
                    const bool bf = o.xt == DT_BF16;
                    xv[r] = u32x4{__float_as_uint(bf ? dec_lo<DT_BF16>(h.x) : dec_lo<DT_F16>(h.x)),
                                  __float_as_uint(bf ? dec_hi<DT_BF16>(h.x) : dec_hi<DT_F16>(h.x)),
                                  __float_as_uint(bf ? dec_lo<DT_BF16>(h.y) : dec_lo<DT_F16>(h.y)),
                                  __float_as_uint(bf ? dec_hi<DT_BF16>(h.y) : dec_hi<DT_F16>(h.y))};
                }
            }
        }
        if constexpr (L::NORM) gv[r] = gld(reinterpret_cast<const u32x2 *>(d.norm + (ok ? k : 0u)));
    }
    // Output lane tid: feature r0 + of, x row om.  Bias and old y requested now.
    const uint32_t of = tid / M, om = tid - of * M;
    const bool live = of < nr;
    const uint32_t n = r0 + (live ? of : 0u);
    const bool yext = (d.flags & LAY_YEXT) != 0;
    uint32_t braw = 0, yw = 0, yw2 = 0;
    const bool y2 = L::Y2 && (d.flags & LAY_Y2) != 0;
    if constexpr (L::BIAS) braw = gld(d.p2 + n);
    if constexpr (L::ACC)  // old y: a tagged word, or the user's y; one load either way (no branch)
        yw = ld32(yext ? reinterpret_cast<const uint32_t *>(d.y) + static_cast<size_t>(om) * d.ldy + n
                       : cx.tags + d.yoff + om * d.yld + n);
    if constexpr (L::Y2)
        if (y2) yw2 = ld32(cx.tags + d.yoff + PL + om * d.yld + n);

    if constexpr (L::ATTX) {
        dit_att_stage<WT, M, L::K>(cx, d, ops[i - 1], att);
    } else {
        // The conversion into the staging, chunk by chunk: tag bit cleared (down's two planes
        // added), x^2 summed, gain applied, split into hi + lo halves of the weights' type.
        // Ops without an early batch convert each chunk as soon as it is current; their rounds
        // request the whole chunk array again, chunks already staged at an offset outside the
        // buffer (they read 0 and fetch nothing), so no chunk's old registers are merged with
        // new ones and the arrays are not held twice over the wait (at M = 6 that spilled 100
        // registers, whose reloads waited for every weight tile in flight).
        static_assert(L::XR <= 16, "pending bits");
        const uint32_t clear = xext ? ~0u : ~1u;
        float tq[L::NORM ? L::XR : 1];  // x^2 of chunk r (per row below, in chunk order)
        bool range_ok = true;
        auto stage = [&](uint32_t r) {
            const uint32_t e = tid + 448 * r;
            const uint32_t m = e / L::K4, k = (e - m * L::K4) * 4;
            float x[4];
            x[0] = __uint_as_float(xv[r].x & clear);
            x[1] = __uint_as_float(xv[r].y & clear);
            x[2] = __uint_as_float(xv[r].z & clear);
            x[3] = __uint_as_float(xv[r].w & clear);
            if constexpr (L::X2) {
                if (x2) {  // the residual: down's first plane + its second, in that order
                    x[0] += untag(xv2[r].x);
                    x[1] += untag(xv2[r].y);
                    x[2] += untag(xv2[r].z);
                    x[3] += untag(xv2[r].w);
                }
            }
            if constexpr (L::NORM) {
                float t = x[0] * x[0];
                t = fmaf(x[1], x[1], t);
                t = fmaf(x[2], x[2], t);
                tq[r] = fmaf(x[3], x[3], t);
                x[0] *= dec_lo<WT>(gv[r].x);
                x[1] *= dec_hi<WT>(gv[r].x);
                x[2] *= dec_lo<WT>(gv[r].y);
                x[3] *= dec_hi<WT>(gv[r].y);
            }
            if constexpr (WT == DT_F16)
                range_ok = range_ok && fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3]))) <= 65504.0f;
            u32x2 hi, lo;
            split4p<WT>(x, hi, lo);
            *reinterpret_cast<u32x2 *>(cx.xs + m * L::KX + k) = hi;
            *reinterpret_cast<u32x2 *>(cx.xs + LayCtx<WT, M>::PLANE + m * L::KX + k) = lo;
        };
        uint32_t pend = 0;  // chunks in range not staged yet
#pragma unroll
        for (uint32_t r = 0; r < L::XR; r++)
            if (tid + 448 * r < L::NCH) pend |= 1u << r;
        uint32_t spins = 0;
        if constexpr (EARLY) {
            // Every chunk current first (stale ones requested again, all at once per round),
            // then the batch, then the conversions: the batch drains meanwhile.  These ops run
            // at M <= 2, where the chunk arrays are small enough to be held over the wait.
            auto stale_bits = [&]() {
                uint32_t st = 0;
#pragma unroll
                for (uint32_t r = 0; r < L::XR; r++) {
                    if (((pend >> r) & 1u) && !tagged4(xv[r], cx.parity)) st |= 1u << r;
                    if constexpr (L::X2)
                        if (x2 && ((pend >> r) & 1u) && !tagged4(xv2[r], cx.parity)) st |= 1u << (16 + r);
                }
                return st;
            };
            uint32_t stale = xext ? 0u : stale_bits();
            while (stale && !cx.gave_up) {
                if (++spins > SPIN_LIMIT) {
                    cx.gave_up = true;
                    raise_flag(cx.sync, SYNC_TIMEOUT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
#pragma unroll
                for (uint32_t r = 0; r < L::XR; r++) {
                    const uint32_t e = tid + 448 * r;
                    const uint32_t m = e / L::K4, k = (e - m * L::K4) * 4;
                    if ((stale >> r) & 1u) xv[r] = ldtag4(cx.rsrc, (d.xoff + m * d.xld + kx0 + k) * 4u);
                    if constexpr (L::X2)
                        if ((stale >> (16 + r)) & 1u) xv2[r] = ldtag4(cx.rsrc, (d.xoff + PL + m * d.xld + k) * 4u);
                }
                stale = stale_bits();
            }
            issue();
#pragma unroll
            for (uint32_t r = 0; r < L::XR; r++)
                if ((pend >> r) & 1u) stage(r);
        } else {
            while (true) {
#pragma unroll
                for (uint32_t r = 0; r < L::XR; r++) {
                    bool cur = ((pend >> r) & 1u) != 0;
                    if (!xext) {
                        cur = cur && tagged4(xv[r], cx.parity);
                        if constexpr (L::X2) cur = cur && (!x2 || tagged4(xv2[r], cx.parity));
                    }
                    if (cur) {
                        stage(r);
                        pend &= ~(1u << r);
                    }
                }
                if (!pend || cx.gave_up) break;
                if (++spins > SPIN_LIMIT) {
                    cx.gave_up = true;
                    raise_flag(cx.sync, SYNC_TIMEOUT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
#pragma unroll
                for (uint32_t r = 0; r < L::XR; r++) {
                    const uint32_t e = tid + 448 * r;
                    const uint32_t m = e / L::K4, k = (e - m * L::K4) * 4;
                    const bool want = ((pend >> r) & 1u) != 0;
                    xv[r] = ldtag4(cx.rsrc, want ? (d.xoff + m * d.xld + kx0 + k) * 4u : 0xFFFFFFF0u);
                    if constexpr (L::X2)
                        if (x2) xv2[r] = ldtag4(cx.rsrc, want ? (d.xoff + PL + m * d.xld + k) * 4u : 0xFFFFFFF0u);
                }
            }
        }
        float ss[M];
#pragma unroll
        for (int mm = 0; mm < M; mm++) ss[mm] = 0.0f;
        if constexpr (L::NORM) {
#pragma unroll
            for (uint32_t r = 0; r < L::XR; r++) {
                const uint32_t e = tid + 448 * r, m = e / L::K4;
                if (e < L::NCH) {
#pragma unroll
                    for (int mm = 0; mm < M; mm++) ss[mm] += m == static_cast<uint32_t>(mm) ? tq[r] : 0.0f;
                }
            }
        }
        if (!range_ok) raise_flag(cx.sync, SYNC_RANGE);
        if constexpr (L::NORM) {
#pragma unroll
            for (int mm = 0; mm < M; mm++) {
                const float t = wave_sum(ss[mm]);
                if (lane == 0) cx.ssw[L::SLOT][mm * 8 + cx.w] = t;
            }
        }
    }
    __syncthreads();  // x staged

    switch (cx.w) {  // the wave's tile range is compile-time in each case
        case 0: lay_mma<WT, M, C, 0>(cx, A); break;
        case 1: lay_mma<WT, M, C, 1>(cx, A); break;
        case 2: lay_mma<WT, M, C, 2>(cx, A); break;
        case 3: lay_mma<WT, M, C, 3>(cx, A); break;
        case 4: lay_mma<WT, M, C, 4>(cx, A); break;
        case 5: lay_mma<WT, M, C, 5>(cx, A); break;
        default: lay_mma<WT, M, C, 6>(cx, A); break;
    }
    __syncthreads();  // every wave's partial sums are in LDS
    // The op's own loads (x, gain, bias, old y) have landed long before this point, and the
    // only later requests are an early batch: waiting for the rest here, where it costs
    // nothing, spares a wait for a load whose value some lanes never use where its registers
    // are next written (the next op's activation loads, behind this op's tile batch).
    __builtin_amdgcn_s_waitcnt(0x0F70 | (EARLY ? NB : 0u));  // vmcnt(NB) or vmcnt(0)

    // Outputs: the 8 slots summed in slot order, norm scale, epilogue, tagged store.
    if (live) {
        auto total = [&](uint32_t rt, uint32_t v) {
            const float *p = cx.part[L::SLOT] + ((rt * M + om) * L::VR + v) * 8;
            const f32x4 a = *reinterpret_cast<const f32x4 *>(p);
            const f32x4 b = *reinterpret_cast<const f32x4 *>(p + 4);
            return ((a[0] + a[1]) + (a[2] + a[3])) + ((b[0] + b[1]) + (b[2] + b[3]));
        };
        float a1, a2 = 0.0f;
        if constexpr (L::GATED) {
            a1 = total(of >> 3, of & 7);
            a2 = total(of >> 3, 8 + (of & 7));
        } else {
            a1 = total(0, of);
        }
        if constexpr (L::NORM) {
            const float *sp = cx.ssw[L::SLOT] + om * 8;
            const f32x4 a = *reinterpret_cast<const f32x4 *>(sp);
            const f32x4 b = *reinterpret_cast<const f32x4 *>(sp + 4);
            const float t = ((a[0] + a[1]) + (a[2] + a[3])) + ((b[0] + b[1]) + (b[2] + b[3]));
            const float scale = rsqrt_hw(t / static_cast<float>(L::K) + d.eps);
            a1 *= scale;
            a2 *= scale;
        }
        // A split op's halves are added by its readers, so its epilogue is linear (bias and
        // the old y only) and the first half alone adds the bias and the old y.
        static_assert(L::KSPLIT == 1 || (L::FLAGS & ~(F_BIAS | F_ACCUM)) == 0, "a split op's epilogue is linear");
        const bool second = L::KSPLIT > 1 && cx.half != 0;
        float bias = 0.0f;
        if constexpr (L::BIAS) {
            asm volatile("" : "+v"(braw));
            bias = second ? 0.0f : dec1<WT>(static_cast<uint16_t>(braw));
        }
        float v = epilogue_fixed<L::FLAGS>(a1, a2, bias);  // on this op's critical path: hardware SiLU / tanh
        // Wait for a tagged word at byte offset off to carry the run's parity.
        auto await_word = [&](uint32_t &word, uint32_t off) {
            uint32_t spins = 0;
            while ((word & 1u) != cx.parity && !cx.gave_up) {
                if (++spins > SPIN_LIMIT) {
                    cx.gave_up = true;
                    raise_flag(cx.sync, SYNC_TIMEOUT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                word = ldtag1(cx.rsrc, off);
            }
        };
        // The second half adds no old y: its plane holds its own sums.
        if constexpr (L::ACC) {
            if (!second) {
                if (!yext) await_word(yw, (d.yoff + om * d.yld + n) * 4u);
                float old = __uint_as_float(yext ? yw : yw & ~1u);
                if constexpr (L::Y2) {
                    if (y2) {
                        await_word(yw2, (d.yoff + PL + om * d.yld + n) * 4u);
                        old += untag(yw2);
                    }
                }
                v += old;
            }
        }
        const uint32_t t = d.tag + (second ? PL : 0u) + om * L::N + n;
        st_tag(cx.tags + t, v, cx.parity);
        if (d.flags & LAY_FINAL) {
            float out = v;
            if constexpr (L::KSPLIT > 1) {
                // The user's value is what the next layer would read: the first plane plus
                // this one, written by the second half once the first half's word is current.
                if (second) {
                    uint32_t w0 = ldtag1(cx.rsrc, (t - PL) * 4u);
                    await_word(w0, (t - PL) * 4u);
                    out = untag(w0) + untag(__float_as_uint(v));  // the stored word's value
                }
            }
            if (L::KSPLIT == 1 || second)
                *reinterpret_cast<__attribute__((address_space(1))) float *>(
                    reinterpret_cast<uintptr_t>(d.y + static_cast<size_t>(om) * d.ldy + n)) = out;
        }
    }
    // Otherwise later ops' weight tiles go behind this op's output stores: they drain while
    // the next op's activations are being produced by the other workgroups.
    if constexpr (!EARLY) issue();
}

// The positions of this workgroup's first attention item of layer op o (its row's and
// pos[0]), requested before the layer's qkv op so the item's cache reads need not wait for them.
template <int M>
__device__ __forceinline__ void lay_attention_pos(const SeqOp &o, uint32_t g, uint32_t (&pos)[2]) {
    const uint32_t hq = o.heads & 0xFFFFu;
    if (g < M * hq) {
        pos[0] = gld(o.pos + g / hq);
        pos[1] = gld(o.pos);
    }
}

// The decode attention item of a layer (the general kernel's attend_item on this kernel's 7
// waves): its (row, head) pairs, M 14 of them, go to workgroups g, g + G, ...; the x staging
// is the item's scratch.  Every other workgroup goes straight on to o, whose activations
// are this item's output.
template <int WT, int M>
__device__ __forceinline__ void lay_attention(LayCtx<WT, M> &cx, const SeqOp &o, uint32_t g, uint32_t G,
                                              const uint32_t (&pos)[2]) {
    const uint32_t hq = o.heads & 0xFFFFu, items = M * hq;
    float *scratch = reinterpret_cast<float *>(cx.xs);
    for (uint32_t it = g; it < items; it += G) {
        const uint32_t *pp = M <= 2 && it == g ? pos : nullptr;
        if (o.cache_t == DT_F32)
            attend_item<DT_F32, LAY_CW>(o, it / hq, it % hq, cx.rsrc, cx.parity, scratch, cx.gave_up, cx.sync, pp);
        else
            attend_item<DT_F16, LAY_CW>(o, it / hq, it % hq, cx.rsrc, cx.parity, scratch, cx.gave_up, cx.sync, pp);
    }
}

// The kernel: n_ops = 4 L ops in the layer pattern, or 5 L with attention items (ATT) (the host
// checks shapes, flags and G); their packed descriptors follow the n_ops op descriptors.
template <int WT, int M, bool ATT>
__global__ __launch_bounds__(LAY_THREADS) void layer_kernel(const SeqOp *__restrict__ ops, uint32_t n_ops,
                                                           uint32_t *sync, const uint32_t *tags, uint32_t tag_bytes) {
    typedef LayCtx<WT, M> X;
    // The x staging; with attention items also their scratch (7168 floats).
    constexpr uint32_t XS = ATT && 2 * X::PLANE < 14336 ? 14336u : 2 * X::PLANE;
    __shared__ __attribute__((aligned(16))) uint16_t xs[XS];
    __shared__ __attribute__((aligned(16))) float p_qkv[LCls<LC_QKV, M>::PART];
    __shared__ __attribute__((aligned(16))) float p_o[LCls<LC_O, M>::PART];
    __shared__ __attribute__((aligned(16))) float p_gu[LCls<LC_GU, M>::PART];
    __shared__ __attribute__((aligned(16))) float p_d[LCls<LC_DOWN, M>::PART];
    __shared__ __attribute__((aligned(16))) float s_qkv[M * 8];
    __shared__ __attribute__((aligned(16))) float s_gu[M * 8];
    const LayOp *__restrict__ lops = reinterpret_cast<const LayOp *>(ops + n_ops);

    X cx;
    cx.xs = xs;
    cx.qs = nullptr;
    cx.rope = nullptr;
    cx.part[LC_QKV] = p_qkv;
    cx.part[LC_O] = p_o;
    cx.part[LC_GU] = p_gu;
    cx.part[LC_DOWN] = p_d;
    cx.ssw[LC_QKV] = s_qkv;
    cx.ssw[LC_GU] = s_gu;
    cx.ssw[LC_O] = s_qkv;
    cx.ssw[LC_DOWN] = s_gu;
    cx.tid = threadIdx.x;
    cx.lane = cx.tid & 63;
    cx.w = __builtin_amdgcn_readfirstlane(cx.tid >> 6);
    cx.sync = sync;
    cx.tags = const_cast<uint32_t *>(tags);
    cx.gave_up = false;
    const uint32_t g = blockIdx.x, G = gridDim.x;
    cx.g = g;
    const uint32_t Ns[4] = {LAY_QKV, LAY_H, LAY_I, LAY_H};
#pragma unroll
    for (int c = 0; c < 4; c++) {
        // down: pair g >> 1 of the G / 2 (G is even) owns the features, half g & 1 of K
        const uint32_t u = c == LC_DOWN ? g >> 1 : g, U = c == LC_DOWN ? G >> 1 : G;
        cx.r0[c] = static_cast<uint32_t>(static_cast<uint64_t>(u) * Ns[c] / U);
        cx.nr[c] = static_cast<uint32_t>(static_cast<uint64_t>(u + 1) * Ns[c] / U) - cx.r0[c];
    }
    cx.half = g & 1u;
    cx.kh = cx.half * LCls<LC_DOWN, M>::KX;
    {
        LRange rq{}, ro{}, rg{}, rd{};
        switch (cx.w) {
#define LAY_RANGES(W)                      \
    case W:                                \
        rq = lay_range<LC_QKV, M>(W);      \
        ro = lay_range<LC_O, M>(W);        \
        rg = lay_range<LC_GU, M>(W);       \
        rd = lay_range<LC_DOWN, M>(W);     \
        break;
            LAY_RANGES(0) LAY_RANGES(1) LAY_RANGES(2) LAY_RANGES(3) LAY_RANGES(4) LAY_RANGES(5)
            default: LAY_RANGES(6)
#undef LAY_RANGES
        }
        cx.ln[LC_QKV] = lay_lane<LC_QKV, M>(cx.r0[LC_QKV], cx.nr[LC_QKV], cx.lane, rq, X::PLANE);
        cx.ln[LC_O] = lay_lane<LC_O, M>(cx.r0[LC_O], cx.nr[LC_O], cx.lane, ro, X::PLANE);
        cx.ln[LC_GU] = lay_lane<LC_GU, M>(cx.r0[LC_GU], cx.nr[LC_GU], cx.lane, rg, X::PLANE);
        cx.ln[LC_DOWN] = lay_lane<LC_DOWN, M>(cx.r0[LC_DOWN], cx.nr[LC_DOWN], cx.lane, rd, X::PLANE, cx.kh);
        cx.up = (cx.lane & 15) >= 8;
    }
    // Slots no compute wave writes (slot 7, and gate|up's row tiles a wave does not reach) stay zero.
    for (uint32_t e = cx.tid; e < LCls<LC_QKV, M>::PART; e += LAY_THREADS) p_qkv[e] = 0.0f;
    for (uint32_t e = cx.tid; e < LCls<LC_O, M>::PART; e += LAY_THREADS) p_o[e] = 0.0f;
    for (uint32_t e = cx.tid; e < LCls<LC_GU, M>::PART; e += LAY_THREADS) p_gu[e] = 0.0f;
    for (uint32_t e = cx.tid; e < LCls<LC_DOWN, M>::PART; e += LAY_THREADS) p_d[e] = 0.0f;
    for (uint32_t e = cx.tid; e < M * 8; e += LAY_THREADS) s_qkv[e] = s_gu[e] = 0.0f;
    const uint32_t epoch = __hip_atomic_load(sync + SYNC_EPOCH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    cx.parity = epoch & 1u;
    cx.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t *>(tags), 0, static_cast<int>(tag_bytes), BUF_DWORD3);

    // Every class has its own tile registers.  A class's tiles for layer l + 1 are requested in
    // batches over the three ops after its layer-l op, so each op requests about the same
    // share of the layer's weight stream (a burst would hold up the loads and stores behind it):
    //   op qkv(l):  gate|up(l) second third, down(l) first sixth
    //   op o(l):    gate|up(l) last third,   down(l) second sixth
    //   op gu(l):   down(l) rest,            qkv(l+1) first half
    //   op down(l): gate|up(l+1) first third, qkv(l+1) second half, o(l+1)
    typedef LCls<LC_QKV, M> LQ;
    typedef LCls<LC_O, M> LO;
    typedef LCls<LC_GU, M> LG;
    typedef LCls<LC_DOWN, M> LD;
    constexpr uint32_t G1 = LG::TA / 3, G2 = 2 * LG::TA / 3, D1 = LD::TA / 6, D2 = 2 * LD::TA / 6, Q1 = LQ::TA / 2;
    // Loads per wave of each op's batch.
    constexpr uint32_t NBQ = (G2 - G1) + D1, NBO = (LG::TA - G2) + (D2 - D1), NBG = (LD::TA - D2) + Q1,
                       NBD = G1 + (LQ::TA - Q1) + LO::TA;
    u32x4 PQ[LQ::TA], PO[LO::TA], PG[LG::TA], PD[LD::TA];
    constexpr uint32_t A = ATT ? 1u : 0u, OPL = 4 + A;  // ops per layer: qkv, [attention,] o, gate|up, down
    const uint32_t L = n_ops / OPL;
    if (L > 0) {
        lay_tiles<WT, M, LC_QKV, 0, LQ::TA>(cx, lops[0], PQ);
        lay_tiles<WT, M, LC_O, 0, LO::TA>(cx, lops[1 + A], PO);
        lay_tiles<WT, M, LC_GU, 0, G1>(cx, lops[2 + A], PG);
    }
    __syncthreads();
    // Each op's packed descriptor is read one op ahead (scalar loads), so no op waits for
    // its own.
    LayOp dq = lops[0], dn;
    for (uint32_t l = 0; l < L; l++) {
        // The last layer's requests for a next layer read layer 0's weights again (unused), so
        // every op requests the same number of tiles.
        const uint32_t i = OPL * l, nx = l + 1 < L ? i + OPL : 0;
        const uint32_t io = i + 1 + A, ig = i + 2 + A, id = i + 3 + A;  // o, gate|up, down
        dn = lops[io];
        // The M = 4 kernel has no registers to spare for them over the qkv op.
        uint32_t apos[2] = {0u, 0u};
        if constexpr (ATT && M <= 2) lay_attention_pos<M>(ops[i + 1], g, apos);
        lay_step<WT, M, LC_QKV, NBQ>(cx, ops, i, dq, PQ, [&]() {
            lay_tiles<WT, M, LC_GU, G1, G2>(cx, lops[ig], PG);
            lay_tiles<WT, M, LC_DOWN, 0, D1>(cx, lops[id], PD);
        });
        if constexpr (ATT) lay_attention<WT, M>(cx, ops[i + 1], g, G, apos);
        dq = lops[ig];
        lay_step<WT, M, LC_O, NBO>(cx, ops, io, dn, PO, [&]() {
            lay_tiles<WT, M, LC_GU, G2, LG::TA>(cx, dq, PG);
            lay_tiles<WT, M, LC_DOWN, D1, D2>(cx, lops[id], PD);
        });
        dn = lops[id];
        lay_step<WT, M, LC_GU, NBG>(cx, ops, ig, dq, PG, [&]() {
            lay_tiles<WT, M, LC_DOWN, D2, LD::TA>(cx, dn, PD);
            lay_tiles<WT, M, LC_QKV, 0, Q1>(cx, lops[nx], PQ);
        });
        dq = lops[nx];
        lay_step<WT, M, LC_DOWN, NBD, ATT>(cx, ops, id, dn, PD, [&]() {
            lay_tiles<WT, M, LC_GU, 0, G1>(cx, lops[nx + 2 + A], PG);
            lay_tiles<WT, M, LC_QKV, Q1, LQ::TA>(cx, dq, PQ);
            lay_tiles<WT, M, LC_O, 0, LO::TA>(cx, lops[nx + 1 + A], PO);
        });
    }
    // The last workgroup out advances the epoch for the next run.
    if (cx.tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(sync + SYNC_EXIT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == G - 1) {
            __hip_atomic_store(sync + SYNC_EXIT, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(sync + SYNC_EPOCH, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// The DiT-block kernel: n_ops = 5 L ops, L DiT blocks of the flow head's shape (dit_pattern:
// qkv, DiT attention, out, ff1, ff2 at M = 6 (batch 2 x seq 3, the flow loop) or M = 2 (1 x 2,
// the aggregator) on DIT_G workgroups, the host checks them), the packed descriptors after
// the op descriptors.  The attention item is not a step of its own: each workgroup computes it
// while staging the out projection's x (dit_att_stage).  Tiling at 256 workgroups: qkv 12 and
// ff1 16 features a workgroup (S = 1, one row tile, 32 block steps as 5 a wave), out and ff2 4
// features (S = 4; at M = 6 three B column groups of two rows).  Each op
// requests the weight tiles of the op two steps on (qkv: ff1, out: ff2, ff1: the next block's
// qkv, ff2: the next block's out) behind its output stores.
template <int WT, int M>
__global__ __launch_bounds__(LAY_THREADS) void dit_block_kernel(const SeqOp *__restrict__ ops, uint32_t n_ops,
                                                               uint32_t *sync, const uint32_t *tags,
                                                               uint32_t tag_bytes) {
    typedef LayCtx<WT, M> X;
    typedef LCls<LC_DQKV, M> LQ;
    typedef LCls<LC_DO, M> LO;
    typedef LCls<LC_FF1, M> LF;
    typedef LCls<LC_FF2, M> LD;
    __shared__ __attribute__((aligned(16))) uint16_t xs[2 * X::PLANE];
    __shared__ __attribute__((aligned(16))) float qs[M * DIT_QKV];
    __shared__ float rope[2 * 32 * DitAtt<M>::S];
    __shared__ __attribute__((aligned(16))) float p_q[LQ::PART];
    __shared__ __attribute__((aligned(16))) float p_o[LO::PART];
    __shared__ __attribute__((aligned(16))) float p_f[LF::PART];
    __shared__ __attribute__((aligned(16))) float p_d[LD::PART];
    __shared__ __attribute__((aligned(16))) float s_q[M * 8];
    __shared__ __attribute__((aligned(16))) float s_f[M * 8];
    const LayOp *__restrict__ lops = reinterpret_cast<const LayOp *>(ops + n_ops);

    X cx;
    cx.xs = xs;
    cx.qs = qs;
    cx.rope = rope;
    cx.part[LQ::SLOT] = p_q;
    cx.part[LO::SLOT] = p_o;
    cx.part[LF::SLOT] = p_f;
    cx.part[LD::SLOT] = p_d;
    cx.ssw[LQ::SLOT] = s_q;
    cx.ssw[LF::SLOT] = s_f;
    cx.ssw[LO::SLOT] = s_q;
    cx.ssw[LD::SLOT] = s_f;
    cx.tid = threadIdx.x;
    cx.lane = cx.tid & 63;
    cx.w = __builtin_amdgcn_readfirstlane(cx.tid >> 6);
    cx.sync = sync;
    cx.tags = const_cast<uint32_t *>(tags);
    cx.gave_up = false;
    const uint32_t g = blockIdx.x, G = gridDim.x;
    cx.g = g;
    // ff2: pair g >> 1 of the G / 2 (G is even) owns the features, half g & 1 of K.
    cx.half = g & 1u;
    cx.kh = cx.half * LD::KX;
    const uint32_t Ns[4] = {LQ::N, LO::N, LF::N, LD::N};
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t u = c == LD::SLOT ? g >> 1 : g, U = c == LD::SLOT ? G >> 1 : G;
        cx.r0[c] = static_cast<uint32_t>(static_cast<uint64_t>(u) * Ns[c] / U);
        cx.nr[c] = static_cast<uint32_t>(static_cast<uint64_t>(u + 1) * Ns[c] / U) - cx.r0[c];
    }
    {
        LRange rq{}, ro{}, rf{}, rd{};
        switch (cx.w) {
#define DIT_RANGES(W)                      \
    case W:                                \
        rq = lay_range<LC_DQKV, M>(W);     \
        ro = lay_range<LC_DO, M>(W);       \
        rf = lay_range<LC_FF1, M>(W);      \
        rd = lay_range<LC_FF2, M>(W);      \
        break;
            DIT_RANGES(0) DIT_RANGES(1) DIT_RANGES(2) DIT_RANGES(3) DIT_RANGES(4) DIT_RANGES(5)
            default: DIT_RANGES(6)
#undef DIT_RANGES
        }
        cx.ln[LQ::SLOT] = lay_lane<LC_DQKV, M>(cx.r0[LQ::SLOT], cx.nr[LQ::SLOT], cx.lane, rq, X::PLANE);
        cx.ln[LO::SLOT] = lay_lane<LC_DO, M>(cx.r0[LO::SLOT], cx.nr[LO::SLOT], cx.lane, ro, X::PLANE);
        cx.ln[LF::SLOT] = lay_lane<LC_FF1, M>(cx.r0[LF::SLOT], cx.nr[LF::SLOT], cx.lane, rf, X::PLANE);
        cx.ln[LD::SLOT] = lay_lane<LC_FF2, M>(cx.r0[LD::SLOT], cx.nr[LD::SLOT], cx.lane, rd, X::PLANE, cx.kh);
        cx.up = false;
    }
    // Slots no compute wave writes stay zero.
    for (uint32_t e = cx.tid; e < LQ::PART; e += LAY_THREADS) p_q[e] = 0.0f;
    for (uint32_t e = cx.tid; e < LO::PART; e += LAY_THREADS) p_o[e] = 0.0f;
    for (uint32_t e = cx.tid; e < LF::PART; e += LAY_THREADS) p_f[e] = 0.0f;
    for (uint32_t e = cx.tid; e < LD::PART; e += LAY_THREADS) p_d[e] = 0.0f;
    for (uint32_t e = cx.tid; e < M * 8; e += LAY_THREADS) s_q[e] = s_f[e] = 0.0f;
    const uint32_t epoch = __hip_atomic_load(sync + SYNC_EPOCH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    cx.parity = epoch & 1u;
    cx.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t *>(tags), 0, static_cast<int>(tag_bytes), BUF_DWORD3);
    // The attention's rotation table (every item shares the first one's frequencies and scale).
    const SeqOp &a0 = ops[1];
    if (cx.tid < 32) {  // pair tid
        float c[DIT_MAXS], sn[DIT_MAXS];
        constexpr uint32_t S = DitAtt<M>::S;
        dit_rope_table(gld(a0.inv_freq + cx.tid), S, c, sn);
#pragma unroll
        for (uint32_t j = 0; j < S; j++) {
            rope[cx.tid * S + j] = c[j];
            rope[(32 + cx.tid) * S + j] = sn[j];
        }
    }
    cx.ascale = a0.eps;

    u32x4 PQ[LQ::TA], PO[LO::TA], PF[LF::TA], PD[LD::TA];
    const uint32_t L = n_ops / 5;
    if (L > 0) {
        lay_tiles<WT, M, LC_DQKV, 0, LQ::TA>(cx, lops[0], PQ);
        lay_tiles<WT, M, LC_DO, 0, LO::TA>(cx, lops[2], PO);
    }
    __syncthreads();
    for (uint32_t l = 0; l < L; l++) {
        // The last block's requests for a next block read block 0's weights again (unused), so
        // every op requests the same number of tiles.
        const uint32_t i = 5 * l, nx = l + 1 < L ? i + 5 : 0;
        const uint32_t io = i + 2, i1 = i + 3, i2 = i + 4;  // out, ff1, ff2 (i + 1: the attention)
        lay_step<WT, M, LC_DQKV, 0>(cx, ops, i, lops[i], PQ, [&]() { lay_tiles<WT, M, LC_FF1, 0, LF::TA>(cx, lops[i1], PF); });
        lay_step<WT, M, LC_DO, 0>(cx, ops, io, lops[io], PO, [&]() { lay_tiles<WT, M, LC_FF2, 0, LD::TA>(cx, lops[i2], PD); });
        lay_step<WT, M, LC_FF1, 0>(cx, ops, i1, lops[i1], PF, [&]() { lay_tiles<WT, M, LC_DQKV, 0, LQ::TA>(cx, lops[nx], PQ); });
        lay_step<WT, M, LC_FF2, 0>(cx, ops, i2, lops[i2], PD,
                                   [&]() { lay_tiles<WT, M, LC_DO, 0, LO::TA>(cx, lops[nx + 2], PO); });
    }
    // The last workgroup out advances the epoch for the next run.
    if (cx.tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(sync + SYNC_EXIT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == G - 1) {
            __hip_atomic_store(sync + SYNC_EXIT, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(sync + SYNC_EPOCH, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

}  // namespace mt
