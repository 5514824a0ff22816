// Linears of 3..8 rows on MFMA (mt_linear with 3 <= M <= 8).
//
// Reference kernel replaced: gemm8_kernel (Shaders.swift:110-283), the reference's path for
// 3 <= M <= 15 (the DiT's M = 6 and the VAE's M = 4, DiT.swift:35-52, VAEDecoder.swift:92).
// Same contract as every mt_linear: y = x W^T with the GemvFlags epilogue, fp32 accumulate.
//
// Why not the lane-group GEMV: there every lane group streaming one weight row also reads
// all M rows of x, so at M = 6 the activation reads outweigh the weights many times over.
// Here x is staged once per workgroup and the weights stream once:
//   - a 512-thread workgroup owns 16 output features (one 16-row MFMA A tile; with the SiLU
//     gate, the 16 matching rows of W2 too) over all of K;
//   - its 8 waves split K in 32-k blocks (pairs of blocks, so that one wave reads both
//     halves of each 128-byte weight line); a wave requests its A
//     tiles (one 16-byte chunk of weights per lane, nontemporal) before it stages x, so the
//     weight stream is in flight while x is converted;
//   - x is staged in LDS in chunks of 1024 k (512 for 64 columns) as hi + lo halves of the
//     weights' 16-bit type (or as it is when x has the weights' type and no norm is fused)
//     (hi rounded toward zero for fp16, to nearest for bf16; lo the rest), the RMSNorm gain
//     applied first and x^2 summed per row when the norm is fused;
//   - v_mfma_f32_16x16x32: B column c = 2 m + h holds half h of x row m (columns past 2 M
//     are zero), so one MFMA covers both halves of every row; neighbouring lanes add the
//     halves;
//   - the waves' partial sums meet in LDS and one lane per output adds them in wave order,
//     applies the norm scale and the epilogue, and stores;
//   - when the 16-feature tiles alone cannot fill the chip (N <= 2032), S workgroups share a
//     tile, each over its own range of 32-k blocks: each stores its partial sums (and
//     its rows' x^2 sums) to the stream's workspace with device-coherent stores, waits for
//     them and counts itself in; the last arrival adds the S records in split order and runs
//     the epilogue.
// Every summation order is fixed, so results are bit-identical from run to run.
#include <algorithm>

#include "dit_attend.hpp"
#include "mt_device.hpp"
#include "mt_internal.hpp"

namespace mt {

namespace {

constexpr int GM_THREADS = 512;
constexpr int GM_NW = GM_THREADS / 64;
constexpr int GM_LDS = 65536 + 2048;  // x staging: 32768 elements per chunk plus row pads (the partial sums reuse it)

typedef uint32_t u32x4g __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2g __attribute__((ext_vector_type(2)));
typedef float f32x4g __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8g __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8g __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(1))) const u32x4g *gw_cp4;

__device__ __attribute__((aligned(16))) uint32_t g_gm_zero[4];

template <int T>
__device__ __forceinline__ f32x4g mfma16x32(const u32x4g a, const u32x4g b, const f32x4g c) {
    if constexpr (T == DT_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8g, a), __builtin_bit_cast(bf16x8g, b),
                                                       c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8g, a), __builtin_bit_cast(f16x8g, b), c,
                                                      0, 0, 0);
}

// x = hi + lo, both of type T, packed in pairs.
template <int T>
__device__ __forceinline__ uint32_t pack_pair(float a, float b) {
    if constexpr (T == DT_BF16) {
        typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
        typedef float f2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, bf2));
    } else {
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
    }
}

// Sum of lane pairs (c, c ^ 1) of a row of 16: the hi and lo columns of one x row.
__device__ __forceinline__ float pair_sum(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}

// Sum over the 64 lanes, the same bits in every lane: quad swaps, half-row and row mirrors
// on DPP (rows of 16), then two exchanges between rows.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum64(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v += dpp_f<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    v += __shfl_xor(v, 16, 64);
    return v + __shfl_xor(v, 32, 64);
}

// Split-K arguments: S workgroups per tile (tile = block % tiles, split = block / tiles), kps
// 32-k blocks each; part / part_bytes / cnt: the stream's workspace (S > 1 only).
struct GmSplit {
    uint32_t tiles, splits, kps, part_bytes;
    float *part;
    uint32_t *cnt;
};

// The DiT attention that produces x (mt_dit_attention_linear): x row m = b S + i is query
// row i of sequence b, attended over qkv (a.x, row stride a.ldx) with H heads of 64.
struct GmAttn {
    const float *inv_freq;
    uint32_t S, H;
    float scale;
};

constexpr int SC1 = 16;  // buffer cache policy: device-coherent

// Shape of one instantiation: NG groups of 16 B columns; H2: x staged as hi + lo halves (x
// of another type than the weights, or a fused norm), so column c is half c & 1 of row c / 2,
// else column c is row c; MM rows at most; KC k per LDS chunk.
template <int NG, bool H2>
struct GmShape {
    static constexpr int HV = H2 ? 2 : 1;
    static constexpr int MM = 16 * NG / HV;
    static constexpr int KC = 32768 / (HV * MM) < 1024 ? 32768 / (HV * MM) : 1024;  // 1024 or 512: at most 4 blocks per wave
    static constexpr int XLD = KC + 16;            // row pad: rows 8 banks apart
    static constexpr int BPW = KC / 32 / GM_NW;  // 32-k blocks per wave per chunk
    static constexpr int XCH = MM * KC / 4 / GM_THREADS;
    static_assert(KC % (64 * GM_NW) == 0 && HV * MM * XLD * 2 <= GM_LDS, "x staging (block pairs per wave)");
};

template <int WT, int XT, bool GATED, bool NORM, int NG, bool ATT = false>
// (The attention-x variants take 2 waves per SIMD: their prologue needs the registers, and
// their few workgroups fill one per CU.)
__global__ __launch_bounds__(GM_THREADS, ATT ? 2 : 4) void gemv_mfma_kernel(LinearArgs a, GmSplit sp, GmAttn att) {
    constexpr bool H2 = XT != WT || NORM;
    typedef GmShape<NG, H2> S;
    constexpr int MM = S::MM, KC = S::KC, XLD = S::XLD, BPW = S::BPW, XCH = S::XCH;
    constexpr int NCT = GATED ? 2 : 1;
    constexpr int REC = NCT * 16 * MM + MM;  // a workgroup's sums: [plane][feature][row], then x^2 per row
    static_assert(GM_NW * NCT * 16 * MM * 4 <= GM_LDS, "partial sums overlay the staging");
    __shared__ __attribute__((aligned(16))) uint8_t smem[GM_LDS];
    uint16_t *xs = reinterpret_cast<uint16_t *>(smem);  // [half][row][k of the chunk], row stride XLD
    float *part = reinterpret_cast<float *>(smem);      // after the K loop: [wave][plane][feature][row]
    __shared__ float ssw[GM_NW][MM];
    __shared__ float tot[REC];
    __shared__ uint32_t last_flag;
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t M = a.M, K = a.K;
    const uint32_t tile = blockIdx.x % sp.tiles, split = blockIdx.x / sp.tiles;
    const uint32_t r0 = tile * 16;
    const uint32_t ks = split * sp.kps * 32, ke = min(K, (split + 1) * sp.kps * 32);  // this split's k range

    // A lane: weight row r0 + (lane & 15), 8 k from 8 (lane >> 4) of each 32-k block.
    const uint32_t arow = r0 + (lane & 15);
    const bool aok = arow < a.N;
    const uint16_t *wrow = a.w + static_cast<size_t>(aok ? arow : 0) * K + 8 * (lane >> 4);
    const uint16_t *w2row = (GATED ? a.w2 : a.w) + static_cast<size_t>(aok ? arow : 0) * K + 8 * (lane >> 4);
    // B lane of group g: column 16 g + (lane & 15).
    const uint32_t bc = lane & 15;
    const u32x4g *zero = reinterpret_cast<const u32x4g *>(g_gm_zero);

    f32x4g acc[NG], acc2[NG];
#pragma unroll
    for (int g = 0; g < NG; g++) acc[g] = acc2[g] = f32x4g{0.0f, 0.0f, 0.0f, 0.0f};
    float ss[MM];
#pragma unroll
    for (int m = 0; m < MM; m++) ss[m] = 0.0f;

    // The epilogue's bias and old y of output lane o = tid + GM_THREADS j (feature o / M, row
    // o % M), requested now so the epilogue does not wait for them (lanes past the outputs
    // read element 0).  Only this tile's final writer stores y, so the old value is the one
    // from before the launch.  PRE: the early requests here and of x below; the gated
    // multi-group variants have no registers to spare for them and request at the point of use.
    constexpr bool PRE = !(GATED && NG > 1);
    constexpr int OPT = (16 * MM + GM_THREADS - 1) / GM_THREADS;
    uint32_t pbias[OPT];
    float pyold[OPT];
#pragma unroll
    for (int j = 0; j < OPT; j++) {
        const uint32_t o = tid + GM_THREADS * j, f = o / M, m = o - f * M, n = r0 + f;
        const bool ok = o < 16 * M && n < a.N;
        pbias[j] = 0;
        pyold[j] = 0.0f;
        if (PRE && (a.flags & F_BIAS)) pbias[j] = a.bias[ok ? n : 0u];
        if (PRE && (a.flags & F_ACCUM)) pyold[j] = a.y[ok ? static_cast<size_t>(m) * a.ldy + n : 0u];
    }

    for (uint32_t kc0 = ks; kc0 < ke; kc0 += KC) {
        const uint32_t kn = min(static_cast<uint32_t>(KC), ke - kc0);
        const uint32_t nkb = (kn + 31) / 32;
        // Attention x: the chunk spans whole heads, items (row, head) go to the 16 half waves;
        // the first two items of each half wave are requested before the weights, so the
        // wait for them does not include the weight stream.
        DitItem di[2];
        float freq = 0.0f;
        const uint32_t hw = tid >> 5, nh = kn / 64, hb = kc0 / 64, items = ATT ? M * nh : 0u;
        auto item_rows = [&](uint32_t it, uint32_t &m, uint32_t &i) {
            const uint32_t hh = it % nh;
            m = it / nh;
            const uint32_t b = m / att.S;
            i = m - b * att.S;
            return static_cast<const float *>(a.x) + static_cast<size_t>(b) * att.S * a.ldx + (hb + hh) * 64 +
                   2 * (tid & 31);
        };
        if constexpr (ATT) {
            static_assert(XT == DT_F32 && !NORM && !GATED, "attention x is fp32, without a norm or gate");
            freq = att.inv_freq[tid & 31];
#pragma unroll
            for (uint32_t u = 0; u < 2; u++) {
                const uint32_t it = hw + 16 * u;
                if (it < items) {
                    uint32_t m, i;
                    const float *rows = item_rows(it, m, i);
                    dit_item_load(rows, a.ldx, att.H * 64, i, att.S, di[u]);
                }
            }
        }
        // The chunk's x (and norm gain) of the first XPF staging rounds (PRE), requested
        // before the weights so that the conversion waits for x alone; lanes past the chunk
        // read element 0.  Later rounds load at the point of use.
        const uint32_t k4 = kn / 4, nch = ATT ? 0u : M * k4;
        const uint32_t rounds = (nch + GM_THREADS - 1) / GM_THREADS;  // uniform
        constexpr int XPF = PRE ? (XCH < 8 ? XCH : 8) : 0;
        u32x4g xf[XT == DT_F32 ? XCH : 1];
        u32x2g xh[XT == DT_F32 ? 1 : XCH];
        u32x2g gn[NORM ? XCH : 1];
        auto fetch = [&](int r) {
            const uint32_t e = tid + GM_THREADS * r, ec = e < nch ? e : 0u;
            const uint32_t m = ec / k4, kk = (ec - m * k4) * 4;
            const size_t xo = static_cast<size_t>(m) * a.ldx + kc0 + kk;
            if constexpr (XT == DT_F32)
                xf[r] = *reinterpret_cast<const u32x4g *>(static_cast<const float *>(a.x) + xo);
            else
                xh[r] = *reinterpret_cast<const u32x2g *>(static_cast<const uint16_t *>(a.x) + xo);
            if constexpr (NORM) gn[r] = *reinterpret_cast<const u32x2g *>(a.norm + kc0 + kk);
        };
#pragma unroll
        for (int r = 0; r < XPF; r++)
            if (static_cast<uint32_t>(r) < rounds) fetch(r);
        // This wave's weight tiles of the chunk: block pairs (2 w, 2 w + 1),
        // (2 w + 16, 2 w + 17), ..., so the two 64-byte halves of each 128-byte weight line
        // come from one wave.
        u32x4g at[BPW], at2[BPW];
#pragma unroll
        for (int u = 0; u < BPW; u++) {
            const uint32_t jb = 2 * GM_NW * (u >> 1) + 2 * w + (u & 1);
            const uint32_t k = kc0 + jb * 32 + 8 * (lane >> 4);  // K % 8 == 0: a chunk is all in or all out
            const bool ok = aok && jb < nkb && k < ke;
            const u32x4g *src = ok ? reinterpret_cast<const u32x4g *>(wrow + kc0 + jb * 32) : zero;
            at[u] = __builtin_nontemporal_load(reinterpret_cast<gw_cp4>(reinterpret_cast<uintptr_t>(src)));
            if constexpr (GATED) {
                const u32x4g *src2 = ok ? reinterpret_cast<const u32x4g *>(w2row + kc0 + jb * 32) : zero;
                at2[u] = __builtin_nontemporal_load(reinterpret_cast<gw_cp4>(reinterpret_cast<uintptr_t>(src2)));
            }
        }
        // Stage x[m][kc0 .. kc0 + kn); the block tail past kn holds zeros.
        if constexpr (ATT) {
            // x is the attention output, staged as hi + lo pairs like any fp32 x.
            float c[DIT_MAXS], s[DIT_MAXS];
            dit_rope_table(freq, att.S, c, s);
            auto stage = [&](uint32_t it, const DitItem &d) {
                uint32_t m, i;
                item_rows(it, m, i);
                const float2 o = dit_item_attend(d, i, att.S, c, s, att.scale);
                const uint32_t hi = pack_pair<WT>(o.x, o.y), lo = pack_pair<WT>(o.x - dec_lo<WT>(hi), o.y - dec_hi<WT>(hi));
                const uint32_t kk = (it % nh) * 64 + 2 * (tid & 31);
                *reinterpret_cast<uint32_t *>(xs + m * XLD + kk) = hi;
                *reinterpret_cast<uint32_t *>(xs + (MM + m) * XLD + kk) = lo;
            };
#pragma unroll
            for (uint32_t u = 0; u < 2; u++)
                if (hw + 16 * u < items) stage(hw + 16 * u, di[u]);
            for (uint32_t it = hw + 32; it < items; it += 16) {  // items past the first two, one at a time
                uint32_t m, i;
                const float *rows = item_rows(it, m, i);
                dit_item_load(rows, a.ldx, att.H * 64, i, att.S, di[0]);
                stage(it, di[0]);
            }
        }
#pragma unroll
        for (int r = 0; r < XCH; r++) {
            const uint32_t e = tid + GM_THREADS * r;
            if (e < nch) {
                if (r >= XPF) fetch(r);
                const uint32_t m = e / k4, kk = (e - m * k4) * 4;
                if constexpr (!H2) {  // x of the weights' type: staged as it is
                    *reinterpret_cast<u32x2g *>(xs + m * XLD + kk) = xh[r];
                } else {
                    float x[4];
                    if constexpr (XT == DT_F32) {
                        x[0] = __uint_as_float(xf[r].x); x[1] = __uint_as_float(xf[r].y);
                        x[2] = __uint_as_float(xf[r].z); x[3] = __uint_as_float(xf[r].w);
                    } else {
                        const u32x2g v = xh[r];
                        x[0] = dec_lo<XT>(v.x); x[1] = dec_hi<XT>(v.x); x[2] = dec_lo<XT>(v.y); x[3] = dec_hi<XT>(v.y);
                    }
                    if constexpr (NORM) {
                        float t = x[0] * x[0];
                        t = fmaf(x[1], x[1], t);
                        t = fmaf(x[2], x[2], t);
                        t = fmaf(x[3], x[3], t);
#pragma unroll
                        for (int mm = 0; mm < MM; mm++) ss[mm] += m == static_cast<uint32_t>(mm) ? t : 0.0f;
                        const u32x2g g = gn[r];
                        x[0] *= dec_lo<WT>(g.x);
                        x[1] *= dec_hi<WT>(g.x);
                        x[2] *= dec_lo<WT>(g.y);
                        x[3] *= dec_hi<WT>(g.y);
                    }
                    const uint32_t h0 = pack_pair<WT>(x[0], x[1]), h1 = pack_pair<WT>(x[2], x[3]);
                    const uint32_t l0 = pack_pair<WT>(x[0] - dec_lo<WT>(h0), x[1] - dec_hi<WT>(h0));
                    const uint32_t l1 = pack_pair<WT>(x[2] - dec_lo<WT>(h1), x[3] - dec_hi<WT>(h1));
                    *reinterpret_cast<u32x2g *>(xs + m * XLD + kk) = u32x2g{h0, h1};
                    *reinterpret_cast<u32x2g *>(xs + (MM + m) * XLD + kk) = u32x2g{l0, l1};
                }
            }
        }
        if (kn % 32) {  // zeros for the last block's k past kn (they meet zero weights)
            const uint32_t tail = nkb * 32 - kn;  // a multiple of 8
            for (uint32_t e = tid; e < S::HV * M * tail; e += GM_THREADS) {
                const uint32_t h = e / (M * tail), rest = e - h * M * tail, m = rest / tail;
                xs[(h * MM + m) * XLD + kn + rest - m * tail] = 0;
            }
        }
        __syncthreads();  // the chunk's x is staged
#pragma unroll
        for (int u = 0; u < BPW; u++) {
            const uint32_t jb = 2 * GM_NW * (u >> 1) + 2 * w + (u & 1);
            if (jb < nkb) {
#pragma unroll
                for (int g = 0; g < NG; g++) {
                    const uint32_t col = 16 * g + bc, m = H2 ? col >> 1 : col, h = H2 ? col & 1 : 0;
                    u32x4g bv = {0u, 0u, 0u, 0u};
                    if (m < M) bv = *reinterpret_cast<const u32x4g *>(xs + (h * MM + m) * XLD + jb * 32 + 8 * (lane >> 4));
                    acc[g] = mfma16x32<WT>(at[u], bv, acc[g]);
                    if constexpr (GATED) acc2[g] = mfma16x32<WT>(at2[u], bv, acc2[g]);
                }
            }
        }
        __syncthreads();  // the chunk's x is no longer read (the partial sums reuse its LDS)
    }

    // Partial sums: lane (column c, row group q) of group g holds D[4 q + i][16 g + c]:
    // feature 4 q + i; with halves, the even lane of each pair stores hi + lo.
    {
        const uint32_t q = lane >> 4;
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const uint32_t col = 16 * g + bc, m = H2 ? col >> 1 : col;
            const bool store = (!H2 || (col & 1) == 0) && m < static_cast<uint32_t>(MM);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float e = H2 ? pair_sum(acc[g][i]) : acc[g][i];
                if (store) part[((w * NCT + 0) * 16 + 4 * q + i) * MM + m] = e;
                if constexpr (GATED) {
                    const float e2 = H2 ? pair_sum(acc2[g][i]) : acc2[g][i];
                    if (store) part[((w * NCT + 1) * 16 + 4 * q + i) * MM + m] = e2;
                }
            }
        }
    }
    if constexpr (NORM) {
#pragma unroll
        for (int m = 0; m < MM; m++) {
            const float t = wave_sum64(ss[m]);
            if (lane == 0) ssw[w][m] = t;
        }
    }
    __syncthreads();
    // The workgroup's sums in wave order, then (split-K) the splits' records in split order.
    constexpr int RPT = (REC + GM_THREADS - 1) / GM_THREADS;  // record elements per thread
    float mine[RPT];
#pragma unroll
    for (int r = 0; r < RPT; r++) {
        const uint32_t e = tid + GM_THREADS * r;
        float t = 0.0f;
        if (e < static_cast<uint32_t>(NCT * 16 * MM)) {
#pragma unroll
            for (int ww = 0; ww < GM_NW; ww++) t += part[ww * NCT * 16 * MM + e];
        } else if (NORM && e < static_cast<uint32_t>(REC)) {
#pragma unroll
            for (int ww = 0; ww < GM_NW; ww++) t += ssw[ww][e - NCT * 16 * MM];
        }
        mine[r] = t;
    }
    if (sp.splits > 1) {
        const __amdgpu_buffer_rsrc_t rsrc =
            __builtin_amdgcn_make_buffer_rsrc(sp.part, 0, static_cast<int>(sp.part_bytes), 0x00020000);
        const uint32_t base = tile * sp.splits * static_cast<uint32_t>(REC) * 4u;
#pragma unroll
        for (int r = 0; r < RPT; r++) {
            const uint32_t e = tid + GM_THREADS * r;
            if (e < static_cast<uint32_t>(REC))
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(mine[r]), rsrc, base + (split * REC + e) * 4u, 0, SC1);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) {
            const uint32_t old = __hip_atomic_fetch_add(sp.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_flag = old == sp.splits - 1;
        }
        __syncthreads();
        if (!last_flag) return;
        if (tid == 0) __hip_atomic_store(sp.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // The splits' records, added in split order: the first SR requested together, the
        // rest one by one.
        constexpr uint32_t SR = 8;
#pragma unroll
        for (int r = 0; r < RPT; r++) {
            const uint32_t e = tid + GM_THREADS * r;
            if (e < static_cast<uint32_t>(REC)) {
                float v[SR];
#pragma unroll
                for (uint32_t s = 0; s < SR; s++)
                    v[s] = s < sp.splits && s != split
                               ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc, base + (s * REC + e) * 4u, 0, SC1))
                               : mine[r];
                float t = 0.0f;
#pragma unroll
                for (uint32_t s = 0; s < SR; s++)
                    if (s < sp.splits) t += v[s];
                for (uint32_t s = SR; s < sp.splits; s++)
                    t += s == split ? mine[r]
                                    : __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc, base + (s * REC + e) * 4u,
                                                                                           0, SC1));
                mine[r] = t;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPT; r++) {
        const uint32_t e = tid + GM_THREADS * r;
        if (e < static_cast<uint32_t>(REC)) tot[e] = mine[r];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < OPT; j++) {
        const uint32_t o = tid + GM_THREADS * j, f = o / M, m = o - f * M, n = r0 + f;
        if (o < 16 * M && n < a.N) {
            float s1 = tot[f * MM + m], s2 = GATED ? tot[16 * MM + f * MM + m] : 0.0f;
            if constexpr (NORM) {
                const float scale = rsqrt_hw(tot[NCT * 16 * MM + m] / static_cast<float>(K) + a.eps);
                s1 *= scale;
                s2 *= scale;
            }
            float *yp = a.y + static_cast<size_t>(m) * a.ldy + n;
            const float b = (a.flags & F_BIAS) ? dec1<WT>(PRE ? static_cast<uint16_t>(pbias[j]) : a.bias[n]) : 0.0f;
            float v = epilogue(s1, s2, b, a.flags);
            if (a.flags & F_ACCUM) v += PRE ? pyold[j] : *yp;
            *yp = v;
        }
    }
}

typedef void (*gm_fn)(LinearArgs, GmSplit, GmAttn);

template <int WT, int XT, int NG>
gm_fn gm_variant(bool gated, bool norm) {
    if constexpr (NG == 1) {
        if (gated) return norm ? gemv_mfma_kernel<WT, XT, true, true, 1> : gemv_mfma_kernel<WT, XT, true, false, 1>;
        return norm ? gemv_mfma_kernel<WT, XT, false, true, 1> : gemv_mfma_kernel<WT, XT, false, false, 1>;
    } else {
        (void)norm;  // a fused norm takes at most 8 rows
        return gated ? gemv_mfma_kernel<WT, XT, true, false, NG> : gemv_mfma_kernel<WT, XT, false, false, NG>;
    }
}

template <int WT, int NG>
gm_fn gm_x(int xt, bool gated, bool norm) {
    switch (xt) {
        case DT_F32: return gm_variant<WT, DT_F32, NG>(gated, norm);
        case DT_F16: return gm_variant<WT, DT_F16, NG>(gated, norm);
        default: return gm_variant<WT, DT_BF16, NG>(gated, norm);
    }
}

template <int NG>
gm_fn gm_w(int wt, int xt, bool gated, bool norm) {
    return wt == DT_BF16 ? gm_x<DT_BF16, NG>(xt, gated, norm) : gm_x<DT_F16, NG>(xt, gated, norm);
}

}  // namespace

// B columns the kernel needs for M rows: M for x of the weights' type without a norm, else
// 2 M (hi + lo halves); 0 if more than 64 (or a fused norm past 8 rows).
int gemv_mfma_columns(uint32_t M, int xt, int wt, bool norm) {
    const bool h2 = xt != wt || norm;
    if (norm && M > 8) return 0;
    const uint32_t cols = h2 ? 2 * M : M;
    return cols <= 64 ? static_cast<int>(cols) : 0;
}

namespace {

// Tiles, splits and (for S > 1) the stream's split-K workspace.  even: splits start at
// multiples of 64 k (whole attention heads).
int gm_splits(const LinearArgs &a, int xt, int wt, bool gated, bool norm, int ng, bool even, hipStream_t stream,
              GmSplit &sp, const FixedWs *fixed = nullptr) {
    sp = GmSplit{};
    sp.tiles = (a.N + 15) / 16;
    const uint32_t kb = (a.K + 31) / 32;
    // Splits: enough workgroups for 256 CUs when the tiles are few, each split at least 8
    // blocks (one per wave); MT_TUNE_GEMM_SPLITK forces a count.
    uint32_t s = 1;
    const int forced = tuning().gemm_splitk;
    if (forced > 0) s = static_cast<uint32_t>(forced);
    else if (sp.tiles < 128) s = std::max(1u, std::min((256u + sp.tiles - 1) / sp.tiles, kb / 8));
    s = std::min(s, std::min(kb, 64u));
    sp.kps = (kb + s - 1) / s;
    if (even) sp.kps += sp.kps & 1u;
    sp.splits = (kb + sp.kps - 1) / sp.kps;  // no empty split
    if (sp.splits > 1) {
        const int mm = 16 * ng / ((xt != wt || norm) ? 2 : 1);
        const int rec = (gated ? 2 : 1) * 16 * mm + mm;
        const size_t pb = static_cast<size_t>(sp.tiles) * sp.splits * rec * 4;
        if (pb > 0x7FFFFFF0u) return set_error(MT_ENOTSUP, "gemv_mfma: split-K workspace beyond 2 GiB");
        void *part = nullptr;
        uint32_t *cnt = nullptr;
        const int rc = split_workspace(fixed, stream, pb, sp.tiles, &part, &cnt, "gemv_mfma");
        if (rc) return rc;
        sp.part = static_cast<float *>(part);
        sp.part_bytes = static_cast<uint32_t>(pb);
        sp.cnt = cnt;
    }
    return MT_OK;
}

template <int WT>
gm_fn gm_attn(int ng) {
    return ng == 1 ? gemv_mfma_kernel<WT, DT_F32, false, false, 1, true>
                   : ng == 2 ? gemv_mfma_kernel<WT, DT_F32, false, false, 2, true>
                             : gemv_mfma_kernel<WT, DT_F32, false, false, 4, true>;
}

}  // namespace

int launch_gemv_mfma(const LinearArgs &a, int xt, int wt, hipStream_t stream, const FixedWs *fixed) {
    const bool gated = (a.flags & F_SILU_GATE) != 0;
    const bool norm = a.norm != nullptr;
    const int cols = gemv_mfma_columns(a.M, xt, wt, norm);
    if (cols == 0) return set_error(MT_ENOTSUP, "gemv_mfma: %u rows exceed the kernel's columns", a.M);
    const int ng = cols <= 16 ? 1 : cols <= 32 ? 2 : 4;
    GmSplit sp;
    const int rc = gm_splits(a, xt, wt, gated, norm, ng, false, stream, sp, fixed);
    if (rc) return rc;
    gm_fn fn = ng == 1 ? gm_w<1>(wt, xt, gated, norm) : ng == 2 ? gm_w<2>(wt, xt, gated, norm) : gm_w<4>(wt, xt, gated, norm);
    hipLaunchKernelGGL(fn, dim3(sp.tiles * sp.splits), dim3(GM_THREADS), 0, stream, a, sp, GmAttn{});
    return check_launch("gemv_mfma");
}

int launch_gemv_mfma_attn(const LinearArgs &a, int wt, const float *inv_freq, uint32_t S, uint32_t H, float scale,
                          hipStream_t stream) {
    const int cols = gemv_mfma_columns(a.M, DT_F32, wt, false);
    if (cols == 0) return set_error(MT_ENOTSUP, "gemv_mfma: %u rows exceed the kernel's columns", a.M);
    if (a.K != H * 64 || a.norm || (a.flags & F_SILU_GATE) || S == 0 || S > DIT_MAXS || a.M % S)
        return set_error(MT_EINVAL, "gemv_mfma: attention x needs K = 64 H, M a multiple of S <= %d, no norm or gate",
                         DIT_MAXS);
    const int ng = cols <= 16 ? 1 : cols <= 32 ? 2 : 4;
    GmSplit sp;
    const int rc = gm_splits(a, DT_F32, wt, false, false, ng, true, stream, sp);
    if (rc) return rc;
    gm_fn fn = wt == DT_BF16 ? gm_attn<DT_BF16>(ng) : gm_attn<DT_F16>(ng);
    hipLaunchKernelGGL(fn, dim3(sp.tiles * sp.splits), dim3(GM_THREADS), 0, stream, a, sp, GmAttn{inv_freq, S, H, scale});
    return check_launch("gemv_mfma");
}

}  // namespace mt
