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
//   - its 8 waves split K in 32-k blocks (block j to wave j mod 8); a wave requests its A
//     tiles (one 16-byte chunk of weights per lane, nontemporal) before it stages x, so the
//     weight stream is in flight while x is converted;
//   - x is staged in LDS in chunks of 2048 k as hi + lo halves of the weights' 16-bit type
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

#include "mt_device.hpp"
#include "mt_internal.hpp"

namespace mt {

namespace {

constexpr int GM_THREADS = 512;
constexpr int GM_NW = GM_THREADS / 64;
constexpr int GM_KC = 2048;               // k per LDS chunk
constexpr int GM_XLD = GM_KC + 32;        // LDS row stride (elements)
constexpr int GM_BPW = GM_KC / 32 / GM_NW;  // 32-k blocks per wave per chunk
constexpr int GM_XCH = 8 * GM_KC / 4 / GM_THREADS;  // 4-element x chunks per thread per chunk (M <= 8)

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

__device__ __forceinline__ float wave_sum64(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Split-K arguments: S workgroups per tile (tile = block % tiles, split = block / tiles), kps
// 32-k blocks each; part / part_bytes / cnt: the stream's workspace (S > 1 only).
struct GmSplit {
    uint32_t tiles, splits, kps, part_bytes;
    float *part;
    uint32_t *cnt;
};

constexpr int SC1 = 16;  // buffer cache policy: device-coherent

template <int WT, int XT, bool GATED, bool NORM>
__global__ __launch_bounds__(GM_THREADS) void gemv_mfma_kernel(LinearArgs a, GmSplit sp) {
    constexpr int NCT = GATED ? 2 : 1;
    constexpr int REC = NCT * 128 + 8;  // a workgroup's sums: [plane][feature][row], then x^2 per row
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][8][GM_XLD];  // [hi, lo][row][k of the chunk]
    __shared__ float part[GM_NW][NCT][16][8];
    __shared__ float ssw[GM_NW][8];
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
    // B lane: column c = lane & 15 is half c & 1 of x row c >> 1.
    const uint32_t bc = lane & 15, bm = bc >> 1, bh = bc & 1;
    const bool bok = bm < M;
    const u32x4g *zero = reinterpret_cast<const u32x4g *>(g_gm_zero);

    f32x4g acc = {0.0f, 0.0f, 0.0f, 0.0f}, acc2 = acc;
    float ss[8];
#pragma unroll
    for (int m = 0; m < 8; m++) ss[m] = 0.0f;

    for (uint32_t kc0 = ks; kc0 < ke; kc0 += GM_KC) {
        const uint32_t kn = min(static_cast<uint32_t>(GM_KC), ke - kc0);
        const uint32_t nkb = (kn + 31) / 32;
        // This wave's weight tiles of the chunk: blocks w, w + 8, ... (requested first).
        u32x4g at[GM_BPW], at2[GM_BPW];
#pragma unroll
        for (int u = 0; u < GM_BPW; u++) {
            const uint32_t jb = w + GM_NW * u;
            const uint32_t k = kc0 + jb * 32 + 8 * (lane >> 4);  // K % 8 == 0: a chunk is all in or all out
            const bool ok = aok && jb < nkb && k < ke;
            const u32x4g *src = ok ? reinterpret_cast<const u32x4g *>(wrow + kc0 + jb * 32) : zero;
            at[u] = __builtin_nontemporal_load(reinterpret_cast<gw_cp4>(reinterpret_cast<uintptr_t>(src)));
            if constexpr (GATED) {
                const u32x4g *src2 = ok ? reinterpret_cast<const u32x4g *>(w2row + kc0 + jb * 32) : zero;
                at2[u] = __builtin_nontemporal_load(reinterpret_cast<gw_cp4>(reinterpret_cast<uintptr_t>(src2)));
            }
        }
        // Stage x[m][kc0 .. kc0 + kn) as hi + lo; the block tail past kn holds zeros.
        const uint32_t k4 = kn / 4, nch = M * k4;
#pragma unroll
        for (int r = 0; r < GM_XCH; r++) {
            const uint32_t e = tid + GM_THREADS * r;
            if (e < nch) {
                const uint32_t m = e / k4, kk = (e - m * k4) * 4;
                float x[4];
                if constexpr (XT == DT_F32) {
                    const float4 v = *reinterpret_cast<const float4 *>(static_cast<const float *>(a.x) +
                                                                       static_cast<size_t>(m) * a.ldx + kc0 + kk);
                    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
                } else {
                    const uint2 v = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(a.x) +
                                                                     static_cast<size_t>(m) * a.ldx + kc0 + kk);
                    x[0] = dec_lo<XT>(v.x); x[1] = dec_hi<XT>(v.x); x[2] = dec_lo<XT>(v.y); x[3] = dec_hi<XT>(v.y);
                }
                if constexpr (NORM) {
                    float t = x[0] * x[0];
                    t = fmaf(x[1], x[1], t);
                    t = fmaf(x[2], x[2], t);
                    t = fmaf(x[3], x[3], t);
#pragma unroll
                    for (int mm = 0; mm < 8; mm++) ss[mm] += m == static_cast<uint32_t>(mm) ? t : 0.0f;
                    const uint2 g = *reinterpret_cast<const uint2 *>(a.norm + kc0 + kk);
                    x[0] *= dec_lo<WT>(g.x);
                    x[1] *= dec_hi<WT>(g.x);
                    x[2] *= dec_lo<WT>(g.y);
                    x[3] *= dec_hi<WT>(g.y);
                }
                const uint32_t h0 = pack_pair<WT>(x[0], x[1]), h1 = pack_pair<WT>(x[2], x[3]);
                const uint32_t l0 = pack_pair<WT>(x[0] - dec_lo<WT>(h0), x[1] - dec_hi<WT>(h0));
                const uint32_t l1 = pack_pair<WT>(x[2] - dec_lo<WT>(h1), x[3] - dec_hi<WT>(h1));
                *reinterpret_cast<u32x2g *>(&xs[0][m][kk]) = u32x2g{h0, h1};
                *reinterpret_cast<u32x2g *>(&xs[1][m][kk]) = u32x2g{l0, l1};
            }
        }
        if (kn % 32) {  // zeros for the last block's k past kn (they meet zero weights)
            const uint32_t tail = nkb * 32 - kn;  // a multiple of 8
            for (uint32_t e = tid; e < 2 * M * tail; e += GM_THREADS) {
                const uint32_t h = e / (M * tail), rest = e - h * M * tail, m = rest / tail;
                xs[h][m][kn + rest - m * tail] = 0;
            }
        }
        __syncthreads();  // the chunk's x is staged
#pragma unroll
        for (int u = 0; u < GM_BPW; u++) {
            const uint32_t jb = w + GM_NW * u;
            if (jb < nkb) {
                u32x4g bv = {0u, 0u, 0u, 0u};
                if (bok) bv = *reinterpret_cast<const u32x4g *>(&xs[bh][bm][jb * 32 + 8 * (lane >> 4)]);
                acc = mfma16x32<WT>(at[u], bv, acc);
                if constexpr (GATED) acc2 = mfma16x32<WT>(at2[u], bv, acc2);
            }
        }
        __syncthreads();  // the chunk's x is no longer read
    }

    // Partial sums: lane (column c, row group q) holds D[4 q + i][c]; features 4 q + i of x
    // row c >> 1, half c & 1: the even lane of each pair stores hi + lo.
    {
        const uint32_t q = lane >> 4;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float e = pair_sum(acc[i]);
            if (bh == 0 && bm < 8) part[w][0][4 * q + i][bm] = e;
            if constexpr (GATED) {
                const float e2 = pair_sum(acc2[i]);
                if (bh == 0 && bm < 8) part[w][1][4 * q + i][bm] = e2;
            }
        }
    }
    if constexpr (NORM) {
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const float t = wave_sum64(ss[m]);
            if (lane == 0) ssw[w][m] = t;
        }
    }
    __syncthreads();
    // The workgroup's sums in wave order: element e of the record.
    float mine = 0.0f;
    if (tid < static_cast<uint32_t>(REC)) {
        if (tid < static_cast<uint32_t>(NCT * 128)) {
            const uint32_t p = tid >> 7, f = (tid >> 3) & 15, m = tid & 7;
#pragma unroll
            for (int ww = 0; ww < GM_NW; ww++) mine += part[ww][p][f][m];
        } else if constexpr (NORM) {
            const uint32_t m = tid - NCT * 128;
#pragma unroll
            for (int ww = 0; ww < GM_NW; ww++) mine += ssw[ww][m];
        }
    }
    if (sp.splits > 1) {
        const __amdgpu_buffer_rsrc_t rsrc =
            __builtin_amdgcn_make_buffer_rsrc(sp.part, 0, static_cast<int>(sp.part_bytes), 0x00020000);
        const uint32_t base = tile * sp.splits * static_cast<uint32_t>(REC) * 4u;
        if (tid < static_cast<uint32_t>(REC))
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(mine), rsrc, base + (split * REC + tid) * 4u, 0, SC1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) {
            const uint32_t old = __hip_atomic_fetch_add(sp.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_flag = old == sp.splits - 1;
        }
        __syncthreads();
        if (!last_flag) return;
        if (tid == 0) __hip_atomic_store(sp.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (tid < static_cast<uint32_t>(REC)) {  // the records in split order
            float t = 0.0f;
            for (uint32_t s = 0; s < sp.splits; s++)
                t += s == split ? mine
                                : __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc, base + (s * REC + tid) * 4u, 0, SC1));
            mine = t;
        }
    }
    if (tid < static_cast<uint32_t>(REC)) tot[tid] = mine;
    __syncthreads();
    if (tid < 16 * M) {
        const uint32_t f = tid / M, m = tid - f * M, n = r0 + f;
        if (n < a.N) {
            float s1 = tot[f * 8 + m], s2 = GATED ? tot[128 + f * 8 + m] : 0.0f;
            if constexpr (NORM) {
                const float scale = 1.0f / sqrtf(tot[NCT * 128 + m] / static_cast<float>(K) + a.eps);
                s1 *= scale;
                s2 *= scale;
            }
            const float b = (a.flags & F_BIAS) ? dec1<WT>(a.bias[n]) : 0.0f;
            float v = epilogue(s1, s2, b, a.flags);
            float *yp = a.y + static_cast<size_t>(m) * a.ldy + n;
            if (a.flags & F_ACCUM) v += *yp;
            *yp = v;
        }
    }
}

typedef void (*gm_fn)(LinearArgs, GmSplit);

template <int WT, int XT>
gm_fn gm_variant(bool gated, bool norm) {
    if (gated) return norm ? gemv_mfma_kernel<WT, XT, true, true> : gemv_mfma_kernel<WT, XT, true, false>;
    return norm ? gemv_mfma_kernel<WT, XT, false, true> : gemv_mfma_kernel<WT, XT, false, false>;
}

template <int WT>
gm_fn gm_x(int xt, bool gated, bool norm) {
    switch (xt) {
        case DT_F32: return gm_variant<WT, DT_F32>(gated, norm);
        case DT_F16: return gm_variant<WT, DT_F16>(gated, norm);
        default: return gm_variant<WT, DT_BF16>(gated, norm);
    }
}

}  // namespace

int launch_gemv_mfma(const LinearArgs &a, int xt, int wt, hipStream_t stream) {
    const bool gated = (a.flags & F_SILU_GATE) != 0;
    const bool norm = a.norm != nullptr;
    GmSplit sp{};
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
    sp.splits = (kb + sp.kps - 1) / sp.kps;  // no empty split
    if (sp.splits > 1) {
        const int rec = (gated ? 2 : 1) * 128 + 8;
        const size_t pb = static_cast<size_t>(sp.tiles) * sp.splits * rec * 4;
        if (pb > 0x7FFFFFF0u) return set_error(MT_ENOTSUP, "gemv_mfma: split-K workspace beyond 2 GiB");
        void *part = nullptr;
        uint32_t *cnt = nullptr;
        const int rc = stream_workspace(stream, pb, sp.tiles, &part, &cnt);
        if (rc) return rc;
        sp.part = static_cast<float *>(part);
        sp.part_bytes = static_cast<uint32_t>(pb);
        sp.cnt = cnt;
    }
    gm_fn fn = wt == DT_BF16 ? gm_x<DT_BF16>(xt, gated, norm) : gm_x<DT_F16>(xt, gated, norm);
    hipLaunchKernelGGL(fn, dim3(sp.tiles * sp.splits), dim3(GM_THREADS), 0, stream, a, sp);
    return check_launch("gemv_mfma");
}

}  // namespace mt
