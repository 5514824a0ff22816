// The C ABI (include/mingtts_hip.h): argument validation, kernel choice, error text.
//
// Validation happens before any HIP call, so a rejected call touches no device state
// and works without a GPU (the CPU tests rely on that).  Shape errors that the reference
// turns into preconditionFailure (Kernels.swift:105, 147) are returned as MT_EINVAL.
#include <errno.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <new>
#include <vector>

#include "mingtts_hip.h"
#include "mt_internal.hpp"

namespace mt {


namespace {
thread_local char g_err[512] = "";
Tuning g_tuning;

size_t dtype_size(int t) { return t == DT_F32 ? 4 : 2; }
bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
const char *dtype_name(int t) { return t == DT_F32 ? "f32" : t == DT_F16 ? "f16" : t == DT_BF16 ? "bf16" : "?"; }
}  // namespace

Tuning &tuning() { return g_tuning; }

int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(MT_EHIP, "%s launch: %s", what, hipGetErrorString(e));
    return MT_OK;
}

// Checks one linear's arguments; fills `a` (with the bias flag set from the pointer,
// Kernels.swift:135).  Returns MT_OK or MT_EINVAL with the reason.
static int validate_linear(const char *who, const void *x, int xt, const void *w, const void *w2, int wt,
                           const void *bias, const void *norm, float *y, const mt_gemv_params &p,
                           LinearArgs &a) {
    if (xt != DT_F32 && xt != DT_F16 && xt != DT_BF16)
        return set_error(MT_EINVAL, "%s: unknown activation dtype %d", who, xt);
    if (wt != DT_F16 && wt != DT_BF16)
        return set_error(MT_EINVAL, "%s: weights must be f16 or bf16, got %s", who, dtype_name(wt));
    const uint32_t known = MT_BIAS | MT_ACCUM | MT_GELU | MT_SILU_GATE | MT_SILU;
    if (p.flags & ~known) return set_error(MT_EINVAL, "%s: unknown flag bits 0x%x", who, p.flags & ~known);
    uint32_t flags = p.flags;
    if (bias) flags |= MT_BIAS;
    if ((flags & MT_BIAS) && !bias) return set_error(MT_EINVAL, "%s: MT_BIAS without a bias pointer", who);
    if ((flags & MT_SILU_GATE) && !w2) return set_error(MT_EINVAL, "%s: MT_SILU_GATE without w2", who);
    if (p.M && p.N) {
        if (!x || !w || !y) return set_error(MT_EINVAL, "%s: null x, w or y", who);
        if (p.K == 0 || p.K % 8) return set_error(MT_EINVAL, "%s: K must be a positive multiple of 8, got %u", who, p.K);
        if (p.ldx < p.K) return set_error(MT_EINVAL, "%s: ldx %u < K %u", who, p.ldx, p.K);
        if (p.ldy < p.N) return set_error(MT_EINVAL, "%s: ldy %u < N %u", who, p.ldy, p.N);
        if (!aligned(x, 16) || (static_cast<size_t>(p.ldx) * dtype_size(xt)) % 16)
            return set_error(MT_EINVAL, "%s: x must be 16-byte aligned with 16-byte row stride", who);
        if (!aligned(w, 16) || (w2 && (flags & MT_SILU_GATE) && !aligned(w2, 16)))
            return set_error(MT_EINVAL, "%s: w / w2 must be 16-byte aligned", who);
        if (!aligned(y, 4)) return set_error(MT_EINVAL, "%s: y must be 4-byte aligned", who);
        if (bias && !aligned(bias, 2)) return set_error(MT_EINVAL, "%s: bias must be 2-byte aligned", who);
        if (norm && !aligned(norm, 16)) return set_error(MT_EINVAL, "%s: norm must be 16-byte aligned", who);
        if (norm && !(p.eps >= 0.0f)) return set_error(MT_EINVAL, "%s: RMSNorm eps must be >= 0", who);
        // x must not overlap y (y may be read-modify-written under MT_ACCUM).
        const char *xb = static_cast<const char *>(x);
        const char *xe = xb + (static_cast<size_t>(p.M - 1) * p.ldx + p.K) * dtype_size(xt);
        const char *yb = reinterpret_cast<const char *>(y);
        const char *ye = yb + (static_cast<size_t>(p.M - 1) * p.ldy + p.N) * 4;
        if (xb < ye && yb < xe) return set_error(MT_EINVAL, "%s: x overlaps y", who);
    }
    a.x = x;
    a.w = static_cast<const uint16_t *>(w);
    a.w2 = static_cast<const uint16_t *>((flags & MT_SILU_GATE) ? w2 : w);
    a.bias = static_cast<const uint16_t *>(bias);
    a.y = y;
    a.M = p.M;
    a.N = p.N;
    a.K = p.K;
    a.ldx = p.ldx;
    a.ldy = p.ldy;
    a.flags = flags;
    a.norm = static_cast<const uint16_t *>(norm);
    a.eps = p.eps;
    return MT_OK;
}

// The kernel family mt_linear (norm false) or mt_linear_rmsnorm (norm true) runs M rows on,
// from one read of each tuning value: mt_linear_kernel reports it, the launchers follow it.
static int linear_family(uint32_t M, int xt, int wt, bool norm) {
    const int rows_max = g_tuning.gemv_rows_max.load(std::memory_order_relaxed);
    const int mode = g_tuning.gemv_mfma.load(std::memory_order_relaxed);
    if (static_cast<int>(M) <= rows_max) return M >= 3 && M <= 8 && mode != 1 ? MT_KERNEL_GEMV_MFMA : MT_KERNEL_GEMV;
    if ((mode == 2 || (mode == 0 && M <= 16)) && gemv_mfma_columns(M, xt, wt, norm) > 0) return MT_KERNEL_GEMV_MFMA;
    return MT_KERNEL_GEMM;
}

static int launch_family(const LinearArgs &a, int xt, int wt, hipStream_t s, const FixedWs *fixed = nullptr) {
    switch (linear_family(a.M, xt, wt, a.norm != nullptr)) {
        case MT_KERNEL_GEMV: return launch_gemv(a, xt, wt, s, g_tuning.gemv_lanes);
        case MT_KERNEL_GEMV_MFMA: return launch_gemv_mfma(a, xt, wt, s, fixed);
        default: return launch_gemm(a, xt, wt, s, fixed);
    }
}

}  // namespace mt

using namespace mt;

extern "C" {

const char *mt_last_error(void) { return g_err; }

const char *mt_version(void) { return "mingtts_hip 0.1.0 gfx950"; }

int mt_linear_kernel(uint32_t M, uint32_t N, uint32_t K, mt_dtype xt, mt_dtype wt) {
    (void)N;
    (void)K;
    return linear_family(M, xt, wt, false);
}

int mt_set_tuning(int key, int value) {
    std::atomic<int> *slot = nullptr;
    int def = 0;
    switch (key) {
        case MT_TUNE_GEMV_ROWS_MAX: slot = &g_tuning.gemv_rows_max; def = 8; break;
        case MT_TUNE_GEMV_LANES: slot = &g_tuning.gemv_lanes; def = 0; break;
        case MT_TUNE_GEMM_SPLITK: slot = &g_tuning.gemm_splitk; def = 0; break;
        case MT_TUNE_SEQ_GROUPS: slot = &g_tuning.seq_groups; def = 0; break;
        case MT_TUNE_SEQ_LAUNCH: slot = &g_tuning.seq_launch; def = 1; break;
        case MT_TUNE_GEMM_TILE: slot = &g_tuning.gemm_tile; def = 0; break;
        case MT_TUNE_GEMM_STAGES: slot = &g_tuning.gemm_stages; def = 0; break;
        case MT_TUNE_GEMV_MFMA: slot = &g_tuning.gemv_mfma; def = 0; break;
        case MT_TUNE_SEQ_LAYER: slot = &g_tuning.seq_layer; def = 0; break;
        default: return set_error(MT_EINVAL, "mt_set_tuning: unknown key %d", key);
    }
    if (key == MT_TUNE_SEQ_LAUNCH && value > 1)
        return set_error(MT_EINVAL, "mt_set_tuning: the sequence launch mode is 0 or 1, got %d", value);
    if (key == MT_TUNE_SEQ_LAYER && value > 1)
        return set_error(MT_EINVAL, "mt_set_tuning: the decode-layer kernel choice is 0 or 1, got %d", value);
    if (key == MT_TUNE_GEMV_MFMA && value > 2)
        return set_error(MT_EINVAL, "mt_set_tuning: the small-M kernel choice is 0, 1 or 2, got %d", value);
    if (key == MT_TUNE_GEMM_STAGES && value > 4)
        return set_error(MT_EINVAL, "mt_set_tuning: the GEMM pipeline depth is 1..4, got %d", value);
    if (key == MT_TUNE_GEMM_TILE && value > 5)
        return set_error(MT_EINVAL, "mt_set_tuning: the GEMM tile choice is 0..5, got %d", value);
    if (key == MT_TUNE_GEMV_ROWS_MAX && value > 8)
        return set_error(MT_EINVAL, "mt_set_tuning: the GEMV takes at most 8 rows per block, got %d", value);
    return slot->exchange(value < 0 ? def : value, std::memory_order_relaxed);
}

int mt_linear(const void *x, mt_dtype xt, const void *w, const void *w2, mt_dtype wt, const void *bias,
              float *y, mt_gemv_params p, mt_stream_t stream) {
    LinearArgs a;
    int rc = validate_linear("mt_linear", x, xt, w, w2, wt, bias, nullptr, y, p, a);
    if (rc) return rc;
    if (p.M == 0 || p.N == 0) return MT_OK;
    return launch_family(a, xt, wt, reinterpret_cast<hipStream_t>(stream));
}

int mt_linear_static(const void *x, mt_dtype xt, const void *w, const void *w2, mt_dtype wt, const void *bias,
                     float *y, mt_gemv_params p, mt_stream_t stream) {
    LinearArgs a;
    int rc = validate_linear("mt_linear_static", x, xt, w, w2, wt, bias, nullptr, y, p, a);
    if (rc) return rc;
    if (p.M == 0 || p.N == 0) return MT_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    FixedWs ws;
    rc = static_scratch(s, ws);
    if (rc) return rc;
    return launch_family(a, xt, wt, s, &ws);
}

int mt_linear_rmsnorm(const void *x, mt_dtype xt, const void *norm, const void *w, const void *w2, mt_dtype wt,
                      const void *bias, float *y, mt_gemv_params p, mt_stream_t stream) {
    if (!norm) return set_error(MT_EINVAL, "mt_linear_rmsnorm: null norm");
    LinearArgs a;
    int rc = validate_linear("mt_linear_rmsnorm", x, xt, w, w2, wt, bias, norm, y, p, a);
    if (rc) return rc;
    if (p.M == 0 || p.N == 0) return MT_OK;
    return launch_family(a, xt, wt, reinterpret_cast<hipStream_t>(stream));
}

// Shared checks of the rope / attention entry points.
static int validate_heads(const char *who, uint32_t hq, uint32_t hkv, int ct, uint32_t cache_len) {
    if (hq == 0 || hkv == 0 || hq % hkv) return set_error(MT_EINVAL, "%s: hq %u must be a positive multiple of hkv %u", who, hq, hkv);
    if (ct != DT_F32 && ct != DT_F16) return set_error(MT_EINVAL, "%s: cache dtype must be f32 or f16", who);
    if (cache_len == 0 || cache_len > 4096) return set_error(MT_EINVAL, "%s: cache_len %u outside 1..4096", who, cache_len);
    return MT_OK;
}

int mt_seq_create_items(const mt_seq_item *items, uint32_t n_items, mt_seq **out) {
    if (!out) return set_error(MT_EINVAL, "mt_seq_create: null out");
    *out = nullptr;
    if (n_items && !items) return set_error(MT_EINVAL, "mt_seq_create: null ops");
    for (uint32_t i = 0; i < n_items; i++) {
        char who[48];
        snprintf(who, sizeof(who), "mt_seq_create: op %u", i);
        if (items[i].kind == MT_SEQ_ATTENTION) {
            const mt_attn_op &a = items[i].attn;
            int rc = validate_heads(who, a.hq, a.hkv, a.cache_t, a.cache_len);
            if (rc) return rc;
            if (a.B == 0 || a.B > 8) return set_error(MT_EINVAL, "%s: an attention item takes 1 <= B <= 8, got %u", who, a.B);
            if (!a.qkv || !a.pos || !a.k_cache || !a.v_cache || !a.inv_freq || !a.out)
                return set_error(MT_EINVAL, "%s: null pointer", who);
            if (a.ldq < (a.hq + 2 * a.hkv) * 64 || a.ldo < a.hq * 64)
                return set_error(MT_EINVAL, "%s: ldq < (hq + 2 hkv) * 64 or ldo < hq * 64", who);
            if (!aligned(a.qkv, 16) || a.ldq % 4 || !aligned(a.out, 16) || a.ldo % 4 || !aligned(a.k_cache, 16) ||
                !aligned(a.v_cache, 16) || a.cache_stride % 8)
                return set_error(MT_EINVAL, "%s: qkv, out and the caches must be 16-byte aligned with 16-byte row strides",
                                 who);
            // Stride 0 with B > 1: rows of one sequence sharing one cache; otherwise one cache a row.
            if (a.B > 1 && a.cache_stride != 0 && a.cache_stride < static_cast<uint64_t>(a.hkv) * a.cache_len * 64)
                return set_error(MT_EINVAL, "%s: cache_stride smaller than one cache (0 for rows of one sequence)",
                                 who);
        } else if (items[i].kind == MT_SEQ_DIT_ATTENTION) {
            const mt_dit_attn_op &a = items[i].dit;
            if (a.B == 0 || a.S == 0 || a.H == 0 || a.S > 8 || a.B * a.S > 8)
                return set_error(MT_EINVAL, "%s: a DiT attention item takes B, S, H >= 1, S <= 8 and B S <= 8", who);
            if (!a.qkv || !a.inv_freq || !a.out) return set_error(MT_EINVAL, "%s: null pointer", who);
            if (a.ldq < 3 * a.H * 64 || a.ldo < a.H * 64)
                return set_error(MT_EINVAL, "%s: ldq < 3 H * 64 or ldo < H * 64", who);
            if (!aligned(a.qkv, 16) || a.ldq % 4 || !aligned(a.out, 16) || a.ldo % 4)
                return set_error(MT_EINVAL, "%s: qkv and out must be 16-byte aligned with 16-byte row strides", who);
        } else if (items[i].kind == MT_SEQ_LINEAR) {
            const mt_linear_op &o = items[i].linear;
            LinearArgs a;
            int rc = validate_linear(who, o.x, o.xt, o.w, o.w2, o.wt, o.bias, o.norm, o.y, o.p, a);
            if (rc) return rc;
            if (o.p.M == 0 || o.p.N == 0) return set_error(MT_EINVAL, "%s: empty op", who);
            if (o.p.M > 8) return set_error(MT_EINVAL, "%s: a sequence takes M <= 8, got %u", who, o.p.M);
        } else {
            return set_error(MT_EINVAL, "%s: unknown kind %d", who, items[i].kind);
        }
    }
    // Plan at a workgroup count: the dataflow form (hazards the reordering could break),
    // then the kernel: the decode-layer kernel when the ops repeat the Qwen2-0.5B decode
    // layer and the count fits its tiling, the DiT-block kernel for the flow head's DiT
    // blocks, else the general kernel within its limits.
    auto plan_at = [&](int g, std::vector<SeqOp> &d, int &w, int &k) {
        int r = seq_plan(items, n_items, g, d, w);
        if (r) return r;
        const bool special = g_tuning.seq_layer == 0;
        k = special && layer_pattern(d.data(), n_items, g)  ? MT_SEQ_DECODE_LAYER
            : special && dit_pattern(d.data(), n_items, g) ? MT_SEQ_DIT_BLOCK
                                                            : MT_SEQ_GENERAL;
        return k != MT_SEQ_GENERAL ? MT_OK : seq_general_limits(items, n_items, g);
    };
    // Plan once with the expected workgroup count before touching the device, so a sequence
    // no kernel can take is rejected without a GPU; re-plan for the device's counts.
    std::vector<SeqOp> dev;
    int wt = DT_F16;
    int kind = MT_SEQ_GENERAL;
    const int want = g_tuning.seq_groups;
    const int guess = want > 0 ? want : 256;
    int rc = plan_at(guess, dev, wt, kind);
    if (rc) return rc;
    if (n_items == 0) return set_error(MT_EINVAL, "mt_seq_create: empty sequence");
    int groups = 0, preferred = 0;
    rc = seq_limits(&groups, &preferred);
    if (rc) return rc;
    // The preferred count when the plan fits it, else every workgroup the device holds.
    std::vector<SeqOp> d2;
    int wt2 = DT_F16;
    int kind2 = MT_SEQ_GENERAL;
    if (plan_at(preferred, d2, wt2, kind2) == MT_OK) {
        groups = preferred;
    } else {
        rc = plan_at(groups, d2, wt2, kind2);
        if (rc) return rc;
    }
    dev.swap(d2);
    wt = wt2;
    kind = kind2;
    SeqPlan *plan = nullptr;
    rc = seq_create(dev.data(), n_items, wt, groups, kind, &plan);
    if (rc) return rc;
    *out = reinterpret_cast<mt_seq *>(plan);
    return MT_OK;
}

int mt_seq_create(const mt_linear_op *ops, uint32_t n_ops, mt_seq **out) {
    if (!out) return set_error(MT_EINVAL, "mt_seq_create: null out");
    *out = nullptr;
    if (n_ops && !ops) return set_error(MT_EINVAL, "mt_seq_create: null ops");
    std::vector<mt_seq_item> items(n_ops);
    for (uint32_t i = 0; i < n_ops; i++) {
        items[i] = mt_seq_item{};
        items[i].kind = MT_SEQ_LINEAR;
        items[i].linear = ops[i];
    }
    return mt_seq_create_items(items.data(), n_ops, out);
}

int mt_seq_run(mt_seq *seq, mt_stream_t stream) {
    if (!seq) return set_error(MT_EINVAL, "mt_seq_run: null plan");
    return seq_run(reinterpret_cast<SeqPlan *>(seq), reinterpret_cast<hipStream_t>(stream));
}

int mt_seq_check(mt_seq *seq) {
    if (!seq) return set_error(MT_EINVAL, "mt_seq_check: null plan");
    return seq_check(reinterpret_cast<SeqPlan *>(seq));
}

int mt_seq_destroy(mt_seq *seq) {
    seq_destroy(reinterpret_cast<SeqPlan *>(seq));
    return MT_OK;
}

int mt_seq_groups(const mt_seq *seq) {
    if (!seq) return set_error(MT_EINVAL, "mt_seq_groups: null plan");
    return seq_groups(reinterpret_cast<const SeqPlan *>(seq));
}

int mt_seq_kernel(const mt_seq *seq) {
    if (!seq) return set_error(MT_EINVAL, "mt_seq_kernel: null plan");
    return seq_kernel_kind(reinterpret_cast<const SeqPlan *>(seq));
}

int mt_rope_cache(float *qkv, uint32_t ldq, uint32_t M, uint32_t hq, uint32_t hkv, uint32_t pos0, void *k_cache,
                  void *v_cache, mt_dtype cache_t, uint32_t cache_len, const float *inv_freq, mt_stream_t stream) {
    int rc = validate_heads("mt_rope_cache", hq, hkv, cache_t, cache_len);
    if (rc) return rc;
    if (M == 0) return MT_OK;
    if (!qkv || !k_cache || !v_cache || !inv_freq) return set_error(MT_EINVAL, "mt_rope_cache: null pointer");
    if (ldq < (hq + 2 * hkv) * 64) return set_error(MT_EINVAL, "mt_rope_cache: ldq %u < (hq + 2 hkv) * 64", ldq);
    if (static_cast<uint64_t>(pos0) + M > cache_len)
        return set_error(MT_EINVAL, "mt_rope_cache: positions %u..%u past cache_len %u", pos0, pos0 + M - 1, cache_len);
    return launch_rope_cache(qkv, ldq, M, hq, hkv, pos0, nullptr, k_cache, v_cache, cache_t, cache_len, 0, inv_freq,
                             reinterpret_cast<hipStream_t>(stream));
}

int mt_rope_cache_decode(float *qkv, uint32_t ldq, uint32_t B, uint32_t hq, uint32_t hkv, const uint32_t *pos,
                         void *k_cache, void *v_cache, mt_dtype cache_t, uint32_t cache_len, uint64_t cache_stride,
                         const float *inv_freq, mt_stream_t stream) {
    int rc = validate_heads("mt_rope_cache_decode", hq, hkv, cache_t, cache_len);
    if (rc) return rc;
    if (B == 0) return MT_OK;
    if (!qkv || !pos || !k_cache || !v_cache || !inv_freq) return set_error(MT_EINVAL, "mt_rope_cache_decode: null pointer");
    if (ldq < (hq + 2 * hkv) * 64) return set_error(MT_EINVAL, "mt_rope_cache_decode: ldq %u < (hq + 2 hkv) * 64", ldq);
    if (B > 1 && cache_stride < static_cast<uint64_t>(hkv) * cache_len * 64)
        return set_error(MT_EINVAL, "mt_rope_cache_decode: cache_stride smaller than one cache");
    return launch_rope_cache(qkv, ldq, B, hq, hkv, 0, pos, k_cache, v_cache, cache_t, cache_len, cache_stride,
                             inv_freq, reinterpret_cast<hipStream_t>(stream));
}

int mt_attention(const float *q, uint32_t ldq, uint32_t M, uint32_t hq, uint32_t hkv, uint32_t pos0, uint32_t window,
                 const void *k_cache, const void *v_cache, mt_dtype cache_t, uint32_t cache_len, float *out,
                 uint32_t ldo, float scale, mt_stream_t stream) {
    int rc = validate_heads("mt_attention", hq, hkv, cache_t, cache_len);
    if (rc) return rc;
    if (M == 0) return MT_OK;
    if (!q || !k_cache || !v_cache || !out) return set_error(MT_EINVAL, "mt_attention: null pointer");
    if (ldq < hq * 64 || ldo < hq * 64) return set_error(MT_EINVAL, "mt_attention: ldq / ldo < hq * 64");
    if (!aligned(q, 16) || ldq % 4 || !aligned(out, 16) || ldo % 4)
        return set_error(MT_EINVAL, "mt_attention: q / out must be 16-byte aligned with 16-byte row strides");
    if (static_cast<uint64_t>(pos0) + M > cache_len)
        return set_error(MT_EINVAL, "mt_attention: positions %u..%u past cache_len %u", pos0, pos0 + M - 1, cache_len);
    return launch_attention(q, ldq, M, hq, hkv, pos0, nullptr, window, k_cache, v_cache, cache_t, cache_len, 0, out,
                            ldo, scale, reinterpret_cast<hipStream_t>(stream));
}

int mt_rope_attention(float *qkv, uint32_t ldq, uint32_t M, uint32_t hq, uint32_t hkv, uint32_t pos0, uint32_t window,
                      void *k_cache, void *v_cache, mt_dtype cache_t, uint32_t cache_len, const float *inv_freq,
                      float *out, uint32_t ldo, float scale, mt_stream_t stream) {
    const char *who = "mt_rope_attention";
    int rc = validate_heads(who, hq, hkv, cache_t, cache_len);
    if (rc) return rc;
    if (M == 0) return MT_OK;
    if (M > 64) return set_error(MT_EINVAL, "%s: at most 64 rows, got %u", who, M);
    if (!qkv || !k_cache || !v_cache || !inv_freq || !out) return set_error(MT_EINVAL, "%s: null pointer", who);
    if (ldq < (hq + 2 * hkv) * 64 || ldo < hq * 64)
        return set_error(MT_EINVAL, "%s: ldq %u < (hq + 2 hkv) * 64 or ldo %u < hq * 64", who, ldq, ldo);
    if (!aligned(out, 16) || ldo % 4) return set_error(MT_EINVAL, "%s: out must be 16-byte aligned with a 16-byte row stride", who);
    if (static_cast<uint64_t>(pos0) + M > cache_len)
        return set_error(MT_EINVAL, "%s: positions %u..%u past cache_len %u", who, pos0, pos0 + M - 1, cache_len);
    // out must not overlap qkv (the kernel rewrites q in place and reads k and v).
    const char *qb = reinterpret_cast<const char *>(qkv), *qe = qb + (static_cast<size_t>(M - 1) * ldq + (hq + 2 * hkv) * 64) * 4;
    const char *ob = reinterpret_cast<const char *>(out), *oe = ob + (static_cast<size_t>(M - 1) * ldo + hq * 64) * 4;
    if (qb < oe && ob < qe) return set_error(MT_EINVAL, "%s: out overlaps qkv", who);
    return launch_rope_attention(qkv, ldq, M, hq, hkv, pos0, window, k_cache, v_cache, cache_t, cache_len, inv_freq, out,
                                 ldo, scale, reinterpret_cast<hipStream_t>(stream));
}

int mt_attention_decode(const float *q, uint32_t ldq, uint32_t B, uint32_t hq, uint32_t hkv, const uint32_t *lens,
                        uint32_t window, const void *k_cache, const void *v_cache, mt_dtype cache_t,
                        uint32_t cache_len, uint64_t cache_stride, float *out, uint32_t ldo, float scale,
                        mt_stream_t stream) {
    int rc = validate_heads("mt_attention_decode", hq, hkv, cache_t, cache_len);
    if (rc) return rc;
    if (B == 0) return MT_OK;
    if (!q || !lens || !k_cache || !v_cache || !out) return set_error(MT_EINVAL, "mt_attention_decode: null pointer");
    if (ldq < hq * 64 || ldo < hq * 64) return set_error(MT_EINVAL, "mt_attention_decode: ldq / ldo < hq * 64");
    if (!aligned(q, 16) || ldq % 4 || !aligned(out, 16) || ldo % 4)
        return set_error(MT_EINVAL, "mt_attention_decode: q / out must be 16-byte aligned with 16-byte row strides");
    if (B > 1 && cache_stride < static_cast<uint64_t>(hkv) * cache_len * 64)
        return set_error(MT_EINVAL, "mt_attention_decode: cache_stride smaller than one cache");
    return launch_attention(q, ldq, B, hq, hkv, 0, lens, window, k_cache, v_cache, cache_t, cache_len, cache_stride,
                            out, ldo, scale, reinterpret_cast<hipStream_t>(stream));
}

int mt_dit_attention(const float *qkv, uint32_t ld, uint32_t B, uint32_t S, uint32_t H, const float *inv_freq,
                     float *out, uint32_t ldo, float scale, mt_stream_t stream) {
    if (B == 0 || S == 0 || H == 0) return MT_OK;
    if (S > 8) return set_error(MT_EINVAL, "mt_dit_attention: at most 8 rows per sequence, got %u", S);
    if (!qkv || !inv_freq || !out) return set_error(MT_EINVAL, "mt_dit_attention: null pointer");
    if (static_cast<uint64_t>(ld) < 3ull * H * 64 || static_cast<uint64_t>(ldo) < static_cast<uint64_t>(H) * 64)
        return set_error(MT_EINVAL, "mt_dit_attention: ld < 3 H 64 or ldo < H 64");
    if (!aligned(qkv, 8) || ld % 2 || !aligned(out, 8) || ldo % 2)
        return set_error(MT_EINVAL, "mt_dit_attention: qkv / out must be 8-byte aligned with even strides");
    if (static_cast<uint64_t>(B) * S * H > 0x7FFFFFFFull) return set_error(MT_EINVAL, "mt_dit_attention: too many items");
    return launch_dit_attention(qkv, ld, B, S, H, inv_freq, out, ldo, scale, reinterpret_cast<hipStream_t>(stream));
}

int mt_dit_attention_linear(const float *qkv, uint32_t B, uint32_t S, uint32_t H, const float *inv_freq, float scale,
                            const void *w, mt_dtype wt, const void *bias, float *y, mt_gemv_params p,
                            mt_stream_t stream) {
    const char *who = "mt_dit_attention_linear";
    if (S > 8) return set_error(MT_EINVAL, "%s: at most 8 rows per sequence, got %u", who, S);
    if (static_cast<uint64_t>(B) * S != p.M) return set_error(MT_EINVAL, "%s: M %u is not B %u x S %u", who, p.M, B, S);
    if (static_cast<uint64_t>(H) * 64 != p.K) return set_error(MT_EINVAL, "%s: K %u is not 64 H (H %u)", who, p.K, H);
    if (p.flags & MT_SILU_GATE) return set_error(MT_EINVAL, "%s: MT_SILU_GATE needs a gate partner", who);
    LinearArgs a;
    int rc = validate_linear(who, qkv, MT_F32, w, nullptr, wt, bias, nullptr, y, p, a);
    if (rc) return rc;
    if (p.M == 0 || p.N == 0) return MT_OK;
    if (!inv_freq) return set_error(MT_EINVAL, "%s: null inv_freq", who);
    if (static_cast<uint64_t>(p.ldx) < 3ull * p.K) return set_error(MT_EINVAL, "%s: qkv row stride %u < 3 K", who, p.ldx);
    // y must not overlap the whole q | k | v span that the prologue reads.
    const char *qb = reinterpret_cast<const char *>(qkv);
    const char *qe = qb + (static_cast<size_t>(p.M - 1) * p.ldx + 3ull * p.K) * 4;
    const char *yb = reinterpret_cast<const char *>(y);
    const char *ye = yb + (static_cast<size_t>(p.M - 1) * p.ldy + p.N) * 4;
    if (qb < ye && yb < qe) return set_error(MT_EINVAL, "%s: qkv overlaps y", who);
    if (gemv_mfma_columns(p.M, MT_F32, wt, false) == 0)
        return set_error(MT_ENOTSUP, "%s: at most 32 rows, got %u", who, p.M);
    return launch_gemv_mfma_attn(a, wt, inv_freq, S, H, scale, reinterpret_cast<hipStream_t>(stream));
}

int mt_flow_assemble(const float *y, const float *history, const float *cemb, const void *cond_bias,
                     const float *temb, const void *x_w, const void *x_b, mt_dtype wt, float *x, uint32_t ldx,
                     uint32_t hidden, uint32_t latent_dim, mt_stream_t stream) {
    if (hidden == 0) return MT_OK;
    if (wt != MT_BF16 && wt != MT_F16) return set_error(MT_EINVAL, "mt_flow_assemble: weights must be f16 or bf16");
    if (!y || !history || !cemb || !cond_bias || !temb || !x_w || !x_b || !x)
        return set_error(MT_EINVAL, "mt_flow_assemble: null pointer");
    if (latent_dim == 0 || latent_dim % 8 || !aligned(x_w, 16))
        return set_error(MT_EINVAL, "mt_flow_assemble: latent_dim must be a positive multiple of 8 and x_w 16-byte aligned");
    if (ldx < hidden) return set_error(MT_EINVAL, "mt_flow_assemble: ldx %u < hidden %u", ldx, hidden);
    return launch_flow_assemble(y, history, cemb, cond_bias, temb, x_w, x_b, wt, x, ldx, hidden, latent_dim,
                                reinterpret_cast<hipStream_t>(stream));
}

int mt_flow_euler(float *y, const float *pred, uint32_t ldp, uint32_t pred_row, uint32_t null_row, float *capture,
                  uint32_t latent_dim, float cfg, float dt, mt_stream_t stream) {
    if (latent_dim == 0) return MT_OK;
    if (!y || !pred) return set_error(MT_EINVAL, "mt_flow_euler: null pointer");
    if (ldp < latent_dim) return set_error(MT_EINVAL, "mt_flow_euler: ldp %u < latent_dim %u", ldp, latent_dim);
    return launch_flow_euler(y, pred, ldp, pred_row, null_row, capture, latent_dim, cfg, dt,
                             reinterpret_cast<hipStream_t>(stream));
}

int mt_flow_euler_assemble(float *y, const float *pred, uint32_t ldp, uint32_t pred_row, uint32_t null_row,
                           float *capture, float cfg, float dt, const float *history, const float *cemb,
                           const void *cond_bias, const float *temb, const void *x_w, const void *x_b, mt_dtype wt,
                           float *x, uint32_t ldx, uint32_t hidden, uint32_t latent_dim, mt_stream_t stream) {
    if (hidden == 0 || latent_dim == 0) return set_error(MT_EINVAL, "mt_flow_euler_assemble: empty hidden or latent");
    if (wt != MT_BF16 && wt != MT_F16) return set_error(MT_EINVAL, "mt_flow_euler_assemble: weights must be f16 or bf16");
    if (!y || !pred || !history || !cemb || !cond_bias || !temb || !x_w || !x_b || !x)
        return set_error(MT_EINVAL, "mt_flow_euler_assemble: null pointer");
    if (latent_dim % 8 || latent_dim > 2048 || !aligned(x_w, 16))
        return set_error(MT_EINVAL,
                         "mt_flow_euler_assemble: latent_dim must be a multiple of 8 up to 2048 and x_w 16-byte aligned");
    if (ldp < latent_dim) return set_error(MT_EINVAL, "mt_flow_euler_assemble: ldp %u < latent_dim %u", ldp, latent_dim);
    if (ldx < hidden) return set_error(MT_EINVAL, "mt_flow_euler_assemble: ldx %u < hidden %u", ldx, hidden);
    return launch_flow_euler_assemble(y, pred, ldp, pred_row, null_row, capture, cfg, dt, history, cemb, cond_bias, temb,
                                      x_w, x_b, wt, x, ldx, hidden, latent_dim, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
