// Plan compiler of mt_seq_create: turns a list of linears and decode attention items
// (serial-encoder semantics, as QwenForward.dispatches issues them, Qwen.swift:72-97) into
// the dataflow form the persistent kernel runs.
//
// For every op it resolves
//   - where x comes from: the tagged output of the latest earlier op that wrote x's region
//     (with the column offset of x inside that output), or the user buffer if nothing
//     earlier wrote it;
//   - where the old y of an accumulate comes from, the same way;
//   - whether the op is the last writer of its output region (only that op writes the
//     user buffer);
// and it checks the hazards the dataflow execution could reorder:
//   - a region read at another layout than it was written (not representable) -> ENOTSUP;
//   - a final write to a region an earlier op read from the user buffer, unless every
//     workgroup has provably finished that earlier op (write-after-read) -> ENOTSUP.
// Overlap between two views with the same row stride is decided element-exactly (column
// slices of one buffer do not conflict); views with different strides are compared as
// byte ranges (conservatively).
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "mingtts_hip.h"
#include "mt_internal.hpp"
#include "seq_tiles.hpp"

namespace mt {

namespace {

struct View {
    const char *base;
    uint64_t ld;     // row stride, bytes
    uint64_t width;  // bytes per row
    uint64_t rows;
    uint64_t begin() const { return reinterpret_cast<uint64_t>(base); }
    uint64_t end() const { return begin() + (rows - 1) * ld + width; }
};

// Do the element sets of a and b intersect?
bool overlap(const View &a, const View &b) {
    if (a.end() <= b.begin() || b.end() <= a.begin()) return false;
    if (a.ld != b.ld || a.width > a.ld || b.width > b.ld) return true;  // conservative
    const View &lo = a.begin() <= b.begin() ? a : b;
    const View &hi = a.begin() <= b.begin() ? b : a;
    const uint64_t ld = a.ld, diff = hi.begin() - lo.begin();
    const uint64_t q = diff / ld, col = diff % ld;
    // hi's row r lies at lo's row r + q, columns [col, col + hi.width) (possibly wrapping
    // into row r + q + 1 when col + hi.width > ld).
    for (uint64_t r = 0; r < hi.rows; r++) {
        const uint64_t lr = r + q;
        if (lr < lo.rows && col < lo.width) return true;
        if (col + hi.width > ld && lr + 1 < lo.rows && (col + hi.width - ld) > 0) return true;
        if (lr >= lo.rows) break;
    }
    return false;
}

// If `in` (fp32 elements) sits inside `out` at one column offset with the same row stride
// and no more rows, returns true and the column offset (elements).
bool covered(const View &in, const View &out, uint32_t &col) {
    if (in.ld != out.ld || in.begin() < out.begin()) return false;
    const uint64_t d = in.begin() - out.begin();
    if (d % 4 || d >= out.ld) return false;
    if (d + in.width > out.width || in.rows > out.rows) return false;
    col = static_cast<uint32_t>(d / 4);
    return true;
}

}  // namespace

int seq_plan(const mt_seq_item *items, uint32_t n, int groups, std::vector<SeqOp> &out, int &wt) {
    if (n > static_cast<uint32_t>(SEQ_OPS_MAX))
        return set_error(MT_ENOTSUP, "mt_seq_create: a sequence takes at most %d ops, got %u", SEQ_OPS_MAX, n);
    out.assign(n, SeqOp{});
    std::vector<View> xv(n), yv(n);
    std::vector<View> caches;  // byte ranges of the attention items' k and v caches
    std::vector<int> done_before(n, -1);
    wt = -1;
    for (uint32_t i = 0; i < n; i++) {
        SeqOp &d = out[i];
        if (items[i].kind == MT_SEQ_ATTENTION) {
            const mt_attn_op &a = items[i].attn;
            const uint32_t K = (a.hq + 2 * a.hkv) * 64, N = a.hq * 64;
            xv[i] = View{reinterpret_cast<const char *>(a.qkv), static_cast<uint64_t>(a.ldq) * 4, uint64_t(K) * 4, a.B};
            yv[i] = View{reinterpret_cast<const char *>(a.out), static_cast<uint64_t>(a.ldo) * 4, uint64_t(N) * 4, a.B};
            const uint64_t es = a.cache_t == MT_F32 ? 4 : 2;
            const uint64_t span = ((a.B - 1) * a.cache_stride + static_cast<uint64_t>(a.hkv) * a.cache_len * 64) * es;
            for (const void *c : {static_cast<const void *>(a.k_cache), static_cast<const void *>(a.v_cache)}) {
                const View cv{static_cast<const char *>(c), span, span, 1};
                for (const View &o : caches)
                    if (overlap(cv, o))
                        return set_error(MT_ENOTSUP, "mt_seq_create: op %u: attention caches overlap", i);
                caches.push_back(cv);
            }
            d.kind = SEQ_ATTN;
            d.x = a.qkv;
            d.xt = MT_F32;
            d.ldx = a.ldq;
            d.w = static_cast<const uint16_t *>(a.k_cache);
            d.w2 = static_cast<const uint16_t *>(a.v_cache);
            d.y = a.out;
            d.ldy = a.ldo;
            d.M = a.B;
            d.N = N;
            d.K = K;
            d.eps = a.scale;
            d.heads = a.hq | (a.hkv << 16);
            d.cache_len = a.cache_len;
            d.window = a.window;
            d.pos = a.pos;
            d.inv_freq = a.inv_freq;
            d.cache_stride = a.cache_stride;
            d.cache_t = a.cache_t;
        } else if (items[i].kind == MT_SEQ_DIT_ATTENTION) {
            const mt_dit_attn_op &a = items[i].dit;
            const uint32_t rows = a.B * a.S, N = a.H * 64;
            xv[i] = View{reinterpret_cast<const char *>(a.qkv), static_cast<uint64_t>(a.ldq) * 4, uint64_t(3 * N) * 4, rows};
            yv[i] = View{reinterpret_cast<const char *>(a.out), static_cast<uint64_t>(a.ldo) * 4, uint64_t(N) * 4, rows};
            d.kind = SEQ_DIT;
            d.x = a.qkv;
            d.xt = MT_F32;
            d.ldx = a.ldq;
            d.y = a.out;
            d.ldy = a.ldo;
            d.M = rows;
            d.N = N;
            d.K = 3 * N;
            d.eps = a.scale;
            d.heads = a.H | (a.S << 16);
            d.inv_freq = a.inv_freq;
        } else {
            const mt_linear_op &o = items[i].linear;
            const mt_gemv_params &p = o.p;
            const size_t xs = o.xt == MT_F32 ? 4 : 2;
            xv[i] = View{static_cast<const char *>(o.x), static_cast<uint64_t>(p.ldx) * xs, static_cast<uint64_t>(p.K) * xs, p.M};
            yv[i] = View{reinterpret_cast<const char *>(o.y), static_cast<uint64_t>(p.ldy) * 4, static_cast<uint64_t>(p.N) * 4, p.M};
            if (wt < 0) wt = o.wt;
            if (o.wt != wt) return set_error(MT_EINVAL, "mt_seq_create: op %u: every op of a sequence must share the weight type", i);
            d.kind = SEQ_LINEAR;
            d.x = o.x;
            d.xt = o.xt;
            d.ldx = p.ldx;
            d.w = static_cast<const uint16_t *>(o.w);
            d.w2 = static_cast<const uint16_t *>((p.flags & MT_SILU_GATE) ? o.w2 : o.w);
            d.bias = static_cast<const uint16_t *>(o.bias);
            d.norm = static_cast<const uint16_t *>(o.norm);
            d.y = o.y;
            d.ldy = p.ldy;
            d.M = p.M;
            d.N = p.N;
            d.K = p.K;
            d.flags = p.flags | (o.bias ? MT_BIAS : 0);
            d.eps = p.eps;
        }

        // x: latest earlier writer.
        d.xsrc = -1;
        for (int j = static_cast<int>(i) - 1; j >= 0; j--) {
            if (!overlap(xv[i], yv[j])) continue;
            uint32_t col = 0;
            if (d.xt != MT_F32 || !covered(xv[i], yv[j], col))
                return set_error(MT_ENOTSUP, "mt_seq_create: op %u reads x from op %d's output at another layout", i, j);
            d.xsrc = j;
            d.xcol = col;
            break;
        }
        // old y of an accumulate: latest earlier writer.
        d.ysrc = -1;
        if (d.flags & MT_ACCUM) {
            for (int j = static_cast<int>(i) - 1; j >= 0; j--) {
                if (!overlap(yv[i], yv[j])) continue;
                uint32_t col = 0;
                if (!covered(yv[i], yv[j], col))
                    return set_error(MT_ENOTSUP, "mt_seq_create: op %u accumulates into op %d's output at another layout", i, j);
                d.ysrc = j;
                d.ycol = col;
                break;
            }
        }
        // every workgroup has finished op done_before[i] before op i computes
        int db = -1;
        if (d.xsrc >= 0) {
            db = std::max(db, done_before[d.xsrc]);
            const SeqOp &src = out[d.xsrc];
            // A linear reads all of x.  When x spans all of a linear producer's features and
            // each workgroup owns at least one, every workgroup has finished the producer.
            // When x spans all heads of an attention item whose own x spans all of a linear
            // producer's features (q, k and v heads), those heads consumed every feature of
            // that producer: every workgroup has finished it.  (The attention item itself
            // runs on a few workgroups; its own x reads prove nothing.)  A DiT attention item
            // is computed by every workgroup from all of its qkv, the same argument.
            if (d.kind == SEQ_LINEAR && d.xcol == 0 && d.K == src.N) {
                if (src.kind == SEQ_LINEAR && src.N >= static_cast<uint32_t>(groups)) db = std::max(db, d.xsrc);
                if ((src.kind == SEQ_ATTN || src.kind == SEQ_DIT) && src.xsrc >= 0) {
                    const SeqOp &pp = out[src.xsrc];
                    if (pp.kind == SEQ_LINEAR && src.xcol == 0 && src.K == pp.N && pp.N >= static_cast<uint32_t>(groups))
                        db = std::max(db, src.xsrc);
                }
            }
        }
        if (d.ysrc >= 0) db = std::max(db, done_before[d.ysrc]);
        done_before[i] = db;
    }
    if (wt < 0) wt = MT_F16;
    // The caches are touched by their attention items alone.
    for (const View &c : caches)
        for (uint32_t i = 0; i < n; i++)
            if (overlap(c, xv[i]) || overlap(c, yv[i]))
                return set_error(MT_ENOTSUP, "mt_seq_create: op %u's x or y overlaps an attention cache", i);
    // final writers and write-after-read
    for (uint32_t i = 0; i < n; i++) {
        out[i].final_out = 1;
        for (uint32_t k = i + 1; k < n; k++) {
            if (!overlap(yv[k], yv[i])) continue;
            uint32_t col = 0;
            if (!covered(yv[i], yv[k], col))
                return set_error(MT_ENOTSUP, "mt_seq_create: op %u partly overwrites op %u's output", k, i);
            out[i].final_out = 0;
            break;
        }
        if (!out[i].final_out) continue;
        for (uint32_t e = 0; e < i; e++) {
            const bool reads_x = out[e].xsrc < 0 && overlap(xv[e], yv[i]);
            const bool reads_y = (out[e].flags & MT_ACCUM) && out[e].ysrc < 0 && e != i && overlap(yv[e], yv[i]);
            if ((reads_x || reads_y) && static_cast<int>(e) > done_before[i])
                return set_error(MT_ENOTSUP,
                                 "mt_seq_create: op %u writes a region op %u read from the user buffer, and not every "
                                 "workgroup is known to be past op %u",
                                 i, e, e);
        }
    }
    return MT_OK;
}

int seq_general_limits(const mt_seq_item *items, uint32_t n, int groups) {
    for (uint32_t i = 0; i < n; i++) {
        if (items[i].kind == MT_SEQ_DIT_ATTENTION)
            return set_error(MT_ENOTSUP,
                             "mt_seq_create: op %u: a DiT attention item runs only in the DiT-block kernel (blocks "
                             "of qkv 3072 x 1024, attention H 16 at B 2 S 3 or B 1 S 2, out, ff1 4096 x 1024 GELU, ff2 on "
                             "%d workgroups)",
                             i, DIT_G);
        if (items[i].kind != MT_SEQ_LINEAR) continue;
        const mt_linear_op &o = items[i].linear;
        const mt_gemv_params &p = o.p;
        if (o.norm && p.K > static_cast<uint32_t>(SEQ_GMAX))
            return set_error(MT_ENOTSUP, "mt_seq_create: op %u: an RMSNorm op takes K <= %d, got %u", i, SEQ_GMAX, p.K);
        // The op's activations are staged whole in the workgroup's LDS (M * K <= XLDS);
        // every workgroup's share of the op at most RMAX features and its partial sums
        // (virtual rows x M per compute wave) within the LDS slice.
        if (static_cast<uint64_t>(p.M) * p.K > static_cast<uint64_t>(SEQ_XLDS))
            return set_error(MT_ENOTSUP, "mt_seq_create: op %u: M * K = %u exceeds the %d activations a workgroup stages",
                             i, p.M * p.K, SEQ_XLDS);
        for (int g = 0; g < groups; g++) {
            const SeqTiles t = seq_tiles(p.N, p.K, p.M, (p.flags & MT_SILU_GATE) != 0, g, groups);
            const uint32_t per_wave = (t.T + SEQ_CW - 1) / SEQ_CW;
            // A wave's contiguous tile range may span at most two row tiles.
            uint32_t span = 1;
            for (int w = 0; w < SEQ_CW; w++) {
                const uint32_t t0 = seq_tile_begin(t.T, w, SEQ_CW), t1 = seq_tile_begin(t.T, w + 1, SEQ_CW);
                if (t1 > t0 && t.KBs) span = std::max(span, (t1 - 1) / t.KBs - t0 / t.KBs + 1);
            }
            if (span > 2)
                return set_error(MT_ENOTSUP,
                                 "mt_seq_create: op %u: a wave's share of the tiles spans %u row tiles of 16 weight "
                                 "rows (K = %u is too short for the sequence kernel's limit of 2)",
                                 i, span, p.K);
            if (t.nr > static_cast<uint32_t>(SEQ_RMAX) || t.V * p.M > static_cast<uint32_t>(SEQ_PARTW) ||
                per_wave > static_cast<uint32_t>(SEQ_TA))
                return set_error(MT_ENOTSUP,
                                 "mt_seq_create: op %u: a workgroup's share (%u features, %u partial sums at M = %u, %u "
                                 "MFMA tiles per compute wave) exceeds the sequence kernel's limits (%d features, %d "
                                 "partial sums, %d tiles)",
                                 i, t.nr, t.V * p.M, p.M, per_wave, SEQ_RMAX, SEQ_PARTW, SEQ_TA);
        }
    }
    return MT_OK;
}

bool layer_pattern(const SeqOp *ops, uint32_t n, int groups) {
    // An even count: down runs on workgroup pairs.
    if (n < 2 || groups < LAY_GMIN || groups > LAY_GMAX || groups % 2) return false;
    const uint32_t M = ops[0].M;
    if (M != 1 && M != 2 && M != 4) return false;
    // With attention items every layer is qkv, attention, o, gate|up, down; the item's rows are
    // the plan's M and its heads the backbone's 14 q / 2 kv (o's K = 14 x 64).
    const bool att = ops[1].kind == SEQ_ATTN;
    const uint32_t per = att ? 5 : 4;
    if (n % per) return false;
    struct Want {
        uint32_t N, K, flags;
        bool norm;
    };
    const Want want[4] = {{LAY_QKV, LAY_H, F_BIAS, true},
                          {LAY_H, LAY_H, F_ACCUM, false},
                          {LAY_I, LAY_H, F_SILU_GATE, true},
                          {LAY_H, LAY_I, F_ACCUM, false}};
    for (uint32_t i = 0; i < n; i++) {
        const SeqOp &o = ops[i];
        uint32_t j = i % per;
        if (att && j == 1) {
            if (o.kind != SEQ_ATTN || o.M != M || o.heads != (14u | (2u << 16)) || o.N != LAY_H) return false;
            continue;
        }
        if (att && j > 1) j--;
        const Want &c = want[j];
        if (o.kind != SEQ_LINEAR || o.M != M || o.N != c.N || o.K != c.K || o.flags != c.flags ||
            (o.norm != nullptr) != c.norm || ((o.flags & F_BIAS) != 0) != (o.bias != nullptr))
            return false;
    }
    // Dataflow: this kernel splits each down over K, so its output is two tagged planes, and
    // only a qkv reading it as x or an o reading it as the old y adds the second plane.  Any
    // other in-plan reader of a down output would read the first half's sums alone.
    auto is_down = [&](int32_t src) { return src >= 0 && static_cast<uint32_t>(src) % per == per - 1; };
    for (uint32_t i = 0; i < n; i++) {
        const uint32_t j = i % per;
        const bool qkv = j == 0, o_proj = j == (att ? 2u : 1u);
        if (is_down(ops[i].xsrc) && !(qkv && ops[i].kind == SEQ_LINEAR)) return false;
        if (is_down(ops[i].ysrc) && !o_proj) return false;
    }
    return true;
}

bool dit_pattern(const SeqOp *ops, uint32_t n, int groups) {
    if (n == 0 || n % 5 || groups != DIT_G) return false;
    struct Want {
        uint32_t N, K, flags;
        bool norm;
    };
    const Want want[5] = {{DIT_QKV, DIT_H, F_BIAS, true},
                          {0, 0, 0, false},
                          {DIT_H, DIT_H, F_BIAS | F_ACCUM, false},
                          {DIT_FF, DIT_H, F_BIAS | F_GELU, true},
                          {DIT_H, DIT_FF, F_BIAS | F_ACCUM, false}};
    // (B, S) = (2, 3) in the flow loop, (1, 2) in the aggregator: the row count fixes both.
    const uint32_t M = ops[0].M, S = M == 6 ? 3u : 2u;
    if (M != 6 && M != 2) return false;
    for (uint32_t i = 0; i < n; i++) {
        const SeqOp &o = ops[i];
        const uint32_t j = i % 5;
        if (o.M != M) return false;
        if (j == 1) {
            // The attention reads all of this block's qkv output; every item shares the first
            // one's frequencies and scale (the kernel builds its rotation table once).
            if (o.kind != SEQ_DIT || o.heads != (DIT_HEADS | (S << 16)) || o.xsrc != static_cast<int32_t>(i - 1) ||
                o.xcol != 0 || o.inv_freq != ops[1].inv_freq || o.eps != ops[1].eps)
                return false;
            continue;
        }
        const Want &c = want[j];
        if (o.kind != SEQ_LINEAR || o.N != c.N || o.K != c.K || o.flags != c.flags || (o.norm != nullptr) != c.norm ||
            o.bias == nullptr)
            return false;
        // The out projection reads exactly the attention's output (it computes it itself).
        if (j == 2 && (o.xsrc != static_cast<int32_t>(i - 1) || o.xcol != 0)) return false;
    }
    // Nothing but that out projection may read a DiT attention item: the kernel never writes
    // the items' outputs to the tagged buffer, so another reader would wait for them forever.
    // ff2 is split over K into two tagged planes, which only a qkv reading them as x or an out
    // projection reading them as the old y adds.
    for (uint32_t i = 0; i < n; i++) {
        const int32_t xs = ops[i].xsrc, ys = ops[i].ysrc;
        if (xs >= 0 && static_cast<uint32_t>(xs) % 5 == 1 && !(i % 5 == 2 && static_cast<uint32_t>(xs) == i - 1))
            return false;
        if (ys >= 0 && static_cast<uint32_t>(ys) % 5 == 1) return false;
        if (xs >= 0 && static_cast<uint32_t>(xs) % 5 == 4 && i % 5 != 0) return false;
        if (ys >= 0 && static_cast<uint32_t>(ys) % 5 == 4 && i % 5 != 2) return false;
    }
    return true;
}

}  // namespace mt
