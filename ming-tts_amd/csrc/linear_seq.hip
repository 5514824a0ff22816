// Host side of the persistent linear sequence (mt_seq_*) and its linear-only kernels; the
// kernel itself is in seq_kernel.hpp.
#include "layer_kernel.hpp"

namespace mt {

struct SeqPlan {
    SeqOp *d_ops = nullptr;
    uint32_t *d_sync = nullptr;
    uint32_t *d_tags = nullptr;
    uint32_t tag_bytes = 0;
    uint32_t n_ops = 0;
    int groups = 0;
    int device = 0;
    seq_fn fn = nullptr;
    bool layer = false;  // runs the decode-layer or DiT-block kernel (packed descriptors follow the ops)
    int kind = MT_SEQ_GENERAL;
    int threads = SEQ_THREADS;
};

int seq_limits(int *groups_out, int *preferred_out) {
    int dev = 0, cus = 0, per_cu = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(seq_attn_kernel(DT_F16, false)),
                                                         SEQ_THREADS, 0);
    if (e != hipSuccess || cus <= 0 || per_cu <= 0)
        return set_error(MT_EHIP, "mt_seq_create: occupancy query failed (%s, cus %d, per_cu %d)", hipGetErrorString(e),
                         cus, per_cu);
    const int want = tuning().seq_groups;
    const int resident = cus * per_cu;
    // Default: one 512-thread workgroup per CU at most, and preferably on 7 of every 8 CUs
    // (a multiple of 8, one share per XCD): fewer workgroups meet in every exchange, and
    // the decode step measured fastest there (557 us at 224 workgroups on 256 CUs against
    // 563-570 us at 216-256).  A plan whose shares do not fit that count takes all CUs.
    *groups_out = want > 0 ? (want < resident ? want : resident) : cus;
    *preferred_out = want > 0 ? *groups_out : ((cus * 7 / 8) & ~7) > 0 ? (cus * 7 / 8) & ~7 : cus;
    return MT_OK;
}

int seq_create(SeqOp *ops, uint32_t n_ops, int wt, int groups, int kind, SeqPlan **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(MT_EHIP, "mt_seq_create: hipGetDevice: %s", hipGetErrorString(e));
    // The decode-layer kernel splits each layer's down over K between workgroup pairs, and the
    // DiT-block kernel each block's ff2: the output is two planes (the layer's or block's last
    // op: every 4th op, every 5th with attention items).
    bool any_attn = false;
    for (uint32_t i = 0; i < n_ops; i++) any_attn = any_attn || ops[i].kind == SEQ_ATTN || ops[i].kind == SEQ_DIT;
    const uint32_t per = any_attn ? 5 : 4;
    const bool split = kind == MT_SEQ_DECODE_LAYER || kind == MT_SEQ_DIT_BLOCK;
    for (uint32_t i = 0; i < n_ops; i++) ops[i].planes = split && i % per == per - 1 ? 2 : 1;
    // Each op's tagged output starts 16-byte aligned (planes M N words apart; M N is a
    // multiple of 4 for every split op).
    size_t tag_words = 0;
    for (uint32_t i = 0; i < n_ops; i++)
        tag_words += (static_cast<size_t>(ops[i].M) * ops[i].N * ops[i].planes + 3) & ~size_t(3);
    if (tag_words * 4 > 0x7FFFFFF0u) return set_error(MT_ENOTSUP, "mt_seq_create: the ops' outputs exceed 2 GiB");
    SeqPlan *p = new SeqPlan();
    p->n_ops = n_ops;
    p->device = dev;
    // One common M of 1 or 2 (the decode step's single row or CFG pair) selects a kernel
    // specialised for it.
    uint32_t m_all = n_ops ? ops[0].M : 0;
    for (uint32_t i = 1; i < n_ops; i++)
        if (ops[i].M != m_all) m_all = 0;
    bool attn = false;
    for (uint32_t i = 0; i < n_ops; i++) attn = attn || ops[i].kind == SEQ_ATTN;
    p->kind = kind;
    if (kind == MT_SEQ_DIT_BLOCK) {
        p->fn = dit_block_kernel_fn(wt, m_all);
        p->layer = true;
        p->threads = LAY_THREADS;
    } else if (kind == MT_SEQ_DECODE_LAYER) {
        p->fn = layer_kernel_fn(wt, m_all, attn);
        p->layer = true;
        p->threads = LAY_THREADS;
    } else if (attn) {
        p->fn = seq_attn_kernel(wt, m_all == 2);
    } else if (wt == DT_BF16) {
        p->fn = m_all == 1   ? seq_kernel<DT_BF16, 1, false>
                : m_all == 2 ? seq_kernel<DT_BF16, 2, false>
                             : seq_kernel<DT_BF16, 0, false>;
    } else {
        p->fn = m_all == 1 ? seq_kernel<DT_F16, 1, false> : m_all == 2 ? seq_kernel<DT_F16, 2, false> : seq_kernel<DT_F16, 0, false>;
    }
    p->groups = groups;
    p->tag_bytes = static_cast<uint32_t>((tag_words ? tag_words : 1) * 4);
    const size_t desc_bytes = (sizeof(SeqOp) + (p->layer ? sizeof(LayOp) : 0)) * (n_ops ? n_ops : 1);
    e = hipMalloc(&p->d_ops, desc_bytes);
    if (e == hipSuccess) e = hipMalloc(&p->d_sync, SYNC_WORDS * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&p->d_tags, p->tag_bytes);
    if (e == hipSuccess) {
        size_t off = 0;
        for (uint32_t i = 0; i < n_ops; i++) {
            ops[i].tag = p->d_tags + off;
            off += (static_cast<size_t>(ops[i].M) * ops[i].N * ops[i].planes + 3) & ~size_t(3);
        }
        // Tagged sources as offsets into the tag buffer (no dependent lookups on the device).
        for (uint32_t i = 0; i < n_ops; i++) {
            if (ops[i].xsrc >= 0) {
                const SeqOp &src = ops[ops[i].xsrc];
                ops[i].xoff = static_cast<uint32_t>(src.tag - p->d_tags) + ops[i].xcol;
                ops[i].xld = src.N;
            }
            if (ops[i].ysrc >= 0) {
                const SeqOp &src = ops[ops[i].ysrc];
                ops[i].yoff = static_cast<uint32_t>(src.tag - p->d_tags) + ops[i].ycol;
                ops[i].yld = src.N;
            }
        }
        e = hipMemcpy(p->d_ops, ops, sizeof(SeqOp) * n_ops, hipMemcpyHostToDevice);
        if (e == hipSuccess && p->layer) {
            // The decode-layer kernel's packed descriptors, right after the op descriptors.
            std::vector<LayOp> lay(n_ops);
            for (uint32_t i = 0; i < n_ops; i++) {
                const SeqOp &o = ops[i];
                LayOp &d = lay[i];
                d.w = o.w;
                d.p2 = (o.flags & F_SILU_GATE) ? o.w2 : o.bias;
                d.norm = o.norm;
                d.y = o.y;
                d.xoff = o.xoff;
                d.xld = o.xld;
                d.yoff = o.yoff;
                d.yld = o.yld;
                d.ldy = o.ldy;
                d.tag = static_cast<uint32_t>(o.tag - p->d_tags);
                d.eps = o.eps;
                d.flags = (o.xsrc < 0 ? LAY_XEXT : 0u) | (o.ysrc < 0 ? LAY_YEXT : 0u) | (o.final_out ? LAY_FINAL : 0u) |
                          (o.xsrc >= 0 && ops[o.xsrc].planes == 2 ? LAY_X2 : 0u) |
                          (o.ysrc >= 0 && ops[o.ysrc].planes == 2 ? LAY_Y2 : 0u);
                // A linear whose x is a DiT attention item's output computes that attention
                // itself: its x is the item's qkv.
                if (o.kind == SEQ_LINEAR && o.xsrc >= 0 && ops[o.xsrc].kind == SEQ_DIT) {
                    d.xoff = ops[o.xsrc].xoff;
                    d.xld = ops[o.xsrc].xld;
                }
            }
            e = hipMemcpy(p->d_ops + n_ops, lay.data(), sizeof(LayOp) * n_ops, hipMemcpyHostToDevice);
        }
    }
    // Tagged words start with parity 0 and the first run uses epoch 1 (parity 1), so no
    // stale word can pass for a current one.
    if (e == hipSuccess) e = hipMemset(p->d_tags, 0, p->tag_bytes);
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
    void *args[] = {&p->d_ops, &p->n_ops, &p->d_sync, &p->d_tags, &p->tag_bytes};
    hipError_t e;
    if (tuning().seq_launch == 1) {
        // Ordinary launch (the default): the workgroups are co-resident while nothing else
        // occupies the CUs; the bounded waits turn a shortfall into the timeout flag.  A
        // cooperative launch guarantees co-residency but starts about 17 us later on MI355X
        // (decode step 393.5 -> 376.3 us, flow stage 2.43 -> 2.25 ms, A/B on one box).
        e = hipLaunchKernel(reinterpret_cast<const void *>(p->fn), dim3(p->groups), dim3(p->threads), args, 0, stream);
    } else {
        e = hipLaunchCooperativeKernel(reinterpret_cast<const void *>(p->fn), dim3(p->groups), dim3(p->threads), args,
                                       0, stream);
    }
    if (e != hipSuccess) return set_error(MT_EHIP, "mt_seq_run: launch: %s", hipGetErrorString(e));
    return MT_OK;
}

int seq_check(SeqPlan *p) {
    uint32_t flags[SYNC_WORDS];
    hipError_t e = hipMemcpy(flags, p->d_sync, sizeof(flags), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return set_error(MT_EHIP, "mt_seq_check: %s", hipGetErrorString(e));
    if (flags[SYNC_TIMEOUT]) return set_error(MT_EHIP, "mt_seq_check: a dataflow wait exceeded its spin bound");
    if (flags[SYNC_RANGE])
        return set_error(MT_ERANGE, "mt_seq_check: an activation exceeded the fp16 range of the weights' type "
                                    "(|x| > 65504); the results of that run are not valid");
    return MT_OK;
}

int seq_groups(const SeqPlan *p) { return p->groups; }

int seq_kernel_kind(const SeqPlan *p) { return p->kind; }

void seq_destroy(SeqPlan *p) {
    if (!p) return;
    (void)hipFree(p->d_ops);
    (void)hipFree(p->d_sync);
    (void)hipFree(p->d_tags);
    delete p;
}

}  // namespace mt
