/*
 * mingtts_hip.h -- C ABI of the MI355X (gfx950) linear hot path of MingTTS.
 *
 * Every entry point takes caller-owned device pointers, enqueues work on the
 * given HIP stream and returns; the caller synchronises.  Device memory is
 * allocated on the call path in two places only: mt_seq_create (the plan, once)
 * and the split-K workspace of the linears (one per device and stream, allocated
 * by the first linear on that stream that splits K, and grown, with a stream
 * synchronisation, when a later one needs more).  A grown workspace replaces the
 * old one without freeing it, so a HIP graph captured earlier on the stream keeps
 * valid addresses; growth is refused under capture (MT_EINVAL: run the same linear
 * once before capturing).  A captured graph uses the capture stream's workspace
 * and arrival counters: replay it on that stream, or make sure no split-K linear
 * runs on the capture stream while it replays elsewhere.  mt_linear_static
 * allocates nothing.  Errors are returned, never raised: 0 on success, a
 * negative code otherwise, with a message in mt_last_error() (thread-local).
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   mt_linear            Encoder.linear            Sources/MingTTS/Engine/Kernels.swift:128-161
 *   mt_rmsnorm           Encoder.rmsnorm           Sources/MingTTS/Engine/Kernels.swift:163-171
 *   mt_gemv_params       GemvParams                Sources/MingTTS/Engine/Shaders.swift:39
 *   MT_BIAS .. MT_SILU   GemvFlags                 Sources/MingTTS/Engine/Kernels.swift:21-28
 *   mt_linear_kernel     Kernels.usesGemm + the    Sources/MingTTS/Engine/Kernels.swift:81-86,
 *                        scalarRowsMax rule                                         126, 137-151
 *   mt_set_tuning        Encoder.kSplitOverride /  Sources/MingTTS/Engine/Kernels.swift:98-126
 *                        columnTilesOverride /
 *                        scalarRowsMax
 *   mt_seq_*             QwenForward.dispatches    Sources/MingTTS/Engine/Qwen.swift:72-97
 *                        encoded on one serial       (each dispatch sees the writes of the
 *                        compute encoder             ones before it)
 *   mt_attn_op           Encoder.ropeCache +       Sources/MingTTS/Engine/Kernels.swift:180-206,
 *   (mt_seq_create_items) Encoder.attention of one Sources/MingTTS/Engine/Qwen.swift:86-87
 *                        decode layer, inside the
 *                        sequence
 *   mt_dit_attn_op       Encoder.ditAttention of   Sources/MingTTS/Engine/Kernels.swift:208-220,
 *   (mt_seq_create_items) DiTForward.encode's      Sources/MingTTS/Engine/DiT.swift:35-52
 *                        blocks, inside the
 *                        sequence
 *   mt_rope_cache        Encoder.ropeCache         Sources/MingTTS/Engine/Kernels.swift:180-191
 *   mt_attention         Encoder.attention         Sources/MingTTS/Engine/Kernels.swift:193-206
 *   mt_rope_attention    Encoder.ropeCache +       Sources/MingTTS/Engine/Kernels.swift:180-206,
 *                        Encoder.attention         Sources/MingTTS/Engine/VAEDecoder.swift:81-107
 *   mt_attention_decode  Encoder.attention over B  Sources/MingTTS/Engine/Kernels.swift:193-206
 *                        independent caches at
 *                        M = 1 each
 *   mt_dit_attention     Encoder.ditAttention      Sources/MingTTS/Engine/Kernels.swift:208-220
 *   mt_dit_attention_    Encoder.ditAttention +    Sources/MingTTS/Engine/DiT.swift:44-45
 *     linear             Encoder.linear(out, +=)
 *   mt_flow_assemble     Encoder.flowAssemble      Sources/MingTTS/Engine/Kernels.swift:222-235
 *   mt_flow_euler        Encoder.flowEuler         Sources/MingTTS/Engine/Kernels.swift:237-246
 *   mt_upsample4         Encoder.upsample4         Sources/MingTTS/Engine/Kernels.swift:247-257
 *   mt_istft_frames      Encoder.istftFrames       Sources/MingTTS/Engine/Kernels.swift:259-270
 *   mt_istft_emit        Encoder.istftEmit         Sources/MingTTS/Engine/Kernels.swift:272-283
 *   mt_st_*              SafeTensors               Sources/MingTTS/Engine/SafeTensors.swift:7-87
 *   mt_arena_*           WeightArena               Sources/MingTTS/Engine/Weights.swift:8-79
 *   mt_last_error        MingTTSError text         Sources/MingTTS/Engine/MetalContext.swift:6-26
 */
#ifndef MINGTTS_HIP_H
#define MINGTTS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI-identical to hipStream_t; NULL is the default stream. */
typedef struct ihipStream_t *mt_stream_t;

/* Return codes. */
#define MT_OK 0
#define MT_EHIP (-5)       /* a HIP runtime error; the text is in mt_last_error() */
#define MT_ENOMEM (-12)
#define MT_EINVAL (-22)    /* a shape, alignment, dtype or pointer the kernels cannot take */
#define MT_ERANGE (-34)     /* mt_seq_check: a run met an activation outside the fp16 range */
#define MT_ENOTSUP (-95)

/* GemvParams, Shaders.swift:39.  y[m, n] = sum_k x[m, k] w[n, k] (+ epilogue).
 * ldx / ldy are row strides in elements of x / y.  eps is unused by linears. */
typedef struct mt_gemv_params {
    uint32_t M, N, K, ldx, ldy, flags;
    float eps;
} mt_gemv_params;

/* GemvFlags, Kernels.swift:21-28.  Epilogue order (Shaders.swift:92-103):
 * v = acc + bias[n]; v = silu(v) * acc2 (SILU_GATE, acc2 = x . w2); v = gelu_tanh(v);
 * v = silu(v); v += y_old (ACCUM); store. */
enum {
    MT_BIAS = 1,
    MT_ACCUM = 2,
    MT_GELU = 4,
    MT_SILU_GATE = 8,
    MT_SILU = 16
};

/* Element types.  Weights and bias are 16-bit; activations x may be any of the
 * three; y is always fp32 (an fp16/bf16 output alone would break 1e-3). */
typedef enum mt_dtype { MT_F32 = 0, MT_F16 = 1, MT_BF16 = 2 } mt_dtype;

/* Kernel families, as reported by mt_linear_kernel: the lane-group GEMV (every 16-byte
 * weight chunk feeds all rows of x), the MFMA GEMM (tiles of x rows and weight rows), and
 * the small-row MFMA kernel that stages x once per 16 output features. */
enum { MT_KERNEL_GEMV = 1, MT_KERNEL_GEMM = 2, MT_KERNEL_GEMV_MFMA = 3 };

/*
 * One linear, Encoder.linear (Kernels.swift:128-161).
 *   x     [M, ldx] of type xt; rows past M are never read.
 *   w     [N, K] of type wt, row-major, 16-byte aligned, K % 8 == 0.
 *   w2    [N, K] gate partner ("up") for MT_SILU_GATE, else NULL.
 *   bias  [N] of type wt, or NULL.  A non-NULL bias sets MT_BIAS (Kernels.swift:135);
 *         MT_BIAS with a NULL bias is an error.
 *   y     [M, ldy] fp32; read first when MT_ACCUM (y may be the residual stream).
 *         x must not overlap y.
 * Requirements (else MT_EINVAL): K % 8 == 0; ldx >= K, ldy >= N; x 16-byte aligned
 * and ldx * sizeof(xt) % 16 == 0; w, w2 16-byte aligned; y 4-byte aligned;
 * wt in {MT_F16, MT_BF16}.  M == 0 or N == 0 is a no-op.
 */
int mt_linear(const void *x, mt_dtype xt, const void *w, const void *w2, mt_dtype wt,
              const void *bias, float *y, mt_gemv_params p, mt_stream_t stream);

/*
 * mt_linear without any allocation.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory on the call path (code under HIP graph capture,
 * serving loops or harnesses that forbid hipMalloc).  Same arguments, semantics and
 * kernels as mt_linear, with the split-K partial sums and arrival counters in a fixed
 * device array of the library (16 MiB of partials and 4096 tiles, held on each device
 * the library runs on until the process ends) instead of the stream's workspace.  A
 * linear whose split needs more is refused with MT_ENOTSUP (mt_linear runs it).  Every
 * call on a device shares that device's array: calls that overlap on one device (on
 * different streams) race, and must be ordered by the caller.
 */
int mt_linear_static(const void *x, mt_dtype xt, const void *w, const void *w2, mt_dtype wt,
                     const void *bias, float *y, mt_gemv_params p, mt_stream_t stream);

/*
 * RMSNorm fused into a linear's prologue: the reference's Encoder.rmsnorm into a scratch
 * row followed by Encoder.linear on it (Kernels.swift:163-171 then 132-161, as Qwen.swift:84-85
 * and 89-90 issue them), computed as one pass:
 *   x'[m, k] = x[m, k] * rsqrt(mean_k x[m, k]^2 + p.eps) * norm[k];   y = linear(x')
 * norm is [K] of type wt, 16-byte aligned.  Everything else is as mt_linear.
 */
int mt_linear_rmsnorm(const void *x, mt_dtype xt, const void *norm, const void *w, const void *w2,
                      mt_dtype wt, const void *bias, float *y, mt_gemv_params p, mt_stream_t stream);

/*
 * Encoder.rmsnorm (Kernels.swift:163-171, Shaders.swift:414-440) on its own: y = x *
 * rsqrt(mean(x^2) + eps) * g over `rows` rows of `width` fp32 values (row strides ldx, ldy),
 * g [width] of type wt (MT_BF16 or MT_F16).  For normalised rows that are read as data (the
 * backbone's final norm, Qwen.swift:94); before a linear use mt_linear_rmsnorm.  width and
 * the strides multiples of 4, x and y 16-byte aligned, g 8-byte aligned; y is x (same
 * stride) or apart from it.
 */
int mt_rmsnorm(const float *x, uint32_t ldx, uint32_t rows, uint32_t width, const void *g, mt_dtype wt, float *y,
               uint32_t ldy, float eps, mt_stream_t stream);

/* The kernel family mt_linear runs for a shape under the current tuning, the analogue of
 * Kernels.usesGemm and scalarRowsMax: M <= MT_TUNE_GEMV_ROWS_MAX (8) -> the GEMV, except
 * 3..8 rows on the small-row MFMA kernel (unless MT_TUNE_GEMV_MFMA = 1); larger M -> the
 * small-row MFMA kernel up to 16 rows (up to 64 under MT_TUNE_GEMV_MFMA = 2, while its
 * columns fit), the GEMM above.  mt_linear_rmsnorm routes the same way, except that its
 * fused norm takes the small-row MFMA kernel up to 8 rows only. */
int mt_linear_kernel(uint32_t M, uint32_t N, uint32_t K, mt_dtype xt, mt_dtype wt);

/* Process-wide tuning overrides, the analogue of Encoder.kSplitOverride /
 * columnTilesOverride / scalarRowsMax (Kernels.swift:98-126).  value < 0 restores
 * the default.  Returns the previous value, or MT_EINVAL for an unknown key. */
enum {
    MT_TUNE_GEMV_ROWS_MAX = 1,   /* M up to this goes to the GEMV family (default 8) */
    MT_TUNE_GEMV_LANES = 2,      /* lanes per output feature in the GEMV, 8..64 (0 = auto) */
    MT_TUNE_GEMM_SPLITK = 3,     /* K splits of the pipelined MFMA GEMM (0 = auto) */
    MT_TUNE_SEQ_GROUPS = 4,      /* workgroups of the persistent sequence kernel (0 = auto) */
    MT_TUNE_SEQ_LAUNCH = 5,      /* 0: cooperative launch; 1: ordinary launch (default), about 17 us
                                    sooner per launch on MI355X; its workgroups (one a CU) are
                                    co-resident while no other kernel holds CUs, as on a device
                                    that runs one stream; a shortfall ends in the bounded waits'
                                    timeout flag (mt_seq_check), never a hang */
    MT_TUNE_GEMM_TILE = 6,       /* MFMA GEMM tile (x rows x weight rows) for fp32 activations and
                                    activations of the weights' type: 0 = auto, 1 = 128 x 128,
                                    2 = 64 x 128, 3 = 64 x 64, 4 = the register-staged 64 x 64 kernel
                                    that the other activation types use, for every type, 5 = the
                                    gated ring kernel (128 x rows x 96 features of W and W2; SiLU-gated
                                    linears only: the auto choice when its tiles fill at least
                                    3/4 of their last wave on the CUs, e.g. gate|up at 448-640
                                    rows on 256 CUs) */
    MT_TUNE_GEMM_STAGES = 7,     /* loads of that GEMM for x of the weights' type: 2..4 = direct-to-LDS
                                    stages of 64 k, 1 = two register-staged stages into two LDS
                                    buffers (0 = auto); fp32 x always stages through registers,
                                    its K loop 1 = committing only the split's stages, 2..4 = the
                                    branch-free loop (64-row tiles; 0 = auto) */
    MT_TUNE_GEMV_MFMA = 8,       /* the MFMA kernel that stages x once per 16 output features: 0 =
                                    for 3..16 rows (default; 3..8 with a fused norm), 1 = never
                                    (lane-group GEMV up to 8 rows, GEMM above), 2 = up to 64 rows of
                                    x of the weights' type (32 otherwise) */
    MT_TUNE_SEQ_LAYER = 9        /* 0: a sequence of Qwen2-0.5B decode layers (qkv 1152 x 896, o,
                                    gate|up 2 x 4864 x 896, down at 1, 2 or 4 rows) runs on the
                                    kernel specialised for those shapes (default); 1: on the
                                    general sequence kernel */
};
int mt_set_tuning(int key, int value);

/*
 * A sequence of linears with the result of executing them in order, each seeing the
 * writes of the ones before it -- QwenForward.dispatches on a serial encoder
 * (Qwen.swift:72-97).  mt_seq_create validates every op, compiles the list into a
 * dataflow plan and uploads it once; mt_seq_run runs the whole sequence as ONE
 * persistent cooperative kernel launch in which ops hand activations to each other
 * through plan-owned tagged buffers (no device-wide barriers).  Dot products run on
 * 16x16x32 MFMA with every fp32 activation split into a hi + lo pair of the weights'
 * 16-bit type; with fp16 weights an activation (times its RMSNorm gain) must stay within
 * the fp16 range, |x| <= 65504, or mt_seq_check reports MT_ERANGE for that run.
 * Requirements, beyond mt_linear's for every op: 1 <= M <= 8; one weight type for all
 * ops; at most 128 ops (linears and attention items); M * K <= 10240 per op (its
 * activations are staged in LDS); K <= 2048 for an op with an RMSNorm gain; a
 * workgroup's share of an op (ceil(N / workgroups) features) at most 64 features, with
 * (features, twice with the gate partner) x M <= 128,
 * and at most 12 MFMA tiles of 16 x 32 weights per wave (eight per workgroup), spanning at
 * most two row tiles of 16 weight rows --
 * every linear of a Qwen2-0.5B decode layer fits at one workgroup per CU on 256 CUs; an
 * op that reads (as x, or as the old y of MT_ACCUM) a
 * region an earlier op wrote must view it with that op's row stride and within its
 * columns; a later write must cover an earlier write of the same region whole; an op
 * may overwrite a region an earlier op read from its buffer only if every workgroup
 * provably finished that earlier op (the later op consumes all of a full-width output
 * in between).  Anything else returns MT_ENOTSUP.
 * User buffers are read where nothing earlier in the sequence wrote them and are left
 * holding the last value written to each region; intermediate values of a region that
 * is written again later never reach the user buffer.  The plan keeps the pointers;
 * the memory behind them may change between runs.  Runs of one plan must not overlap
 * in time.
 */
typedef struct mt_linear_op {
    const void *x;
    const void *w;
    const void *w2;
    const void *bias;
    const void *norm;   /* RMSNorm gain as in mt_linear_rmsnorm (eps = p.eps), or NULL */
    float *y;
    mt_gemv_params p;
    int32_t xt;   /* mt_dtype */
    int32_t wt;   /* mt_dtype */
} mt_linear_op;

typedef struct mt_seq mt_seq;
int mt_seq_create(const mt_linear_op *ops, uint32_t n_ops, mt_seq **out);

/*
 * The decode attention of one layer as an item of a sequence: mt_rope_cache_decode then
 * mt_attention_decode (Encoder.ropeCache + Encoder.attention, Kernels.swift:180-206;
 * Qwen.swift:86-87) for B independent rows, one query each.  Row b sits at position
 * pos[b] (a device array of B uint32, read at run time): its k head(s) rotated by NeoX
 * RoPE and its raw v heads are appended to sequence b's caches (k_cache / v_cache + b *
 * cache_stride elements, layout [hkv, cache_len, 64]) at pos[b], and its hq query heads,
 * rotated, attend over keys [max(0, len_b - window), len_b), len_b = min(pos[b] + 1,
 * cache_len) (window 0 = unlimited; a pos[b] >= cache_len appends nothing), with scores
 * scaled by `scale`; out row b (stride ldo) gets the hq heads of 64.  qkv rows are
 * [q (hq*64) | k (hkv*64) | v (hkv*64)] at stride ldq; they are read, not modified (the
 * rotated q stays inside the kernel).  With cache_stride 0 and B > 1 the rows are
 * instead B consecutive positions of one sequence sharing one cache, pos[b] = pos[0] + b
 * (mt_rope_attention's rows, as the VAE decoder's layers issue them): row b appends its k
 * and v at pos[b] and attends over [max(0, pos[b] + 1 - window), pos[b]], rows 0 .. b - 1's
 * new keys included.  Requirements: as mt_rope_cache_decode and mt_attention_decode (or
 * mt_rope_attention for rows of one sequence); B <= 8; the caches of the sequence's
 * attention items must not overlap each other or any linear's x or y.
 */
typedef struct mt_attn_op {
    const float *qkv;
    uint32_t ldq, B, hq, hkv;
    const uint32_t *pos;
    void *k_cache;
    void *v_cache;
    int32_t cache_t;      /* mt_dtype: MT_F32 or MT_F16 */
    uint32_t cache_len;   /* <= 4096 */
    uint64_t cache_stride;
    const float *inv_freq;  /* 32 floats: 1 / theta^(2i / 64) */
    float *out;
    uint32_t ldo;
    uint32_t window;
    float scale;
} mt_attn_op;

/*
 * The DiT's full attention of mt_dit_attention as an item of a sequence (Encoder.ditAttention,
 * Kernels.swift:208-220; DiTForward.encode, DiT.swift:35-52): B sequences of S rows, H heads of
 * 64, interleaved RoPE at positions 0 .. S - 1, scores scaled by `scale`; qkv rows [q | k | v]
 * (H*64 each) at stride ldq, out rows (H*64) at stride ldo.  It runs only in the DiT-block
 * kernel (mt_seq_kernel = MT_SEQ_DIT_BLOCK), where every workgroup computes it while staging
 * the out projection's activations.
 */
typedef struct mt_dit_attn_op {
    const float *qkv;
    uint32_t ldq, B, S, H;
    const float *inv_freq;  /* 32 floats: 1 / theta^(2i / 64) */
    float *out;
    uint32_t ldo;
    float scale;
} mt_dit_attn_op;

enum { MT_SEQ_LINEAR = 0, MT_SEQ_ATTENTION = 1, MT_SEQ_DIT_ATTENTION = 2 };
typedef struct mt_seq_item {
    int32_t kind;          /* MT_SEQ_LINEAR: `linear` is the op; MT_SEQ_ATTENTION: `attn`;
                              MT_SEQ_DIT_ATTENTION: `dit` */
    mt_linear_op linear;
    mt_attn_op attn;
    mt_dit_attn_op dit;
} mt_seq_item;
/* mt_seq_create over a list of linears and attention items: the whole decode layer
 * (QwenForward.dispatches, Qwen.swift:84-91) as one persistent launch.  An attention
 * item's output is an activation like a linear's (a later linear reads it as x).
 * DiT attention items are taken in one pattern only: DiT blocks at the flow head's shape
 * (DiTForward.encode, DiT.swift:35-52), each rmsnorm+qkv 3072 x 1024 + bias, the DiT
 * attention (H 16; B 2 x S 3 = 6 rows as in the flow loop, or B 1 x S 2 = 2 rows as in the
 * aggregator) of that qkv, out 1024 x 1024 + bias += reading the attention's output,
 * rmsnorm+ff1 4096 x 1024 + bias GELU, ff2 1024 x 4096 + bias +=, at M = B S rows, every
 * attention item with the same inv_freq and scale, on a device with 256 CUs (one workgroup
 * each); anything else with a DiT attention item returns MT_ENOTSUP. */
int mt_seq_create_items(const mt_seq_item *items, uint32_t n_items, mt_seq **out);
int mt_seq_run(mt_seq *seq, mt_stream_t stream);
int mt_seq_destroy(mt_seq *seq);
/* Workgroups the plan's kernel runs with (after mt_seq_create). */
int mt_seq_groups(const mt_seq *seq);
/* The kernel the plan runs: MT_SEQ_DECODE_LAYER when its linears repeat the Qwen2-0.5B
 * decode layer of QwenForward.dispatches (Qwen.swift:84-91; qkv 1152 x 896 + bias with the
 * first RMSNorm, o 896 x 896 +=, gate|up 2 x 4864 x 896 SiLU-gate with the second RMSNorm,
 * down 896 x 4864 +=) at 1, 2 or 4 rows, with or without decode attention items;
 * MT_SEQ_DIT_BLOCK for the DiT blocks described at mt_seq_create_items; MT_SEQ_GENERAL
 * otherwise (or under MT_TUNE_SEQ_LAYER = 1, which refuses DiT attention items).  All compute
 * the same sequence. */
enum { MT_SEQ_GENERAL = 0, MT_SEQ_DECODE_LAYER = 1, MT_SEQ_DIT_BLOCK = 2 };
int mt_seq_kernel(const mt_seq *seq);
/* Synchronous health check of a plan after its runs completed: MT_EHIP if a dataflow wait
 * of a run gave up after its spin bound (co-residency was lost), MT_ERANGE if an fp16-weight
 * run met an activation beyond the fp16 range, else MT_OK.  Both flags stay set for the
 * plan's life.  No counterpart in the reference (Metal has no in-kernel grid waits). */
int mt_seq_check(mt_seq *seq);

/*
 * Encoder.ropeCache (Kernels.swift:180-191, Shaders.swift:451-486): NeoX RoPE
 * (pairs i, i + 32 of each 64-wide head, angle = pos * inv_freq[i]) on the hq query
 * heads of qkv in place, and the rotated k heads plus the raw v heads appended to
 * the caches at positions pos0 .. pos0 + M - 1.  qkv rows are [q(hq*64) | k(hkv*64) |
 * v(hkv*64)] with row stride ldq floats.  Caches are [hkv, cache_len, 64] of type
 * cache_t (MT_F32 as the reference, or MT_F16).
 */
int mt_rope_cache(float *qkv, uint32_t ldq, uint32_t M, uint32_t hq, uint32_t hkv, uint32_t pos0,
                  void *k_cache, void *v_cache, mt_dtype cache_t, uint32_t cache_len,
                  const float *inv_freq, mt_stream_t stream);

/*
 * Batched decode form of mt_rope_cache: B independent sequences, one qkv row each.
 * Row b is rotated at position pos[b] (a device array of B uint32) and its k / v land
 * in sequence b's caches (k_cache / v_cache + b * cache_stride elements) at pos[b].
 * A pos[b] >= cache_len appends nothing (the q heads are still rotated).
 */
int mt_rope_cache_decode(float *qkv, uint32_t ldq, uint32_t B, uint32_t hq, uint32_t hkv,
                         const uint32_t *pos, void *k_cache, void *v_cache, mt_dtype cache_t,
                         uint32_t cache_len, uint64_t cache_stride, const float *inv_freq,
                         mt_stream_t stream);

/*
 * Encoder.attention (Kernels.swift:193-206, Shaders.swift:490-596): causal GQA of
 * the M query rows at positions pos0 .. pos0 + M - 1 over the cache, keys
 * [max(0, pos + 1 - window), pos] (window 0 = unlimited), scores scaled by `scale`,
 * max-subtracted softmax, out = sum p v.  q rows hold hq heads of 64 (stride ldq),
 * out rows stride ldo.  pos0 + M <= cache_len <= 4096.  Rows of a prefill (M >= 8, every
 * row's keys starting at 0, pos0 + M <= 1024) are attended 4 to a workgroup; the results
 * are bit-identical to attending the rows one call each.
 */
int mt_attention(const float *q, uint32_t ldq, uint32_t M, uint32_t hq, uint32_t hkv,
                 uint32_t pos0, uint32_t window, const void *k_cache, const void *v_cache,
                 mt_dtype cache_t, uint32_t cache_len, float *out, uint32_t ldo, float scale,
                 mt_stream_t stream);

/*
 * mt_rope_cache then mt_attention over the same M rows (Encoder.ropeCache then
 * Encoder.attention, Kernels.swift:180-206, as VAEDecoder.decodeDispatches issues them for the
 * decoder's sliding-window layers, VAEDecoder.swift:81-107) in one launch, with the same
 * effects and the same bits: q of every row is rotated in place in qkv, row m's rotated k and
 * raw v are appended at pos0 + m, and out row m attends over [max(0, pos0 + m + 1 - window),
 * pos0 + m].  M <= 64; out 16-byte aligned with a 16-byte row stride and apart from qkv;
 * otherwise as the two calls.
 */
int mt_rope_attention(float *qkv, uint32_t ldq, uint32_t M, uint32_t hq, uint32_t hkv, uint32_t pos0,
                      uint32_t window, void *k_cache, void *v_cache, mt_dtype cache_t, uint32_t cache_len,
                      const float *inv_freq, float *out, uint32_t ldo, float scale, mt_stream_t stream);

/*
 * Batched decode attention: B independent sequences, one query row each (the CFG
 * cond/uncond pair at B = 2).  Sequence b attends over its own cache (k_cache +
 * b * cache_stride elements, layout [hkv, cache_len, 64]) at keys
 * [max(0, len_b - window), len_b), len_b = lens[b] (a device array of B uint32,
 * 1 <= len_b <= cache_len).  q / out rows b at stride ldq / ldo.
 */
int mt_attention_decode(const float *q, uint32_t ldq, uint32_t B, uint32_t hq, uint32_t hkv,
                        const uint32_t *lens, uint32_t window, const void *k_cache,
                        const void *v_cache, mt_dtype cache_t, uint32_t cache_len,
                        uint64_t cache_stride, float *out, uint32_t ldo, float scale,
                        mt_stream_t stream);

/*
 * The DiT flow step around its linears (MingEngine.encodeStep's flow loop,
 * Engine.swift:395-402; DiTForward.encode, DiT.swift:35-52).
 *
 * mt_dit_attention -- Encoder.ditAttention (Kernels.swift:208-220, Shaders.swift:598-648):
 * full attention inside each of B sequences of S <= 8 rows.  qkv rows (stride ld floats) are
 * [q (H*64) | k (H*64) | v (H*64)]; q and k of row i (position i in its sequence) are rotated
 * by interleaved RoPE (pairs 2p, 2p + 1, angle = i * inv_freq[p], 32 frequencies); scores
 * q.k * scale, max-subtracted softmax over the sequence's S keys, out = sum p v (row stride
 * ldo).  qkv / out 8-byte aligned with even strides.
 */
int mt_dit_attention(const float *qkv, uint32_t ld, uint32_t B, uint32_t S, uint32_t H, const float *inv_freq,
                     float *out, uint32_t ldo, float scale, mt_stream_t stream);

/*
 * mt_dit_attention_linear -- the DiT block's Encoder.ditAttention followed by the out
 * projection Encoder.linear(attn, block.out, x, flags: .accumulate) (DiT.swift:44-45) in one
 * launch: y (op)= att W^T with the GemvFlags epilogue, where att = mt_dit_attention(qkv, p.ldx,
 * B, S, H, inv_freq, ..., scale) is computed inside the linear's prologue and never stored.
 * p.M = B * S (<= 32), p.K = 64 H, p.ldx = the qkv row stride (>= 3 K); the rest of p, w, wt,
 * bias and y as mt_linear with fp32 x (no MT_SILU_GATE).  qkv 16-byte aligned with a 16-byte
 * row stride; y must not overlap qkv.  Gives the same bits as mt_dit_attention into a buffer
 * followed by mt_linear of that buffer.
 */
int mt_dit_attention_linear(const float *qkv, uint32_t B, uint32_t S, uint32_t H, const float *inv_freq, float scale,
                            const void *w, mt_dtype wt, const void *bias, float *y, mt_gemv_params p,
                            mt_stream_t stream);

/*
 * mt_flow_assemble -- Encoder.flowAssemble (Kernels.swift:222-235, Shaders.swift:650-676):
 * the six flow-input rows x (stride ldx floats, hidden wide): row r, slot r % 3 = 0: temb +
 * cemb (r < 3) or temb + cond_bias (r >= 3); 1: x_b + x_w history; 2: x_b + x_w y.  x_w is
 * the x-embedder [hidden, latent_dim] and x_b / cond_bias [hidden], all of type wt (MT_BF16
 * as the reference, or MT_F16); y, history [latent_dim], cemb, temb [hidden] fp32.
 * latent_dim a multiple of 8 and x_w 16-byte aligned.
 */
int mt_flow_assemble(const float *y, const float *history, const float *cemb, const void *cond_bias,
                     const float *temb, const void *x_w, const void *x_b, mt_dtype wt, float *x, uint32_t ldx,
                     uint32_t hidden, uint32_t latent_dim, mt_stream_t stream);

/*
 * mt_flow_euler -- Encoder.flowEuler (Kernels.swift:237-246, Shaders.swift:678-693): with c
 * = pred[pred_row], u = pred[null_row] (row stride ldp), y += (c + (c - u) cfg) dt; capture
 * (2 * latent_dim floats, or NULL) receives c then u.
 */
int mt_flow_euler(float *y, const float *pred, uint32_t ldp, uint32_t pred_row, uint32_t null_row, float *capture,
                  uint32_t latent_dim, float cfg, float dt, mt_stream_t stream);

/*
 * mt_flow_euler_assemble -- Encoder.flowEuler of ODE step k followed by Encoder.flowAssemble
 * of step k + 1 (Kernels.swift:222-246; the ODE loop of Engine.swift:395-402) in one launch:
 * exactly mt_flow_euler(y, pred, ldp, pred_row, null_row, capture, latent_dim, cfg, dt) then
 * mt_flow_assemble(y, history, cemb, cond_bias, temb, x_w, x_b, wt, x, ldx, hidden,
 * latent_dim), the same arithmetic and bits, one workgroup.  No counterpart in the reference
 * (two dispatches there): it spares one launch per ODE step.  latent_dim a multiple of 8 up
 * to 2048; x must not overlap y, pred, history or capture.
 */
int mt_flow_euler_assemble(float *y, const float *pred, uint32_t ldp, uint32_t pred_row, uint32_t null_row,
                           float *capture, float cfg, float dt, const float *history, const float *cemb,
                           const void *cond_bias, const float *temb, const void *x_w, const void *x_b, mt_dtype wt,
                           float *x, uint32_t ldx, uint32_t hidden, uint32_t latent_dim, mt_stream_t stream);

/*
 * The audio VAE decoder's tail (VAEDecoder.decodeDispatches, VAEDecoder.swift:81-107).
 *
 * mt_upsample4 -- Encoder.upsample4 (Kernels.swift:247-257, Shaders.swift:700-718): the four
 * frames of a latent from fc1 outputs prev / cur / next ([hidden] each; prev or next NULL when
 * absent, then clamped to cur), torch's linear upsample (align_corners = false, scale 4):
 * rows 0..3 = 0.625 cur + 0.375 prev, 0.875 cur + 0.125 prev, 0.875 cur + 0.125 next,
 * 0.625 cur + 0.375 next; frames row stride ldf.
 *
 * mt_istft_frames -- Encoder.istftFrames (Kernels.swift:259-270, Shaders.swift:720-759):
 * spectrum rows (stride ld_spec) hold [log-magnitude, phase] of nfft / 2 + 1 bins each; frame
 * f = irfft(min(e^logmag, 100) e^{i phase}) / nfft * window lands in ring slot (frame0 + f) %
 * ring of ring_frames ([ring][nfft]).  cos_table[t] = cos(2 pi t / nfft).  nfft a multiple of
 * 4, at most 4096; count <= ring.
 *
 * mt_istft_emit -- Encoder.istftEmit (Kernels.swift:272-283, Shaders.swift:761-787): samples
 * s0 .. s0 + count - 1 of the stream: for s = s0 + i + (nfft - hop) / 2, out[i] = the sum of
 * frames f <= last_frame with 0 <= s - f hop < nfft of their sample s - f hop, over the sum of
 * window^2 at those samples.
 */
int mt_upsample4(const float *prev, const float *cur, const float *next, float *frames, uint32_t ldf,
                 uint32_t hidden, mt_stream_t stream);
int mt_istft_frames(const float *spec, uint32_t ld_spec, uint32_t count, uint32_t nfft,
                    const float *cos_table, const float *window, float *ring_frames, uint32_t frame0,
                    uint32_t ring, mt_stream_t stream);
int mt_istft_emit(const float *ring_frames, const float *window, uint32_t nfft, uint32_t hop, uint32_t s0,
                  uint32_t count, uint32_t last_frame, uint32_t ring, float *out, mt_stream_t stream);

/*
 * The weight path (setup time; these calls read files and allocate host memory, and
 * mt_arena_upload allocates pinned staging and a small counter buffer for its duration).
 *
 * mt_st_* -- SafeTensors (SafeTensors.swift:7-87): a memory-mapped .safetensors file (an
 * 8-byte little-endian header length, a JSON header of {name: {dtype, shape, data_offsets}},
 * the data).  A malformed header, or a file shorter than the header needs, is refused with
 * MT_EINVAL and the reference's message.  Entries are listed in header order; mt_st_find
 * gives a tensor's dtype (MT_BF16 / MT_F16 / MT_F32, or -1 for another), shape (up to 8
 * dims), byte size and its bytes in the mapping (valid until mt_st_close).
 */
typedef struct mt_st mt_st;
typedef struct mt_st_entry {
    int32_t dtype;
    uint32_t ndim;
    uint64_t shape[8];
    uint64_t bytes;
    const void *host;
} mt_st_entry;
int mt_st_open(const char *path, mt_st **out);
int mt_st_close(mt_st *st);
int mt_st_count(const mt_st *st);
int mt_st_name(const mt_st *st, uint32_t index, const char **name);
int mt_st_find(const mt_st *st, const char *name, mt_st_entry *out);

/*
 * mt_arena_* -- WeightArena (Weights.swift:8-79): one module's 16-bit weights in one device
 * buffer.  Plan with mt_arena_tensor (a bf16 tensor, or several concatenated along their
 * first axis, e.g. q, k and v rows; Weights.swift:34-50) and mt_arena_padded (a bf16 [n,
 * stored_k] weight laid out as [n, k] with zero columns past stored_k; Weights.swift:59-71);
 * each lands at the next 256-byte-aligned offset in call order.  Then allocate
 * mt_arena_bytes() of device memory (256-byte aligned) and mt_arena_upload it: synchronous on
 * `stream`; the arena reads as zeros outside the tensors.  convert_to MT_F16 converts the
 * uploaded bf16 weights to fp16 in place (round to nearest even); mt_arena_audit then gives
 * the count of finite values that became +-inf and of nonzero values that became zero.  The
 * st file must stay open until the upload.  No counterpart for the conversion in the
 * reference (its kernels read bf16 only).
 */
typedef struct mt_arena mt_arena;
int mt_arena_create(const mt_st *st, mt_dtype convert_to, mt_arena **out);
int mt_arena_tensor(mt_arena *arena, const char *const *names, uint32_t n_names, uint64_t *offset,
                    uint64_t *count);
int mt_arena_padded(mt_arena *arena, const char *name, uint32_t n, uint32_t k, uint32_t stored_k,
                    uint64_t *offset);
uint64_t mt_arena_bytes(const mt_arena *arena);
int mt_arena_upload(mt_arena *arena, void *device_base, mt_stream_t stream);
int mt_arena_audit(const mt_arena *arena, uint64_t *overflow, uint64_t *underflow);
int mt_arena_destroy(mt_arena *arena);

/* Text of the last error on this thread ("" if none). */
const char *mt_last_error(void);
/* Library version string. */
const char *mt_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MINGTTS_HIP_H */
