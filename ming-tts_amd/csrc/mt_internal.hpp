// Host-side internals shared by the launchers and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <vector>

#include "mingtts_hip.h"
#include "mt_device.hpp"

namespace mt {

struct FixedWs;  // a fixed split-K scratch (below)

// Error reporting: the message lands in the thread-local buffer read by mt_last_error().
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// hipGetLastError after a launch, as an ABI return code.
int check_launch(const char *what);

// Process-wide tuning (mt_set_tuning).  Every field is read and written atomically
// (relaxed), so host threads launching on distinct streams may call mt_set_tuning
// concurrently; a change applies to calls that read the field after it.
struct Tuning {
    std::atomic<int> gemv_rows_max{8};
    std::atomic<int> gemv_lanes{0};
    std::atomic<int> gemm_splitk{0};
    std::atomic<int> gemm_tile{0};
    std::atomic<int> gemm_stages{0};
    std::atomic<int> gemv_mfma{0};
    std::atomic<int> seq_groups{0};
    std::atomic<int> seq_launch{1};
    std::atomic<int> seq_layer{0};
};
Tuning &tuning();

// One op of a persistent linear sequence, as the kernel reads it.  Activations produced
// inside the sequence travel through the plan's tagged buffers (fp32 words whose lowest
// mantissa bit carries the run's parity, one per output element); user buffers are read
// only where nothing in the sequence wrote them before, and written only by the last op
// that writes each region.
struct SeqOp {
    const void *x;          // external x (when xsrc < 0), element type xt
    const uint16_t *w;
    const uint16_t *w2;
    const uint16_t *bias;
    const uint16_t *norm;
    float *y;               // user output (written only when final != 0)
    uint32_t *tag;          // this op's tagged output [M][N]
    uint32_t M, N, K, ldx, ldy, flags;
    float eps;
    int32_t xsrc;           // op producing x, or -1
    uint32_t xcol;          // column of x[.][0] in that op's output
    int32_t ysrc;           // op producing y's old value (accumulate), or -1 (read y)
    uint32_t ycol;
    int32_t xt;             // element type of an external x
    int32_t final_out;      // nonzero: this op's output is the last write of its region
    uint32_t xoff, xld;     // tagged x: word offset of x[0][0] in the plan's tag buffer, row stride
    uint32_t yoff, yld;     // tagged old y: the same
    int32_t kind;           // SEQ_LINEAR, or SEQ_ATTN (below)
    // A decode attention item (kind SEQ_ATTN): x is the qkv rows (M = B rows, K = (hq + 2 hkv)
    // 64 words read), y the output (N = hq 64), w / w2 the k / v caches, eps the score scale;
    // no weights, bias, norm or flags.
    uint32_t heads;         // hq | hkv << 16
    uint32_t cache_len, window;
    const uint32_t *pos;    // [M] positions
    const float *inv_freq;  // 32 RoPE frequencies
    uint64_t cache_stride;  // elements between row b's caches and row b + 1's
    int32_t cache_t;        // cache element type
    int32_t planes;         // tagged output planes: 2 for the decode-layer kernel's down (split over K), else 1
};
static_assert(sizeof(SeqOp) % 16 == 0, "SeqOp is staged into LDS in 16-byte pieces");
// A DiT attention item (kind SEQ_DIT): x the qkv rows (M = B S rows, K = 3 H 64), y the output
// (N = H 64), eps the score scale, heads = H | S << 16, inv_freq its 32 RoPE frequencies.
enum : int32_t { SEQ_LINEAR = 0, SEQ_ATTN = 1, SEQ_DIT = 2 };
struct SeqPlan;
// Limits of the persistent sequence kernel: threads per workgroup, output features per
// workgroup per op, and the LDS areas of its waves.
constexpr int SEQ_THREADS_N = 512;
constexpr int SEQ_RMAX = 64;
constexpr int SEQ_PARTW = 128;     // partial sums per compute wave per op: virtual rows * M
constexpr int SEQ_XLDS = 10240;    // M * K of an op: its activations staged in LDS (hi + lo)
constexpr int SEQ_OPS_MAX = 128;   // ops of a sequence (their descriptors are staged in LDS)
constexpr int SEQ_CW = 8;          // waves per workgroup, each computing a share of every op
constexpr int SEQ_TA = 12;         // MFMA tiles of one op a wave holds in registers
constexpr int SEQ_GMAX = 2048;     // K of an op with an RMSNorm gain (staged in LDS)
// The Qwen2-0.5B decode layer (Weights.swift:81-92) the decode-layer kernel is specialised
// for, and the workgroup counts its tiling takes.
constexpr uint32_t LAY_H = 896, LAY_QKV = 1152, LAY_I = 4864;
constexpr int LAY_GMIN = 224, LAY_GMAX = 256;
// Workgroup count of the persistent kernel on the current device.
int seq_limits(int *groups, int *preferred);
// Dataflow plan of a serial list of linears and attention items for `groups` workgroups
// (host only; no HIP calls).
int seq_plan(const mt_seq_item *items, uint32_t n, int groups, std::vector<SeqOp> &out, int &wt);
// The general sequence kernel's limits on each linear's share at `groups` workgroups
// (MT_ENOTSUP with the reason when one is exceeded).
int seq_general_limits(const mt_seq_item *items, uint32_t n, int groups);
// Do the planned ops repeat the Qwen2-0.5B decode layer (qkv 1152 x 896 with bias and
// RMSNorm, o 896 x 896 accumulating, gate|up 2 x 4864 x 896 SiLU-gate with RMSNorm, down
// 896 x 4864 accumulating) at one M of 1, 2 or 4, with `groups` in the decode-layer
// kernel's range?
bool layer_pattern(const SeqOp *ops, uint32_t n, int groups);
// The DiT blocks of the flow head (DiTForward.encode, DiT.swift:35-52) the DiT-block kernel is
// specialised for: per block rmsnorm+qkv 3072 x 1024 + bias, DiT attention (H 16) of that qkv,
// out 1024 x 1024 + bias += of the attention's output, rmsnorm+ff1 4096 x 1024 + bias GELU, ff2
// 1024 x 4096 + bias +=, at B 2 x S 3 = 6 rows (the flow loop) or B 1 x S 2 = 2 rows (the
// aggregator), on exactly DIT_G workgroups.
constexpr uint32_t DIT_H = 1024, DIT_QKV = 3072, DIT_FF = 4096, DIT_HEADS = 16;
constexpr int DIT_G = 256;
bool dit_pattern(const SeqOp *ops, uint32_t n, int groups);
// The kernel of a plan: MT_SEQ_GENERAL, MT_SEQ_DECODE_LAYER or MT_SEQ_DIT_BLOCK.
int seq_create(SeqOp *ops, uint32_t n_ops, int wt, int groups, int kind, SeqPlan **out);
int seq_run(SeqPlan *p, hipStream_t stream);
int seq_check(SeqPlan *p);
void seq_destroy(SeqPlan *p);
int seq_groups(const SeqPlan *p);
int seq_kernel_kind(const SeqPlan *p);

int launch_flow_euler_assemble(float *y, const float *pred, uint32_t ldp, uint32_t pred_row, uint32_t null_row,
                               float *capture, float cfg, float dt, const float *history, const float *cemb,
                               const void *cbias, const float *temb, const void *xw, const void *xb, int wt, float *x,
                               uint32_t ldx, uint32_t hidden, uint32_t latent, hipStream_t stream);
int launch_rope_cache(float *qkv, uint32_t ldq, uint32_t rows, uint32_t hq, uint32_t hkv, uint32_t pos0,
                      const uint32_t *pos_arr, void *kc, void *vc, int ct, uint32_t cache_len,
                      uint64_t cache_stride, const float *inv_freq, hipStream_t stream);
int launch_rope_attention(float *qkv, uint32_t ldq, uint32_t rows, uint32_t hq, uint32_t hkv, uint32_t pos0,
                          uint32_t window, void *kc, void *vc, int ct, uint32_t cache_len, const float *inv_freq,
                          float *out, uint32_t ldo, float scale, hipStream_t stream);
int launch_attention(const float *q, uint32_t ldq, uint32_t rows, uint32_t hq, uint32_t hkv, uint32_t pos0,
                     const uint32_t *lens, uint32_t window, const void *kc, const void *vc, int ct,
                     uint32_t cache_len, uint64_t cache_stride, float *out, uint32_t ldo, float scale,
                     hipStream_t stream);

int launch_dit_attention(const float *qkv, uint32_t ld, uint32_t B, uint32_t S, uint32_t H, const float *inv_freq,
                         float *out, uint32_t ldo, float scale, hipStream_t stream);
int launch_flow_assemble(const float *y, const float *history, const float *cemb, const void *cbias, const float *temb,
                         const void *xw, const void *xb, int wt, float *x, uint32_t ldx, uint32_t hidden,
                         uint32_t latent, hipStream_t stream);
int launch_flow_euler(float *y, const float *pred, uint32_t ldp, uint32_t pred_row, uint32_t null_row, float *capture,
                      uint32_t latent, float cfg, float dt, hipStream_t stream);

int gemv_lanes_log2(uint32_t K, int override_lanes, uint32_t M);
int launch_gemv(const LinearArgs &a, int xt, int wt, hipStream_t stream, int override_lanes);
// Up to 64 B columns (M rows of x of the weights' type, or 2 M with hi + lo halves; a fused
// norm at most 8 rows) on MFMA, x staged once per workgroup of 16 output features.
int gemv_mfma_columns(uint32_t M, int xt, int wt, bool norm);
int launch_gemv_mfma(const LinearArgs &a, int xt, int wt, hipStream_t stream, const FixedWs *fixed = nullptr);
// The same kernel with x computed in its prologue as the DiT attention of qkv = a.x (row
// stride a.ldx): mt_dit_attention_linear.
int launch_gemv_mfma_attn(const LinearArgs &a, int wt, const float *inv_freq, uint32_t S, uint32_t H, float scale,
                          hipStream_t stream);
// The lane-group GEMV, and the MFMA GEMM (pipelined for x of the weights' type without a
// norm, register-staged otherwise); mt_linear's routing between them and the small-row MFMA
// kernel is linear_family in api.cpp.  The small-row kernel runs up to 16 rows because it
// measured faster than the pipelined GEMM at M = 16 on every Qwen linear, even at 32, and
// slower at 64.
int launch_gemm(const LinearArgs &a, int xt, int wt, hipStream_t stream, const FixedWs *fixed = nullptr);

// A fixed split-K scratch (mt_linear_static): arrival counters (zero between launches) and
// room for partial sums.  A launcher given one uses it instead of the stream's workspace and
// refuses a linear that needs more.
struct FixedWs {
    uint32_t *cnt;
    uint32_t counters;
    void *part;
    size_t part_bytes;
};
// The fixed scratch of the current device (set up on the first call on a device), or an error.
int static_scratch(hipStream_t stream, FixedWs &ws);
// The split-K workspace of a launch: the fixed scratch when fixed != null, else the stream's.
int split_workspace(const FixedWs *fixed, hipStream_t stream, size_t part_bytes, uint32_t counters, void **part,
                    uint32_t **cnt, const char *who);

// Compute units of the current device (cached per device), or <= 0 when it cannot be queried.
int device_cus();
// Split-K workspace of `stream` on the current device: at least `part_bytes` of partial sums
// and `counters` zeroed arrival counters (the kernels leave them zero again).  Grows by
// synchronising the stream, so it is not for use under graph capture once it must grow.
int stream_workspace(hipStream_t stream, size_t part_bytes, uint32_t counters, void **part, uint32_t **cnt);

// Pipelined MFMA GEMM for activations of the weights' type, or fp32 (split into hi + lo).
struct TiledPlan {
    int shape;                // index of the (bm, bn) tile shape
    uint32_t bm, bn;          // x rows and weight rows per tile
    uint32_t tiles_m, tiles_n, splits, kps;
    int stages;               // LDS pipeline depth (64-k stages; 1: two register-staged buffers)
};
TiledPlan tiled_plan(uint32_t M, uint32_t N, uint32_t K, bool gated, int cus, int shape_override, int splitk_override,
                     bool split);
// x of the weights' type without a norm, or fp32 x with or without one (a.norm).
int launch_gemm_tiled(const LinearArgs &a, int xt, int wt, hipStream_t stream, const FixedWs *fixed = nullptr);

}  // namespace mt
