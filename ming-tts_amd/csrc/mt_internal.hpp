// Host-side internals shared by the launchers and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mt_device.hpp"

namespace mt {

// Error reporting: the message lands in the thread-local buffer read by mt_last_error().
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// hipGetLastError after a launch, as an ABI return code.
int check_launch(const char *what);

// Process-wide tuning (mt_set_tuning).
struct Tuning {
    int gemv_rows_max = 8;
    int gemv_lanes = 0;
    int gemm_splitk = 0;
    int seq_groups = 0;
};
Tuning &tuning();

// One op of a persistent linear sequence, as the kernel reads it.
struct SeqOp {
    const void *x;
    const uint16_t *w;
    const uint16_t *w2;
    const uint16_t *bias;
    float *y;
    const uint16_t *norm;
    uint32_t M, N, K, ldx, ldy, flags;
    float eps;
    int32_t lanes_log2;
};
struct SeqPlan;
int seq_create(const SeqOp *ops, uint32_t n_ops, int mr, int wt, int xt, SeqPlan **out);
int seq_run(SeqPlan *p, hipStream_t stream);
int seq_check(SeqPlan *p);
void seq_destroy(SeqPlan *p);
int seq_groups(const SeqPlan *p);

int launch_rope_cache(float *qkv, uint32_t ldq, uint32_t rows, uint32_t hq, uint32_t hkv, uint32_t pos0,
                      const uint32_t *pos_arr, void *kc, void *vc, int ct, uint32_t cache_len,
                      uint64_t cache_stride, const float *inv_freq, hipStream_t stream);
int launch_attention(const float *q, uint32_t ldq, uint32_t rows, uint32_t hq, uint32_t hkv, uint32_t pos0,
                     const uint32_t *lens, uint32_t window, const void *kc, const void *vc, int ct,
                     uint32_t cache_len, uint64_t cache_stride, float *out, uint32_t ldo, float scale,
                     hipStream_t stream);

int gemv_lanes_log2(uint32_t K, int override_lanes);
int launch_gemv(const LinearArgs &a, int xt, int wt, hipStream_t stream, int override_lanes);
int launch_gemm(const LinearArgs &a, int xt, int wt, hipStream_t stream, int splitk_override);

}  // namespace mt
