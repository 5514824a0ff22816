// Persistent execution of a linear sequence (mt_seq_*): the decode step's chain of
// dependent GEMVs as ONE cooperative launch.
//
// Reference counterpart: QwenForward.dispatches encoded on one serial compute encoder
// (Qwen.swift:72-97); every dispatch sees the writes of the ones before it.  On MI355X a
// launch per linear costs microseconds of dispatch and drain against 0.2-2.2 us of weight
// streaming per decode linear, so the whole chain runs inside one grid of resident
// workgroups:
//   - op i's output features are split evenly over the G workgroups (rows r0..r1 of W);
//     inside a workgroup, groups of L lanes own one feature each (gemv_feature);
//   - between ops, a device-wide barrier: every wave releases its stores at agent scope,
//     thread 0 bumps a counter and spins (bounded) until all G have arrived, every wave
//     acquires at agent scope before reading the next op's activations;
//   - the last workgroup to leave resets the counters, so the plan can be re-run (and
//     captured) without any memset.
// A spin that exceeds its bound sets a flag (read by mt_seq_check) and lets the wave go
// on, so a broken co-residency assumption ends the kernel instead of hanging it.
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "gemv_core.hpp"
#include "mt_internal.hpp"
#include "mingtts_hip.h"

namespace mt {


// Words of the sync area, each on its own 128-byte line.
enum : int { SYNC_COUNT = 0, SYNC_EXIT = 32, SYNC_TIMEOUT = 64, SYNC_WORDS = 96 };
constexpr int SEQ_THREADS = 512;
// Polls before a barrier gives up; each poll is at least one memory round trip (~1 us),
// against a normal wait of a few microseconds.
constexpr uint32_t SPIN_LIMIT = 1u << 20;

// `abandoned` (thread 0's register) is set after a timeout: the workgroup then stops waiting
// at later barriers, so a lost co-residency costs one spin bound, not one per op.
__device__ __forceinline__ void grid_barrier(uint32_t *sync, uint32_t target, bool &abandoned) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(sync + SYNC_COUNT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t spins = 0;
        while (!abandoned &&
               __hip_atomic_load(sync + SYNC_COUNT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (++spins > SPIN_LIMIT) {
                __hip_atomic_store(sync + SYNC_TIMEOUT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                abandoned = true;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

template <int MR, int WT, int XT>
__global__ __launch_bounds__(SEQ_THREADS) void seq_kernel(const SeqOp *__restrict__ ops, uint32_t n_ops,
                                                         uint32_t *sync) {
    const uint32_t G = gridDim.x, g = blockIdx.x;
    bool abandoned = false;
    for (uint32_t i = 0; i < n_ops; i++) {
        const SeqOp o = ops[i];
        const LinearArgs a{o.x, o.w, o.w2, o.bias, o.y, o.M, o.N, o.K, o.ldx, o.ldy, o.flags, o.norm, o.eps};
        const int l2 = o.lanes_log2, L = 1 << l2;
        const int groups = SEQ_THREADS >> l2;
        const int grp = static_cast<int>(threadIdx.x) >> l2, j = static_cast<int>(threadIdx.x) & (L - 1);
        const uint32_t r0 = static_cast<uint32_t>(static_cast<uint64_t>(g) * o.N / G);
        const uint32_t r1 = static_cast<uint32_t>(static_cast<uint64_t>(g + 1) * o.N / G);
        const int rows = static_cast<int>(o.M);
        const bool gated = (o.flags & F_SILU_GATE) != 0, norm = o.norm != nullptr;
        if (gated && norm) {
            for (uint32_t n = r0 + grp; n < r1; n += groups) gemv_feature<MR, WT, XT, true, true, 4>(a, n, 0, rows, L, j);
        } else if (gated) {
            for (uint32_t n = r0 + grp; n < r1; n += groups) gemv_feature<MR, WT, XT, true, false, 4>(a, n, 0, rows, L, j);
        } else if (norm) {
            for (uint32_t n = r0 + grp; n < r1; n += groups) gemv_feature<MR, WT, XT, false, true, 4>(a, n, 0, rows, L, j);
        } else {
            for (uint32_t n = r0 + grp; n < r1; n += groups) gemv_feature<MR, WT, XT, false, false, 4>(a, n, 0, rows, L, j);
        }
        if (i + 1 < n_ops) grid_barrier(sync, (i + 1) * G, abandoned);
    }
    // The last workgroup out resets the counters for the next run.
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(sync + SYNC_EXIT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == G - 1) {
            __hip_atomic_store(sync + SYNC_COUNT, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(sync + SYNC_EXIT, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

typedef void (*seq_fn)(const SeqOp *, uint32_t, uint32_t *);

namespace {

template <int MR, int WT>
seq_fn pick_x(int xt) {
    switch (xt) {
        case DT_F32: return seq_kernel<MR, WT, DT_F32>;
        case DT_F16: return seq_kernel<MR, WT, DT_F16>;
        default: return seq_kernel<MR, WT, DT_BF16>;
    }
}

template <int MR>
seq_fn pick_w(int wt, int xt) { return wt == DT_BF16 ? pick_x<MR, DT_BF16>(xt) : pick_x<MR, DT_F16>(xt); }

seq_fn pick(int mr, int wt, int xt) {
    switch (mr) {
        case 1: return pick_w<1>(wt, xt);
        case 2: return pick_w<2>(wt, xt);
        case 4: return pick_w<4>(wt, xt);
        default: return pick_w<8>(wt, xt);
    }
}

}  // namespace

struct SeqPlan {
    SeqOp *d_ops = nullptr;
    uint32_t *d_sync = nullptr;
    uint32_t n_ops = 0;
    int groups = 0;
    int device = 0;
    seq_fn fn = nullptr;
};

int seq_create(const SeqOp *ops, uint32_t n_ops, int mr, int wt, int xt, SeqPlan **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(MT_EHIP, "mt_seq_create: hipGetDevice: %s", hipGetErrorString(e));
    SeqPlan *p = new SeqPlan();
    p->n_ops = n_ops;
    p->device = dev;
    p->fn = pick(mr, wt, xt);
    int cus = 0, per_cu = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(p->fn), SEQ_THREADS, 0);
    if (e != hipSuccess || cus <= 0 || per_cu <= 0) {
        delete p;
        return set_error(MT_EHIP, "mt_seq_create: occupancy query failed (%s, cus %d, per_cu %d)",
                         hipGetErrorString(e), cus, per_cu);
    }
    int want = tuning().seq_groups;
    const int resident = cus * per_cu;
    // Default: one 512-thread workgroup per CU.
    p->groups = want > 0 ? (want < resident ? want : resident) : cus;
    e = hipMalloc(&p->d_ops, sizeof(SeqOp) * (n_ops ? n_ops : 1));
    if (e == hipSuccess) e = hipMalloc(&p->d_sync, SYNC_WORDS * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemcpy(p->d_ops, ops, sizeof(SeqOp) * n_ops, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(p->d_sync, 0, SYNC_WORDS * sizeof(uint32_t));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(p->d_ops);
        (void)hipFree(p->d_sync);
        delete p;
        return set_error(MT_EHIP, "mt_seq_create: %s", hipGetErrorString(e));
    }
    *out = p;
    return MT_OK;
}

int seq_run(SeqPlan *p, hipStream_t stream) {
    if (p->n_ops == 0) return MT_OK;
    void *args[] = {&p->d_ops, &p->n_ops, &p->d_sync};
    hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void *>(p->fn), dim3(p->groups),
                                              dim3(SEQ_THREADS), args, 0, stream);
    if (e != hipSuccess) return set_error(MT_EHIP, "mt_seq_run: cooperative launch: %s", hipGetErrorString(e));
    return MT_OK;
}

int seq_check(SeqPlan *p) {
    uint32_t flag = 0;
    hipError_t e = hipMemcpy(&flag, p->d_sync + SYNC_TIMEOUT, sizeof(flag), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return set_error(MT_EHIP, "mt_seq_check: %s", hipGetErrorString(e));
    if (flag) return set_error(MT_EHIP, "mt_seq_check: a device-wide barrier exceeded its spin bound");
    return MT_OK;
}

int seq_groups(const SeqPlan *p) { return p->groups; }

void seq_destroy(SeqPlan *p) {
    if (!p) return;
    (void)hipFree(p->d_ops);
    (void)hipFree(p->d_sync);
    delete p;
}

}  // namespace mt
