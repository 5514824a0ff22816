// Per-(device, stream) device workspace of the split-K GEMM, and the device CU count.
//
// Launches on one stream run in order, so one workspace per stream is never used by two
// launches at once; launches on different streams get different workspaces.  The first
// bytes hold the arrival counters (zeroed once at allocation and left zero by every
// launch), the partial sums follow.  A workspace that has to grow is replaced, never freed:
// a HIP graph captured on the stream keeps the old buffer's addresses in its nodes, and a
// replay must still find that memory there (the retired buffers are at most as large as the
// live one, since each growth at least doubles it).
#include <algorithm>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "mt_internal.hpp"

namespace mt {

namespace {

constexpr size_t COUNTER_BYTES_ALIGN = 256;

struct Workspace {
    void *base = nullptr;
    size_t part_bytes = 0;
    uint32_t counters = 0;
};

std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;
std::vector<void *> g_retired;  // replaced workspaces, kept until the process ends

int g_cus[64];

}  // namespace

int device_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return -1;
    if (dev < 64 && g_cus[dev] > 0) return g_cus[dev];
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
    if (dev < 64) g_cus[dev] = cus;
    return cus;
}

int split_workspace(const FixedWs *fixed, hipStream_t stream, size_t part_bytes, uint32_t counters, void **part,
                    uint32_t **cnt, const char *who) {
    if (!fixed) return stream_workspace(stream, part_bytes, counters, part, cnt);
    if (part_bytes > fixed->part_bytes || counters > fixed->counters)
        return set_error(MT_ENOTSUP,
                         "%s: the split-K partials (%zu bytes, %u tiles) exceed the static scratch (%zu bytes, %u "
                         "tiles); use mt_linear",
                         who, part_bytes, counters, fixed->part_bytes, fixed->counters);
    *part = fixed->part;
    *cnt = fixed->cnt;
    return MT_OK;
}

int stream_workspace(hipStream_t stream, size_t part_bytes, uint32_t counters, void **part, uint32_t **cnt) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(MT_EHIP, "workspace: no current device");
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Workspace &w = g_ws[std::make_pair(dev, stream)];
    if (!w.base || w.part_bytes < part_bytes || w.counters < counters) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
            return set_error(MT_EINVAL, "workspace: the split-K workspace must grow, which cannot happen under "
                                        "graph capture; run the same linear once before capturing");
        const size_t pb = std::max(part_bytes, w.part_bytes * 2);
        const uint32_t nc = std::max<uint32_t>(std::max(counters, w.counters * 2), 1024);
        const size_t cb = (static_cast<size_t>(nc) * 4 + COUNTER_BYTES_ALIGN - 1) / COUNTER_BYTES_ALIGN * COUNTER_BYTES_ALIGN;
        if (w.base) {
            g_retired.push_back(w.base);  // graphs captured on this stream may still use it
            w.base = nullptr;
        }
        void *p = nullptr;
        hipError_t e = hipMalloc(&p, cb + pb);
        if (e != hipSuccess) return set_error(MT_ENOMEM, "workspace: hipMalloc(%zu): %s", cb + pb, hipGetErrorString(e));
        // Ordered on the stream itself (which need not synchronise with the null stream).
        e = hipMemsetAsync(p, 0, cb, stream);
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
        if (e != hipSuccess) {
            (void)hipFree(p);
            return set_error(MT_EHIP, "workspace: hipMemset: %s", hipGetErrorString(e));
        }
        w.base = p;
        w.part_bytes = pb;
        w.counters = static_cast<uint32_t>(cb / 4);
    }
    const size_t cb = static_cast<size_t>(w.counters) * 4;
    *cnt = static_cast<uint32_t *>(w.base);
    *part = static_cast<char *>(w.base) + cb;
    return MT_OK;
}

}  // namespace mt
