// The fixed split-K scratch of mt_linear_static: the linear's split-K partial sums and
// arrival counters in one file-scope device array instead of a per-stream allocation, for
// callers that cannot allocate (code under HIP graph capture, serving loops that forbid
// hipMalloc).  Every call on a device shares that device's array; each launch leaves the
// counters zero again, so nothing has to be cleared between calls, and calls that overlap on
// one device race.
#include <mutex>

#include "mt_internal.hpp"

namespace mt {

namespace {

constexpr uint32_t STATIC_COUNTERS = 4096;         // arrival counters: tiles of one split linear
constexpr size_t STATIC_PART_BYTES = 16u << 20;    // partial sums: 16 MiB
constexpr size_t STATIC_BYTES = STATIC_COUNTERS * 4 + STATIC_PART_BYTES;

}  // namespace

// Host code never passes this symbol to a kernel (in host code it names no device address):
// it uses the address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) uint8_t scratch[STATIC_BYTES];

namespace {

std::mutex g_mu;
void *g_ptr[64];  // the array's address on each device, set at the device's first call

}  // namespace

int static_scratch(hipStream_t stream, FixedWs &ws) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return set_error(MT_EHIP, "mt_linear_static: no current device (or device index past 63)");
    void *p = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        if (!g_ptr[dev]) {
            hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p)
                return set_error(MT_EHIP, "mt_linear_static: hipGetSymbolAddress: %s", hipGetErrorString(e));
            // The array starts zero (a device global) and every launch leaves its counters zero,
            // so no clear is issued: one here could still be running on this stream while
            // another stream's first call already counts tiles in.
            g_ptr[dev] = p;
        }
        p = g_ptr[dev];
    }
    ws.cnt = static_cast<uint32_t *>(p);
    ws.counters = STATIC_COUNTERS;
    ws.part = static_cast<uint8_t *>(p) + STATIC_COUNTERS * 4;
    ws.part_bytes = STATIC_PART_BYTES;
    return MT_OK;
}

}  // namespace mt
