// Diagnose outputs of dispatch and combine (the reference's waitRecvCostStats / sendCostStats,
// moe_dispatch_normal.h:489-529, moe_combine_normal.h:197): per source rank, the microseconds
// the phase spent on that rank's data, accumulated across calls.  With one EP rank every row comes
// from rank 0, so entry 0 receives the phase's wall time on the stream: a one-thread kernel stamps
// the 100 MHz constant clock when the stream reaches the phase, another one after it, and adds the
// difference.  Both are ordinary stream-ordered kernels (no host synchronisation, graph-capturable).
#include <atomic>

#include "cam_device.h"
#include "launchers.h"

namespace cam {

__global__ void phase_begin_kernel(uint64_t *stamp) { stamp[0] = wall_clock64(); }

__global__ void phase_end_kernel(const uint64_t *stamp, int32_t *stats, int idx, long long ticks_per_us)
{
    const uint64_t dt = wall_clock64() - stamp[0];
    atomicAdd(stats + idx, (int32_t)(dt / (uint64_t)ticks_per_us));
}

// Constant-clock ticks per microsecond of the current device, cached per device (a racing first call only
// repeats the idempotent query).
static long long ticks_per_us()
{
    constexpr int MAX_DEV = 64;
    static std::atomic<long long> cache[MAX_DEV];
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0)
        dev = 0;
    if (dev < MAX_DEV) {
        const long long c = cache[dev].load(std::memory_order_relaxed);
        if (c > 0)
            return c;
    }
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0)
        khz = 100000;  // gfx9: 100 MHz
    const long long t = khz >= 1000 ? khz / 1000 : 1;
    if (dev < MAX_DEV)
        cache[dev].store(t, std::memory_order_relaxed);
    return t;
}

hipError_t launch_phase_begin(uint64_t *stamp, hipStream_t s)
{
    hipLaunchKernelGGL(phase_begin_kernel, dim3(1), dim3(1), 0, s, stamp);
    return hipGetLastError();
}

hipError_t launch_phase_end(const uint64_t *stamp, int32_t *stats, int idx, hipStream_t s)
{
    hipLaunchKernelGGL(phase_end_kernel, dim3(1), dim3(1), 0, s, stamp, stats, idx, ticks_per_us());
    return hipGetLastError();
}

}  // namespace cam
