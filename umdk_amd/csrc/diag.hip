// Diagnose outputs of dispatch and combine (the reference's waitRecvCostStats / sendCostStats,
// moe_dispatch_normal.h:489-529, moe_combine_normal.h:197): per source rank, the microseconds
// the phase spent on that rank's data, accumulated across calls.  With one EP rank every row comes
// from rank 0, so entry 0 receives the phase's wall time on the stream: a one-thread kernel stamps
// the 100 MHz constant clock when the stream reaches the phase, another one after it, and adds the
// difference.  Both are ordinary stream-ordered kernels (no host synchronisation, graph-capturable).
#include "cam_device.h"
#include "launchers.h"

namespace cam {

__global__ void phase_begin_kernel(uint64_t *stamp) { stamp[0] = wall_clock64(); }

__global__ void phase_end_kernel(const uint64_t *stamp, int32_t *stats, int idx, long long ticks_per_us)
{
    const uint64_t dt = wall_clock64() - stamp[0];
    atomicAdd(stats + idx, (int32_t)(dt / (uint64_t)ticks_per_us));
}

static long long ticks_per_us()
{
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0)
        khz = 100000;  // gfx9: 100 MHz
    return khz >= 1000 ? khz / 1000 : 1;
}

hipError_t launch_phase_begin(uint64_t *stamp, hipStream_t s)
{
    hipLaunchKernelGGL(phase_begin_kernel, dim3(1), dim3(1), 0, s, stamp);
    return hipGetLastError();
}

hipError_t launch_phase_end(const uint64_t *stamp, int32_t *stats, int idx, hipStream_t s)
{
    static const long long tpu = ticks_per_us();
    hipLaunchKernelGGL(phase_end_kernel, dim3(1), dim3(1), 0, s, stamp, stats, idx, tpu);
    return hipGetLastError();
}

}  // namespace cam
