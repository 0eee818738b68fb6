// Device helpers of the fused decode entry (fused_deep_moe): expert-id
// preparation and small fills.  The composition itself is host code in
// fused_api.cpp.
#include "cam_device.h"
#include "launchers.h"

namespace cam {

// ids_eff[t,k] = expert_ids[t,k] - first_local when the token is active (x_active_mask is a
// true-prefix mask, API guide doc/en/cam/CAM API Guide.md:197) and the expert is one of this
// rank's local experts; otherwise -1 (not routed here).
__global__ void prepare_ids_kernel(const int32_t *__restrict__ ids, const uint8_t *__restrict__ active, int T, int K,
                                   int first_local, int L, int32_t *__restrict__ out)
{
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < T * K; i += gridDim.x * blockDim.x) {
        const int t = i / K;
        const int e = ids[i] - first_local;
        const bool on = (active == nullptr || active[t] != 0) && e >= 0 && e < L && ids[i] >= 0;
        out[i] = on ? e : -1;
    }
}

hipError_t launch_prepare_ids(const int32_t *ids, const uint8_t *active, int T, int K, int first_local, int L,
                              int32_t *out, hipStream_t s)
{
    if (T * K == 0)
        return hipSuccess;
    const int blocks = (T * K + 255) / 256 < 1024 ? (T * K + 255) / 256 : 1024;
    hipLaunchKernelGGL(prepare_ids_kernel, dim3(blocks), dim3(256), 0, s, ids, active, T, K, first_local, L, out);
    return hipGetLastError();
}

__global__ void fill_i64_kernel(int64_t *p, int64_t v, long n)
{
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
        p[i] = v;
}

hipError_t launch_fill_i64(int64_t *p, int64_t v, long n, hipStream_t s)
{
    if (n <= 0)
        return hipSuccess;
    hipLaunchKernelGGL(fill_i64_kernel, dim3(1), dim3(256), 0, s, p, v, n);
    return hipGetLastError();
}

}  // namespace cam
