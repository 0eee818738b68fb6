// D2: the count exchange of notify_dispatch for a single rank, plus a fill
// utility.  With one rank the all-to-all of (count, offset, numTokens)
// triples (notify_dispatch.h:163-254) is the identity, so only the builders
// remain:
//   send_offset[e]            = exclusive prefix of counts (notify_dispatch.h:143-152)
//   recv_count[e]             = inclusive prefix, expert-major (notify_dispatch.h:340-360)
//   recv_offset[e]            = the sender's send_offset[e]
//   total_recv, max_bs        = sum of counts, numTokens
//   recv_tokens_per_expert[l] = counts as int64 (notify_dispatch.h:389-412)
#include "cam_device.h"
#include "launchers.h"

namespace cam {

constexpr int NOTIFY_THREADS = 512;  // one thread per expert, E <= 512

__global__ void fill_i32_kernel(int32_t *p, int32_t v, long n)
{
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
        p[i] = v;
}

hipError_t launch_fill_i32(int32_t *p, int32_t v, long n, hipStream_t s)
{
    if (n <= 0)
        return hipSuccess;
    long blocks = (n + 255) / 256;
    if (blocks > 4096)
        blocks = 4096;
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p, v, n);
    return hipGetLastError();
}

__global__ __launch_bounds__(NOTIFY_THREADS) void notify_kernel(const int32_t *__restrict__ counts, int E, int T,
                                                                int32_t *send_offset, int32_t *total_recv,
                                                                int32_t *recv_count, int32_t *recv_offset,
                                                                int32_t *max_bs, int64_t *recv_tokens_per_expert,
                                                                int local_experts)
{
    __shared__ int32_t wave_sum[NOTIFY_THREADS / 64];
    const int e = threadIdx.x;
    const int lane = e & 63, w = e >> 6;
    const int32_t c = e < E ? counts[e] : 0;
    // inclusive scan within the wave
    int32_t v = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int32_t u = __shfl_up(v, o, 64);
        if (lane >= o)
            v += u;
    }
    if (lane == 63)
        wave_sum[w] = v;
    __syncthreads();
    int32_t before = 0;
    for (int ww = 0; ww < w; ++ww)
        before += wave_sum[ww];
    const int32_t incl = before + v;
    if (e < E) {
        send_offset[e] = incl - c;
        if (recv_offset)
            recv_offset[e] = incl - c;
        if (recv_count)
            recv_count[e] = incl;
        if (recv_tokens_per_expert && e < local_experts)
            recv_tokens_per_expert[e] = c;
    }
    if (e == E - 1) {
        if (total_recv)
            *total_recv = incl;
        if (max_bs)
            *max_bs = T;
    }
}

hipError_t launch_notify(const int32_t *counts, int E, int T, int32_t *send_offset, int32_t *total_recv,
                         int32_t *recv_count, int32_t *recv_offset, int32_t *max_bs, int64_t *recv_tokens_per_expert,
                         int local_experts, hipStream_t s)
{
    hipLaunchKernelGGL(notify_kernel, dim3(1), dim3(NOTIFY_THREADS), 0, s, counts, E, T, send_offset, total_recv,
                       recv_count, recv_offset, max_bs, recv_tokens_per_expert, local_experts);
    return hipGetLastError();
}

}  // namespace cam
