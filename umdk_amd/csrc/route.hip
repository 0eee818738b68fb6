// R0: top-K routing kernels over chunks of 16 tokens; the routing itself (16-lane rows, DPP max reductions
// over order-preserving score keys, ties to the lower expert id, renormalised softmax gates) is route_block in
// prefill_dev.h.  There is no reference routing kernel (callers pass topk_idx; see
// src/cam/examples/moe_dispatch_combine_prefill_sample.py:87-93).
#include "cam_device.h"
#include "launchers.h"
#include "prefill_dev.h"

namespace cam {

// The routing kernels: one block per chunk of 16 tokens (route_block in prefill_dev.h).
template <int PER, bool HIST = false>
__global__ __launch_bounds__(ROUTE_WAVES * 64) void route_kernel(const float *__restrict__ logits,
                                                                 const float *__restrict__ bias, int T, int E,
                                                                 int K, int32_t *__restrict__ topk_idx,
                                                                 float *__restrict__ topk_w,
                                                                 int64_t *__restrict__ topk_idx64,
                                                                 int Ec = 0, int32_t *__restrict__ chunk_counts = nullptr,
                                                                 int32_t *__restrict__ chunk_pref = nullptr,
                                                                 int32_t *__restrict__ chunk_rank = nullptr)
{
    route_block<PER, HIST>(logits, bias, T, E, K, topk_idx, topk_w, topk_idx64, Ec, chunk_counts, chunk_pref,
                           chunk_rank, (int)blockIdx.x, (int)gridDim.x);
}

hipError_t launch_route(const float *logits, const float *bias, int T, int E, int K, int32_t *topk_idx,
                        float *topk_w, hipStream_t s, int64_t *topk_idx64)
{
    if (T == 0)
        return hipSuccess;
    if (E > 16 * ROUTE_MAX_PER_LANE || K > 16)
        return hipErrorInvalidValue;
    const int tokens_per_block = ROUTE_WAVES * 4;
    const int grid = (T + tokens_per_block - 1) / tokens_per_block;
    const dim3 g(grid), b(ROUTE_WAVES * 64);
    const int per = (E + 15) >> 4;
    if (per <= 1)
        hipLaunchKernelGGL(route_kernel<1>, g, b, 0, s, logits, bias, T, E, K, topk_idx, topk_w, topk_idx64);
    else if (per <= 2)
        hipLaunchKernelGGL(route_kernel<2>, g, b, 0, s, logits, bias, T, E, K, topk_idx, topk_w, topk_idx64);
    else if (per <= 4)
        hipLaunchKernelGGL(route_kernel<4>, g, b, 0, s, logits, bias, T, E, K, topk_idx, topk_w, topk_idx64);
    else if (per <= 8)
        hipLaunchKernelGGL(route_kernel<8>, g, b, 0, s, logits, bias, T, E, K, topk_idx, topk_w, topk_idx64);
    else if (per <= 16)
        hipLaunchKernelGGL(route_kernel<16>, g, b, 0, s, logits, bias, T, E, K, topk_idx, topk_w, topk_idx64);
    else
        hipLaunchKernelGGL(route_kernel<32>, g, b, 0, s, logits, bias, T, E, K, topk_idx, topk_w, topk_idx64);
    return hipGetLastError();
}

int route_tokens_per_block() { return ROUTE_WAVES * 4; }

hipError_t launch_route_hist(const float *logits, const float *bias, int T, int E, int K, int Ec, int32_t *topk_idx,
                             float *topk_w, int32_t *chunk_counts, int32_t *chunk_pref, int32_t *chunk_rank,
                             hipStream_t s)
{
    if (T == 0)
        return hipSuccess;
    if (E > 16 * ROUTE_MAX_PER_LANE || K > 16 || Ec > E || Ec < 1 || !chunk_rank)
        return hipErrorInvalidValue;
    const int grid = (T + ROUTE_WAVES * 4 - 1) / (ROUTE_WAVES * 4);
    const dim3 g(grid), b(ROUTE_WAVES * 64);
    const int per = (E + 15) >> 4;
#define ROUTE_HIST_CASE(P)                                                                                          \
    hipLaunchKernelGGL((route_kernel<P, true>), g, b, 0, s, logits, bias, T, E, K, topk_idx, topk_w, nullptr, Ec,   \
                       chunk_counts, chunk_pref, chunk_rank)
    if (per <= 1)
        ROUTE_HIST_CASE(1);
    else if (per <= 2)
        ROUTE_HIST_CASE(2);
    else if (per <= 4)
        ROUTE_HIST_CASE(4);
    else if (per <= 8)
        ROUTE_HIST_CASE(8);
    else if (per <= 16)
        ROUTE_HIST_CASE(16);
    else
        ROUTE_HIST_CASE(32);
#undef ROUTE_HIST_CASE
    return hipGetLastError();
}

}  // namespace cam
