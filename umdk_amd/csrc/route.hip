// R0: top-K routing.  One wave per token; experts are spread over the 64
// lanes (lane l holds experts l, l+64, ...).  Each of the K rounds is a wave
// arg-max on (score, -index), so ties go to the lower expert id.  Gates are
// softmax(logits) at the selected experts, renormalised over the K picks:
// w_k = exp(l_k - max_l) / sum_j exp(l_j - max_l), summed in pick order.
// There is no reference routing kernel (callers pass topk_idx; see
// src/cam/examples/moe_dispatch_combine_prefill_sample.py:87-93).
#include "cam_device.h"
#include "launchers.h"

namespace cam {

constexpr int ROUTE_MAX_PER_LANE = 8;  // E <= 512
constexpr int ROUTE_WAVES = 4;

__global__ __launch_bounds__(ROUTE_WAVES * 64) void route_kernel(const float *__restrict__ logits,
                                                                 const float *__restrict__ bias, int T, int E,
                                                                 int K, int32_t *__restrict__ topk_idx,
                                                                 float *__restrict__ topk_w)
{
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * ROUTE_WAVES + (threadIdx.x >> 6);
    if (t >= T)
        return;
    const float *l = logits + (size_t)t * E;
    float lg[ROUTE_MAX_PER_LANE], sc[ROUTE_MAX_PER_LANE];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < ROUTE_MAX_PER_LANE; ++j) {
        const int e = lane + 64 * j;
        if (e < E) {
            lg[j] = l[e];
            sc[j] = bias ? lg[j] + bias[e] : lg[j];
            mx = fmaxf(mx, lg[j]);
        } else {
            lg[j] = 0.0f;
            sc[j] = -INFINITY;
        }
    }
    mx = group_max<64>(mx);
    uint32_t taken = 0;  // bit j: expert lane+64j already picked
    float my_ex = 0.0f;  // lane k keeps the k-th pick's exp
    int my_idx = 0;
    for (int k = 0; k < K; ++k) {
        float bs = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < ROUTE_MAX_PER_LANE; ++j) {
            const int e = lane + 64 * j;
            if (e < E && !(taken & (1u << j)) && (sc[j] > bs || bi == 0x7fffffff)) {
                bs = sc[j];
                bi = e;
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float os = __shfl_xor(bs, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (oi != 0x7fffffff && (bi == 0x7fffffff || os > bs || (os == bs && oi < bi))) {
                bs = os;
                bi = oi;
            }
        }
        // owner lane marks it taken and evaluates the exponent
        float ex = 0.0f;
        if ((bi & 63) == lane) {
            const int j = bi >> 6;
#pragma unroll
            for (int jj = 0; jj < ROUTE_MAX_PER_LANE; ++jj)
                if (jj == j) {
                    taken |= 1u << jj;
                    ex = expf(lg[jj] - mx);
                }
        }
        ex = __shfl(ex, bi & 63, 64);
        if (lane == k) {
            my_ex = ex;
            my_idx = bi;
        }
    }
    // sum of the K exponents in pick order
    float denom = 0.0f;
    for (int k = 0; k < K; ++k)
        denom += __shfl(my_ex, k, 64);
    if (lane < K) {
        topk_idx[(size_t)t * K + lane] = my_idx;
        topk_w[(size_t)t * K + lane] = my_ex / denom;
    }
}

hipError_t launch_route(const float *logits, const float *bias, int T, int E, int K, int32_t *topk_idx,
                        float *topk_w, hipStream_t s)
{
    if (T == 0)
        return hipSuccess;
    const int grid = (T + ROUTE_WAVES - 1) / ROUTE_WAVES;
    hipLaunchKernelGGL(route_kernel, dim3(grid), dim3(ROUTE_WAVES * 64), 0, s, logits, bias, T, E, K, topk_idx,
                       topk_w);
    return hipGetLastError();
}

}  // namespace cam
