// R0: top-K routing.  A token is handled by a 16-lane row of a wave (four
// tokens per wave); lane l of the row holds experts l, l+16, l+32, ...
// Each (score, expert) pair is a 64-bit key: the score's bits mapped to an
// order-preserving unsigned integer, then ~expert, so the largest key is the
// largest score with ties going to the lower expert id.  Each of the K
// rounds takes the row-wide maximum of the score part, then of ~expert over
// the lanes holding that score, each with four DPP max steps (quad xor 1,
// quad xor 2, half-row mirror, row mirror; no LDS traffic, no branches), and
// the owning lane retires that expert by zeroing its key.
// Gates are softmax(logits) at the picks renormalised over the K picks:
// w_k = exp(l_k - max_l) / sum_j exp(l_j - max_l), summed in pick order.
// There is no reference routing kernel (callers pass topk_idx; see
// src/cam/examples/moe_dispatch_combine_prefill_sample.py:87-93).
#include "cam_device.h"
#include "launchers.h"

namespace cam {

constexpr int ROUTE_WAVES = 4;
constexpr int ROUTE_MAX_PER_LANE = 32;  // E <= 512 over 16 lanes

// dpp_ctrl codes (GCN/CDNA DPP): quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror
constexpr int DPP_QUAD_XOR1 = 0xB1;
constexpr int DPP_QUAD_XOR2 = 0x4E;
constexpr int DPP_HALF_MIRROR = 0x141;
constexpr int DPP_MIRROR = 0x140;

template <int CTRL> __device__ __forceinline__ uint32_t dpp(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

template <int CTRL> __device__ __forceinline__ uint32_t umax_step(uint32_t v)
{
    return max(v, dpp<CTRL>(v));
}

template <int CTRL> __device__ __forceinline__ float fmax_step(float v)
{
    return fmaxf(v, __uint_as_float(dpp<CTRL>(__float_as_uint(v))));
}

__device__ __forceinline__ uint32_t order_key(float s)
{
    const uint32_t u = __float_as_uint(s);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// HIST: the block's 16 tokens are one layout chunk; it also writes the chunk's histogram of the picked
// ids below Ec (the local experts), chunk_counts[e * gridDim.x + blockIdx.x] for every e < Ec, the chunk's
// exclusive prefix of that histogram over the experts, chunk_pref[e * gridDim.x + blockIdx.x] (summed over the
// chunks it is expert e's offset among the received rows, so no step after this launch needs every expert's
// total), and each such
// pick's rank among the chunk's picks of the same expert in (t,k) order, chunk_rank[t * K + k].  A token's K
// picks are distinct experts, so that rank is the number of earlier tokens of the chunk that picked the
// expert: each expert gets a 16-bit mask of the chunk's tokens that picked it (an LDS atomic OR, which no
// order of the ORs changes), the rank is the popcount of the mask below the token, the count that of the
// whole mask.
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
    const int lane = threadIdx.x & 63;
    const int l16 = lane & 15;
    const int t = (blockIdx.x * ROUTE_WAVES + (threadIdx.x >> 6)) * 4 + (lane >> 4);
    const bool live = t < T;  // dead rows still run the DPP steps (they read only their own row)
    const float *l = logits + (size_t)(live ? t : 0) * E;
    uint32_t khi[PER];
    float lg[PER], bs[PER];
    // loads first, all unconditional (clamped index) so they are in flight together
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = min(l16 + 16 * j, E - 1);
        lg[j] = l[e];
        bs[j] = bias ? bias[e] : 0.0f;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const bool valid = live && l16 + 16 * j < E;
        // + 0.0f turns -0.0 into +0.0, so the integer key orders zeros as a float compare does
        const float sc = (bias ? lg[j] + bs[j] : lg[j]) + 0.0f;
        mx = valid ? fmaxf(mx, lg[j]) : mx;
        khi[j] = valid ? order_key(sc) : 0u;
    }
    mx = fmax_step<DPP_QUAD_XOR1>(mx);
    mx = fmax_step<DPP_QUAD_XOR2>(mx);
    mx = fmax_step<DPP_HALF_MIRROR>(mx);
    mx = fmax_step<DPP_MIRROR>(mx);

    int my_idx = 0;
#pragma unroll 1
    for (int k = 0; k < K; ++k) {
        // row-wide best score key, then the lowest expert id holding it (picked slots are zeroed):
        // two branch-free 32-bit max reductions instead of one 64-bit one
        uint32_t hi = 0;
#pragma unroll
        for (int j = 0; j < PER; ++j)
            hi = max(hi, khi[j]);
        hi = umax_step<DPP_QUAD_XOR1>(hi);
        hi = umax_step<DPP_QUAD_XOR2>(hi);
        hi = umax_step<DPP_HALF_MIRROR>(hi);
        hi = umax_step<DPP_MIRROR>(hi);
        int jb = PER;  // this lane's lowest slot holding the row maximum (slots ascend in expert id)
#pragma unroll
        for (int j = PER - 1; j >= 0; --j)
            jb = khi[j] == hi ? j : jb;
        uint32_t lo = (hi != 0 && jb < PER) ? ~(uint32_t)(l16 + 16 * jb) : 0u;
        lo = umax_step<DPP_QUAD_XOR1>(lo);
        lo = umax_step<DPP_QUAD_XOR2>(lo);
        lo = umax_step<DPP_HALF_MIRROR>(lo);
        lo = umax_step<DPP_MIRROR>(lo);
        const int best = (int)~lo;
        const int clear = (best & 15) == l16 ? best >> 4 : -1;
#pragma unroll
        for (int j = 0; j < PER; ++j)
            khi[j] = j == clear ? 0u : khi[j];
        if (l16 == k)
            my_idx = best;
    }
    float my_ex = 0.0f;
    if (l16 < K && live)
        my_ex = expf(l[my_idx] - mx);
    float denom = 0.0f;
    for (int k = 0; k < K; ++k)
        denom += __shfl(my_ex, (lane & 48) | k, 64);
    if (l16 < K && live) {
        topk_idx[(size_t)t * K + l16] = my_idx;
        topk_w[(size_t)t * K + l16] = my_ex / denom;
        if (topk_idx64)
            topk_idx64[(size_t)t * K + l16] = my_idx;
    }
    if constexpr (HIST) {
        static_assert(ROUTE_WAVES * 4 <= 32, "a chunk's tokens fit a 32-bit mask");
        __shared__ uint32_t picked[ROUTE_MAX_PER_LANE * 16];  // per expert: the chunk's tokens that picked it
        for (int e = threadIdx.x; e < Ec; e += ROUTE_WAVES * 64)
            picked[e] = 0u;
        __syncthreads();
        const int tl = t - blockIdx.x * ROUTE_WAVES * 4;  // the token's place in the chunk
        const bool local = l16 < K && live && my_idx < Ec;
        if (local)
            atomicOr(&picked[my_idx], 1u << tl);
        __syncthreads();
        if (local)
            chunk_rank[(size_t)t * K + l16] = __popc(picked[my_idx] & ((1u << tl) - 1u));
        // the histogram, and its exclusive prefix over the experts: thread i owns experts [i PE, (i + 1) PE)
        constexpr int NT = ROUTE_WAVES * 64, PE = (ROUTE_MAX_PER_LANE * 16 + NT - 1) / NT;
        __shared__ int32_t wsum[ROUTE_WAVES];
        int cnt[PE], own = 0;
#pragma unroll
        for (int q = 0; q < PE; ++q) {
            const int e = threadIdx.x * PE + q;
            cnt[q] = e < Ec ? __popc(picked[e]) : 0;
            own += cnt[q];
        }
        int incl = own;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int u = __shfl_up(incl, o, 64);
            if (lane >= o)
                incl += u;
        }
        if (lane == 63)
            wsum[threadIdx.x >> 6] = incl;
        __syncthreads();
        int run = incl - own;
        for (int v = 0; v < (int)(threadIdx.x >> 6); ++v)
            run += wsum[v];
#pragma unroll
        for (int q = 0; q < PE; ++q) {
            const int e = threadIdx.x * PE + q;
            if (e < Ec) {
                chunk_counts[(size_t)e * gridDim.x + blockIdx.x] = cnt[q];
                chunk_pref[(size_t)e * gridDim.x + blockIdx.x] = run;
            }
            run += cnt[q];
        }
    }
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
