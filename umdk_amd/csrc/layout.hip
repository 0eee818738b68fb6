// D1: dispatch layout.  For every (t,k): send_token_idx = number of earlier
// (t',k') in row-major order routed to the same expert (a stable rank), plus
// per-expert and per-rank token counts and the token->rank membership table.
// Restates dispatch_layout.h:112-161 (count, cross-core prefix, rank).
//
// Two launches over token-aligned chunks of about 1024 (t,k) entries:
//   1. layout_hist_kernel: per-chunk expert/rank histograms (LDS atomics;
//      order does not matter for counts) and is_token_in_rank rows.
//   2. layout_rank_kernel: each chunk sums the histograms of the chunks
//      before it (its per-expert base), then ranks its entries in order,
//      512 at a time: within a wave the lanes sharing an expert are found
//      with one ballot per bit of the expert id, and waves are ordered
//      through per-wave counts in LDS.  No atomics decide an order, so the
//      result is deterministic and identical to the serial loop.
// Expert ids outside [0,E) are not routed: send_token_idx = -1, not counted.
#include "cam_device.h"
#include "launchers.h"

namespace cam {

constexpr int CHUNK_ENTRIES = 1024;
constexpr int HIST_THREADS = 256;
constexpr int RANK_THREADS = 512;
constexpr int RANK_WAVES = RANK_THREADS / 64;
constexpr int MAX_E = 512;
constexpr int MAX_R = 384;

LayoutPlan layout_plan(int T, int K)
{
    LayoutPlan p;
    p.tokens_per_chunk = CHUNK_ENTRIES / K > 0 ? CHUNK_ENTRIES / K : 1;
    p.n_chunks = T > 0 ? (T + p.tokens_per_chunk - 1) / p.tokens_per_chunk : 0;
    return p;
}

size_t layout_workspace_bytes(int T, int K, int E, int R)
{
    LayoutPlan p = layout_plan(T, K);
    return sizeof(int32_t) * (size_t)p.n_chunks * (size_t)(E + R);
}

template <typename IdxT>
__global__ __launch_bounds__(HIST_THREADS) void layout_hist_kernel(const IdxT *__restrict__ topk_idx, int T, int K,
                                                                   int E, int R, int tpc,
                                                                   int32_t *__restrict__ is_token_in_rank,
                                                                   int32_t *__restrict__ chunk_counts)
{
    __shared__ int32_t hist[MAX_E + MAX_R];
    int32_t *rhist = hist + E;
    for (int i = threadIdx.x; i < E + R; i += HIST_THREADS)
        hist[i] = 0;
    __syncthreads();
    const int c = blockIdx.x;
    const int t0 = c * tpc, t1 = min(T, t0 + tpc);
    const int per_rank = E / R;
    for (int t = t0 + threadIdx.x; t < t1; t += HIST_THREADS) {
        const IdxT *row = topk_idx + (size_t)t * K;
        if (is_token_in_rank)
            for (int r = 0; r < R; ++r)
                is_token_in_rank[(size_t)t * R + r] = 0;
        for (int k = 0; k < K; ++k) {
            const int64_t e = row[k];
            if (e < 0 || e >= E)
                continue;
            atomicAdd(&hist[e], 1);
            const int r = (int)e / per_rank;
            bool first = true;
            for (int kk = 0; kk < k; ++kk) {
                const int64_t ee = row[kk];
                if (ee >= 0 && ee < E && (int)ee / per_rank == r)
                    first = false;
            }
            if (first) {
                atomicAdd(&rhist[r], 1);
                if (is_token_in_rank)
                    is_token_in_rank[(size_t)t * R + r] = 1;
            }
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < E + R; i += HIST_THREADS)
        chunk_counts[(size_t)c * (E + R) + i] = hist[i];
}

template <typename IdxT>
__global__ __launch_bounds__(RANK_THREADS) void layout_rank_kernel(const IdxT *__restrict__ topk_idx, int T, int K,
                                                                   int E, int R, int tpc,
                                                                   const int32_t *__restrict__ chunk_counts,
                                                                   int32_t *__restrict__ ntok_per_expert,
                                                                   int32_t *__restrict__ ntok_per_rank,
                                                                   int32_t *__restrict__ send_token_idx)
{
    __shared__ int32_t run[MAX_E];
    __shared__ int32_t wave_hist[RANK_WAVES][MAX_E];
    const int c = blockIdx.x;
    const int nc = gridDim.x;
    const int ER = E + R;
    for (int e = threadIdx.x; e < E; e += RANK_THREADS) {
        int32_t base = 0;
        for (int cc = 0; cc < c; ++cc)
            base += chunk_counts[(size_t)cc * ER + e];
        run[e] = base;
        if (c == nc - 1 && ntok_per_expert)
            ntok_per_expert[e] = base + chunk_counts[(size_t)c * ER + e];
    }
    if (c == nc - 1 && ntok_per_rank)
        for (int r = threadIdx.x; r < R; r += RANK_THREADS) {
            int32_t tot = 0;
            for (int cc = 0; cc < nc; ++cc)
                tot += chunk_counts[(size_t)cc * ER + E + r];
            ntok_per_rank[r] = tot;
        }
    const int nbits = E > 1 ? 32 - __clz(E - 1) : 1;
    const int w = threadIdx.x >> 6;
    const uint64_t lt = lanemask_lt();
    const long i0 = (long)c * tpc * K;
    const long i1 = (long)min(T, (c + 1) * tpc) * K;
    for (long base = i0; base < i1; base += RANK_THREADS) {
        for (int j = threadIdx.x; j < RANK_WAVES * E; j += RANK_THREADS)
            (&wave_hist[0][0])[(j / E) * MAX_E + (j % E)] = 0;
        __syncthreads();
        const long i = base + threadIdx.x;
        int e = -1;
        if (i < i1) {
            const int64_t v = topk_idx[i];
            e = (v >= 0 && v < E) ? (int)v : -1;
        }
        const bool valid = e >= 0;
        uint64_t peers = __ballot(valid);
        for (int b = 0; b < nbits; ++b) {
            const bool bit = valid && ((e >> b) & 1);
            const uint64_t m = __ballot(bit);
            peers &= bit ? m : ~m;
        }
        const int inrank = __popcll(peers & lt);
        if (valid && inrank == 0)
            wave_hist[w][e] = __popcll(peers);
        __syncthreads();
        if (i < i1) {
            int32_t rank = -1;
            if (valid) {
                rank = run[e] + inrank;
                for (int ww = 0; ww < w; ++ww)
                    rank += wave_hist[ww][e];
            }
            send_token_idx[i] = rank;
        }
        __syncthreads();
        for (int ee = threadIdx.x; ee < E; ee += RANK_THREADS) {
            int32_t s = 0;
#pragma unroll
            for (int ww = 0; ww < RANK_WAVES; ++ww)
                s += wave_hist[ww][ee];
            run[ee] += s;
        }
        __syncthreads();
    }
}

template <typename IdxT>
static hipError_t layout_impl(const IdxT *topk_idx, int T, int K, int E, int R, int32_t *ntok_per_rank,
                              int32_t *ntok_per_expert, int32_t *is_token_in_rank, int32_t *send_token_idx, void *ws,
                              hipStream_t s)
{
    LayoutPlan p = layout_plan(T, K);
    if (p.n_chunks == 0) {
        // no tokens: counts are all zero (a fill kernel, never a memset node,
        // so the launch stays safe under graph capture)
        hipError_t err = hipSuccess;
        if (ntok_per_expert)
            err = launch_fill_i32(ntok_per_expert, 0, E, s);
        if (err == hipSuccess && ntok_per_rank)
            err = launch_fill_i32(ntok_per_rank, 0, R, s);
        return err;
    }
    int32_t *chunk_counts = (int32_t *)ws;
    hipLaunchKernelGGL((layout_hist_kernel<IdxT>), dim3(p.n_chunks), dim3(HIST_THREADS), 0, s, topk_idx, T, K, E, R,
                       p.tokens_per_chunk, is_token_in_rank, chunk_counts);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return err;
    hipLaunchKernelGGL((layout_rank_kernel<IdxT>), dim3(p.n_chunks), dim3(RANK_THREADS), 0, s, topk_idx, T, K, E, R,
                       p.tokens_per_chunk, chunk_counts, ntok_per_expert, ntok_per_rank, send_token_idx);
    return hipGetLastError();
}

hipError_t launch_layout(const int64_t *topk_idx, int T, int K, int E, int R, int32_t *ntok_per_rank,
                         int32_t *ntok_per_expert, int32_t *is_token_in_rank, int32_t *send_token_idx, void *ws,
                         hipStream_t s)
{
    return layout_impl<int64_t>(topk_idx, T, K, E, R, ntok_per_rank, ntok_per_expert, is_token_in_rank,
                                send_token_idx, ws, s);
}

hipError_t launch_layout_i32(const int32_t *topk_idx, int T, int K, int E, int32_t *ntok_per_expert,
                             int32_t *send_token_idx, void *ws, hipStream_t s)
{
    return layout_impl<int32_t>(topk_idx, T, K, E, 1, nullptr, ntok_per_expert, nullptr, send_token_idx, ws, s);
}

}  // namespace cam
