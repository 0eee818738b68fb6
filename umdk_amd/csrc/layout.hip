// D1: dispatch layout.  For every (t,k): send_token_idx = number of earlier
// (t',k') in row-major order routed to the same expert (a stable rank), plus
// per-expert and per-rank token counts and the token->rank membership table.
// Restates dispatch_layout.h:112-161 (count, cross-core prefix, rank).
//
// Three launches over token-aligned chunks of at most 256 (t,k) entries:
//   1. layout_hist_kernel: per-chunk expert/rank histograms (LDS atomics;
//      order does not matter for counts) and is_token_in_rank rows, stored
//      transposed: counts[e][chunk].
//   2. layout_scan_kernel: one wave per expert (and per rank) turns its row
//      of chunk counts into exclusive chunk bases (wave prefix scan) and
//      writes the totals.
//   3. layout_rank_kernel: one block per chunk ranks its entries in order:
//      within a wave the lanes sharing an expert are found with one ballot
//      per bit of the expert id, and waves are ordered through per-wave
//      counts in LDS.  No atomics decide an order, so the result is
//      deterministic and identical to the serial loop.
// Expert ids outside [0,E) are not routed: send_token_idx = -1, not counted.
#include "cam_device.h"
#include "launchers.h"
#include "prefill_dev.h"

namespace cam {

constexpr int CHUNK_ENTRIES = 256;
constexpr int HIST_THREADS = 256;
constexpr int RANK_THREADS = 256;
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
                                                                   int E, int R, int Rc, int tpc,
                                                                   int32_t *__restrict__ is_token_in_rank,
                                                                   int32_t *__restrict__ counts)
{
    // Rc = R when per-rank token counts are requested, else 0 (no rank rows, no per-token rank dedup)
    __shared__ int32_t hist[MAX_E + MAX_R];
    int32_t *rhist = hist + E;
    for (int i = threadIdx.x; i < E + Rc; i += HIST_THREADS)
        hist[i] = 0;
    __syncthreads();
    const int c = blockIdx.x, nc = gridDim.x;
    const int t0 = c * tpc, t1 = min(T, t0 + tpc);
    const int per_rank = E / R;
    // entries of the chunk, one per thread (tpc*K <= 256)
    const int i = threadIdx.x;
    const int t = t0 + i / K, k = i % K;
    if (t < t1) {
        const IdxT *row = topk_idx + (size_t)t * K;
        const int64_t e = row[k];
        if (e >= 0 && e < E)
            atomicAdd(&hist[e], 1);
        if (Rc > 0 && e >= 0 && e < E) {
            const int r = (int)e / per_rank;
            bool first = true;
            for (int kk = 0; kk < k; ++kk) {
                const int64_t ee = row[kk];
                if (ee >= 0 && ee < E && (int)ee / per_rank == r)
                    first = false;
            }
            if (first)
                atomicAdd(&rhist[r], 1);
        }
    }
    if (is_token_in_rank) {
        // rows of this chunk's tokens: 0/1 membership, written once each
        for (long q = threadIdx.x; q < (long)(t1 - t0) * R; q += HIST_THREADS) {
            const int tt = t0 + (int)(q / R), r = (int)(q % R);
            const IdxT *row = topk_idx + (size_t)tt * K;
            int in = 0;
            for (int kk = 0; kk < K; ++kk) {
                const int64_t ee = row[kk];
                in |= (ee >= 0 && ee < E && (int)ee / per_rank == r);
            }
            is_token_in_rank[(size_t)tt * R + r] = in;
        }
    }
    __syncthreads();
    for (int q = threadIdx.x; q < E + Rc; q += HIST_THREADS)
        counts[(size_t)q * nc + c] = hist[q];
}

// One wave per counter row (experts, then ranks): exclusive scan over chunks.
__global__ __launch_bounds__(256) void layout_scan_kernel(int E, int R, int nc, int32_t *__restrict__ counts,
                                                          int32_t *__restrict__ ntok_per_expert,
                                                          int32_t *__restrict__ ntok_per_rank)
{
    const int lane = threadIdx.x & 63;
    const int q = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (q >= E + R)
        return;
    int32_t *row = counts + (size_t)q * nc;
    int32_t carry = 0;
    // the first 256 chunks' counts are loaded before any is scanned (one memory round trip for them)
    int32_t pre[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
        pre[u] = u * 64 + lane < nc ? row[u * 64 + lane] : 0;
    for (int c0 = 0; c0 < nc; c0 += 64) {
        const int c = c0 + lane;
        int32_t v = 0;
        if (c0 < 256) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
                v = c0 == u * 64 ? pre[u] : v;
        } else {
            v = c < nc ? row[c] : 0;
        }
        int32_t incl = v;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int32_t u = __shfl_up(incl, o, 64);
            if (lane >= o)
                incl += u;
        }
        if (c < nc)
            row[c] = carry + incl - v;
        carry += __shfl(incl, 63, 64);
    }
    if (lane == 0) {
        if (q < E) {
            if (ntok_per_expert)
                ntok_per_expert[q] = carry;
        } else if (ntok_per_rank) {
            ntok_per_rank[q - E] = carry;
        }
    }
}

template <typename IdxT>
__global__ __launch_bounds__(RANK_THREADS) void layout_rank_kernel(const IdxT *__restrict__ topk_idx, int T, int K,
                                                                   int E, int tpc,
                                                                   const int32_t *__restrict__ chunk_base,
                                                                   int32_t *__restrict__ send_token_idx)
{
    __shared__ int32_t wave_hist[RANK_WAVES][MAX_E];
    __shared__ int32_t base[MAX_E];  // this chunk's exclusive base per expert, loaded beside the ids
    const int c = blockIdx.x, nc = gridDim.x;
    const int w = threadIdx.x >> 6;
    for (int j = threadIdx.x; j < E; j += RANK_THREADS)
        base[j] = chunk_base[(size_t)j * nc + c];
    for (int j = threadIdx.x; j < RANK_WAVES * E; j += RANK_THREADS)
        wave_hist[j / E][j % E] = 0;
    const long i0 = (long)c * tpc * K;
    const long i1 = (long)min(T, (c + 1) * tpc) * K;
    const long i = i0 + threadIdx.x;   // tpc*K <= RANK_THREADS: one entry per thread
    int e = -1;
    if (i < i1) {
        const int64_t v = topk_idx[i];
        e = (v >= 0 && v < E) ? (int)v : -1;
    }
    __syncthreads();  // wave_hist cleared and base loaded
    const bool valid = e >= 0;
    const int nbits = E > 1 ? 32 - __clz(E - 1) : 1;
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
        const bool bit = valid && ((e >> b) & 1);
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    const int inrank = __popcll(peers & lanemask_lt());
    if (valid && inrank == 0)
        wave_hist[w][e] = __popcll(peers);
    __syncthreads();
    if (i < i1) {
        int32_t rank = -1;
        if (valid) {
            rank = base[e] + inrank;
            for (int ww = 0; ww < w; ++ww)
                rank += wave_hist[ww][e];
        }
        send_token_idx[i] = rank;
    }
}

// The prefill step's bookkeeping after route_kernel<.., HIST> (chunks of 16 tokens): one wave per local
// expert (four per block, all blocks in parallel: a single block would be bound by one CU's outstanding
// memory requests) runs scan_expert (prefill_dev.h): chunk bases in place, send offset, count exchange.
constexpr int SN_THREADS = 256;
constexpr int SN_WAVES = SN_THREADS / 64;
__global__ __launch_bounds__(SN_THREADS) void scan_notify_kernel(int E, int nc, int32_t *__restrict__ counts,
                                                                 const int32_t *__restrict__ pref,
                                                                 int32_t *__restrict__ send_offset,
                                                                 int32_t *__restrict__ recv_count,
                                                                 int64_t *__restrict__ tokens_per_expert)
{
    const int e = blockIdx.x * SN_WAVES + (int)(threadIdx.x >> 6);
    if (e >= E)
        return;
    scan_expert(e, nc, counts, pref, send_offset, recv_count, tokens_per_expert);
}

hipError_t launch_scan_notify(int E, int nc, int32_t *counts, const int32_t *pref, int32_t *send_offset,
                              int32_t *recv_count, int64_t *tokens_per_expert, hipStream_t s)
{
    if (E < 1 || E > MAX_E || nc < 1)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(scan_notify_kernel, dim3((E + SN_WAVES - 1) / SN_WAVES), dim3(SN_THREADS), 0, s, E, nc,
                       counts, pref, send_offset, recv_count, tokens_per_expert);
    return hipGetLastError();
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
    int32_t *counts = (int32_t *)ws;
    const int Rc = ntok_per_rank ? R : 0;
    hipLaunchKernelGGL((layout_hist_kernel<IdxT>), dim3(p.n_chunks), dim3(HIST_THREADS), 0, s, topk_idx, T, K, E, R,
                       Rc, p.tokens_per_chunk, is_token_in_rank, counts);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return err;
    hipLaunchKernelGGL(layout_scan_kernel, dim3((E + Rc + 3) / 4), dim3(256), 0, s, E, Rc, p.n_chunks, counts,
                       ntok_per_expert, ntok_per_rank);
    err = hipGetLastError();
    if (err != hipSuccess)
        return err;
    hipLaunchKernelGGL((layout_rank_kernel<IdxT>), dim3(p.n_chunks), dim3(RANK_THREADS), 0, s, topk_idx, T, K, E,
                       p.tokens_per_chunk, counts, send_token_idx);
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

namespace cam {

// Decode-sized fused bookkeeping (T*K <= 8192 entries): one block of 1024 threads does what
// prepare_ids + the three layout launches + the count exchange do for the prefill path:
//   ids_eff[t,k] = expert id if the token is active and the id is in [0,E), else -1;
//   send_token_idx = stable rank within the expert (same ballot ranking as layout_rank_kernel,
//   1024 entries per round, rounds in order); counts, exclusive offsets, inclusive recv_count,
//   int64 tokens per expert and the total.
constexpr int SMALL_THREADS = 1024;
constexpr int SMALL_WAVES = SMALL_THREADS / 64;

__global__ __launch_bounds__(SMALL_THREADS) void layout_small_kernel(
    const int32_t *__restrict__ ids, const uint8_t *__restrict__ active, int T, int K, int E,
    int32_t *__restrict__ ids_eff, int32_t *__restrict__ counts, int32_t *__restrict__ sti,
    int32_t *__restrict__ send_offset, int32_t *__restrict__ recv_count, int32_t *__restrict__ total,
    int64_t *__restrict__ tokens_per_expert, int32_t *__restrict__ zero, int nzero)
{
    for (int i = threadIdx.x; i < nzero; i += SMALL_THREADS)
        zero[i] = 0;
    __shared__ int32_t run[MAX_E];
    __shared__ int32_t wave_hist[SMALL_WAVES][MAX_E];
    __shared__ int32_t wsum[SMALL_WAVES];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int TK = T * K;
    for (int e = tid; e < E; e += SMALL_THREADS)
        run[e] = 0;
    const int nbits = E > 1 ? 32 - __clz(E - 1) : 1;
    const uint64_t lt = lanemask_lt();
    for (int base = 0; base < TK; base += SMALL_THREADS) {
        for (int j = tid; j < SMALL_WAVES * E; j += SMALL_THREADS)
            wave_hist[j / E][j % E] = 0;
        __syncthreads();
        const int i = base + tid;
        int e = -1;
        if (i < TK) {
            const int id = ids[i];
            const bool on = (active == nullptr || active[i / K] != 0) && id >= 0 && id < E;
            e = on ? id : -1;
            ids_eff[i] = e;
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
        if (i < TK) {
            int32_t r = -1;
            if (valid) {
                r = run[e] + inrank;
                for (int ww = 0; ww < w; ++ww)
                    r += wave_hist[ww][e];
            }
            sti[i] = r;
        }
        __syncthreads();
        for (int ee = tid; ee < E; ee += SMALL_THREADS) {
            int32_t sacc = 0;
#pragma unroll
            for (int ww = 0; ww < SMALL_WAVES; ++ww)
                sacc += wave_hist[ww][ee];
            run[ee] += sacc;
        }
        __syncthreads();
    }
    // count exchange of one rank: exclusive / inclusive prefix over the experts
    const int c = tid < E ? run[tid] : 0;
    int32_t v = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int32_t u = __shfl_up(v, o, 64);
        if (lane >= o)
            v += u;
    }
    if (lane == 63)
        wsum[w] = v;
    __syncthreads();
    int32_t before = 0;
    for (int ww = 0; ww < w; ++ww)
        before += wsum[ww];
    const int32_t incl = before + v;
    if (tid < E) {
        counts[tid] = c;
        send_offset[tid] = incl - c;
        recv_count[tid] = incl;
        tokens_per_expert[tid] = c;
        if (tid == E - 1)
            *total = incl;
    }
}

hipError_t launch_layout_small(const int32_t *ids, const uint8_t *active, int T, int K, int E, int32_t *ids_eff,
                               int32_t *counts, int32_t *sti, int32_t *send_offset, int32_t *recv_count,
                               int32_t *total, int64_t *tokens_per_expert, hipStream_t s, int32_t *zero,
                               int nzero)
{
    if (T * K > 8192 || E > MAX_E || E > SMALL_THREADS || nzero < 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(layout_small_kernel, dim3(1), dim3(SMALL_THREADS), 0, s, ids, active, T, K, E, ids_eff, counts,
                       sti, send_offset, recv_count, total, tokens_per_expert, zero, nzero);
    return hipGetLastError();
}

}  // namespace cam
