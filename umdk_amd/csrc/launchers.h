// Internal host launchers, one per kernel family.  Not exported: the public
// surface is the two-phase C ABI in include/camhip.h (implemented in api.cpp).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cam {

// QUANT_INT8_FUSED: the fused decode op's int8 recipe (no epsilon, optional smooth scales); internal only
enum QuantMode { QUANT_NONE = 0, QUANT_INT8_TOKEN = 2, QUANT_FP8_BLOCK = 3, QUANT_INT8_FUSED = 4 };

// ---- routing (route.hip)
// topk_idx64 (optional): the same ids as int64, the layout op's input type
hipError_t launch_route(const float *logits, const float *bias, int T, int E, int K, int32_t *topk_idx,
                        float *topk_w, hipStream_t s, int64_t *topk_idx64 = nullptr);

// routing that also writes per-chunk histograms of the ids below Ec: chunks of route_tokens_per_block() tokens,
// chunk_counts[e * nc + c], each chunk's exclusive prefix of its histogram over the experts, chunk_pref[e * nc +
// c], and each such pick's rank among its chunk's picks of the same expert, chunk_rank[t * K + k] (the prefill
// step)
int route_tokens_per_block();
hipError_t launch_route_hist(const float *logits, const float *bias, int T, int E, int K, int Ec, int32_t *topk_idx,
                             float *topk_w, int32_t *chunk_counts, int32_t *chunk_pref, int32_t *chunk_rank,
                             hipStream_t s);

// ---- dispatch layout (layout.hip)
struct LayoutPlan {
    int tokens_per_chunk;
    int n_chunks;
};
LayoutPlan layout_plan(int T, int K);
size_t layout_workspace_bytes(int T, int K, int E, int R);
hipError_t launch_layout(const int64_t *topk_idx, int T, int K, int E, int R, int32_t *ntok_per_rank,
                         int32_t *ntok_per_expert, int32_t *is_token_in_rank, int32_t *send_token_idx,
                         void *ws, hipStream_t s);
// the prefill step: chunk counts [E][nc] -> exclusive chunk bases in place, and the one-rank count exchange from
// the row totals and the summed chunk prefixes [E][nc] of launch_route_hist
hipError_t launch_scan_notify(int E, int nc, int32_t *counts, const int32_t *pref, int32_t *send_offset,
                              int32_t *recv_count, int64_t *tokens_per_expert, hipStream_t s);
// int32 topk ids, used by the fused path
hipError_t launch_layout_i32(const int32_t *topk_idx, int T, int K, int E, int32_t *ntok_per_expert,
                             int32_t *send_token_idx, void *ws, hipStream_t s);

// decode-sized layout + count exchange in one launch (T*K <= 8192; ids masked by `active`); it also zeroes
// zero[0, nzero) (a later launch's counters)
hipError_t launch_layout_small(const int32_t *ids, const uint8_t *active, int T, int K, int E, int32_t *ids_eff,
                               int32_t *counts, int32_t *sti, int32_t *send_offset, int32_t *recv_count,
                               int32_t *total, int64_t *tokens_per_expert, hipStream_t s, int32_t *zero = nullptr,
                               int nzero = 0);

// ---- small utilities (notify.hip)
hipError_t launch_fill_i32(int32_t *p, int32_t v, long n, hipStream_t s);

// ---- count exchange for one rank (notify.hip)
hipError_t launch_notify(const int32_t *counts, int E, int T, int32_t *send_offset, int32_t *total_recv,
                         int32_t *recv_count, int32_t *recv_offset, int32_t *max_bs,
                         int64_t *recv_tokens_per_expert, int local_experts, hipStream_t s);

// ---- permute + quantise (dispatch.hip); topk_idx == nullptr: identity rows (K must be 1)
hipError_t launch_dispatch(const uint16_t *x, const int32_t *topk_idx, const int32_t *send_offset,
                           const int32_t *send_token_idx, int T, int H, int K, int E, int rank, int cap, int quant_mode,
                           void *expand_x, float *scales, int32_t *expand_idx, hipStream_t s,
                           int32_t *inv_out = nullptr, const float *smooth = nullptr, bool kmajor_scales = false,
                           const int32_t *chunk_base = nullptr, int tpc = 0, const int32_t *chunk_rank = nullptr,
                           bool skip_unrouted = false);
// decode sizes (dispatch_decode_fits: T*K <= 2048, E <= 512; bf16 or fp8 rows): layout + count exchange +
// dispatch as one launch (the arguments of launch_layout_small and launch_dispatch; the ranks and effective ids
// stay in LDS)
hipError_t launch_dispatch_decode(const int32_t *ids, const uint8_t *active, const uint16_t *x, int T, int H, int K,
                                  int E, int cap, int quant_mode, void *expand_x, float *scales, int32_t *expand_idx,
                                  int32_t *inv_out, bool kmajor_scales, int32_t *counts, int32_t *send_offset,
                                  int32_t *recv_count, int32_t *total, int64_t *tokens_per_expert, hipStream_t s,
                                  int32_t *zero, int nzero);
bool dispatch_decode_fits(int T, int K, int E);
// (send_token_idx == nullptr: the rank within the expert is chunk_base[e * nc + t / tpc] plus chunk_rank[t * K + k],
// the rank inside the token's chunk of tpc tokens; skip_unrouted: tokens with no pick in [0, E) read nothing, for a
// rank that holds only some of the experts)
// (fp8: kmajor_scales writes the block scales as [H/128, cap], the layout the grouped GEMMs read)
// combine without the scatter launch, for callers whose dispatch already wrote inv
hipError_t launch_combine_gather(const uint16_t *y, const int32_t *expand_idx, int N, const int32_t *recv_count_last,
                                 const float *topk_w, int T, int K, int H, uint16_t *out, const int32_t *inv,
                                 hipStream_t s);

// ---- diagnose outputs (diag.hip): stats[idx] += microseconds between the two stream points
hipError_t launch_phase_begin(uint64_t *stamp, hipStream_t s);
hipError_t launch_phase_end(const uint64_t *stamp, int32_t *stats, int idx, hipStream_t s);

// ---- fused decode helpers (fused.hip)
hipError_t launch_prepare_ids(const int32_t *ids, const uint8_t *active, int T, int K, int first_local, int L,
                              int32_t *out, hipStream_t s);
hipError_t launch_fill_i64(int64_t *p, int64_t v, long n, hipStream_t s);

// ---- weighted unpermute (combine.hip)
hipError_t launch_combine(const uint16_t *y, const int32_t *expand_idx, int N, const int32_t *recv_count_last,
                          const float *topk_w, int T, int K, int H, uint16_t *out, int32_t *inv_ws,
                          hipStream_t s);
// the same combine with its row map (and diagnose stamp) in the library's static per-device scratch:
// no workspace, no allocation; T*K <= COMBINE_NOALLOC_MAX_SLOTS
constexpr long COMBINE_NOALLOC_MAX_SLOTS = 1L << 18;
hipError_t launch_combine_noalloc(const uint16_t *y, const int32_t *expand_idx, int N, const int32_t *recv_count_last,
                                  const float *topk_w, int T, int K, int H, uint16_t *out, int32_t *cost_stats,
                                  int stats_idx, hipStream_t s);

}  // namespace cam
