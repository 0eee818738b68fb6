// D3 + Q1/Q2: permute-by-expert dispatch with fused quantisation.
// Row of (t,k) = send_offset[e] + send_token_idx[t,k]  (moe_dispatch_normal.h:381-398)
// expand_idx[row] = (rank, t, k)                       (moe_dispatch_normal.h:335-344)
//
// One wave per (token, 1024-column chunk) for bf16 and fp8 rows (one wave
// per token for int8, whose scale needs the whole row).  The wave reads its
// slice of the token's row once (16-byte loads, lane l owns columns
// [1024 j + 16 l, +16)), quantises it once in registers, and writes the same
// bytes to each of the token's K destination rows as 16-byte stores: HBM
// traffic is one read of x and one write per routed row, the minimum.
//   quant_mode 0: bf16 copy.
//   quant_mode 2: int8 per token, s = 127/(amax+1e-12), q = rint(x*s), scale = 1/s
//                 (moe_dispatch_normal.h:295-332).
//   QUANT_INT8_FUSED (internal, the fused decode op): int8 per token, optional
//                 per-expert smooth scales, s = 127/amax (dispatch_int8_kernel).
//   quant_mode 3: fp8 e4m3fn per 1x128 block: amax clamped to >= 1e-4,
//                 q = e4m3_rne_sat(x * (448/amax)), scale = amax/448.  A block
//                 is 8 adjacent lanes, so its amax is a 3-step xor shuffle.
// Entries whose expert id is outside [0,E) are skipped.
#include "cam_device.h"
#include "launchers.h"
#include "prefill_dev.h"

namespace cam {

constexpr int DISP_WAVES = 4;
constexpr int DISP_NIT = 7;  // H <= 7168 = 7 * 1024
constexpr int DISP_MAX_K = 16;

// bf16 copy and fp8 1x128 quantisation: one wave per (token, 1024-column chunk) (dispatch_wave in
// prefill_dev.h).
template <int MODE>
__global__ __launch_bounds__(DISP_WAVES * 64) void dispatch_chunk_kernel(
    const uint16_t *__restrict__ x, const int32_t *__restrict__ topk_idx, const int32_t *__restrict__ send_offset,
    RankSrc rs, int T, int H, int K, int E, int rank, int cap, int nchunk,
    uint8_t *__restrict__ expand_x, float *__restrict__ scales, int32_t *__restrict__ expand_idx,
    int32_t *__restrict__ inv_out, int kmajor, int skip_unrouted)
{
    const long item = (long)blockIdx.x * DISP_WAVES + (threadIdx.x >> 6);
    if (item >= (long)T * nchunk)
        return;
    const int t = (int)(item / nchunk), j = (int)(item % nchunk);
    dispatch_wave<MODE>(x, topk_idx, send_offset, rs, t, j, T, H, K, E, rank, cap, expand_x, scales, expand_idx,
                        inv_out, kmajor, skip_unrouted, [] {});
}

// int8 per-token quantisation needs the whole row's amax: one wave per token,
// the row held in registers (lane l owns columns [1024 j + 16 l, +16)).
// FUSED = false: the prefill recipe, s = 127/(amax+1e-12) (moe_dispatch_normal.h:295-332).
// FUSED = true: the fused decode recipe (cam_moe_distribute_dispatch.h:640-681 and the shared-expert
// QuantToken, grouped_matmul_slice_m_per_token_dequant_swiglu_quant_multistage_workspace.h): optional
// smooth scales smooth[e, :] multiply x first (e = the destination expert, 0 in identity mode), then
// s = 127/amax with no epsilon; a row of zeros gets q = 0 and scale 0.  With smooth scales the
// quantised row differs per destination, so it is recomputed for each of the token's K rows.
template <bool FUSED>
__global__ __launch_bounds__(DISP_WAVES * 64) void dispatch_int8_kernel(
    const uint16_t *__restrict__ x, const int32_t *__restrict__ topk_idx, const int32_t *__restrict__ send_offset,
    RankSrc rs, int T, int H, int K, int E, int rank, int cap,
    uint8_t *__restrict__ expand_x, float *__restrict__ scales, int32_t *__restrict__ expand_idx,
    int32_t *__restrict__ inv_out, const float *__restrict__ smooth)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * DISP_WAVES + (threadIdx.x >> 6);
    if (t >= T)
        return;
    const int dst = dispatch_dest(topk_idx, send_offset, rs, t, T, K, E, cap, lane);
    if (inv_out && lane < K)
        inv_out[(size_t)t * K + lane] = dst;
    const u32x4 *xr = reinterpret_cast<const u32x4 *>(x + (size_t)t * H);
    u32x4 raw[DISP_NIT][2];
#pragma unroll
    for (int j = 0; j < DISP_NIT; ++j) {
        const int col = j * 1024 + lane * 16;
        if (col < H) {
            raw[j][0] = __builtin_nontemporal_load(xr + (col >> 3));
            raw[j][1] = __builtin_nontemporal_load(xr + (col >> 3) + 1);
        } else {
            raw[j][0] = u32x4{0, 0, 0, 0};
            raw[j][1] = u32x4{0, 0, 0, 0};
        }
    }
    u32x4 q[DISP_NIT];
    float tok_scale = 0.0f;
    // quantises the register row, multiplied by sm[col] when sm is given
    auto quantise = [&](const float *sm) {
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < DISP_NIT; ++j) {
            float f[16];
            unpack_bf16x8(raw[j][0], f);
            unpack_bf16x8(raw[j][1], f + 8);
            const int col = j * 1024 + lane * 16;
            if (sm && col < H) {
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    f[i] = f[i] * sm[col + i];
            }
#pragma unroll
            for (int i = 0; i < 16; ++i)
                amax = fmaxf(amax, fabsf(f[i]));
        }
        amax = group_max<64>(amax);
        float sc;
        if (FUSED) {
            sc = amax > 0.0f ? 127.0f / amax : 0.0f;
            tok_scale = amax > 0.0f ? 1.0f / sc : 0.0f;
        } else {
            sc = 127.0f / (amax + 1e-12f);
            tok_scale = 1.0f / sc;
        }
#pragma unroll
        for (int j = 0; j < DISP_NIT; ++j) {
            float f[16];
            unpack_bf16x8(raw[j][0], f);
            unpack_bf16x8(raw[j][1], f + 8);
            const int col = j * 1024 + lane * 16;
            if (sm && col < H) {
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    f[i] = f[i] * sm[col + i];
            }
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t pk = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int v = (int)rintf(f[4 * w + b] * sc);
                    pk |= (uint32_t)(v & 0xff) << (8 * b);
                }
                q[j][w] = pk;
            }
        }
    };
    const bool per_dest = FUSED && smooth != nullptr;
    if (!per_dest)
        quantise(nullptr);
    for (int k = 0; k < K; ++k) {
        const int row = __shfl(dst, k, 64);
        if (row < 0)
            continue;
        if (per_dest) {
            const int e = topk_idx ? topk_idx[(size_t)t * K + k] : 0;
            quantise(smooth + (size_t)e * H);
        }
        u32x4 *out = reinterpret_cast<u32x4 *>(expand_x + (size_t)row * H);
#pragma unroll
        for (int j = 0; j < DISP_NIT; ++j) {
            const int col = j * 1024 + lane * 16;
            if (col < H)
                out[col >> 4] = q[j];
        }
        if (lane == 0) {
            scales[row] = tok_scale;
            if (expand_idx) {
                expand_idx[(size_t)row * 3 + 0] = rank;
                expand_idx[(size_t)row * 3 + 1] = t;
                expand_idx[(size_t)row * 3 + 2] = k;
            }
        }
    }
}

// Decode sizes (T*K <= DEC_MAX_TK): the layout (D1, the id preparation of the fused op and the count exchange
// of one rank) folded into the dispatch launch.  Every block (16 waves) computes the whole layout of the T*K
// picks in LDS -- the same stable per-expert ranks as layout_small_kernel: lanes sharing an expert found with
// one ballot per bit of its id, waves ordered by per-wave counts -- while its waves' loads of x are in flight,
// then dispatches its (token, chunk) items from the LDS copy.  Block 0 also writes the layout's outputs
// (counts, send offsets, inclusive counts, total, int64 tokens per expert); the grid clears `zero` (the
// chained GEMMs' counters).
constexpr int DEC_WAVES = 16;
constexpr int DEC_THREADS = DEC_WAVES * 64;
constexpr int DEC_MAX_TK = LAYOUT_LDS_MAX_TK;
constexpr int DEC_MAX_E = LAYOUT_LDS_MAX_E;

template <int MODE>
__global__ __launch_bounds__(DEC_THREADS) void dispatch_decode_kernel(
    const int32_t *__restrict__ ids, const uint8_t *__restrict__ active, const uint16_t *__restrict__ x, int T,
    int H, int K, int E, int cap, int nchunk, uint8_t *__restrict__ expand_x, float *__restrict__ scales,
    int32_t *__restrict__ expand_idx, int32_t *__restrict__ inv_out, int kmajor, int32_t *__restrict__ counts,
    int32_t *__restrict__ send_offset, int32_t *__restrict__ recv_count, int32_t *__restrict__ total,
    int64_t *__restrict__ tokens_per_expert, int32_t *__restrict__ zero, int nzero)
{
    __shared__ LayoutLds<DEC_THREADS> s;
    for (long i = (long)blockIdx.x * DEC_THREADS + threadIdx.x; i < nzero; i += (long)gridDim.x * DEC_THREADS)
        zero[i] = 0;
    auto layout = [&]() {
        layout_lds<DEC_THREADS>(ids, active, T, K, E, s);
        if (blockIdx.x == 0)
            layout_lds_store(s, E, counts, send_offset, recv_count, total, tokens_per_expert);
    };
    const long item = (long)blockIdx.x * DEC_WAVES + (threadIdx.x >> 6);
    if (item >= (long)T * nchunk) {  // a wave without an item still takes its part in the block's layout
        layout();
        return;
    }
    const int t = (int)(item / nchunk), j = (int)(item % nchunk);
    const RankSrc rs{s.rank, nullptr, nullptr, 0};
    dispatch_wave<MODE>(x, s.ids, s.off, rs, t, j, T, H, K, E, 0, cap, expand_x, scales, expand_idx, inv_out,
                        kmajor, 0, layout);
}

hipError_t launch_dispatch_decode(const int32_t *ids, const uint8_t *active, const uint16_t *x, int T, int H, int K,
                                  int E, int cap, int quant_mode, void *expand_x, float *scales, int32_t *expand_idx,
                                  int32_t *inv_out, bool kmajor_scales, int32_t *counts, int32_t *send_offset,
                                  int32_t *recv_count, int32_t *total, int64_t *tokens_per_expert, hipStream_t s,
                                  int32_t *zero, int nzero)
{
    if (!dispatch_decode_fits(T, K, E) || K > DISP_MAX_K || H > DISP_NIT * 1024 || (H & 15) || nzero < 0 ||
        (quant_mode != QUANT_NONE && quant_mode != QUANT_FP8_BLOCK) || (quant_mode == QUANT_FP8_BLOCK && (H & 127)))
        return hipErrorInvalidValue;
    const int nchunk = (H + 1023) / 1024;
    const dim3 grid((unsigned)(((long)T * nchunk + DEC_WAVES - 1) / DEC_WAVES)), block(DEC_THREADS);
    uint8_t *ex = (uint8_t *)expand_x;
    if (quant_mode == QUANT_NONE)
        hipLaunchKernelGGL(dispatch_decode_kernel<QUANT_NONE>, grid, block, 0, s, ids, active, x, T, H, K, E, cap,
                           nchunk, ex, scales, expand_idx, inv_out, kmajor_scales ? 1 : 0, counts, send_offset,
                           recv_count, total, tokens_per_expert, zero, nzero);
    else
        hipLaunchKernelGGL(dispatch_decode_kernel<QUANT_FP8_BLOCK>, grid, block, 0, s, ids, active, x, T, H, K, E,
                           cap, nchunk, ex, scales, expand_idx, inv_out, kmajor_scales ? 1 : 0, counts, send_offset,
                           recv_count, total, tokens_per_expert, zero, nzero);
    return hipGetLastError();
}
bool dispatch_decode_fits(int T, int K, int E) { return T >= 1 && (long)T * K <= DEC_MAX_TK && E >= 1 && E <= DEC_MAX_E; }

hipError_t launch_dispatch(const uint16_t *x, const int32_t *topk_idx, const int32_t *send_offset,
                           const int32_t *send_token_idx, int T, int H, int K, int E, int rank, int cap, int quant_mode,
                           void *expand_x, float *scales, int32_t *expand_idx, hipStream_t s, int32_t *inv_out,
                           const float *smooth, bool kmajor_scales, const int32_t *chunk_base, int tpc,
                           const int32_t *chunk_rank, bool skip_unrouted)
{
    if (topk_idx && !send_token_idx && (!chunk_base || !chunk_rank || tpc < 1))
        return hipErrorInvalidValue;
    const RankSrc rs{send_token_idx, chunk_base, chunk_rank, tpc};
    if (T == 0)
        return hipSuccess;
    if (H > DISP_NIT * 1024 || K > DISP_MAX_K || (H & 15))
        return hipErrorInvalidValue;
    const dim3 block(DISP_WAVES * 64);
    const int nchunk = (H + 1023) / 1024;
    const dim3 grid_chunk((unsigned)(((long)T * nchunk + DISP_WAVES - 1) / DISP_WAVES));
    uint8_t *ex = (uint8_t *)expand_x;
    switch (quant_mode) {
    case QUANT_NONE:
        hipLaunchKernelGGL(dispatch_chunk_kernel<QUANT_NONE>, grid_chunk, block, 0, s, x, topk_idx, send_offset,
                           rs, T, H, K, E, rank, cap, nchunk, ex, scales, expand_idx, inv_out, 0, skip_unrouted ? 1 : 0);
        break;
    case QUANT_INT8_TOKEN:
        hipLaunchKernelGGL(dispatch_int8_kernel<false>, dim3((T + DISP_WAVES - 1) / DISP_WAVES), block, 0, s, x,
                           topk_idx, send_offset, rs, T, H, K, E, rank, cap, ex, scales, expand_idx,
                           inv_out, nullptr);
        break;
    case QUANT_INT8_FUSED:
        hipLaunchKernelGGL(dispatch_int8_kernel<true>, dim3((T + DISP_WAVES - 1) / DISP_WAVES), block, 0, s, x,
                           topk_idx, send_offset, rs, T, H, K, E, rank, cap, ex, scales, expand_idx,
                           inv_out, smooth);
        break;
    case QUANT_FP8_BLOCK:
        if (H & 127)
            return hipErrorInvalidValue;
        hipLaunchKernelGGL(dispatch_chunk_kernel<QUANT_FP8_BLOCK>, grid_chunk, block, 0, s, x, topk_idx,
                           send_offset, rs, T, H, K, E, rank, cap, nchunk, ex, scales, expand_idx, inv_out,
                           kmajor_scales ? 1 : 0, skip_unrouted ? 1 : 0);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace cam
