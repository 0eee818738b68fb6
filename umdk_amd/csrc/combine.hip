// C1: weighted unpermute (combine).
//   out[t] = bf16_rne( sum_{k ascending} float(y[row(t,k)]) * w[t,k] )
// fp32 accumulation starting from +0, multiply then add, never fused
// (moe_combine_normal.h:343-377; cam_moe_distribute_combine.h:654-716).
//
// Two launches:
//   1. combine_scatter_kernel: inv[t*K+k] = row for every received row
//      (the single-rank form of CopyBufferToShare, moe_combine_normal.h:286-303,
//      which moves whole rows; here only the 4-byte row index moves).
//   2. combine_gather_kernel: one wave per (token, 1024-column chunk) reads
//      its K row slices with 16-byte loads (all K in flight together),
//      accumulates in k order and writes the bf16 slice once.
// inv needs no clearing: the gather accepts inv[t*K+k] = r only when
// 0 <= r < rows and expand_idx[r] names (t,k) back, so stale workspace
// contents can never select a row; such slots are skipped, as the fused
// combine skips expert ids < 0.
#include <atomic>
#include <mutex>

#include "cam_device.h"
#include "launchers.h"

namespace cam {

#ifndef CAM_COMB_WAVES
#define CAM_COMB_WAVES 4
#endif
#ifndef CAM_COMB_NTLD
#define CAM_COMB_NTLD 1
#endif
#ifndef CAM_COMB_NTST
#define CAM_COMB_NTST 1
#endif
constexpr int COMB_WAVES = CAM_COMB_WAVES;
constexpr int COMB_NIT = 7;   // H <= 7168
constexpr int COMB_KB = 8;    // rows in flight per batch

__global__ void combine_scatter_kernel(const int32_t *__restrict__ expand_idx, int N,
                                       const int32_t *__restrict__ recv_count_last, int T, int K,
                                       int32_t *__restrict__ inv)
{
    const int lim = recv_count_last ? min(N, *recv_count_last) : N;
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < lim; r += gridDim.x * blockDim.x) {
        const int t = expand_idx[(size_t)r * 3 + 1], k = expand_idx[(size_t)r * 3 + 2];
        if (t >= 0 && t < T && k >= 0 && k < K)
            inv[(size_t)t * K + k] = r;
    }
}

__global__ __launch_bounds__(COMB_WAVES * 64) void combine_gather_kernel(
    const uint16_t *__restrict__ y, const int32_t *__restrict__ expand_idx, int N,
    const int32_t *__restrict__ recv_count_last, const float *__restrict__ topk_w, int T, int K, int H, int nchunk,
    uint16_t *__restrict__ out, const int32_t *__restrict__ inv)
{
#pragma clang fp contract(off)
    // one wave per (token, 1024-column chunk): lane l owns columns [1024 j + 8 l, +8) and
    // [1024 j + 512 + 8 l, +8), so each 16-byte load or store instruction of the wave covers
    // one contiguous kilobyte (whole cache lines, no partial-line writes)
    const int lane = threadIdx.x & 63;
    const long item = (long)blockIdx.x * COMB_WAVES + (threadIdx.x >> 6);
    if (item >= (long)T * nchunk)
        return;
    const int t = (int)(item / nchunk), j = (int)(item % nchunk);
    const int lim = recv_count_last ? min(N, *recv_count_last) : N;
    int row = -1;
    float w = 0.0f;
    if (lane < K) {
        const int r = inv[(size_t)t * K + lane];
        if (r >= 0 && r < lim && expand_idx[(size_t)r * 3 + 1] == t && expand_idx[(size_t)r * 3 + 2] == lane) {
            row = r;
            w = topk_w[(size_t)t * K + lane];
        }
    }
    const int col = j * 1024 + lane * 8;
    const bool act = col < H;         // H % 16 == 0 and 1024-aligned chunks: both halves or neither
    const bool act1 = col + 512 < H;
    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
        acc[i] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += COMB_KB) {
        u32x4 v[COMB_KB][2];
        int rk[COMB_KB];
        float wk[COMB_KB];
#pragma unroll
        for (int b = 0; b < COMB_KB; ++b) {
            const int k = k0 + b;
            rk[b] = k < K ? __shfl(row, k, 64) : -1;
            wk[b] = __shfl(w, k < K ? k : 0, 64);
            if (rk[b] >= 0 && act) {
                const uint16_t *src = y + (size_t)rk[b] * H + col;
#if CAM_COMB_NTLD
                v[b][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src));
                v[b][1] = act1 ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src + 512))
                               : u32x4{0, 0, 0, 0};
#else
                v[b][0] = *reinterpret_cast<const u32x4 *>(src);
                v[b][1] = act1 ? *reinterpret_cast<const u32x4 *>(src + 512) : u32x4{0, 0, 0, 0};
#endif
            }
        }
#pragma unroll
        for (int b = 0; b < COMB_KB; ++b) {
            if (rk[b] < 0 || !act)
                continue;
            float f[16];
            unpack_bf16x8(v[b][0], f);
            unpack_bf16x8(v[b][1], f + 8);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float p = f[i] * wk[b];
                acc[i] = acc[i] + p;
            }
        }
    }
    if (act) {
        uint16_t *orow = out + (size_t)t * H + col;
#if CAM_COMB_NTST
        __builtin_nontemporal_store(pack_bf16x8(acc), reinterpret_cast<u32x4 *>(orow));
        if (act1)
            __builtin_nontemporal_store(pack_bf16x8(acc + 8), reinterpret_cast<u32x4 *>(orow + 512));
#else
        *reinterpret_cast<u32x4 *>(orow) = pack_bf16x8(acc);
        if (act1)
            *reinterpret_cast<u32x4 *>(orow + 512) = pack_bf16x8(acc + 8);
#endif
    }
}

hipError_t launch_combine_gather(const uint16_t *y, const int32_t *expand_idx, int N, const int32_t *recv_count_last,
                                 const float *topk_w, int T, int K, int H, uint16_t *out, const int32_t *inv,
                                 hipStream_t s)
{
    if (T == 0)
        return hipSuccess;
    if (H > COMB_NIT * 1024 || (H & 15) || K > 64)
        return hipErrorInvalidValue;
    const int nchunk = (H + 1023) / 1024;
    const long items = (long)T * nchunk;
    hipLaunchKernelGGL(combine_gather_kernel, dim3((unsigned)((items + COMB_WAVES - 1) / COMB_WAVES)),
                       dim3(COMB_WAVES * 64), 0, s, y, expand_idx, N, recv_count_last, topk_w, T, K, H, nchunk, out,
                       inv);
    return hipGetLastError();
}

hipError_t launch_combine(const uint16_t *y, const int32_t *expand_idx, int N, const int32_t *recv_count_last,
                          const float *topk_w, int T, int K, int H, uint16_t *out, int32_t *inv_ws, hipStream_t s)
{
    if (T == 0)
        return hipSuccess;
    if (H > COMB_NIT * 1024 || (H & 15) || K > 64)
        return hipErrorInvalidValue;
    if (N > 0) {
        int blocks = (N + 255) / 256;
        if (blocks > 2048)
            blocks = 2048;
        hipLaunchKernelGGL(combine_scatter_kernel, dim3(blocks), dim3(256), 0, s, expand_idx, N, recv_count_last, T,
                           K, inv_ws);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess)
            return err;
    }
    const int nchunk = (H + 1023) / 1024;
    const long items = (long)T * nchunk;
    hipLaunchKernelGGL(combine_gather_kernel, dim3((unsigned)((items + COMB_WAVES - 1) / COMB_WAVES)),
                       dim3(COMB_WAVES * 64), 0, s, y, expand_idx, N, recv_count_last, topk_w, T, K, H, nchunk, out,
                       inv_ws);
    return hipGetLastError();
}

// ---------------------------------------------------------------- allocation-free combine
// Scratch of the allocation-free entry point: the row map (T*K int32, at most
// COMBINE_NOALLOC_MAX_SLOTS) and, past it, the diagnose output's 8-byte start stamp.  One copy
// per GPU, held until the process ends; every call on a GPU shares it, so calls that overlap on
// one GPU race.  Nothing in it needs clearing: the gather validates every map entry against
// expand_idx, and the stamp is written before it is read.
constexpr size_t NOALLOC_MAP_BYTES = sizeof(int32_t) * (size_t)COMBINE_NOALLOC_MAX_SLOTS;
static __device__ __align__(256) uint8_t scratch[NOALLOC_MAP_BYTES + 256];

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
std::atomic<void *> g_scratch[NOALLOC_MAX_DEVICES];
std::mutex g_scratch_mu;
}  // namespace

// Device address of `scratch` on the current device.  Host code never uses the array's name as
// an address (on the host it is only a stand-in for the symbol): it asks the runtime once per
// device, with that device current, and keeps the answer.
hipError_t combine_noalloc_scratch(void **ptr)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return e;
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
        return hipErrorInvalidDevice;
    void *p = g_scratch[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess)
                return e;
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *ptr = p;
    return hipSuccess;
}

hipError_t launch_combine_noalloc(const uint16_t *y, const int32_t *expand_idx, int N, const int32_t *recv_count_last,
                                  const float *topk_w, int T, int K, int H, uint16_t *out, int32_t *cost_stats,
                                  int stats_idx, hipStream_t s)
{
    if ((long)T * K > COMBINE_NOALLOC_MAX_SLOTS)
        return hipErrorInvalidValue;
    void *base = nullptr;
    hipError_t e = combine_noalloc_scratch(&base);
    if (e != hipSuccess)
        return e;
    int32_t *inv = (int32_t *)base;
    uint64_t *stamp = (uint64_t *)((uint8_t *)base + NOALLOC_MAP_BYTES);
    if (cost_stats) {
        e = launch_phase_begin(stamp, s);
        if (e != hipSuccess)
            return e;
    }
    e = launch_combine(y, expand_idx, N, recv_count_last, topk_w, T, K, H, out, inv, s);
    if (e != hipSuccess || !cost_stats)
        return e;
    return launch_phase_end(stamp, cost_stats, stats_idx, s);
}

}  // namespace cam
