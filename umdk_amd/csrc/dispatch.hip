// D3 + Q1/Q2: permute-by-expert dispatch with fused quantisation.
// Row of (t,k) = send_offset[e] + send_token_idx[t,k]  (moe_dispatch_normal.h:381-398)
// expand_idx[row] = (rank, t, k)                       (moe_dispatch_normal.h:335-344)
//
// One wave per token.  The wave reads the token's row once (16-byte loads,
// lane l owns elements [1024 j + 16 l, +16) of iteration j), quantises it
// once in registers, and writes the same bytes to each of the token's K
// destination rows as 16-byte stores: HBM traffic is one read of x and one
// write per routed row, the algorithmic minimum.
//   quant_mode 0: bf16 copy.
//   quant_mode 2: int8 per token, s = 127/(amax+1e-12), q = rint(x*s), scale = 1/s
//                 (moe_dispatch_normal.h:295-332).
//   quant_mode 3: fp8 e4m3fn per 1x128 block: amax clamped to >= 1e-4,
//                 q = e4m3_rne_sat(x * (448/amax)), scale = amax/448.  A block
//                 is 8 adjacent lanes, so its amax is a 3-step xor shuffle.
// Entries whose expert id is outside [0,E) are skipped.
#include "cam_device.h"
#include "launchers.h"

namespace cam {

constexpr int DISP_WAVES = 4;
constexpr int DISP_NIT = 7;  // H <= 7168 = 7 * 1024
constexpr int DISP_MAX_K = 16;

template <int MODE>
__global__ __launch_bounds__(DISP_WAVES * 64) void dispatch_kernel(
    const uint16_t *__restrict__ x, const int32_t *__restrict__ topk_idx, const int32_t *__restrict__ send_offset,
    const int32_t *__restrict__ send_token_idx, int T, int H, int K, int E, int rank, uint8_t *__restrict__ expand_x,
    float *__restrict__ scales, int32_t *__restrict__ expand_idx)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * DISP_WAVES + (threadIdx.x >> 6);
    if (t >= T)
        return;

    // destinations: lane k < K resolves entry (t,k)
    int dst = -1;
    if (lane < K) {
        const int e = topk_idx[(size_t)t * K + lane];
        if (e >= 0 && e < E)
            dst = send_offset[e] + send_token_idx[(size_t)t * K + lane];
    }

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

    if constexpr (MODE == QUANT_NONE) {
        for (int k = 0; k < K; ++k) {
            const int row = __shfl(dst, k, 64);
            if (row < 0)
                continue;
            u32x4 *out = reinterpret_cast<u32x4 *>(expand_x + (size_t)row * H * 2);
#pragma unroll
            for (int j = 0; j < DISP_NIT; ++j) {
                const int col = j * 1024 + lane * 16;
                if (col < H) {
                    out[(col >> 3)] = raw[j][0];
                    out[(col >> 3) + 1] = raw[j][1];
                }
            }
            if (lane == 0) {
                expand_idx[(size_t)row * 3 + 0] = rank;
                expand_idx[(size_t)row * 3 + 1] = t;
                expand_idx[(size_t)row * 3 + 2] = k;
            }
        }
    } else {
        u32x4 q[DISP_NIT];
        float blk_scale[DISP_NIT];
        float tok_scale = 0.0f;
        if constexpr (MODE == QUANT_INT8_TOKEN) {
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < DISP_NIT; ++j) {
                float f[16];
                unpack_bf16x8(raw[j][0], f);
                unpack_bf16x8(raw[j][1], f + 8);
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    amax = fmaxf(amax, fabsf(f[i]));
            }
            amax = group_max<64>(amax);
            const float sc = 127.0f / (amax + 1e-12f);
            tok_scale = 1.0f / sc;
#pragma unroll
            for (int j = 0; j < DISP_NIT; ++j) {
                float f[16];
                unpack_bf16x8(raw[j][0], f);
                unpack_bf16x8(raw[j][1], f + 8);
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
                blk_scale[j] = 0.0f;
            }
        } else {
#pragma unroll
            for (int j = 0; j < DISP_NIT; ++j) {
                float f[16];
                unpack_bf16x8(raw[j][0], f);
                unpack_bf16x8(raw[j][1], f + 8);
                float amax = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    amax = fmaxf(amax, fabsf(f[i]));
                amax = fmaxf(group_max<8>(amax), 1e-4f);
                const float inv = 448.0f / amax;
                blk_scale[j] = amax / 448.0f;
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    q[j][w] = f32x4_to_e4m3(f[4 * w] * inv, f[4 * w + 1] * inv, f[4 * w + 2] * inv,
                                            f[4 * w + 3] * inv);
            }
        }
        const int nb = H >> 7;
        for (int k = 0; k < K; ++k) {
            const int row = __shfl(dst, k, 64);
            if (row < 0)
                continue;
            u32x4 *out = reinterpret_cast<u32x4 *>(expand_x + (size_t)row * H);
#pragma unroll
            for (int j = 0; j < DISP_NIT; ++j) {
                const int col = j * 1024 + lane * 16;
                if (col < H) {
                    out[col >> 4] = q[j];
                    if constexpr (MODE == QUANT_FP8_BLOCK) {
                        if ((lane & 7) == 0)
                            scales[(size_t)row * nb + (col >> 7)] = blk_scale[j];
                    }
                }
            }
            if (lane == 0) {
                if constexpr (MODE == QUANT_INT8_TOKEN)
                    scales[row] = tok_scale;
                expand_idx[(size_t)row * 3 + 0] = rank;
                expand_idx[(size_t)row * 3 + 1] = t;
                expand_idx[(size_t)row * 3 + 2] = k;
            }
        }
    }
}

hipError_t launch_dispatch(const uint16_t *x, const int32_t *topk_idx, const int32_t *send_offset,
                           const int32_t *send_token_idx, int T, int H, int K, int E, int rank, int quant_mode,
                           void *expand_x, float *scales, int32_t *expand_idx, hipStream_t s)
{
    if (T == 0)
        return hipSuccess;
    if (H > DISP_NIT * 1024 || K > DISP_MAX_K || (H & 15))
        return hipErrorInvalidValue;
    const dim3 grid((T + DISP_WAVES - 1) / DISP_WAVES), block(DISP_WAVES * 64);
    uint8_t *ex = (uint8_t *)expand_x;
    switch (quant_mode) {
    case QUANT_NONE:
        hipLaunchKernelGGL(dispatch_kernel<QUANT_NONE>, grid, block, 0, s, x, topk_idx, send_offset, send_token_idx,
                           T, H, K, E, rank, ex, scales, expand_idx);
        break;
    case QUANT_INT8_TOKEN:
        hipLaunchKernelGGL(dispatch_kernel<QUANT_INT8_TOKEN>, grid, block, 0, s, x, topk_idx, send_offset,
                           send_token_idx, T, H, K, E, rank, ex, scales, expand_idx);
        break;
    case QUANT_FP8_BLOCK:
        if (H & 127)
            return hipErrorInvalidValue;
        hipLaunchKernelGGL(dispatch_kernel<QUANT_FP8_BLOCK>, grid, block, 0, s, x, topk_idx, send_offset,
                           send_token_idx, T, H, K, E, rank, ex, scales, expand_idx);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace cam
