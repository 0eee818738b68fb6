// Device-side helpers shared by the CAM MoE kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define CAM_WAVE 64

namespace cam {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_to_f32(uint32_t h16) { return __uint_as_float(h16 << 16); }

// fp32 -> bf16 bits, round to nearest even (NaN-free inputs).
__device__ __forceinline__ uint32_t f32_to_bf16(float f)
{
    uint32_t u = __float_as_uint(f);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// Two fp32 -> two bf16 (round to nearest even) packed little-endian, by the hardware conversion
// (v_cvt_pk_bf16_f32): one instruction for what f32_to_bf16 takes four for, the same bits for every
// finite input.
typedef __bf16 cam_bf16x2 __attribute__((ext_vector_type(2)));
typedef float cam_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((cam_f32x2{a, b}), cam_bf16x2));
}

// Unpack 8 bf16 held in a 16-byte vector into fp32.
__device__ __forceinline__ void unpack_bf16x8(const u32x4 v, float *f)
{
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(v[i] << 16);
        f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
    }
}

__device__ __forceinline__ u32x4 pack_bf16x8(const float *f)
{
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        r[i] = f32_to_bf16(f[2 * i]) | (f32_to_bf16(f[2 * i + 1]) << 16);
    return r;
}

// Four fp32 -> four OCP e4m3fn codes (round to nearest even), packed little-endian.
// Values are clamped to +-448 first, so the conversion saturates.
__device__ __forceinline__ uint32_t f32x4_to_e4m3(float a, float b, float c, float d)
{
    a = fminf(fmaxf(a, -448.0f), 448.0f);
    b = fminf(fmaxf(b, -448.0f), 448.0f);
    c = fminf(fmaxf(c, -448.0f), 448.0f);
    d = fminf(fmaxf(d, -448.0f), 448.0f);
    int r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
    return (uint32_t)r;
}

// Max over groups of `width` adjacent lanes (width a power of two <= 64).
template <int width> __device__ __forceinline__ float group_max(float v)
{
#pragma unroll
    for (int o = width / 2; o > 0; o >>= 1)
        v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ uint64_t lanemask_lt()
{
    const int lane = threadIdx.x & 63;
    return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

}  // namespace cam
