// G1-G3: grouped expert GEMMs over ragged expert segments, bf16 or fp8 e4m3
// with 128x128 weight block scales and 1x128 activation scales.
//
// Semantics (CPU restatement in oracle/cam_oracle.c):
//   rows of A are in dispatch order; expert e owns rows [off_e, off_e+cnt_e),
//   off = exclusive prefix of group_list (tokens per local expert);
//   weights are stored N-major, K contiguous: W [L, N, K] (fp8 scales
//   [L, N/128, K/128]).
//   GMM1+SwiGLU (EPI_SWIGLU_*): N = 2I, rows [0,I) of W are the gate and
//     [I,2I) the up projection (block_epilogue_per_token_dequant_swiglu.h:256-286:
//     silu on the left half); h = silu(g) * u, silu(g) = g / (1 + exp(-g)),
//     stored as bf16, or requantised to fp8 per 1x128 block of h exactly like
//     the dispatch quantiser (post_swiglu_dynamic_quant.h:164-231 requantises
//     per token in int8).
//   GMM2 (EPI_PLAIN): out = bf16(A W^T) per expert
//     (block_epilogue_per_token_dequant.hpp:338-361).
//
// Kernel design (gfx950):
//   * 256 x 256 output tiles (for SwiGLU: 256 rows x 128 h-columns, i.e. 128
//     gate + 128 up rows of W), 8 waves in a 2 x 4 grid, 128 x 64 per wave
//     as 8 x 4 MFMA 16x16 tiles (v_mfma_f32_16x16x32_bf16, or
//     v_mfma_scale_f32_16x16x128_f8f6f4 with unit scales for fp8); the 128
//     accumulators per lane leave room for the fp8 per-block rescale in VALU.
//   * Each k-step moves 128 bytes of every A and W row (64 bf16 / 128 fp8)
//     through LDS, double buffered, one barrier per k-step; global loads of
//     the next k-step are in flight while the current one is multiplied.
//     LDS rows are 128 B with the 16-byte chunks XOR-swizzled by (row & 7),
//     so fragment reads spread over all banks.
//   * MFMA operands are (W fragment, A fragment), so each lane's four
//     accumulators are four consecutive output columns of one row: the
//     epilogue stores 8 contiguous bytes per lane without a transpose.
//   * fp8: one MFMA of K=128 per (i,j) per k-step covers exactly one scale
//     block, so acc += mfma(...) * (a_scale[m] * w_scale[n-block]).
//   * Persistent grid (one block per CU) walking tiles expert by expert,
//     N-tile by N-tile, M-tiles fastest, remapped so that the blocks of one
//     XCD take consecutive tiles (they share W tiles in that XCD's L2).
#include "cam_device.h"
#include "gmm.h"

namespace cam {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) int i32x8;

constexpr int GBM = 256, GBN = 256, GKB = 128;  // tile rows, tile W-rows, bytes per row per k-step
constexpr int GTHREADS = 512;
constexpr int G_MAX_L = 512;
constexpr int LDS_TILE = GBM * GKB;  // 32 KiB per operand per buffer

struct GroupTable {
    int tile_prefix[G_MAX_L + 1];  // exclusive prefix of M-tiles per expert
    int row_off[G_MAX_L + 1];      // exclusive prefix of rows per expert
};

// Block-wide exclusive scans of ceil(cnt/GBM) and cnt over the L experts.
__device__ void build_group_table(const int64_t *__restrict__ group_list, int L, GroupTable &gt, int *scratch)
{
    // scratch: 2 * GTHREADS ints
    const int tid = threadIdx.x;
    const int per = (L + GTHREADS - 1) / GTHREADS;
    int tsum = 0, rsum = 0;
    for (int q = 0; q < per; ++q) {
        const int e = tid * per + q;
        if (e < L) {
            const int c = (int)group_list[e];
            tsum += (c + GBM - 1) / GBM;
            rsum += c;
        }
    }
    scratch[tid] = tsum;
    scratch[GTHREADS + tid] = rsum;
    __syncthreads();
    if (tid == 0) {
        int a = 0, b = 0;
        for (int i = 0; i < GTHREADS; ++i) {
            const int x = scratch[i], y = scratch[GTHREADS + i];
            scratch[i] = a;
            scratch[GTHREADS + i] = b;
            a += x;
            b += y;
        }
        gt.tile_prefix[L] = a;
        gt.row_off[L] = b;
    }
    __syncthreads();
    int ta = scratch[tid], ra = scratch[GTHREADS + tid];
    for (int q = 0; q < per; ++q) {
        const int e = tid * per + q;
        if (e < L) {
            const int c = (int)group_list[e];
            gt.tile_prefix[e] = ta;
            gt.row_off[e] = ra;
            ta += (c + GBM - 1) / GBM;
            ra += c;
        }
    }
    __syncthreads();
}

__device__ __forceinline__ int swz(int row, int chunk) { return row * GKB + ((chunk ^ (row & 7)) << 4); }

template <int DT, int EPI>
__global__ __launch_bounds__(GTHREADS, 1) void gmm_kernel(GmmArgs p)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t *lds_a = smem;                   // [2][GBM][GKB]
    uint8_t *lds_b = smem + 2 * LDS_TILE;    // [2][GBN][GKB]
    GroupTable *gt = reinterpret_cast<GroupTable *>(smem + 4 * LDS_TILE);
    int *scratch = reinterpret_cast<int *>(gt + 1);  // 2*GTHREADS ints; reused for the fp8 amax exchange

    build_group_table(p.group_list, p.L, *gt, scratch);

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = w >> 2, wn = w & 3;  // 2 row waves x 4 column waves
    const int l16 = lane & 15, lg = lane >> 4;
    constexpr bool SWIGLU = EPI != EPI_PLAIN;
    const int esz = DT == DT_FP8 ? 1 : 2;
    const int kbytes = p.K * esz;  // bytes per row
    const int nk = kbytes / GKB;
    const int half_n = p.N / 2;    // I for SwiGLU
    const int ntn = SWIGLU ? half_n / 128 : p.N / GBN;
    const int total = gt->tile_prefix[p.L] * ntn;

    // XCD-aware order: blocks b, b+8, b+16, ... run on the same XCD; give them consecutive tiles
    const int G = gridDim.x;
    const int logical = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);

    for (int tile = (G & 7) ? (int)blockIdx.x : logical; tile < total; tile += G) {
        // ---- tile -> (expert, n-tile, m-tile)
        int lo = 0, hi = p.L - 1;
        while (lo < hi) {  // last e with tile_prefix[e]*ntn <= tile
            const int mid = (lo + hi + 1) >> 1;
            if (gt->tile_prefix[mid] * ntn <= tile)
                lo = mid;
            else
                hi = mid - 1;
        }
        const int e = lo;
        const int mt_e = gt->tile_prefix[e + 1] - gt->tile_prefix[e];
        const int local = tile - gt->tile_prefix[e] * ntn;
        const int nt = local / mt_e, mt = local % mt_e;
        const int seg0 = gt->row_off[e], seg1 = min(gt->row_off[e + 1], p.M);  // never write past row M
        const int row0 = seg0 + mt * GBM;
        const int n0 = SWIGLU ? nt * 128 : nt * GBN;  // first h-column (SwiGLU) or W row (plain)

        // ---- byte offsets of this thread's 4 A chunks and 4 W chunks of k-step 0 (32-bit:
        // the host checks that A and one expert's W are below 4 GiB)
        uint32_t ga[4], gb[4];
        const uint8_t *wbase = p.W + (size_t)e * p.N * kbytes;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = (tid >> 3) + 64 * i, c = tid & 7;
            const int arow = min(row0 + r, p.M - 1);
            ga[i] = (uint32_t)arow * (uint32_t)kbytes + c * 16;
            int wrow;
            if (SWIGLU) {
                // LDS row r belongs to column wave r/64: 32 gate rows then the 32 up rows
                // of the same h-columns
                const int wnn = r >> 6, jj = r & 63;
                const int hcol = n0 + 32 * wnn + (jj & 31);
                wrow = jj < 32 ? hcol : half_n + hcol;
            } else {
                wrow = n0 + r;
            }
            gb[i] = (uint32_t)wrow * (uint32_t)kbytes + c * 16;
        }

        f32x4 acc[8][4];
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

        u32x4 ra[4], rb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ra[i] = *reinterpret_cast<const u32x4 *>(p.A + ga[i]);
            rb[i] = *reinterpret_cast<const u32x4 *>(wbase + gb[i]);
        }
        __syncthreads();  // previous tile's readers are done with both buffers
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = (tid >> 3) + 64 * i, c = tid & 7;
            *reinterpret_cast<u32x4 *>(lds_a + swz(r, c)) = ra[i];
            *reinterpret_cast<u32x4 *>(lds_b + swz(r, c)) = rb[i];
        }
        __syncthreads();

        // fp8 scale bookkeeping
        const float *ws_g = nullptr, *ws_u = nullptr;
        const int am0 = row0 + wm * 128 + l16;  // activation-scale row of fragment i: am0 + 16 i
        if constexpr (DT == DT_FP8) {
            const float *wsb = p.Ws + (size_t)e * (p.N / 128) * nk;
            if (SWIGLU) {
                ws_g = wsb + (size_t)(n0 / 128) * nk;
                ws_u = wsb + (size_t)((half_n + n0) / 128) * nk;
            } else {
                ws_g = wsb + (size_t)((n0 + wn * 64) / 128) * nk;
            }
        }

        for (int ks = 0; ks < nk; ++ks) {
            const int cur = ks & 1;
            const bool more = ks + 1 < nk;
            if (more) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    ra[i] = *reinterpret_cast<const u32x4 *>(p.A + ga[i] + (uint32_t)(ks + 1) * GKB);
                    rb[i] = *reinterpret_cast<const u32x4 *>(wbase + gb[i] + (uint32_t)(ks + 1) * GKB);
                }
            }
            const uint8_t *la = lds_a + cur * LDS_TILE + (wm * 128) * GKB;
            const uint8_t *lb = lds_b + cur * LDS_TILE + (wn * 64) * GKB;
            if constexpr (DT == DT_BF16) {
#pragma unroll
                for (int sub = 0; sub < 2; ++sub) {
                    bf16x8 bfr[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        bfr[j] = *reinterpret_cast<const bf16x8 *>(lb + swz(j * 16 + l16, sub * 4 + lg));
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const bf16x8 afr = *reinterpret_cast<const bf16x8 *>(la + swz(i * 16 + l16, sub * 4 + lg));
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[j], afr, acc[i][j], 0, 0, 0);
                    }
                }
            } else {
                float sa[8];
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    sa[i] = p.As[(uint32_t)min(am0 + 16 * i, p.M - 1) * (uint32_t)nk + ks];
                const float sg = ws_g[ks];
                const float su = SWIGLU ? ws_u[ks] : sg;
                i32x8 bfr[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const u32x4 v0 = *reinterpret_cast<const u32x4 *>(lb + swz(j * 16 + l16, 2 * lg));
                    const u32x4 v1 = *reinterpret_cast<const u32x4 *>(lb + swz(j * 16 + l16, 2 * lg + 1));
                    bfr[j] = i32x8{(int)v0[0], (int)v0[1], (int)v0[2], (int)v0[3],
                                   (int)v1[0], (int)v1[1], (int)v1[2], (int)v1[3]};
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const u32x4 v0 = *reinterpret_cast<const u32x4 *>(la + swz(i * 16 + l16, 2 * lg));
                    const u32x4 v1 = *reinterpret_cast<const u32x4 *>(la + swz(i * 16 + l16, 2 * lg + 1));
                    const i32x8 afr = i32x8{(int)v0[0], (int)v0[1], (int)v0[2], (int)v0[3],
                                            (int)v1[0], (int)v1[1], (int)v1[2], (int)v1[3]};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                        const f32x4 d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bfr[j], afr, z, 0, 0, 0,
                                                                                         127, 0, 127);
                        // in SwiGLU tiles a wave's columns j<2 are gate rows, j>=2 up rows
                        const float s = sa[i] * ((SWIGLU && j >= 2) ? su : sg);
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            acc[i][j][q] += d[q] * s;
                    }
                    // keep each fragment row's MFMA results short-lived (no hoisting of all 32)
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            if (more) {
                uint8_t *na = lds_a + (cur ^ 1) * LDS_TILE;
                uint8_t *nb = lds_b + (cur ^ 1) * LDS_TILE;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = (tid >> 3) + 64 * i, c = tid & 7;
                    *reinterpret_cast<u32x4 *>(na + swz(r, c)) = ra[i];
                    *reinterpret_cast<u32x4 *>(nb + swz(r, c)) = rb[i];
                }
            }
            __syncthreads();
        }

        // ---- epilogue: lane holds rows m = row0 + wm*128 + 16 i + l16 and, per j, four
        // consecutive columns 16 j + 4 lg + q of the wave's 64-wide column range
        if constexpr (EPI == EPI_PLAIN) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int m = row0 + wm * 128 + i * 16 + l16;
                if (m >= seg1)
                    continue;
                uint16_t *crow = reinterpret_cast<uint16_t *>(p.C) + (size_t)m * p.N + n0 + wn * 64 + 4 * lg;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    u32x2 v;
                    v[0] = f32_to_bf16(acc[i][j][0]) | (f32_to_bf16(acc[i][j][1]) << 16);
                    v[1] = f32_to_bf16(acc[i][j][2]) | (f32_to_bf16(acc[i][j][3]) << 16);
                    *reinterpret_cast<u32x2 *>(crow + 16 * j) = v;
                }
            }
        } else {
            // h-columns of this wave: n0 + 32 wn + 16 j + 4 lg + q, j < 2 (gate j, up j+2)
            float h[8][2][4];
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float g = acc[i][j][q], u = acc[i][j + 2][q];
                        h[i][j][q] = g / (1.0f + expf(-g)) * u;
                    }
            if constexpr (EPI == EPI_SWIGLU_BF16) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int m = row0 + wm * 128 + i * 16 + l16;
                    if (m >= seg1)
                        continue;
                    uint16_t *hrow = reinterpret_cast<uint16_t *>(p.C) + (size_t)m * half_n + n0 + 32 * wn + 4 * lg;
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        u32x2 v;
                        v[0] = f32_to_bf16(h[i][j][0]) | (f32_to_bf16(h[i][j][1]) << 16);
                        v[1] = f32_to_bf16(h[i][j][2]) | (f32_to_bf16(h[i][j][3]) << 16);
                        *reinterpret_cast<u32x2 *>(hrow + 16 * j) = v;
                    }
                }
            } else {
                // fp8 1x128 requant: the tile's 128 h-columns of a row are one scale block,
                // split over the four column waves; exchange partial amax through LDS
                float *red = reinterpret_cast<float *>(scratch);  // [4][256]
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    float mx = 0.0f;
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            mx = fmaxf(mx, fabsf(h[i][j][q]));
                    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                    if (lg == 0)
                        red[wn * 256 + wm * 128 + i * 16 + l16] = mx;
                }
                __syncthreads();
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int r = wm * 128 + i * 16 + l16;
                    const int m = row0 + r;
                    const float amax = fmaxf(fmaxf(fmaxf(red[r], red[256 + r]), fmaxf(red[512 + r], red[768 + r])), 1e-4f);
                    const float inv = 448.0f / amax;
                    if (m < seg1) {
                        uint8_t *hrow = p.C + (size_t)m * half_n + n0 + 32 * wn + 4 * lg;
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            *reinterpret_cast<uint32_t *>(hrow + 16 * j) = f32x4_to_e4m3(
                                h[i][j][0] * inv, h[i][j][1] * inv, h[i][j][2] * inv, h[i][j][3] * inv);
                        if (wn == 0 && lg == 0)
                            p.Cs[(size_t)m * (half_n / 128) + n0 / 128] = amax / 448.0f;
                    }
                }
                __syncthreads();  // red is reused by the next tile
            }
        }
    }
}

size_t gmm_lds_bytes() { return 4 * LDS_TILE + sizeof(GroupTable) + 2 * GTHREADS * sizeof(int); }
// scratch holds 2*GTHREADS = 1024 ints: the group-table scan and the [4][256] fp8 amax exchange

static int g_num_cus = 0;

template <int DT, int EPI> static hipError_t launch_one(const GmmArgs &a, hipStream_t s)
{
    static bool attr_set = false;
    const size_t lds = gmm_lds_bytes();
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void *)gmm_kernel<DT, EPI>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess)
            return e;
        attr_set = true;
    }
    if (g_num_cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&g_num_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            g_num_cus = 0;
        if (g_num_cus <= 0)
            g_num_cus = 256;
    }
    const int grid = (g_num_cus + 7) / 8 * 8;
    hipLaunchKernelGGL((gmm_kernel<DT, EPI>), dim3(grid), dim3(GTHREADS), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_gmm(const GmmArgs &a, int dt, int epi, hipStream_t s)
{
    if (a.L <= 0 || a.L > G_MAX_L || a.M <= 0)
        return hipErrorInvalidValue;
    if (dt == DT_BF16) {
        if (epi == EPI_PLAIN)
            return launch_one<DT_BF16, EPI_PLAIN>(a, s);
        if (epi == EPI_SWIGLU_BF16)
            return launch_one<DT_BF16, EPI_SWIGLU_BF16>(a, s);
    } else if (dt == DT_FP8) {
        if (epi == EPI_PLAIN)
            return launch_one<DT_FP8, EPI_PLAIN>(a, s);
        if (epi == EPI_SWIGLU_FP8)
            return launch_one<DT_FP8, EPI_SWIGLU_FP8>(a, s);
        if (epi == EPI_SWIGLU_BF16)
            return launch_one<DT_FP8, EPI_SWIGLU_BF16>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace cam
