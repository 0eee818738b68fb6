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
//     silu on the left half); h = silu(g) * u, silu(g) = g / (1 + exp(-g)) (hardware exp and reciprocal),
//     stored as bf16, or requantised to fp8 per 1x128 block of h exactly like
//     the dispatch quantiser (post_swiglu_dynamic_quant.h:164-231 requantises
//     per token in int8).
//   GMM2 (EPI_PLAIN): out = bf16(A W^T) per expert
//     (block_epilogue_per_token_dequant.hpp:338-361).
//
// Kernel design (gfx950):
//   * Output tiles of 256, 128 or 32 rows x 256 W rows (SwiGLU: the gate and up rows of one 128-column
//     block of h; the decode plain GEMM 128 W rows), picked per expert from its row count (the Tile
//     struct below); the 128/256-row tiles run 8 waves in a 2 x 4 grid, the 32-row tile 4 waves.  MFMA
//     16x16: v_mfma_f32_16x16x32_bf16, v_mfma_i32_16x16x64_i8, or v_mfma_scale_f32_16x16x128_f8f6f4 with
//     unit scales for fp8.
//   * Operands stream through a ring of LDS stages by direct global->LDS DMA (global_load_lds_dwordx4, or
//     buffer_load_dwordx4 ... lds through a buffer resource for the 128/256-row tiles): no staging
//     registers, and further k-steps stay in flight while one is multiplied.  Each k-step is 128 bytes of
//     every A and W row (64 bf16 / 128 one-byte elements); the fp8 activation scales of the k-step ride the
//     same DMA (4-byte lanes, read k-major [K/128, M] so that one k-step's scales of 64 rows are one
//     contiguous 256-byte run; row-major scales are transposed first).  A wave's loads are counted with
//     s_waitcnt vmcnt and published with a bare s_barrier (no fence, so outstanding prefetches are not
//     drained).
//   * LDS rows are 128 B with the 16-byte chunks XOR-swizzled by (row >> 1) & 7:
//     each lane fetches the global chunk that belongs at its DMA slot, so
//     fragment reads spread over all banks.
//   * MFMA operands are (W fragment, A fragment), so a lane's four
//     accumulators are four consecutive output columns of one row: the
//     epilogue stores 8 contiguous bytes per lane without a transpose.
//   * fp8: one MFMA of K=128 per (i,j) per k-step covers exactly one scale
//     block, so acc += mfma(...) * (a_scale[m] * w_scale[n-block]), applied by the VALU one fragment row
//     after the MFMA that produced it.
//   * Persistent grid (one block per CU) walking tiles expert by expert in
//     groups of 8 M-tiles x all N-tiles (M fastest), remapped so that the
//     blocks of one XCD take consecutive tiles: they share A and W tiles in
//     that XCD's L2.
#include <algorithm>
#include <cstdlib>
#include <atomic>
#include <type_traits>

#include "cam_device.h"
#include "gmm.h"
#include "launchers.h"

namespace cam {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) int i32x8;

#ifndef CAM_GMM_MIN_NK256
#define CAM_GMM_MIN_NK256 16
#endif
#ifndef CAM_GMM_UNROLL2
// the 256-row tile's k-loop unrolled by two, so that the ring slot of each step is a constant and every LDS
// address an immediate offset (measured: the M = 65536 fp8 GMM1 2.18 vs 2.13 PFLOPS, config 3's bf16 GEMMs
// 1.31 vs 1.27 PFLOPS, config 4's 278-284 vs 286 us; fewer address and scalar instructions per k-step)
#define CAM_GMM_UNROLL2 1
#endif
#ifndef CAM_GMM_NT_MAXBM
#define CAM_GMM_NT_MAXBM 32  // tile heights up to this stream their weights nontemporally
#endif

constexpr int GBN = 256, GKB = 128;  // tile W-rows, bytes per row per k-step
constexpr int GMAX_THREADS = 512;    // block size of the largest tile
constexpr int G_MAX_L = 512;

// Tile shapes (BM rows x BN W rows, 128-byte k-steps):
//   BM = 256: 8 waves, 2 x 4 of 128 x 64, 2-stage ring -- half the L2->LDS bytes per FLOP of the
//             128-row tile, for compute-bound prefill;
//   BM = 128: 8 waves, 2 x 4 of 64 x 64, 3-stage ring;
//   BM = 32:  4 waves, 1 x 4 of 32 x 64, 4-stage ring (decode: a handful of rows per expert, the k-loop
//             is a weight stream and the extra stage keeps more of it in flight);
//   BM = 32, BN = 128: 4 waves of 32 x 32, 6-stage ring (the same bytes in flight) -- the decode GEMM
//             without SwiGLU, whose tiles then divide evenly over the CUs.
template <int BM_, int BN_ = GBN> struct Tile {
    static constexpr int BM = BM_, BN = BN_;
    static constexpr int NWAVES = BM >= 128 ? 8 : 4;
    static constexpr int THREADS = 64 * NWAVES;
    static constexpr int WAVES_M = BM >= 128 ? 2 : 1;
    static constexpr int WAVES_N = NWAVES / WAVES_M;
    static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;  // wave tile
    static constexpr int IF = WM / 16, JF = WN / 16;              // MFMA fragments per wave
    static constexpr int STAGES = BM >= 256 ? 2 : BM >= 128 ? 3 : BN >= 256 ? 4 : 6;
    static constexpr int A_BYTES = BM * GKB;
    static constexpr int B_BYTES = BN * GKB;
    static constexpr int S_ROWS = WM > 64 ? WM : 64;  // activation-scale rows a wave DMAs (64 per instruction)
    static constexpr int S_DMAS = S_ROWS / 64;
    static constexpr int S_BYTES = NWAVES * S_ROWS * 4;  // per-wave copies of its rows' activation scales
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES + S_BYTES;
    static constexpr int A_LOADS = A_BYTES / 1024 / NWAVES;  // DMA instructions per wave per stage (1 KiB each)
    static constexpr int B_LOADS = B_BYTES / 1024 / NWAVES;
};

// W rows per tile: 256, except the decode tile (BM = 32) of the plain GEMM (a SwiGLU tile holds the gate and
// up rows of one 128-column scale block of h)
#ifndef CAM_GMM_SMALL_PLAIN_BN
#define CAM_GMM_SMALL_PLAIN_BN 128
#endif
constexpr int small_bn(int bm, int epi) { return bm == 32 && epi == 0 ? CAM_GMM_SMALL_PLAIN_BN : GBN; }

// Expert tables of a launch, built once at kernel start: per tile class (256-, 128- and 32-row tiles) the
// inclusive prefix of M-tiles per expert, and the inclusive prefix of rows per expert (the exclusive prefix
// of expert e is entry e-1, or 0 for e = 0; no entry for it keeps the tables within the LDS budget).
constexpr int G_NCLASS = 3;
constexpr int tile_class(int bm) { return bm >= 256 ? 0 : bm >= 128 ? 1 : 2; }
struct GroupTables {
    int tile_end[G_NCLASS][G_MAX_L];
    int row_end[G_MAX_L];
};
// the experts each class takes: a row count in [lo, hi) (lo >= hi: the class is not used)
struct ClassRanges {
    int lo[G_NCLASS], hi[G_NCLASS];
};

// Readiness between the two GEMMs of a chained launch (launch_gmm_chain): the GMM1 tiles of an M-tile
// produce its h rows, the GMM2 tiles of that M-tile consume them.  Counters are indexed by M-tile over the
// classes in turn (the 256-row M-tiles, then the 128-row ones, then the 32-row ones), the same in both GEMMs
// because both split every expert into the same tile height.
enum SyncRole { SYNC_NONE = 0, SYNC_PRODUCE = 1, SYNC_CONSUME = 2 };
struct GmmSync {
    int *ready;       // per M-tile: GMM1 tiles whose h rows have been stored
    int target;       // GMM1 tiles per M-tile (I / 128); one more when a test makes every wait give up
    long long ticks;  // wait bound in constant-clock ticks
};
// nonzero once a readiness wait has given up (sticky; read and cleared by the host, sync_status_read)
__device__ int g_cam_sync_status;

// The one argument of a chained kernel.  The GEMM loops already hold every scalar register they have, so the
// chained kernels keep nothing of it resident: each use re-reads the field from the kernel-argument segment
// through a pointer the compiler cannot see through (a scalar load), and each phase loads its own GEMM's
// arguments when it starts.
struct ChainParams {
    GmmArgs g1, g2;
    GmmSync sy;
};
__device__ __forceinline__ const ChainParams *chain_params()
{
    uint64_t a = (uint64_t)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(a));
    // (a constant-address-space origin: the loads stay scalar loads)
    return (const ChainParams *)(const __attribute__((address_space(4))) ChainParams *)a;
}

// readiness counters of a chained launch: the M-tiles (at most M/32 + L), then one arrival counter per XCD,
// then one heavy-tile queue per XCD
__host__ __device__ constexpr int chain_arrival_index(int M, int L) { return M / 32 + L + 1; }
__host__ __device__ constexpr int chain_queue_index(int M, int L) { return chain_arrival_index(M, L) + 8; }

// h stores of a producing GMM1 tile: agent-coherent (sc1, written through to memory), so that a GMM2 tile on
// another XCD, whose L2 has never held these lines during the launch, reads them from memory
// (global address-space pointers: the atomics then need no aperture check of a flat address)
template <typename T> __device__ __forceinline__ __attribute__((address_space(1))) T *gptr(T *p)
{
    return (__attribute__((address_space(1))) T *)p;
}
template <bool CO, typename T> __device__ __forceinline__ void st_h(T *p, T v)
{
    if constexpr (CO)
        __hip_atomic_store(gptr(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        *p = v;
}

// Diagnostic build only (-DCAM_GMM_TIMELINE): every block records, per tile, its wall-clock start and end
// (100 MHz constant clock) with the tile's class, expert and index, into 128 slots per block;
// camhipDebugGmmTimeline copies them out.  Off in every product build.
#ifdef CAM_GMM_TIMELINE
constexpr int G_TL_SLOTS = 128, G_TL_BLOCKS = 1024;
__device__ uint64_t g_cam_tl[G_TL_BLOCKS * G_TL_SLOTS][3];
#define CAM_TL_DECL                                                                                             \
    int tl_k = (BM >= 256 ? 0 : BM >= 128 ? 32 : 64) + (ROLE == SYNC_CONSUME ? 16 : 0);                         \
    uint64_t tl_t0 = wall_clock64();
#define CAM_TL_REC(e, tile)                                                                                     \
    do {                                                                                                        \
        const uint64_t tl_t1 = wall_clock64();                                                                  \
        if (threadIdx.x == 0 && blockIdx.x < G_TL_BLOCKS && tl_k < G_TL_SLOTS) {                                \
            uint64_t *r = g_cam_tl[blockIdx.x * G_TL_SLOTS + tl_k];                                              \
            r[0] = ((uint64_t)blockIdx.x << 48) | ((uint64_t)BM << 36) | ((uint64_t)EPI << 32) |                 \
                   ((uint64_t)(e) << 20) | (uint64_t)(tile);                                                    \
            r[1] = tl_t0;                                                                                       \
            r[2] = tl_t1;                                                                                       \
        }                                                                                                       \
        ++tl_k;                                                                                                 \
        tl_t0 = tl_t1;                                                                                          \
    } while (0)
#else
#define CAM_TL_DECL
#define CAM_TL_REC(e, tile)
#endif

// Block-wide exclusive scans of the M-tiles of each tile class and of the rows per expert, from one read of
// the counts.  Only experts with a row count in a class's [lo, hi) get tiles of that class (a launch may
// split the experts between tile heights); the row offsets count every expert (they locate segments in
// dispatch order).
template <int GTHREADS>
__device__ void build_group_tables(const int64_t *__restrict__ group_list, int L, GroupTables &gt, int *scratch,
                                   const ClassRanges &cr)
{
    constexpr int NQ = G_NCLASS + 1;  // tile counts per class, then rows
    constexpr int BMS[G_NCLASS] = {256, 128, 32};
    const int tid = threadIdx.x;
    const int per = (L + GTHREADS - 1) / GTHREADS;
    int cnt[4] = {0, 0, 0, 0};
    auto add = [&](int c, int *v) {
#pragma unroll
        for (int k = 0; k < G_NCLASS; ++k)
            v[k] += (c >= cr.lo[k] && c < cr.hi[k]) ? (c + BMS[k] - 1) / BMS[k] : 0;
        v[G_NCLASS] += c;
    };
    for (int q = 0; q < per; ++q) {
        const int e = tid * per + q;
        if (e < L)
            add((int)group_list[e], cnt);
    }
    // exclusive scan: within each wave by lane shuffles, then over the waves' totals
    constexpr int NWV = GTHREADS / 64;
    const int lane = tid & 63, wv = tid >> 6;
    int inc[NQ];
#pragma unroll
    for (int k = 0; k < NQ; ++k)
        inc[k] = cnt[k];
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
#pragma unroll
        for (int k = 0; k < NQ; ++k) {
            const int u = __shfl_up(inc[k], d, 64);
            if (lane >= d)
                inc[k] += u;
        }
    }
    if (lane == 63) {
#pragma unroll
        for (int k = 0; k < NQ; ++k)
            scratch[k * NWV + wv] = inc[k];
    }
    __syncthreads();
    int run[NQ];
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        int ex = inc[k] - cnt[k];
#pragma unroll
        for (int v = 0; v < NWV; ++v)
            ex += v < wv ? scratch[k * NWV + v] : 0;
        run[k] = ex;
    }
    for (int q = 0; q < per; ++q) {
        const int e = tid * per + q;
        if (e < L) {
            add((int)group_list[e], run);
#pragma unroll
            for (int k = 0; k < G_NCLASS; ++k)
                gt.tile_end[k][e] = run[k];
            gt.row_end[e] = run[G_NCLASS];
        }
    }
    __syncthreads();
}

// LDS byte offset of 16-byte chunk `chunk` of row `row`.  Chunks are XOR-swizzled by (row >> 1) & 7:
// two 128-byte rows share one 256-byte bank row, so the 16 rows of a fragment read (same logical
// chunk) land on 16 distinct 16-byte bank groups.
__device__ __forceinline__ int swz(int row, int chunk) { return row * GKB + ((chunk ^ ((row >> 1) & 7)) << 4); }

// the lane's index in its wave, from mbcnt (no work-item id register)
__device__ __forceinline__ int lane_id() { return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// s_waitcnt with only vmcnt constrained (expcnt and lgkmcnt at their maxima)
template <int N> __device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (7 << 4) | (0xF << 8));
}

// s_waitcnt vmcnt(N) and lgkmcnt(0): this wave's older DMAs and all of its LDS reads are done
template <int N> __device__ __forceinline__ void wait_vmcnt_lgkm0()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (7 << 4));
}

// barrier without a memory fence: prefetches in flight stay in flight
__device__ __forceinline__ void bar()
{
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ void dma16(const void *g, void *lds)
{
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)lds, 16, 0, 0);
}
// the same with the nontemporal cache policy: a stream read once (decode weights) is not kept in L2
__device__ __forceinline__ void dma16_nt(const void *g, void *lds)
{
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)lds, 16, 0, 2);
}
__device__ __forceinline__ void dma4(const void *g, void *lds)
{
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)lds, 4, 0, 0);
}
// agent-coherent (sc1): data another XCD may have written during the launch
__device__ __forceinline__ void dma4_sc1(const void *g, void *lds)
{
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)lds, 4, 0, 16);
}

// The same DMAs through a buffer resource: the base sits in four SGPRs, the lane's 32-bit byte offset in one
// VGPR and the k-step's offset in an SGPR, so a DMA needs no 64-bit address registers and no address
// arithmetic per k-step.  Offsets are 32-bit, as the flat addresses' per-lane offsets already are: the C ABI
// rejects activations or one expert's weights of 4 GiB or more, and the activation scales are a 32nd of the
// activations.  The record count is unbounded (no range check, as with flat addresses).
#ifndef CAM_GMM_BUFDMA
#define CAM_GMM_BUFDMA 1
#endif
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *base)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, -1, 0x00020000);
}
template <int BYTES, int AUX>
__device__ __forceinline__ void bdma(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, void *lds)
{
    auto *l = (__attribute__((address_space(3))) void *)lds;
    if constexpr (BYTES == 4 && AUX == 16)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, l, 4, voff, soff, 0, 16);
    else if constexpr (BYTES == 4)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, l, 4, voff, soff, 0, 0);
    else if constexpr (AUX == 2)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, l, 16, voff, soff, 0, 2);
    else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, l, 16, voff, soff, 0, 0);
}

// scalar (SMEM) load of a block-uniform element of read-only data: it counts on lgkmcnt, not on the
// vmcnt of the DMA ring, so it never makes a wait drain prefetches
__device__ __forceinline__ float sload(const float *p, int idx)
{
    return ((const __attribute__((address_space(4))) float *)p)[idx];
}

// LDS-only barrier: this wave's LDS traffic has completed, then every wave meets; DMAs in flight stay
// in flight
__device__ __forceinline__ void lds_sync()
{
    __builtin_amdgcn_s_waitcnt(0xF | (3 << 14) | (7 << 4));  // lgkmcnt(0), vmcnt and expcnt at their maxima
    bar();
}

// Tiles of the experts with a row count in [lo, hi); this block takes tiles first, first + G, ...
// (first == -1: balanced placement, see below; G_DYN: a dynamic queue), preceded by a run of rn tiles rs, rs + rstride, ... (an
// increasing sequence: the first index past the class's tiles ends it).
// ROLE (chained launches only): SYNC_PRODUCE tiles store h agent-coherently and count each finished tile in
// sy.ready; SYNC_CONSUME tiles start their DMAs only once sy.ready of their M-tile has reached sy.target.  Waves
// beyond the tile's own (a 32-row class run by an 8-wave block) are spectators: they issue no DMA, MFMA or store
// and only meet the block's barriers.
constexpr int G_DYN = -2;  // gmm_body's `first` for a dynamic tile queue (see there)

// EAGER (the 4-wave chained kernel): a producer's primed tile counts its predecessor at k-step edge STAGES-2
// instead of after its k-loop (a branch inside the k-loop, which the 8-wave kernels cannot afford).  bid: the
// block's position for balanced placement (a chained consumer passes its arrival order), -1: blockIdx.x.
// wv: the wave's index in the block (a scalar the kernel computes once; -1: from threadIdx.x).  The body
// takes the lane from mbcnt and never reads the work-item id: a register holding it through the whole kernel
// gets spilled, and each reload before a k-loop makes the loop wait for it at every iteration.
template <int DT, int EPI, int BM, bool NTW = (BM <= CAM_GMM_NT_MAXBM), int ROLE = SYNC_NONE, bool EAGER = false>
__device__ __forceinline__ void gmm_body(const GmmArgs &p, const GroupTables *gtab, int first, int rs = 0, int rn = 0,
                                         int rstride = 1, int bid = -1, int wv = -1)
{
    using TC = Tile<BM, small_bn(BM, EPI)>;
    constexpr int TBN = TC::BN;
    constexpr int NW = TC::NWAVES;
    constexpr int GBM = TC::BM, WM = TC::WM, WN = TC::WN, IF = TC::IF, JF = TC::JF;
    constexpr int GSTAGES = TC::STAGES, STAGE_BYTES = TC::STAGE_BYTES;
    constexpr int A_BYTES = TC::A_BYTES, B_BYTES = TC::B_BYTES, A_LOADS = TC::A_LOADS, B_LOADS = TC::B_LOADS;
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    // the epilogue's exchange area (fp8 amax, int8 row maxima) follows this class's ring
    int *scratch = reinterpret_cast<int *>(smem + GSTAGES * STAGE_BYTES);
    const int *tile_end = gtab->tile_end[tile_class(BM)];
    auto tile_prefix = [&](int e) { return e > 0 ? tile_end[e - 1] : 0; };
    auto row_off = [&](int e) { return e > 0 ? gtab->row_end[e - 1] : 0; };

    const int lane = lane_id();
    const int w = wv >= 0 ? wv : __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const bool first_thread = w == 0 && lane == 0;
    const int wm = w / TC::WAVES_N, wn = w % TC::WAVES_N;
    const int l16 = lane & 15, lg = lane >> 4;
    constexpr bool PRODUCE = ROLE == SYNC_PRODUCE, CONSUME = ROLE == SYNC_CONSUME;
    const bool spect = ROLE != SYNC_NONE && NW < 8 && w >= NW;  // (8-wave tiles never have spectators)
    // M-tiles of the classes before this one (the readiness counters' index base), read when needed
    auto cls_base = [&]() {
        int b = 0;
#pragma unroll
        for (int k = 0; k < tile_class(BM); ++k)
            b += gtab->tile_end[k][p.L - 1];
        return __builtin_amdgcn_readfirstlane(b);
    };
    constexpr bool SWIGLU = EPI != EPI_PLAIN;
    constexpr bool FP8 = DT == DT_FP8;
    constexpr bool INT8 = DT == DT_INT8;
    constexpr int LOADS = A_LOADS + B_LOADS + (FP8 ? TC::S_DMAS : 0);  // DMA instructions per wave per stage
    const int esz = DT == DT_BF16 ? 2 : 1;
    const uint32_t kbytes = (uint32_t)p.K * esz;  // bytes per row
    const int nk = (int)(kbytes / GKB);
    const int half_n = p.N / 2;                    // I for SwiGLU
    const int ntn = SWIGLU ? half_n / 128 : p.N / TBN;
    const int total = __builtin_amdgcn_readfirstlane(tile_prefix(p.L)) * ntn;

    // first == -1: this launch has one tile class, so balance it: with R = ceil(total / grid) rounds, only
    // the first ceil(total / R) blocks (rounded up to whole XCDs) take tiles, R each at most.  A weight
    // stream is bound by aggregate HBM bandwidth, which that many CUs still saturate, and no CU is left
    // streaming a final partial round alone.  Otherwise the caller's position and the full grid stride.
    int G = gridDim.x, logical = first;
    // G_DYN (chained consumer, 256-row tiles): tiles rs, rs + 1, ... rs + rn - 1 handed out one at a time by
    // the queue counter SY().ready[rstride], shared by the blocks of one XCD
    const bool dyn = CONSUME && BM >= 256 && first == G_DYN;
    if (first == -1) {
        const int b = bid >= 0 ? bid : (int)blockIdx.x;
        const int rounds = max((total + G - 1) / G, 1);
        const int g_eff = min(G, ((total + rounds - 1) / rounds + 7) / 8 * 8);
        if (b >= g_eff)
            return;
        G = g_eff;
        logical = (b & 7) * (G >> 3) + (b >> 3);
    }
    // the block's k-th tile: the run, then the strided sequence
    auto seq = [&](int k) { return k < rn ? rs + k * rstride : logical + (k - rn) * G; };

    // DMA slot of this lane inside a 1 KiB band (8 rows x 128 B): row l/8, physical chunk l%8,
    // which holds logical chunk (l%8) ^ ((row >> 1) & 7) -- see swz()
    const int band_row = lane >> 3;
    auto chunk_off = [&](int r) { return (uint32_t)(((lane & 7) ^ ((r >> 1) & 7)) << 4); };

    // ---- one tile's coordinates and the per-lane sources of this wave's DMA bands
    struct Ctx {
        int e, row0, seg1, n0;
        const uint8_t *wbase;
        const float *wsb;  // this expert's weight scales (fp8 block or int8 per-channel), or null
        uint32_t ga[A_LOADS], gb[B_LOADS], gs[TC::S_DMAS];
        int wsg, wsu;  // fp8: weight-scale row offsets (gate / up n-blocks, or the wave's column block)
        int active;    // some row of this wave lies inside the segment (an int: a bool tail makes struct copies go through scratch)
    };
    auto setup = [&](int tile, Ctx &c) {
        int lo = 0, hi = p.L - 1;
        while (lo < hi) {  // last e with tile_prefix[e]*ntn <= tile
            const int mid = (lo + hi + 1) >> 1;
            if (tile_end[mid - 1] * ntn <= tile)
                lo = mid;
            else
                hi = mid - 1;
        }
        const int e = __builtin_amdgcn_readfirstlane(lo);
        c.e = e;
        const int mt_e = __builtin_amdgcn_readfirstlane(tile_end[e] - tile_prefix(e));
        const int local = __builtin_amdgcn_readfirstlane(tile - tile_prefix(e) * ntn);
        // within the expert: groups of up to 8 M-tiles, N-tiles in turn, the group's M-tiles
        // fastest -- a run of consecutive tiles (one XCD's share of a round) covers ~8 A row blocks
        // x a few W column blocks, so both operands are re-read from that XCD's L2
        constexpr int GM = 8;
        const int grp = local / (GM * ntn), rem = local % (GM * ntn);
        const int gm = min(GM, mt_e - grp * GM);
        const int nt = rem / gm, mt = grp * GM + rem % gm;
        const int seg0 = __builtin_amdgcn_readfirstlane(row_off(e));
        c.seg1 = min(__builtin_amdgcn_readfirstlane(gtab->row_end[e]), p.M);  // never write past row M
        c.row0 = seg0 + mt * GBM;
        c.n0 = SWIGLU ? nt * 128 : nt * TBN;  // first h-column (SwiGLU) or W row (plain)
        // a wave whose rows all lie past the segment skips its MFMAs (it still moves its share of the
        // DMA and meets every barrier): a tile of a short segment costs little more than its weights
        c.active = !spect && c.row0 + wm * WM < c.seg1;

        if (p.Wl) {  // separated weights: one allocation per expert, pointers read by scalar loads (a vector
                     // load here would make the tile switch wait for every DMA in flight)
            c.wbase = reinterpret_cast<const uint8_t *>(
                ((const __attribute__((address_space(4))) uint64_t *)p.Wl)[e]);
            c.wsb = p.Wsl ? reinterpret_cast<const float *>(((const __attribute__((address_space(4))) uint64_t *)p.Wsl)[e])
                          : nullptr;
        } else {
            c.wbase = p.W + (size_t)e * p.N * kbytes;
            c.wsb = !p.Ws ? nullptr : p.Ws + (INT8 ? (size_t)e * p.N : (size_t)e * (p.N / 128) * nk);
        }
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) {
            const int r = (i * NW + w) * 8 + band_row;  // tile row 0..GBM-1
            c.ga[i] = (uint32_t)min(c.row0 + r, c.seg1 - 1) * kbytes + chunk_off(r);
        }
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) {
            const int r = (i * NW + w) * 8 + band_row;  // LDS W row 0..255
            int wrow;
            if (SWIGLU) {
                // LDS rows [WN c, WN c + WN) feed column wave c: WN/2 gate rows, then the
                // WN/2 up rows of the same h-columns
                const int cw = r / WN, jj = r % WN;
                const int hcol = c.n0 + (WN / 2) * cw + (jj % (WN / 2));
                wrow = jj < WN / 2 ? hcol : half_n + hcol;
            } else {
                wrow = c.n0 + r;
            }
            c.gb[i] = (uint32_t)wrow * kbytes + chunk_off(r);
        }
        // fp8: this wave's activation-scale rows (the WM rows of its row block wm, 64 per DMA), placed so that
        // the IF rows a lane multiplies (16 i + l16, i < IF) sit next to each other: LDS slot p holds row
        // (p % IF) 16 + p / IF, and a lane reads its IF scales with one or two vector reads per k-step
        // (per-row 4-byte reads interleaved with the MFMAs: the M = 65536 fp8 GEMMs ~3% slower)
#pragma unroll
        for (int d = 0; d < TC::S_DMAS; ++d) {
            const int p = d * 64 + lane;
            const int r = p < WM ? (p % IF) * 16 + p / IF : p;
            c.gs[d] = (uint32_t)min(c.row0 + wm * WM + r, c.seg1 - 1);  // k-major: + kc * M
        }
        c.wsg = ((SWIGLU ? c.n0 : c.n0 + wn * WN) / 128) * nk;
        c.wsu = SWIGLU ? ((half_n + c.n0) / 128) * nk : c.wsg;
    };
    // DMA instruction q (0 <= q < LOADS) of k-step kc of tile c into ring slot `slot`: A bands, then
    // W bands, then (fp8) the activation scales
    auto dma_one = [&](const Ctx &c, int kc, int slot, int q) {
        if (spect)
            return;
        uint8_t *st = smem + slot * STAGE_BYTES;
        if constexpr (CAM_GMM_BUFDMA && BM >= 128) {  // (the decode tile measured 0.4 us slower per step this way)
            if (q < A_LOADS) {
                bdma<16, 0>(buf_rsrc(p.A), c.ga[q], (uint32_t)kc * GKB, st + (q * NW + w) * 1024);
            } else if (q < A_LOADS + B_LOADS) {
                const int i = q - A_LOADS;
                bdma<16, NTW ? 2 : 0>(buf_rsrc(c.wbase), c.gb[i], (uint32_t)kc * GKB,
                                      st + A_BYTES + (i * NW + w) * 1024);
            } else {
                const int d = q - A_LOADS - B_LOADS;
                bdma<4, CONSUME ? 16 : 0>(buf_rsrc(p.As), c.gs[d] * 4u, (uint32_t)kc * (uint32_t)p.M * 4u,
                                          st + A_BYTES + B_BYTES + w * TC::S_ROWS * 4 + d * 256);
            }
            return;
        }
        if (q < A_LOADS) {
            dma16(p.A + c.ga[q] + (uint32_t)kc * GKB, st + (q * NW + w) * 1024);
        } else if (q < A_LOADS + B_LOADS) {
            const int i = q - A_LOADS;
            // decode tiles and the light experts' tiles of a skewed prefill launch (NTW): the weights are a
            // stream read about once, fetched nontemporally (measured: the config-5 decode step 244 vs
            // 274 us, config 4's GMM1 216 vs 222 us)
            if constexpr (NTW)
                dma16_nt(c.wbase + c.gb[i] + (uint32_t)kc * GKB, st + A_BYTES + (i * NW + w) * 1024);
            else
                dma16(c.wbase + c.gb[i] + (uint32_t)kc * GKB, st + A_BYTES + (i * NW + w) * 1024);
        } else {
            const int d = q - A_LOADS - B_LOADS;
            if constexpr (CONSUME)
                dma4_sc1(p.As + c.gs[d] + (size_t)kc * p.M, st + A_BYTES + B_BYTES + w * TC::S_ROWS * 4 + d * 256);
            else
                dma4(p.As + c.gs[d] + (size_t)kc * p.M, st + A_BYTES + B_BYTES + w * TC::S_ROWS * 4 + d * 256);
        }
    };

    f32x4 acc[IF][JF];
    // fp8: the lane's IF activation scales of a stage (rows 16 i + l16), contiguous in the wave's scale slot
    auto rd_scales = [&](const uint8_t *st, float *sa) {
        const float *sp = reinterpret_cast<const float *>(st + A_BYTES + B_BYTES + w * TC::S_ROWS * 4) + l16 * IF;
        if constexpr (IF % 4 == 0) {
#pragma unroll
            for (int q = 0; q < IF / 4; ++q) {
                const f32x4 v = reinterpret_cast<const f32x4 *>(sp)[q];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    sa[4 * q + u] = v[u];
            }
        } else {
#pragma unroll
            for (int q = 0; q < IF; ++q)
                sa[q] = sp[q];
        }
    };

    // ---- epilogue: lane holds rows m = row0 + wm*WM + 16 i + l16 and, per j, four
    // consecutive columns 16 j + 4 lg + q of the wave's WN-wide column range
    auto epilogue = [&](const Ctx &c) {
        if (spect) {
            if constexpr (EPI == EPI_SWIGLU_FP8) {
                lds_sync();  // the two exchange barriers of the fp8 requantisation
                lds_sync();
            }
            return;
        }
        const int row0 = c.row0, seg1 = c.seg1, n0 = c.n0;
        if constexpr (EPI == EPI_PLAIN) {
#pragma unroll
            for (int i = 0; i < IF; ++i) {
                const int m = row0 + wm * WM + i * 16 + l16;
                if (m >= seg1)
                    continue;
                uint16_t *crow = reinterpret_cast<uint16_t *>(p.C) + (size_t)m * p.N + n0 + wn * WN + 4 * lg;
#pragma unroll
                for (int j = 0; j < JF; ++j) {
                    u32x2 v;
                    v[0] = f32x2_to_bf16x2(acc[i][j][0], acc[i][j][1]);
                    v[1] = f32x2_to_bf16x2(acc[i][j][2], acc[i][j][3]);
                    *reinterpret_cast<u32x2 *>(crow + 16 * j) = v;
                }
            }
        } else {
            // h-columns of this wave: n0 + (WN/2) wn + 16 j + 4 lg + q, j < JF/2 (gate j, up j+JF/2)
            constexpr int HF = JF / 2;
            float h[IF][HF][4];
#pragma unroll
            for (int i = 0; i < IF; ++i)
#pragma unroll
                for (int j = 0; j < HF; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float g = acc[i][j][q], u = acc[i][j + HF][q];
                        // silu(g) = g / (1 + exp(-g)) with the hardware exp and reciprocal (about 1 ulp
                        // each; measured: the decode step 1 us and the M = 65536 fp8 GMM1 4% faster than
                        // the correctly rounded division)
                        h[i][j][q] = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
                    }
            if constexpr (EPI == EPI_SWIGLU_F32AMAX) {
                // fp32 h and this wave's partial row maximum of |h| (its 32 h-columns), one slot per wave and
                // row, so the requantisation needs no zeroed buffer and no atomics
#pragma unroll
                for (int i = 0; i < IF; ++i) {
                    const int m = row0 + wm * WM + i * 16 + l16;
                    float mx = 0.0f;
#pragma unroll
                    for (int j = 0; j < HF; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            mx = fmaxf(mx, fabsf(h[i][j][q]));
                    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                    if (m < seg1) {
                        float *hrow = reinterpret_cast<float *>(p.C) + (size_t)m * half_n + n0 + (WN / 2) * wn + 4 * lg;
#pragma unroll
                        for (int j = 0; j < HF; ++j)
                            *reinterpret_cast<f32x4 *>(hrow + 16 * j) =
                                f32x4{h[i][j][0], h[i][j][1], h[i][j][2], h[i][j][3]};
                        static_assert(WN / 2 == GMM_AMAX_COLS, "one partial maximum per wave's h-columns");
                        if (lg == 0)
                            p.Cs[(size_t)m * (half_n / GMM_AMAX_COLS) + n0 / GMM_AMAX_COLS + wn] = mx;
                    }
                }
            } else if constexpr (EPI == EPI_SWIGLU_BF16) {
#pragma unroll
                for (int i = 0; i < IF; ++i) {
                    const int m = row0 + wm * WM + i * 16 + l16;
                    if (m >= seg1)
                        continue;
                    uint16_t *hrow =
                        reinterpret_cast<uint16_t *>(p.C) + (size_t)m * half_n + n0 + (WN / 2) * wn + 4 * lg;
#pragma unroll
                    for (int j = 0; j < HF; ++j) {
                        const uint64_t v = (uint64_t)f32x2_to_bf16x2(h[i][j][0], h[i][j][1]) |
                                           ((uint64_t)f32x2_to_bf16x2(h[i][j][2], h[i][j][3]) << 32);
                        st_h<PRODUCE>(reinterpret_cast<uint64_t *>(hrow + 16 * j), v);
                    }
                }
            } else {
                // fp8 1x128 requant: the tile's 128 h-columns of a row are one scale block,
                // split over the column waves; exchange partial amax through LDS.  The lane's row and
                // column offsets are recomputed here from the lane id (mbcnt): values kept from the kernel's
                // start are spilled by the k-loop, and each reload would wait on every store issued before it
                const int lid = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
                const int l16 = lid & 15, lg = lid >> 4;
                float *red = reinterpret_cast<float *>(scratch);  // [WAVES_N][GBM]
#pragma unroll
                for (int i = 0; i < IF; ++i) {
                    float mx = 0.0f;
#pragma unroll
                    for (int j = 0; j < HF; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            mx = fmaxf(mx, fabsf(h[i][j][q]));
                    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                    if (lg == 0)
                        red[wn * GBM + wm * WM + i * 16 + l16] = mx;
                }
                lds_sync();
                // every row's block maximum first, then all the stores back to back: a register reload
                // between two rows' stores would wait for the earlier stores to complete (vmcnt counts both)
                float amx[IF];
#pragma unroll
                for (int i = 0; i < IF; ++i) {
                    const int r = wm * WM + i * 16 + l16;
                    float amax = 1e-4f;
#pragma unroll
                    for (int cc = 0; cc < TC::WAVES_N; ++cc)
                        amax = fmaxf(amax, red[cc * GBM + r]);
                    amx[i] = amax;
                }
#pragma unroll
                for (int i = 0; i < IF; ++i) {
                    const int m = row0 + wm * WM + i * 16 + l16;
                    const float inv = 448.0f / amx[i];
                    if (m < seg1) {
                        uint8_t *hrow = p.C + (size_t)m * half_n + n0 + (WN / 2) * wn + 4 * lg;
#pragma unroll
                        for (int j = 0; j < HF; ++j)
                            st_h<PRODUCE>(reinterpret_cast<uint32_t *>(hrow + 16 * j),
                                          f32x4_to_e4m3(h[i][j][0] * inv, h[i][j][1] * inv, h[i][j][2] * inv,
                                                        h[i][j][3] * inv));
                        if (wn == 0 && lg == 0)
                            st_h<PRODUCE>(p.Cs + (size_t)(n0 / 128) * p.M + m, amx[i] / 448.0f);  // k-major h scales
                    }
                }
                lds_sync();  // red is reused by the next tile
            }
        }
    };
    auto clear_acc = [&]() {
#pragma unroll
        for (int i = 0; i < IF; ++i)
#pragma unroll
            for (int j = 0; j < JF; ++j)
                acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    };

    // int8: per-channel x per-token dequantisation of the exact int32 sums:
    // v = ((float)acc * w_scale[n]) * x_scale[m]  (block_epilogue_per_token_dequant*.h)
    auto dequant_int8 = [&](const Ctx &cur) {
        if constexpr (INT8) {
            const float *wsr = cur.wsb;
#pragma unroll
            for (int j = 0; j < JF; ++j) {
                int c0;
                if (SWIGLU) {
                    const int jj = j % (JF / 2);
                    c0 = cur.n0 + (WN / 2) * wn + 16 * jj + 4 * lg + (j >= JF / 2 ? half_n : 0);
                } else {
                    c0 = cur.n0 + wn * WN + 16 * j + 4 * lg;
                }
                const f32x4 wv = *reinterpret_cast<const f32x4 *>(wsr + c0);
#pragma unroll
                for (int i = 0; i < IF; ++i) {
                    const float xs = p.As[min(cur.row0 + wm * WM + i * 16 + l16, p.M - 1)];
                    const i32x4 iv = __builtin_bit_cast(i32x4, acc[i][j]);
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        acc[i][j][q] = ((float)iv[q] * wv[q]) * xs;
                }
            }
        }
    };

    // ---- readiness (chained launches).  A producer counts a tile once every wave's h stores have completed:
    // each wave's vmcnt wait that covers them, then a barrier, then one atomic add by thread 0.  A consumer
    // wave polls the counter of the tile's M-tile (lane 0, agent-coherent load) before the tile's first DMA.
    auto SY = [&]() -> GmmSync { return chain_params()->sy; };  // (chained kernels only)
    // the counter of a tile's M-tile, from its context
    auto mti_ctx = [&](const Ctx &c) {
        return __builtin_amdgcn_readfirstlane(cls_base() + tile_prefix(c.e) + (c.row0 - row_off(c.e)) / GBM);
    };
    int sig = -1;      // producer: counter of the tile whose stores are still to be counted
    int gave_up = 0;   // consumer: a wait of this wave gave up (the launch's outputs are void; no more waits)
    auto signal = [&]() {
        if constexpr (PRODUCE) {
            if (sig >= 0 && first_thread)
                __hip_atomic_fetch_add(gptr(SY().ready + sig), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            sig = -1;
        }
    };
    auto poll = [&](int m) -> int {
        int v = 0;
        if (lane == 0)
            v = __hip_atomic_load(gptr(SY().ready + m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return __builtin_amdgcn_readfirstlane(v);
    };
    auto wait_ready = [&](int m) {
        if constexpr (CONSUME) {
            if (spect || gave_up)
                return;
            const uint64_t t0 = wall_clock64();
            while (poll(m) < SY().target) {
                if ((long long)(wall_clock64() - t0) > SY().ticks) {
                    if (lane == 0)
                        __hip_atomic_fetch_or(gptr(&g_cam_sync_status), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    gave_up = 1;
                    return;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        }
    };
    // the M-tile counter of a tile index (the expert search of setup, nothing else)
    auto mti_of = [&](int tile) {
        int lo = 0, hi = p.L - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (tile_end[mid - 1] * ntn <= tile)
                lo = mid;
            else
                hi = mid - 1;
        }
        const int e = __builtin_amdgcn_readfirstlane(lo);
        const int local = tile - tile_prefix(e) * ntn;
        constexpr int GM = 8;
        const int mt_e = tile_end[e] - tile_prefix(e);
        const int grp = local / (GM * ntn), rem = local % (GM * ntn);
        const int gm = min(GM, mt_e - grp * GM);
        return __builtin_amdgcn_readfirstlane(cls_base() + tile_prefix(e) + grp * GM + rem % gm);
    };

    if constexpr (BM >= 256) {
        // 256-row tile (8 waves of 128 x 64; fp8, bf16 or int8): half the L2->LDS bytes per FLOP of the 128-row
        // tile.  Its accumulators leave no room for a second register set, so: two LDS stages, the
        // W fragments of a k-step read once after the barrier, the A fragments streamed AHEAD rows
        // in front of the MFMAs that use them (the other wave on the SIMD covers the W read), the
        // next k-step's A bands issued during the first half of this k-step's MFMAs and the W bands
        // of the k-step after it from the middle on (a second barrier frees the W slot as soon as the
        // fragments are in registers).  Tiles do not overlap: each starts with its own first DMA and
        // drains at its end.  bf16 and int8 run the same loop with two chained K-half MFMAs per fragment pair
        // and no block scaling (measured against the generic two-stage loop, which waits for the whole ring
        // at every k-step: config 3's bf16 GEMMs 1.16 -> 1.27 PFLOPS, the int8 M-sweep's GMM1 +11%).
        static_assert(GSTAGES == 2, "two-stage ring");
        // A rows read ahead of their MFMAs (1, 2 or 3 measured within 1% of each other); the chained kernel
        // reads one row ahead, whose registers its scalar spill lanes need
        constexpr int AHEAD = ROLE == SYNC_NONE ? 2 : 1;
        // a tile's first DMAs: the W bands of k-step 0, its A bands and scales, then the W bands of k-step 1
        auto prime = [&](const Ctx &c) {
#pragma unroll
            for (int q = A_LOADS; q < A_LOADS + B_LOADS; ++q)
                dma_one(c, 0, 0, q);
#pragma unroll
            for (int q = 0; q < LOADS; ++q)
                if (q < A_LOADS || q >= A_LOADS + B_LOADS)
                    dma_one(c, 0, 0, q);
#pragma unroll
            for (int q = A_LOADS; q < A_LOADS + B_LOADS; ++q)
                dma_one(c, min(1, nk - 1), 1, q);
        };
        // dynamic queue: thread 0 takes the next index and publishes the tile through the (plain-epilogue,
        // so unused) exchange area; past the queue's end, `total`
        int *qslot = reinterpret_cast<int *>(scratch) + 128;
        auto take = [&]() {
            if constexpr (CONSUME) {
                return __hip_atomic_fetch_add(gptr(SY().ready + rstride), 1, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
            }
            return 0;
        };
        auto publish = [&](int k) {
            if (first_thread)
                *qslot = k < rn ? rs + k : total;
            lds_sync();
            return __builtin_amdgcn_readfirstlane(*qslot);
        };
        int kt = 0, tile;
        if (dyn) {
            const int k = first_thread ? take() : 0;
            tile = publish(k);
        } else {
            tile = seq(0);
        }
        Ctx c;
        CAM_TL_DECL
        if (tile < total) {
            setup(tile, c);
            wait_ready(mti_ctx(c));
            prime(c);
        }
        int next_ready = 0;  // consumer: the next tile's counter, polled while this tile's ring drains
        while (tile < total) {
            if constexpr (PRODUCE) {
                // the previous tile's h stores preceded this tile's first LOADS + B_LOADS DMAs (prime): once
                // no more than those are in flight in any wave, the stores have completed
                if (sig >= 0) {
                    wait_vmcnt<LOADS + B_LOADS>();
                    bar();
                    signal();
                }
            }
            clear_acc();
            f32x4 pend[JF];
            float ps[JF];
#pragma unroll
            for (int j = 0; j < JF; ++j) {
                pend[j] = f32x4{0.f, 0.f, 0.f, 0.f};
                ps[j] = 0.0f;
            }
            // one k-step; SL = ks & 1, the ring slot (a compile-time constant under CAM_GMM_UNROLL2, so that
            // every LDS address of the step is an immediate offset)
            auto kstep = [&](auto act, int ks, auto slc) {
                {
                    constexpr int SL0 = decltype(slc)::value;
                    const int SL = SL0 >= 0 ? SL0 : (ks & 1);
                    // k-step ks has landed (only the W bands of ks+1, issued last, may still be in flight);
                    // this wave's reads of k-step ks-1 are done
                    wait_vmcnt_lgkm0<B_LOADS>();
                    bar();  // ... for every wave: the A/scale slot (ks+1)%2 is free
                    const uint8_t *st = smem + SL * STAGE_BYTES;
                    const uint8_t *la = st + (wm * WM) * GKB;
                    const uint8_t *lb = st + A_BYTES + (wn * WN) * GKB;
                    i32x8 b[JF], a[IF];
                    float sa[IF];
                    auto rd_a = [&](int i) {
                        const u32x4 v0 = *reinterpret_cast<const u32x4 *>(la + swz(i * 16 + l16, lg));
                        const u32x4 v1 = *reinterpret_cast<const u32x4 *>(la + swz(i * 16 + l16, 4 + lg));
                        a[i] = i32x8{(int)v0[0], (int)v0[1], (int)v0[2], (int)v0[3],
                                     (int)v1[0], (int)v1[1], (int)v1[2], (int)v1[3]};
                    };
                    if constexpr (FP8)
                        rd_scales(st, sa);
#pragma unroll
                    for (int j = 0; j < JF; ++j) {
                        const u32x4 v0 = *reinterpret_cast<const u32x4 *>(lb + swz(j * 16 + l16, lg));
                        const u32x4 v1 = *reinterpret_cast<const u32x4 *>(lb + swz(j * 16 + l16, 4 + lg));
                        b[j] = i32x8{(int)v0[0], (int)v0[1], (int)v0[2], (int)v0[3],
                                     (int)v1[0], (int)v1[1], (int)v1[2], (int)v1[3]};
                    }
                    float sg = 0.0f, su = 0.0f;
                    if constexpr (FP8) {
                        sg = sload(c.wsb, c.wsg + ks);
                        su = SWIGLU ? sload(c.wsb, c.wsu + ks) : sg;
                    }
                    const int kn = min(ks + 1, nk - 1);  // past the end: reload the last k-step
#pragma unroll
                    for (int i = 0; i < AHEAD; ++i)
                        rd_a(i);
#pragma unroll
                    for (int i = 0; i < IF; ++i) {
                        if (i + AHEAD < IF)
                            rd_a(i + AHEAD);
                        const float sgi = FP8 ? sa[i] * sg : 0.0f, sui = FP8 ? sa[i] * su : 0.0f;
                        const int pi = i == 0 ? IF - 1 : i - 1;  // row of the pending results
#pragma unroll
                        for (int j = 0; j < JF; ++j) {
                            if constexpr (decltype(act)::value && !FP8) {
                                // bf16 / int8: the lane's two 16-byte chunks are the k-step's two K halves
                                // (32 bf16 or 64 int8 elements each); int8 accumulates exact int32 sums
                                const i32x4 b0 = {b[j][0], b[j][1], b[j][2], b[j][3]}, b1 = {b[j][4], b[j][5], b[j][6], b[j][7]};
                                const i32x4 a0 = {a[i][0], a[i][1], a[i][2], a[i][3]}, a1 = {a[i][4], a[i][5], a[i][6], a[i][7]};
                                if constexpr (INT8) {
                                    i32x4 t = __builtin_bit_cast(i32x4, acc[i][j]);
                                    t = __builtin_amdgcn_mfma_i32_16x16x64_i8(b0, a0, t, 0, 0, 0);
                                    t = __builtin_amdgcn_mfma_i32_16x16x64_i8(b1, a1, t, 0, 0, 0);
                                    acc[i][j] = __builtin_bit_cast(f32x4, t);
                                } else {
                                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                        __builtin_bit_cast(bf16x8, b0), __builtin_bit_cast(bf16x8, a0), acc[i][j], 0, 0, 0);
                                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                        __builtin_bit_cast(bf16x8, b1), __builtin_bit_cast(bf16x8, a1), acc[i][j], 0, 0, 0);
                                }
                            } else if constexpr (decltype(act)::value) {
                                const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                                const f32x4 d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b[j], a[i], z, 0,
                                                                                                 0, 0, 127, 0, 127);
#pragma unroll
                                for (int q = 0; q < 4; ++q)
                                    acc[pi][j][q] += pend[j][q] * ps[j];
                                pend[j] = d;
                                ps[j] = (SWIGLU && j >= JF / 2) ? sui : sgi;
                            }
                            // the A bands and scales of k-step ks+1 over the first half of the MFMAs; at the
                            // middle, when every wave has consumed its W fragments of ks, a barrier frees W
                            // slot ks%2 and the W bands of ks+2 go into it: the W stream runs 1.5 k-steps
                            // ahead in the same LDS.  All A/scale DMAs precede them (the wait above counts
                            // on the W bands being the last B_LOADS issued).
                            const int n = i * JF + j;
                            constexpr int HALF = IF * JF / 2, AS = LOADS - B_LOADS;
                            if (n < HALF) {
#pragma unroll
                                for (int u = n * AS / HALF; u < (n + 1) * AS / HALF; ++u)
                                    dma_one(c, kn, 1 - SL, u < A_LOADS ? u : u + B_LOADS);
                            }
                            if (n == HALF) {
                                bar();
#pragma unroll
                                for (int q = A_LOADS; q < A_LOADS + B_LOADS; ++q)
                                    dma_one(c, min(ks + 2, nk - 1), SL, q);
                            }
                            if constexpr (FP8) {
                                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
                                __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // 4 VALU
                            } else {
                                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // 2 MFMA
                            }
                            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // a DMA, where one follows
                        }
                    }
                }
            };
            auto kloop = [&](auto act) {
#if CAM_GMM_UNROLL2
                int ks = 0;
                for (; ks + 1 < nk; ks += 2) {
                    kstep(act, ks, std::integral_constant<int, 0>{});
                    kstep(act, ks + 1, std::integral_constant<int, 1>{});
                }
                if (ks < nk)
                    kstep(act, ks, std::integral_constant<int, 0>{});
#else
                for (int ks = 0; ks < nk; ++ks)
                    kstep(act, ks, std::integral_constant<int, -1>{});
#endif
            };
            if (c.active)
                kloop(std::true_type{});
            else
                kloop(std::false_type{});
            if constexpr (FP8) {
#pragma unroll
                for (int j = 0; j < JF; ++j)  // the last row's pending results
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        acc[IF - 1][j][q] += pend[j][q] * ps[j];
            }
            int ntile = 0;
            if (dyn) {
                // the queue's answer arrives while the ring drains; then the next tile's counter, answered
                // during the epilogue
                const int k = first_thread ? take() : 0;
                wait_vmcnt<0>();
                ntile = publish(k);
                if (ntile < total && !gave_up)
                    next_ready = poll(mti_of(ntile));
            } else {
                if constexpr (CONSUME) {
                    ntile = seq(kt + 1);
                    if (ntile < total && !gave_up && !spect)
                        next_ready = poll(mti_of(ntile));  // answered while the ring drains
                }
                wait_vmcnt<0>();  // the tail's reload has landed before the next tile reuses the ring
                bar();
            }
            dequant_int8(c);
            epilogue(c);
            if constexpr (PRODUCE)
                sig = mti_ctx(c);
            CAM_TL_REC(c.e, tile);
            // int8: the dequantisation's loads have landed before the next tile (otherwise the compiler,
            // unsure of them, waits for every DMA in flight inside the k-loop)
            if constexpr (INT8)
                wait_vmcnt<0>();
            ++kt;
            tile = dyn ? ntile : seq(kt);
            if (tile < total) {
                setup(tile, c);
                if constexpr (CONSUME) {
                    if (next_ready < SY().target)
                        wait_ready(mti_ctx(c));
                }
                prime(c);
            }
        }
        if constexpr (PRODUCE) {
            wait_vmcnt<0>();
            bar();
            signal();
        }
        return;
    } else {
        // ---- 128/32-row tiles: software-pipelined k-loop over a ring of STAGES slots, continued
        // across the block's tiles.  Ring slots are indexed by the block's running k-step count kb+ks,
        // and the DMA of k-step ks+STAGES is spread over the MFMAs of k-step ks (or of its second
        // half); past the end of a tile it fetches the next tile's first k-steps, so a tile starts
        // with its operands already in flight.  With fewer k-steps than stages, or no next tile, the
        // past-the-end DMAs reload the tile's last k-step (the DMA count per k-step, and so every
        // vmcnt wait, stays uniform) and the ring is drained before the next tile.
        int kt = 0;
        int tile = seq(0);
        if (tile >= total)
            return;
        Ctx cur, nxt;
        setup(tile, cur);
        CAM_TL_DECL
        int kb = 0;          // the block's k-steps before the current tile
        bool primed = false;  // the current tile's first STAGES k-steps were issued by the previous tile
        int cur_ready = 0;    // consumer: the current tile's counter as polled before the previous tile's epilogue
        const bool can_chain = nk >= GSTAGES && (!(CONSUME && EAGER) || nk >= 2 * GSTAGES - 2);
        // A consumer chains into its next tile only when that tile's rows are ready.  Nothing of this runs
        // inside the k-loop (a branch there makes the compiler duplicate the loop): wave 0 copies the counter
        // of the tile after next into an LDS slot by DMA at each tile's start, and every wave reads the next
        // tile's slot after the tile's first barrier -- the copy was issued a whole tile earlier, and that
        // tile's k-step waits have covered it.  The block's second tile's counter is copied before its first
        // tile's DMAs.  Two slots of 64 ints (a DMA writes one per lane) in the exchange area, which the plain
        // epilogue does not use; tile k's counter goes to slot k & 1.
        int *rslot = scratch;
        // EAGER consumer (the 4-wave kernel, which affords a branch in its k-loop): the copy goes out at k-step
        // edge nk - 2 STAGES + 2 and is read at edge nk - STAGES, just before the first past-the-end DMA, so the
        // decision uses a counter value from late in the current tile
        constexpr bool EAGER_C = CONSUME && EAGER;
        const int e_copy = nk - 2 * GSTAGES + 2, e_read = nk - GSTAGES;
        if constexpr (CONSUME && !EAGER) {
            const int t1 = seq(1);
            if (t1 < total && w == 0)
                dma4_sc1(SY().ready + mti_of(t1), rslot + 64);
        }
        while (true) {
            const int ntile = seq(++kt);
            const bool has_next = ntile < total;
            // (int8 chains too: its dequantisation's vector loads then wait for the next tile's first DMAs,
            // which land meanwhile -- measured 8 us faster on the int8 decode step than draining first)
            int chain = has_next && can_chain;
            if (has_next)
                setup(ntile, nxt);
            else
                nxt = cur;
            auto slot = [&](int ks) { return (kb + ks) % GSTAGES; };
            auto stage_ptr = [&](int ks) { return smem + slot(ks) * STAGE_BYTES; };
            // DMA instruction q of the current tile's k-step ksx (ksx may run past the end)
            auto dma_ks = [&](int ksx, int q) {
                // a uniform branch between two direct calls: selecting the context by reference would
                // place one of them in scratch memory, and every reload from there waits for the whole
                // DMA ring (vmcnt(0))
                if (ksx >= nk && chain)
                    dma_one(nxt, ksx - nk, slot(ksx), q);
                else
                    dma_one(cur, min(ksx, nk - 1), slot(ksx), q);
            };
            // the DMAs that follow MFMA n of NMF in a phase: spread evenly, so that a wave stalled on
            // a DMA issue still has MFMAs in the pipe
            auto dma_after = [&](int n, int nmf, int ksx) {
#pragma unroll
                for (int q = n * LOADS / nmf; q < (n + 1) * LOADS / nmf; ++q)
                    dma_ks(ksx, q);
            };
            if (!primed) {
                if constexpr (CONSUME) {
                    if (cur_ready < SY().target)
                        wait_ready(mti_ctx(cur));
                }
#pragma unroll
                for (int s0 = 0; s0 < GSTAGES; ++s0)
#pragma unroll
                    for (int q = 0; q < LOADS; ++q)
                        dma_one(cur, min(s0, nk - 1), slot(s0), q);
            }
            wait_vmcnt<LOADS *(GSTAGES - 1)>();  // k-step 0 has landed
            bar();
            // producer, unprimed tile: the previous tile's stores preceded these STAGES k-steps of DMAs
            if constexpr (PRODUCE) {
                if (!primed)
                    signal();
            }
            const bool poll_next = chain;  // EAGER consumer: decided inside the k-loop
            if constexpr (EAGER_C)
                chain = 0;
            if constexpr (CONSUME && !EAGER) {
                // the next tile's counter (bar() is a compiler memory barrier: the slot is read afresh), then
                // the copy of the one after it into the slot this tile's counter occupied
                if (chain)
                    chain = __builtin_amdgcn_readfirstlane(rslot[(kt & 1) * 64]) >= SY().target;
                const int t2 = seq(kt + 1);
                if (t2 < total && w == 0)
                    dma4_sc1(SY().ready + mti_of(t2), rslot + ((kt + 1) & 1) * 64);
            }
            clear_acc();
            // end of a k-step: k-step ks+1 has landed for every wave and every wave has read k-step ks
            int edge = 0;
            auto step_edge = [&]() {
                wait_vmcnt_lgkm0<LOADS *(GSTAGES - 2)>();
                bar();
                if constexpr (PRODUCE && EAGER) {
                    // edge STAGES-2: only LOADS (STAGES - 2) DMAs, all issued during this k-loop, may still be in
                    // flight in any wave, so the previous tile's h stores (issued before) have completed
                    if (edge == GSTAGES - 2)
                        signal();
                }
                if constexpr (EAGER_C) {
                    if (poll_next) {
                        // the copy issued at e_copy has landed by e_read: STAGES - 2 k-steps of DMAs came after it
                        if (edge == e_copy && w == 0)
                            dma4_sc1(SY().ready + mti_ctx(nxt), scratch);
                        if (edge == e_read)
                            chain = __builtin_amdgcn_readfirstlane(scratch[0]) >= SY().target;  // (bar(): read afresh)
                    }
                }
                if constexpr (EAGER)
                    ++edge;
            };

            if constexpr (FP8) {
                // One K=128 MFMA per fragment pair and k-step, and each is one scale block, so its result
                // is scaled on the VALU.  W fragments are double-buffered; A fragments are refilled row by
                // row right after the row's MFMAs have issued (one register set plus one W set in flight).
                // The scaling lags one fragment row behind (row i-1's results are scaled while row i's MFMAs
                // issue, 4 VALU : 1 MFMA), so the MFMA pipe never waits for a result it has just produced.
                // A lane's 32 K-bytes are the 16-byte chunks lg and 4+lg of the 128-byte row (not 2lg, 2lg+1):
                // the same K permutation in both operands leaves each block's dot products unchanged, and
                // this pattern reads LDS at twice the rate (no 2-way bank conflict).
                struct WRegs {
                    i32x8 b[JF];
                    float sg, su;  // weight scales of the wave's gate / up column blocks
                };
                i32x8 a[IF];
                float sa[IF];  // activation scales of the lane's rows
                f32x4 pend[JF];
                float ps[JF];
#pragma unroll
                for (int j = 0; j < JF; ++j) {
                    pend[j] = f32x4{0.f, 0.f, 0.f, 0.f};
                    ps[j] = 0.0f;
                }
                auto rd_w = [&](WRegs &r, int ks) {
                    const uint8_t *lb = stage_ptr(ks) + A_BYTES + (wn * WN) * GKB;
#pragma unroll
                    for (int j = 0; j < JF; ++j) {
                        const u32x4 v0 = *reinterpret_cast<const u32x4 *>(lb + swz(j * 16 + l16, lg));
                        const u32x4 v1 = *reinterpret_cast<const u32x4 *>(lb + swz(j * 16 + l16, 4 + lg));
                        r.b[j] = i32x8{(int)v0[0], (int)v0[1], (int)v0[2], (int)v0[3],
                                       (int)v1[0], (int)v1[1], (int)v1[2], (int)v1[3]};
                    }
                    const int kc = min(ks, nk - 1);
                    r.sg = sload(cur.wsb, cur.wsg + kc);
                    r.su = SWIGLU ? sload(cur.wsb, cur.wsu + kc) : r.sg;
                };
                auto rd_a = [&](int i, int ks) {
                    const uint8_t *st = stage_ptr(ks);
                    const uint8_t *la = st + (wm * WM) * GKB;
                    const u32x4 v0 = *reinterpret_cast<const u32x4 *>(la + swz(i * 16 + l16, lg));
                    const u32x4 v1 = *reinterpret_cast<const u32x4 *>(la + swz(i * 16 + l16, 4 + lg));
                    a[i] = i32x8{(int)v0[0], (int)v0[1], (int)v0[2], (int)v0[3],
                                 (int)v1[0], (int)v1[1], (int)v1[2], (int)v1[3]};
                    // with the last row: every row's scale of the k-step, read together (each row's scale
                    // product for the k-step before has been formed by then)
                    if (i == IF - 1)
                        rd_scales(st, sa);
                };
                // MFMAs of the k-step held in (a, wr); A rows of k-step ks_next are read behind them and
                // the DMA of k-step ks_next-1+STAGES is spread between them
                auto mm = [&](const WRegs &wr, int ks_next, auto act) {
                    const int ks_dma = ks_next - 1 + GSTAGES;
#pragma unroll
                    for (int i = 0; i < IF; ++i) {
                        const float sgi = sa[i] * wr.sg, sui = sa[i] * wr.su;
                        const int pi = i == 0 ? IF - 1 : i - 1;  // row of the pending results
#pragma unroll
                        for (int j = 0; j < JF; ++j) {
                            if constexpr (decltype(act)::value) {
                                const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                                const f32x4 d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wr.b[j], a[i], z, 0,
                                                                                                 0, 0, 127, 0, 127);
#pragma unroll
                                for (int q = 0; q < 4; ++q)
                                    acc[pi][j][q] += pend[j][q] * ps[j];
                                pend[j] = d;
                                // in SwiGLU tiles a wave's columns j < JF/2 are gate rows, the rest up rows
                                ps[j] = (SWIGLU && j >= JF / 2) ? sui : sgi;
                            }
                            dma_after(i * JF + j, IF * JF, ks_dma);
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
                            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // 4 VALU
                            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // a DMA, where one follows
                        }
                        rd_a(i, ks_next);
                    }
                };
                WRegs w0, w1;
#pragma unroll
                for (int i = 0; i < IF; ++i)
                    rd_a(i, 0);
                rd_w(w0, 0);
                auto kloop = [&](auto act) {
                    int ks = 0;
                    for (; ks + 1 < nk; ks += 2) {
                        step_edge();
                        rd_w(w1, ks + 1);
                        mm(w0, ks + 1, act);
                        step_edge();
                        rd_w(w0, ks + 2);
                        mm(w1, ks + 2, act);
                    }
                    if (ks < nk) {
                        step_edge();
                        mm(w0, ks + 1, act);
                    }
                };
                if (!spect && (TC::WAVES_M == 1 || cur.active))  // (one row-wave: a tile always has rows for it)
                    kloop(std::true_type{});
                else if constexpr (TC::WAVES_M > 1 || ROLE != SYNC_NONE)
                    kloop(std::false_type{});
#pragma unroll
                for (int j = 0; j < JF; ++j)  // the last row's pending results
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        acc[IF - 1][j][q] += pend[j][q] * ps[j];
            } else {
                // bf16 / int8: two phases per k-step (the K=32 / K=64 halves of the 128-byte step), each
                // phase's fragments read into the register set the previous phase is not using
                struct Regs {
                    i32x4 a[IF];
                    i32x4 b[JF];
                };
                auto rd = [&](Regs &f, int ks, int ph) {
                    const uint8_t *st = stage_ptr(ks);
                    const uint8_t *la = st + (wm * WM) * GKB;
                    const uint8_t *lb = st + A_BYTES + (wn * WN) * GKB;
#pragma unroll
                    for (int i = 0; i < IF; ++i)
                        f.a[i] = *reinterpret_cast<const i32x4 *>(la + swz(i * 16 + l16, ph * 4 + lg));
#pragma unroll
                    for (int j = 0; j < JF; ++j)
                        f.b[j] = *reinterpret_cast<const i32x4 *>(lb + swz(j * 16 + l16, ph * 4 + lg));
                };
                // MFMAs of one phase; with ks_dma >= 0 the DMA of that k-step is spread between them
                auto mm = [&](const Regs &f, int ks_dma, auto act) {
#pragma unroll
                    for (int i = 0; i < IF; ++i)
#pragma unroll
                        for (int j = 0; j < JF; ++j) {
                            if (ks_dma >= 0)
                                dma_after(i * JF + j, IF * JF, ks_dma);
                            if constexpr (!decltype(act)::value)
                                ;
                            else if constexpr (INT8)
                                acc[i][j] = __builtin_bit_cast(
                                    f32x4, __builtin_amdgcn_mfma_i32_16x16x64_i8(
                                               f.b[j], f.a[i], __builtin_bit_cast(i32x4, acc[i][j]), 0, 0, 0));
                            else
                                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, f.b[j]),
                                                                                    __builtin_bit_cast(bf16x8, f.a[i]),
                                                                                    acc[i][j], 0, 0, 0);
                        }
                };
                Regs r0, r1;
                rd(r0, 0, 0);
                auto kloop = [&](auto act) {
                    for (int ks = 0; ks < nk; ++ks) {
                        rd(r1, ks, 1);
                        mm(r0, -1, act);
                        step_edge();
                        rd(r0, ks + 1, 0);
                        mm(r1, ks + GSTAGES, act);
                    }
                };
                if (!spect && (TC::WAVES_M == 1 || cur.active))  // (one row-wave: a tile always has rows for it)
                    kloop(std::true_type{});
                else if constexpr (TC::WAVES_M > 1 || ROLE != SYNC_NONE)
                    kloop(std::false_type{});
            }

            // producer, primed tile: the previous tile's stores are counted now -- the k-loop's last edge left
            // at most LOADS (STAGES - 2) DMAs in flight in every wave, all issued after those stores
            signal();
            dequant_int8(cur);
            if (!chain) {
                if constexpr (CONSUME) {
                    if (has_next && !gave_up && !spect)
                        cur_ready = poll(mti_ctx(nxt));  // answered while the ring drains
                }
                wait_vmcnt<0>();  // the tail's reloads have landed before the next tile reuses the ring
                bar();
            }
            epilogue(cur);
            if constexpr (PRODUCE)
                sig = mti_ctx(cur);
            CAM_TL_REC(cur.e, tile);
            kb += nk;
            if (!has_next)
                break;
            primed = chain;
            tile = ntile;
            cur = nxt;
        }
        wait_vmcnt<0>();  // every DMA has landed before the block exits
        if constexpr (PRODUCE) {
            bar();
            signal();
        }
    }
}

// XCD-aware order: blocks b, b+8, b+16, ... run on the same XCD; give them consecutive positions,
// so that a run of consecutive tiles shares that XCD's L2
__device__ __forceinline__ int xcd_position()
{
    const int G = gridDim.x;
    return (G & 7) ? (int)blockIdx.x : (int)((blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3));
}

// LDS of a launch: a class's ring of stages, then that class's epilogue exchange area; the expert tables
// sit at the end of the launch's LDS (the same place for every class of a launch).
template <int BM, int BN = GBN> constexpr size_t ring_bytes() { return Tile<BM, BN>::STAGES * Tile<BM, BN>::STAGE_BYTES; }
template <int BM, int BN = GBN> constexpr size_t exchange_bytes()
{
    return (size_t)Tile<BM, BN>::WAVES_N * BM * sizeof(float);  // [WAVES_N][BM] row maxima
}
template <int BM, int BN = GBN> constexpr size_t class_bytes() { return ring_bytes<BM, BN>() + exchange_bytes<BM, BN>(); }
constexpr size_t cmax(size_t a, size_t b) { return a > b ? a : b; }
constexpr size_t G_LDS_SMALL_BYTES = cmax(class_bytes<32, GBN>(), class_bytes<32, 128>()) + sizeof(GroupTables);
constexpr size_t G_LDS_BIG_BYTES =
    cmax(cmax(class_bytes<256>(), class_bytes<128>()), cmax(class_bytes<32, GBN>(), class_bytes<32, 128>())) +
    sizeof(GroupTables);
static_assert(G_LDS_SMALL_BYTES <= 163840 && G_LDS_BIG_BYTES <= 163840, "LDS budget of a gfx950 workgroup");
// the table scan's per-wave totals (before any ring use)
static_assert(sizeof(int) * 4 * (GMAX_THREADS / 64) <= ring_bytes<32, 128>(), "table-scan scratch");

// Decode-sized segments: the 32-row tile (4 waves).
template <int DT, int EPI> __global__ __launch_bounds__(256, 1) void gmm_kernel_small(GmmArgs p)
{
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    GroupTables *gt = reinterpret_cast<GroupTables *>(smem + G_LDS_SMALL_BYTES - sizeof(GroupTables));
    const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    build_group_tables<Tile<32>::THREADS>(p.group_list, p.L, *gt, reinterpret_cast<int *>(smem),
                                          ClassRanges{{0, 0, 0}, {0, 0, 0x7fffffff}});
    gmm_body<DT, EPI, 32>(p, gt, -1, 0, 0, 1, -1, wv);
}

// Prefill: 8 waves, 128- or 256-row tile picked per launch from the actual rows per touched
// expert (counts are on the device).  The choice is block-uniform and identical in every block.
// Experts with at least this many rows take the 256-row tile (when the launch allows it).
constexpr int G_HEAVY_ROWS = 384;
// In a launch with heavy experts (fp8 and bf16), the experts with fewer rows than this take the 32-row tile on
// four of the block's waves: their tiles are a weight stream, and that tile's four-stage ring keeps half as
// many weight bytes again in flight per CU as the 128-row tile's three stages (measured on config 4's fp8
// GMM1: such a tile streams its 1.8 MB in 46-58 us against 51-65 us, the GEMM 186 vs 193 us; the int8 GEMM
// measured 1-2% slower and keeps the 128-row tile).
#ifndef CAM_GMM_SMALL_ROWS
#define CAM_GMM_SMALL_ROWS 64
#endif
constexpr int G_SMALL_ROWS = CAM_GMM_SMALL_ROWS;
#ifndef CAM_GMM_RUN32
#define CAM_GMM_RUN32 3
#endif

// Between two tile classes the block meets at an LDS-only barrier (lds_sync): both prefill loops have drained
// their DMAs before the last epilogue, so only the ring's LDS reads must be complete (__syncthreads would also
// wait for the epilogue's global stores; the next class's first DMAs queue behind those stores either way).
// Prefill: 8 waves.  With the 256-row tile allowed, the experts holding at least G_HEAVY_ROWS rows run
// 256-row tiles first, then the rest 128-row tiles -- one launch, the longest tiles first, the tile
// sequence of each block continuing round-robin from the first class into the second, and (fp8, bf16) from
// there into a third, the experts with fewer than G_SMALL_ROWS rows on 32-row tiles.  A layer whose
// load is skewed (a few experts with a thousand rows, many with a handful) gets tall tiles where they
// halve the operand traffic and short ones where a tall tile would multiply padding.  The light experts'
// (at most three M-tiles each) weights are fetched nontemporally.
// short reductions keep the 128-row tile: the 256-row tile's per-tile ring fill and drain would
// not amortise over fewer than 16 k-steps (at 16, GMM2 of DeepSeek-V3's shapes: the M = 65536 fp8 GMM2
// 1.71 vs 1.57 PFLOPS, int8 1.97 vs 1.67 POPS, config 4's fp8 GMM2 116 vs 122 us)
__host__ __device__ constexpr bool big_tall(int allow256, int K, int dt)
{
    return allow256 && (int)((uint32_t)K * (dt == DT_BF16 ? 2 : 1) / GKB) >= CAM_GMM_MIN_NK256;
}
template <int DT> __device__ __forceinline__ ClassRanges big_ranges(bool tall)
{
    constexpr int SMALL = DT == DT_INT8 ? 1 : G_SMALL_ROWS;  // rows below: the 32-row tile class
    return tall ? ClassRanges{{G_HEAVY_ROWS, SMALL, 1}, {0x7fffffff, G_HEAVY_ROWS, SMALL}}
                : ClassRanges{{0, 0, 0}, {0, 0x7fffffff, 0}};
}

// The 8-wave schedule of one GEMM over the tile classes of the launch's tables (gmm_kernel_big).  ROLE !=
// SYNC_NONE (the chained kernel): the 32-row class keeps the block's other four waves as spectators instead of
// ending them, since the block has more work after it.
// bid: the block's id for the placement (blockIdx.x; a chained consumer passes its arrival order, so that the
// blocks that finish GMM1 first take the positions with the most GMM2 work).
template <int DT, int EPI, int ROLE>
__device__ __forceinline__ void big_schedule(const GmmArgs &p, const GroupTables *gt, bool tall, int bid, int wv)
{
    const int pos = (gridDim.x & 7) ? bid : (bid & 7) * (int)(gridDim.x >> 3) + (bid >> 3);  // XCD-aware order
    constexpr int SMALL = DT == DT_INT8 ? 1 : G_SMALL_ROWS;  // rows below: the 32-row tile class
    constexpr bool KEEP = ROLE != SYNC_NONE;
    if (!tall) {
        gmm_body<DT, EPI, 128, false, ROLE>(p, gt, -1, 0, 0, 1, bid, wv);
        return;
    }
    // light tiles worth about one heavy tile: a 256-row tile against 128-row tiles (2 for 1-byte operands, 1
    // for bf16) or 32-row tiles (a plain one holds 128 W rows, a SwiGLU one 256: measured 35 and 105 us per
    // heavy tile against 9 and 45-55 us per light one)
    constexpr int run = DT == DT_BF16 ? 1 : 2;
    constexpr int run32 = EPI == EPI_PLAIN ? 4 : CAM_GMM_RUN32;
    // (uniform values read from LDS go to scalar registers at once: a VGPR holding one across the classes gets
    // spilled, and its reload after a tile's k-loop makes the next k-loop wait for it at every iteration)
    const int n_heavy = __builtin_amdgcn_readfirstlane(gt->tile_end[0][p.L - 1]);  // 256-row M-tiles (heavy)
    const bool has_mid = __builtin_amdgcn_readfirstlane(gt->tile_end[1][p.L - 1]) > 0;
    const bool has_small = __builtin_amdgcn_readfirstlane(gt->tile_end[2][p.L - 1]) > 0;
    const int G = gridDim.x;
    // 256-row tiles: heavy M-tiles x N-tiles
    const int heavy_tiles = n_heavy * (EPI != EPI_PLAIN ? p.N / 2 / 128 : p.N / 256);
    if constexpr (ROLE == SYNC_CONSUME) {
        // Chained GMM2: the blocks reach it at different times (their GMM1 work differs), so the heavy tiles go
        // out through dynamic queues, one per XCD over that XCD's consecutive share (tiles sharing its L2), to
        // whichever of its blocks is free; the light tiles follow round-robin by the blocks' arrival order.
        if (heavy_tiles > 0) {
            const int nq = (G & 7) ? 1 : 8, x = nq == 1 ? 0 : (bid & 7);
            const int hx = (heavy_tiles + nq - 1) / nq;
            const int len = max(0, min(hx, heavy_tiles - x * hx));
            gmm_body<DT, EPI, 256, false, ROLE>(p, gt, G_DYN, x * hx, len, chain_queue_index(p.M, p.L) + x, -1, wv);
            lds_sync();
        }
        if (has_mid)
            gmm_body<DT, EPI, 128, true, ROLE>(p, gt, pos, 0, 0, 1, -1, wv);
        if constexpr (SMALL > 1) {
            if (has_small) {
                lds_sync();
                gmm_body<DT, EPI, 32, true, ROLE>(p, gt, pos, 0, 0, 1, -1, wv);
            }
        }
        return;
    }
    if (heavy_tiles > 0 && heavy_tiles < G && (G & 7) == 0) {
        // Fewer heavy tiles than blocks.  They are split evenly over the 8 XCDs (XCD x takes the run
        // [x hx, (x + 1) hx), consecutive tiles sharing that XCD's L2), so each XCD keeps some blocks free.
        // The free blocks start on the light tiles at once, `run` (or `run32`) in a row each; the rest of
        // the light tiles go round-robin over all blocks in launch order (every XCD in turn), reaching the
        // heavy blocks as they finish.
        const int xcd = bid & 7, slot = bid >> 3, S = G >> 3;
        const int hx = (heavy_tiles + 7) / 8;
        auto heavy_in = [&](int x) { return max(0, min(hx, heavy_tiles - x * hx)); };
        const int len = heavy_in(xcd);
        if (slot < len) {
            gmm_body<DT, EPI, 256, false, ROLE>(p, gt, 0x3fffffff, xcd * hx + slot, (len - slot + S - 1) / S, S, -1, wv);
            lds_sync();  // every wave is done with the first class's ring
        }
        int free_before = 0, free_all = 0;
        for (int x = 0; x < 8; ++x) {
            const int fx = max(0, S - heavy_in(x));
            free_before += x < xcd ? fx : 0;
            free_all += fx;
        }
        const bool is_free = slot >= len;
        const int fpos = free_before + slot - len;  // the block's rank among the free blocks
        if (has_mid)
            gmm_body<DT, EPI, 128, true, ROLE>(p, gt, run * free_all + bid, is_free ? fpos * run : 0, is_free ? run : 0, 1, -1, wv);
        if constexpr (SMALL > 1) {
            if (has_small) {
                lds_sync();
                if (!KEEP && wv >= Tile<32>::NWAVES)
                    return;  // the 32-row tile's four waves go on (a barrier only counts the waves still running)
                gmm_body<DT, EPI, 32, true, ROLE>(p, gt, run32 * free_all + bid, is_free ? fpos * run32 : 0, is_free ? run32 : 0, 1, -1, wv);
            }
        }
        return;
    }
    if (n_heavy == 0) {  // one class after another, each balanced over the blocks
        if (has_mid)
            gmm_body<DT, EPI, 128, true, ROLE>(p, gt, -1, 0, 0, 1, bid, wv);
        if constexpr (SMALL > 1) {
            if (has_small) {
                lds_sync();
                if (!KEEP && wv >= Tile<32>::NWAVES)
                    return;
                gmm_body<DT, EPI, 32, true, ROLE>(p, gt, -1, 0, 0, 1, bid, wv);
            }
        }
        return;
    }
    // At least as many heavy tiles as blocks: they go round-robin over the blocks, so the first
    // heavy_tiles % G blocks run one more of them than the rest.  Those others (the free blocks) start the
    // light tiles with a run of about one heavy tile's worth each; the rest of the light tiles go
    // round-robin over all blocks (measured on config 4's GMM2, 364 heavy tiles on 256 blocks: the light
    // tiles' round-robin then no longer lands on blocks still busy with their second heavy tile).
    gmm_body<DT, EPI, 256, false, ROLE>(p, gt, pos, 0, 0, 1, -1, wv);
    lds_sync();  // every wave is done with the first class's ring
    const int r = heavy_tiles % G;
    const int nfree = r > 0 ? G - r : 0;
    const bool is_free = nfree > 0 && pos >= r;
    const int fpos = pos - r;
    if (has_mid)
        gmm_body<DT, EPI, 128, true, ROLE>(p, gt, run * nfree + pos, is_free ? fpos * run : 0, is_free ? run : 0, 1, -1, wv);
    if constexpr (SMALL > 1) {
        if (has_small) {
            lds_sync();
            if (!KEEP && wv >= Tile<32>::NWAVES)
                return;
            gmm_body<DT, EPI, 32, true, ROLE>(p, gt, run32 * nfree + pos, is_free ? fpos * run32 : 0, is_free ? run32 : 0, 1, -1, wv);
        }
    }
}

template <int DT, int EPI> __global__ __launch_bounds__(512, 1) void gmm_kernel_big(GmmArgs p)
{
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    GroupTables *gt = reinterpret_cast<GroupTables *>(smem + G_LDS_BIG_BYTES - sizeof(GroupTables));
    const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const bool tall = big_tall(p.allow256, p.K, DT);
    // every class's expert table, from one read of the counts
    build_group_tables<GMAX_THREADS>(p.group_list, p.L, *gt, reinterpret_cast<int *>(smem), big_ranges<DT>(tall));
    big_schedule<DT, EPI, SYNC_NONE>(p, gt, tall, (int)blockIdx.x, wv);
}

// Chained GMM1 + SwiGLU -> GMM2 (launch_gmm_chain): one table build, every block's GMM1 tiles (producing), then
// its GMM2 tiles (consuming).  A block only ever waits for GMM1 tiles, and every block runs all of its GMM1
// tiles before its first wait, so with every block resident each wait ends; a wait that outlasts the bound
// gives up instead (and the host reads the sync status).  The grid is one block per CU, the blocks' LDS keeps
// them to one per CU.
// The block's arrival order at the GMM1 -> GMM2 boundary, as a block id: its rank among the blocks of its XCD
// (one counter per XCD, after the M-tile counters) in place of blockIdx.x >> 3.  The consumer phase places its
// tiles by it: the blocks that finish GMM1 first take the positions that hold the most GMM2 work.
__device__ __forceinline__ int arrival_bid(int M, int L, uint8_t *smem, int wv)
{
    int *slot = reinterpret_cast<int *>(smem);  // the ring is idle between the phases
    const int xcd = blockIdx.x & 7;
    if (wv == 0 && lane_id() == 0) {
        int *ctr = chain_params()->sy.ready + chain_arrival_index(M, L) + xcd;
        *slot = __hip_atomic_fetch_add(gptr(ctr), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    const int r = *slot;
    __syncthreads();  // (the slot is ring memory again)
    return (gridDim.x & 7) ? (int)blockIdx.x : r * 8 + xcd;
}

template <int DT, int EPI1> __global__ __launch_bounds__(512, 1) void gmm_chain_big(ChainParams cp)
{
    (void)cp;  // read through chain_params()
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    GroupTables *gt = reinterpret_cast<GroupTables *>(smem + G_LDS_BIG_BYTES - sizeof(GroupTables));
    const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    bool tall;
    {
        const GmmArgs p1 = chain_params()->g1;
        tall = big_tall(p1.allow256, p1.K, DT);  // the host checked that GMM2 makes the same choice
        build_group_tables<GMAX_THREADS>(p1.group_list, p1.L, *gt, reinterpret_cast<int *>(smem),
                                         big_ranges<DT>(tall));
        big_schedule<DT, EPI1, SYNC_PRODUCE>(p1, gt, tall, (int)blockIdx.x, wv);
    }
    lds_sync();  // every wave is done with GMM1's last ring
    const GmmArgs p2 = chain_params()->g2;
    const int bid = arrival_bid(p2.M, p2.L, smem, wv);
    big_schedule<DT, EPI_PLAIN, SYNC_CONSUME>(p2, gt, tall, bid, wv);
}
template <int DT, int EPI1> __global__ __launch_bounds__(256, 1) void gmm_chain_small(ChainParams cp)
{
    (void)cp;
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    GroupTables *gt = reinterpret_cast<GroupTables *>(smem + G_LDS_SMALL_BYTES - sizeof(GroupTables));
    // Decode tiles are weight streams of fixed size, so the two phases are balanced statically: GMM1's tiles go
    // round-robin over every block, and the blocks left with one GMM1 tile fewer start GMM2 with a run of R
    // tiles, R = a GMM1 tile's weight bytes over a GMM2 tile's (256 rows of K1 against 128 rows of K2).  Those
    // first GMM2 tiles (the first experts) depend only on GMM1's first round.
    const int pos = xcd_position(), G = gridDim.x;
    const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    int t1;
    {
        const GmmArgs p1 = chain_params()->g1;
        build_group_tables<Tile<32>::THREADS>(p1.group_list, p1.L, *gt, reinterpret_cast<int *>(smem),
                                              ClassRanges{{0, 0, 0}, {0, 0, 0x7fffffff}});
        t1 = gt->tile_end[2][p1.L - 1] * (p1.N / 2 / 128);
        gmm_body<DT, EPI1, 32, true, SYNC_PRODUCE, true>(p1, gt, pos, 0, 0, 1, -1, wv);
    }
    lds_sync();
    const GmmArgs p2 = chain_params()->g2;
    const int r1 = t1 % G, nfree = r1 ? G - r1 : 0;
    const bool is_free = nfree > 0 && pos >= r1;
    constexpr int BN2 = small_bn(32, EPI_PLAIN);
    const int R = max(1, (GBN * chain_params()->g1.K + BN2 * p2.K / 2) / (BN2 * p2.K));
    gmm_body<DT, EPI_PLAIN, 32, true, SYNC_CONSUME, true>(p2, gt, R * nfree + pos, is_free ? (pos - r1) * R : 0,
                                                          is_free ? R : 0, 1, -1, wv);
}

// Per-device launch state: the CU count and whether a kernel's dynamic-LDS limit has been raised.
// Both are cached per device in atomics, so concurrent first calls and several GPUs are safe (a
// racing first call only repeats the idempotent query or attribute set).
constexpr int G_MAX_DEVICES = 64;

static int current_device()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0)
        dev = 0;
    return dev;
}

static int num_cus(int dev)
{
    static std::atomic<int> cache[G_MAX_DEVICES];
    if (dev < G_MAX_DEVICES) {
        const int c = cache[dev].load(std::memory_order_relaxed);
        if (c > 0)
            return c;
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        n = 256;
    if (dev < G_MAX_DEVICES)
        cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

// one flag per device and kernel instantiation (the caller passes its own static array)
template <typename K> static hipError_t set_lds(K kernel, size_t lds, int dev, std::atomic<bool> *done)
{
    if (dev < G_MAX_DEVICES && done[dev].load(std::memory_order_acquire))
        return hipSuccess;
    hipError_t e = hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e == hipSuccess && dev < G_MAX_DEVICES)
        done[dev].store(true, std::memory_order_release);
    return e;
}

// Tile choice.  A row capacity of at most 48 rows per expert (decode) can only hold short
// segments: the 32-row kernel.  Otherwise the 8-wave kernel, which picks the 128- or 256-row
// tile on the device from the actual counts (a prefill-sized capacity may still hold short
// segments when most rows are routed elsewhere).  One launch, no host synchronisation.
template <int DT, int EPI> static hipError_t launch_one(GmmArgs a, hipStream_t s)
{
    const int dev = current_device();
    const int grid = (num_cus(dev) + 7) / 8 * 8;
    if (a.M <= 48 * a.L) {
        static std::atomic<bool> done[G_MAX_DEVICES];
        const size_t lds = G_LDS_SMALL_BYTES;
        hipError_t e = set_lds(gmm_kernel_small<DT, EPI>, lds, dev, done);
        if (e != hipSuccess)
            return e;
        hipLaunchKernelGGL((gmm_kernel_small<DT, EPI>), dim3(grid), dim3(256), lds, s, a);
        return hipGetLastError();
    }
    a.allow256 = a.M >= G_HEAVY_ROWS;  // some expert may reach the 256-row tile class
    static std::atomic<bool> done[G_MAX_DEVICES];
    const size_t lds = G_LDS_BIG_BYTES;
    hipError_t e = set_lds(gmm_kernel_big<DT, EPI>, lds, dev, done);
    if (e != hipSuccess)
        return e;
    hipLaunchKernelGGL((gmm_kernel_big<DT, EPI>), dim3(grid), dim3(512), lds, s, a);
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
    } else if (dt == DT_INT8) {
        if (epi == EPI_PLAIN)
            return launch_one<DT_INT8, EPI_PLAIN>(a, s);
        if (epi == EPI_SWIGLU_F32AMAX)
            return launch_one<DT_INT8, EPI_SWIGLU_F32AMAX>(a, s);
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

// ---- chained GMM1 -> GMM2
#ifndef CAM_GMM_CHAIN_BIG
#define CAM_GMM_CHAIN_BIG 1  // the prefill-sized chained kernel (8 waves, all tile classes)
#endif
int gmm_chain_counters(int M, int L) { return chain_queue_index(M, L) + 8; }

static bool chain_small(const GmmArgs &g) { return g.M <= 48 * g.L; }

// CAMHIP_GMM_CHAIN=0 in the environment turns the chained launch off (the two-launch path runs instead; for
// measuring one against the other)
static bool chain_enabled()
{
    static const bool on = [] {
        const char *v = getenv("CAMHIP_GMM_CHAIN");
        return !(v && v[0] == '0');
    }();
    return on;
}

// h above this size is not chained: the producing tiles store it agent-coherently (written through to
// memory), which for h of hundreds of MB (Mixtral-sized prefill) costs more than the overlap gains
constexpr long long G_CHAIN_MAX_H_BYTES = 64ll << 20;

bool gmm_chain_supported(const GmmArgs &g1, const GmmArgs &g2, int dt)
{
    if (dt != DT_FP8 && dt != DT_BF16)
        return false;  // int8 requantises h per token in a launch of its own
    if (!chain_enabled() || (long long)g1.M * (g1.N / 2) * (dt == DT_BF16 ? 2 : 1) > G_CHAIN_MAX_H_BYTES)
        return false;
    if (g1.M != g2.M || g1.L != g2.L || g1.group_list != g2.group_list || g2.K * 2 != g1.N)
        return false;
    if (chain_small(g1))
        return true;
#if !CAM_GMM_CHAIN_BIG
    return false;
#endif
    const int allow = g1.M >= G_HEAVY_ROWS;
    return big_tall(allow, g1.K, dt) == big_tall(allow, g2.K, dt);  // both GEMMs split every expert alike
}

static std::atomic<long long> g_sync_ticks{0};
static std::atomic<int> g_sync_unreach{0};
void sync_debug_set(long long wait_ticks, int unreachable)
{
    g_sync_ticks.store(wait_ticks, std::memory_order_relaxed);
    g_sync_unreach.store(unreachable ? 1 : 0, std::memory_order_relaxed);
}

hipError_t sync_status_read(int *status, bool clear)
{
    int v = 0;
    hipError_t e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_cam_sync_status), sizeof(int), 0, hipMemcpyDeviceToHost);
    if (e != hipSuccess)
        return e;
    if (clear && v != 0) {
        const int zero = 0;
        e = hipMemcpyToSymbol(HIP_SYMBOL(g_cam_sync_status), &zero, sizeof(int), 0, hipMemcpyHostToDevice);
        if (e != hipSuccess)
            return e;
    }
    *status = v;
    return hipSuccess;
}

template <int DT, int EPI1> static hipError_t launch_chain_t(GmmArgs g1, GmmArgs g2, GmmSync sy, hipStream_t s)
{
    const int dev = current_device();
    // one block per CU at most (a block's GMM2 tiles wait for GMM1 tiles of other blocks, so every block must be
    // resident at once), in whole XCD rounds where the CU count allows
    const int cus = num_cus(dev), grid = cus >= 8 ? cus / 8 * 8 : cus;
    if (chain_small(g1)) {
        static std::atomic<bool> done[G_MAX_DEVICES];
        hipError_t e = set_lds(gmm_chain_small<DT, EPI1>, G_LDS_SMALL_BYTES, dev, done);
        if (e != hipSuccess)
            return e;
        hipLaunchKernelGGL((gmm_chain_small<DT, EPI1>), dim3(grid), dim3(256), G_LDS_SMALL_BYTES, s, ChainParams{g1, g2, sy});
        return hipGetLastError();
    }
#if CAM_GMM_CHAIN_BIG
    g1.allow256 = g2.allow256 = g1.M >= G_HEAVY_ROWS;
    static std::atomic<bool> done[G_MAX_DEVICES];
    hipError_t e = set_lds(gmm_chain_big<DT, EPI1>, G_LDS_BIG_BYTES, dev, done);
    if (e != hipSuccess)
        return e;
    hipLaunchKernelGGL((gmm_chain_big<DT, EPI1>), dim3(grid), dim3(512), G_LDS_BIG_BYTES, s, ChainParams{g1, g2, sy});
    return hipGetLastError();
#else
    return hipErrorNotSupported;
#endif
}

hipError_t launch_gmm_chain(const GmmArgs &g1, const GmmArgs &g2, int dt, int *ready, hipStream_t s)
{
    if (g1.L <= 0 || g1.L > G_MAX_L || g1.M <= 0 || ready == nullptr)
        return hipErrorInvalidValue;
    if (!gmm_chain_supported(g1, g2, dt))
        return hipErrorNotSupported;
    const long long t = g_sync_ticks.load(std::memory_order_relaxed);
    const GmmSync sy{ready, g1.N / 2 / 128 + g_sync_unreach.load(std::memory_order_relaxed),
                     t > 0 ? t : 200000000LL};  // 2 s of the 100 MHz constant clock
    if (dt == DT_FP8)
        return launch_chain_t<DT_FP8, EPI_SWIGLU_FP8>(g1, g2, sy, s);
    return launch_chain_t<DT_BF16, EPI_SWIGLU_BF16>(g1, g2, sy, s);
}

#ifdef CAM_GMM_TIMELINE
}  // namespace cam
// diagnostic build only: copy the per-tile records out and clear them
extern "C" __attribute__((visibility("default"))) int camhipDebugGmmTimeline(void *host_dst, size_t bytes)
{
    const size_t n = std::min(bytes, sizeof(cam::g_cam_tl));
    if (hipMemcpyFromSymbol(host_dst, HIP_SYMBOL(cam::g_cam_tl), n, 0, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    static uint8_t zeros[sizeof(cam::g_cam_tl)];
    return hipMemcpyToSymbol(HIP_SYMBOL(cam::g_cam_tl), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice) == hipSuccess
               ? (int)(n / sizeof(cam::g_cam_tl[0]))
               : -1;
}
namespace cam {
#endif

// Per-token int8 requantisation of h (post_swiglu_dynamic_quant.h:164-231): one block per row.
__global__ __launch_bounds__(256) void quant_rows_int8_kernel(const float *__restrict__ h,
                                                              const float *__restrict__ amax_in,
                                                              const int64_t *__restrict__ group_list, int L, int M,
                                                              int I, int8_t *__restrict__ q, float *__restrict__ scale)
{
    __shared__ int tot;
    __shared__ float red[256 / 64];
    if (threadIdx.x == 0)
        tot = 0;
    __syncthreads();
    int part = 0;
    for (int e = threadIdx.x; e < L; e += blockDim.x)
        part += (int)group_list[e];
    if (part)
        atomicAdd(&tot, part);
    __syncthreads();
    const int total = min(tot, M);
    const int S = I / GMM_AMAX_COLS;  // partial maxima per row
    for (int m = blockIdx.x; m < total; m += gridDim.x) {
        float pm = 0.0f;
        for (int c = threadIdx.x; c < S; c += blockDim.x)
            pm = fmaxf(pm, amax_in[(size_t)m * S + c]);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
            pm = fmaxf(pm, __shfl_xor(pm, o, 64));
        if ((threadIdx.x & 63) == 0)
            red[threadIdx.x >> 6] = pm;
        __syncthreads();
        const float a = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __syncthreads();  // red is rewritten for the next row
        const float inv = a > 0.0f ? 1.0f / a : 0.0f;  // rows of zeros quantise to 0 with scale 0
        const f32x4 *hr = reinterpret_cast<const f32x4 *>(h + (size_t)m * I);
        uint32_t *qr = reinterpret_cast<uint32_t *>(q + (size_t)m * I);
        for (int c = threadIdx.x; c < I / 4; c += blockDim.x) {
            const f32x4 v = hr[c];
            uint32_t pk = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b)
                pk |= (uint32_t)((int)rintf((v[b] * 127.0f) * inv) & 0xff) << (8 * b);
            qr[c] = pk;
        }
        if (threadIdx.x == 0)
            scale[m] = a * (1.0f / 127.0f);
    }
}

hipError_t launch_quant_rows_int8(const float *h, const float *amax, const int64_t *group_list, int L, int M, int I,
                                  int8_t *q, float *scale, hipStream_t s)
{
    if (M <= 0 || L <= 0 || (I % GMM_AMAX_COLS))
        return hipErrorInvalidValue;
    const int grid = M < 4096 ? M : 4096;
    hipLaunchKernelGGL(quant_rows_int8_kernel, dim3(grid), dim3(256), 0, s, h, amax, group_list, L, M, I, q, scale);
    return hipGetLastError();
}

// fp8 activation scales row-major [M, nb] -> k-major [nb, M] through an LDS tile: 64 rows x nb per block,
// read and written in contiguous runs
// One block per 64 x 64 tile of (rows, scale blocks): every load of the tile is issued at once (16 per
// thread, consecutive blocks of a row on consecutive lanes), the tile turns in LDS, and the stores run
// along the rows.  Rows at or past sum(group_list) are neither read nor written.
__global__ __launch_bounds__(256) void scales_kmajor_kernel(const float *__restrict__ src,
                                                          const int64_t *__restrict__ group_list, int L, int M,
                                                          int nb, float *__restrict__ dst)
{
    __shared__ float tile[64][65];
    __shared__ int tot;
    const int tid = threadIdx.x;
    if (tid < 64) {
        int part = 0;
#pragma unroll
        for (int q = 0; q < G_MAX_L / 64; ++q) {
            const int e = q * 64 + tid;
            part += e < L ? (int)group_list[e] : 0;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
            part += __shfl_xor(part, o, 64);
        if (tid == 0)
            tot = part;
    }
    __syncthreads();
    const int rows = min(tot, M);
    const int r0 = blockIdx.x * 64, b0 = blockIdx.y * 64;
    if (r0 >= rows)
        return;
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int idx = i * 256 + tid, r = idx >> 6, b = idx & 63;
        v[i] = (r0 + r < rows && b0 + b < nb) ? src[(size_t)(r0 + r) * nb + b0 + b] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int idx = i * 256 + tid;
        tile[idx >> 6][idx & 63] = v[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int idx = i * 256 + tid, b = idx >> 6, r = idx & 63;
        if (r0 + r < rows && b0 + b < nb)
            dst[(size_t)(b0 + b) * M + r0 + r] = tile[r][b];
    }
}

hipError_t launch_scales_to_kmajor(const float *src, const int64_t *group_list, int L, int M, int nb, float *dst,
                                   hipStream_t s)
{
    if (M < 0 || nb <= 0 || L <= 0 || L > G_MAX_L)
        return hipErrorInvalidValue;
    if (M == 0)
        return hipSuccess;
    hipLaunchKernelGGL(scales_kmajor_kernel, dim3((M + 63) / 64, (nb + 63) / 64), dim3(256), 0, s, src, group_list, L,
                       M, nb, dst);
    return hipGetLastError();
}

}  // namespace cam
