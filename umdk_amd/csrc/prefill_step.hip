// The prefill step's route -> chunk scan + count exchange -> dispatch (R0, D1, D2, D3 + Q1) in one launch.
//
// The grid's blocks take roles by index: the first ceil(T/16) route a 16-token chunk each (route_block), the
// next ceil(Ec/4) scan one expert per wave (scan_expert), the rest dispatch one (token, 1024-column chunk)
// per wave (dispatch_wave).  Blocks start in index order on every XCD, so the route and scan blocks are
// resident before any dispatch block waits for them.  A dispatch wave issues its loads of x first and only then
// waits for the routing and the scan, so the routing's latency, the scan's and the two launch gaps of the
// three-launch step overlap with the first resident dispatch waves' reads of x.  The stages' results are
// bit-identical to the three launches: the same device bodies run, their cross-stage outputs stored and read
// agent-coherently.
//
// Readiness: a static per-device array of counters -- route blocks done, experts scanned, dispatch blocks past
// their wait -- published after each stage's stores have completed (vmcnt(0), then an agent-scope atomic).
// Device-scope atomics on one address serialise (~30 ns each: one counter bumped by each of 7168 dispatch
// blocks measured 0.9 ms), so every counter is split into shards on cache lines of their own: 8 for the route
// blocks and 8 for the scan waves (a waiter sums them), 64 for the dispatch blocks, whose completing blocks
// bump one top counter.  Dispatch blocks wait for the scan only (every scan wave waited for the routing).  The
// block that completes the top counter resets everything, so every launch starts from zero (the array is zero
// when the library is loaded).  Launches that overlap on one GPU therefore race (the reference's prefill ops
// do not support concurrent use either, doc/en/cam/CAM API Guide.md:38-39).  A wait gives up after a bound
// (2 s), sets the status word and lets the launch end; the host reads it with step_status_read.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <mutex>

#include "cam_device.h"
#include "launchers.h"
#include "prefill_dev.h"

namespace cam {

// Counters, one per 128-byte line (SY_STRIDE ints): route shards, scan shards, dispatch-block shards, the top
// counter of completed dispatch shards, the status word (1: a wait gave up)
constexpr int SY_STRIDE = 32, SY_RSH = 8, SY_SSH = 8, SY_DSH = 64;
constexpr int SY_ROUTED = 0, SY_SCANNED = SY_ROUTED + SY_RSH, SY_PASSED = SY_SCANNED + SY_SSH,
              SY_TOP = SY_PASSED + SY_DSH, SY_RTOP = SY_TOP + 1, SY_STOP = SY_RTOP + 1, SY_RDONE = SY_STOP + 1,
              SY_SDONE = SY_RDONE + 1, SY_STATUS = SY_SDONE + 1, SY_SLOTS = SY_STATUS + 1;
static __device__ __align__(256) int step_sync[SY_SLOTS * SY_STRIDE];
__device__ __forceinline__ int *sy_slot(int *base, int i) { return base + i * SY_STRIDE; }

// dispatch blocks at most: about what the GPU holds at once (256 CUs x 8 blocks of 4 waves)
constexpr int STEP_MAX_DISP_BLOCKS = 2048;
constexpr int STEP_DEFAULT_MODE = 1;

struct StepArgs {
    const float *logits;
    const float *bias;
    const uint16_t *x;
    int T, H, E, Ec, K, cap, nchunk, kmajor, skip_unrouted;
    int32_t *topk_idx;
    float *topk_w;
    int32_t *counts, *pref, *chunk_rank, *send_offset, *recv_count;
    int64_t *tokens_per_expert;
    uint8_t *expand_x;
    float *scales;
    int32_t *expand_idx, *inv;
    int nroute, nscan, ndisp_waves, ndisp_blocks;
    int extra;  // added to the wait targets: 1 makes every wait give up (a test hook)
    int *sync;
    long long ticks;
};

// Waits until the flag in `slot` reaches target (lane 0 polls, agent-coherent, a long sleep between polls:
// coherent reads of one line are served one at a time at the memory side, and thousands of waves polling it
// slow down the very stages they wait for); false when the bound ran out (status set).
template <int SLEEP>
__device__ __forceinline__ bool step_wait(int *sync, int slot, int target, long long ticks)
{
    const int lane = threadIdx.x & 63;
    const uint64_t t0 = wall_clock64();
    while (true) {
        int v = 0;
        if (lane == 0)
            v = __hip_atomic_load(gp(sy_slot(sync, slot)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__builtin_amdgcn_readfirstlane(v) >= target)
            return true;
        if ((long long)(wall_clock64() - t0) > ticks) {
            if (lane == 0)
                __hip_atomic_fetch_or(gp(sy_slot(sync, SY_STATUS)), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        __builtin_amdgcn_s_sleep(SLEEP);
    }
}

template <int PER, int MODE> __global__ __launch_bounds__(256) void prefill_step_kernel(StepArgs a)
{
    const int b = blockIdx.x;
    int *sync = a.sync;
    auto bump = [&](int slot) {
        return __hip_atomic_fetch_add(gp(sy_slot(sync, slot)), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    // counts one of `total` items in shard i of `nsh` (items i, i + nsh, ...); the item completing a shard bumps
    // `top`, the one completing `top` raises `done` (so waiters read one flag)
    auto count = [&](int shard_base, int nsh, int i, int total, int top, int done) {
        const int sh = i % nsh, in_shard = (total - sh + nsh - 1) / nsh;
        if (bump(shard_base + sh) == in_shard - 1 && bump(top) == min(total, nsh) - 1)
            __hip_atomic_store(gp(sy_slot(sync, done)), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    if (b < a.nroute) {
        route_block<PER, true, true>(a.logits, a.bias, a.T, a.E, a.K, a.topk_idx, a.topk_w, nullptr, a.Ec, a.counts,
                                     a.pref, a.chunk_rank, b, a.nroute);
        __builtin_amdgcn_s_waitcnt(0);  // this wave's coherent stores have completed
        __syncthreads();                 // ... every wave's
        if (threadIdx.x == 0)
            count(SY_ROUTED, SY_RSH, b, a.nroute, SY_RTOP, SY_RDONE);
        return;
    }
    if (b < a.nroute + a.nscan) {
        const int e = (b - a.nroute) * 4 + (int)(threadIdx.x >> 6);
#if defined(CAM_STEP_PHASES) && CAM_STEP_PHASES == 1
        return;
#endif
        if (e >= a.Ec)
            return;
        step_wait<16>(sync, SY_RDONE, 1 + a.extra, a.ticks);
        scan_expert<true>(e, a.nroute, a.counts, a.pref, a.send_offset, a.recv_count, a.tokens_per_expert);
        __builtin_amdgcn_s_waitcnt(0);
        if ((threadIdx.x & 63) == 0) {
            if (a.ndisp_blocks > 0) {
                count(SY_SCANNED, SY_SSH, e, a.Ec, SY_STOP, SY_SDONE);
            } else {
                // routing + scan only (the dispatch is a launch of its own): the wave completing the scan
                // resets the counters -- every scan wave has read the routing flag by then
                const int sh = e % SY_SSH, in_shard = (a.Ec - sh + SY_SSH - 1) / SY_SSH;
                if (bump(SY_SCANNED + sh) == in_shard - 1 && bump(SY_STOP) == min(a.Ec, SY_SSH) - 1) {
                    for (int i = 0; i < SY_STATUS; ++i)
                        __hip_atomic_store(gp(sy_slot(sync, i)), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        return;
    }
    // dispatch blocks loop over (token, chunk) items, item = i * 4 ndb + 4 db + wave: the wait, the count and the
    // barrier happen once per block (every block paying a poll and an atomic round trip measured 76 vs 62 us)
    const int db = b - a.nroute - a.nscan, ndb = a.ndisp_blocks;
    // Wave 0 waits for the scan for the whole block (a few thousand resident waves polling would slow the stages
    // they wait for), then the block meets.  Past the wait the block reads no counter again: wave 0 counts it in
    // its shard; the block completing a shard bumps the top counter, the one completing that resets all.
    auto ready = [&]() {
        if (threadIdx.x < 64) {
            step_wait<64>(sync, SY_SDONE, 1 + a.extra, a.ticks);
            if (threadIdx.x == 0) {
                const int sh = db % SY_DSH, in_shard = (ndb - sh + SY_DSH - 1) / SY_DSH;
                if (bump(SY_PASSED + sh) == in_shard - 1 && bump(SY_TOP) == min(ndb, SY_DSH) - 1) {
                    for (int i = 0; i < SY_STATUS; ++i)
                        __hip_atomic_store(gp(sy_slot(sync, i)), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        __syncthreads();
    };
    const RankSrc rs{nullptr, a.counts, a.chunk_rank, ROUTE_WAVES * 4};
    long item = (long)db * 4 + (threadIdx.x >> 6);
#ifdef CAM_STEP_PHASES  // diagnostic variants: routing and scan (and the dispatch blocks' wait), no dispatch
    ready();
    return;
#endif
    if (item >= (long)a.ndisp_waves) {
        ready();  // a wave without an item still meets the block's barrier
        return;
    }
    // the first item waits (after its loads of x are in flight), the others find the stages done
    dispatch_wave<MODE, true>(a.x, a.topk_idx, a.send_offset, rs, (int)(item / a.nchunk), (int)(item % a.nchunk),
                              a.T, a.H, a.K, a.Ec, 0, a.cap, a.expand_x, a.scales, a.expand_idx, a.inv, a.kmajor,
                              a.skip_unrouted, ready);
    for (item += 4l * ndb; item < (long)a.ndisp_waves; item += 4l * ndb)
        dispatch_wave<MODE, true>(a.x, a.topk_idx, a.send_offset, rs, (int)(item / a.nchunk),
                                  (int)(item % a.nchunk), a.T, a.H, a.K, a.Ec, 0, a.cap, a.expand_x, a.scales,
                                  a.expand_idx, a.inv, a.kmajor, a.skip_unrouted, [] {});
}

// The array's device address on the current device, looked up once per device (host code never uses the
// array's name as an address)
static hipError_t step_sync_ptr(int **out)
{
    constexpr int MAXD = 64;
    static std::atomic<void *> cache[MAXD];
    static std::mutex mu;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return e;
    if (dev < 0 || dev >= MAXD)
        return hipErrorInvalidDevice;
    void *p = cache[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(mu);
        p = cache[dev].load(std::memory_order_relaxed);
        if (!p) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(step_sync));
            if (e != hipSuccess)
                return e;
            cache[dev].store(p, std::memory_order_release);
        }
    }
    *out = (int *)p;
    return hipSuccess;
}

// CAMHIP_STEP_FUSED in the environment (for measuring the forms against each other): 0 -- three launches,
// 1 -- routing + scan in one launch, then the dispatch, 2 -- all three stages in one launch
int step_fused_mode()
{
    static const int mode = [] {
        const char *v = getenv("CAMHIP_STEP_FUSED");
        return v && v[0] >= '0' && v[0] <= '2' ? v[0] - '0' : STEP_DEFAULT_MODE;
    }();
    return mode;
}

static std::atomic<long long> g_step_ticks{0};
static std::atomic<int> g_step_unreach{0};
void step_debug_set(long long wait_ticks, int unreachable)
{
    g_step_ticks.store(wait_ticks, std::memory_order_relaxed);
    g_step_unreach.store(unreachable ? 1 : 0, std::memory_order_relaxed);
}

hipError_t step_status_read(int *status, bool clear)
{
    int *p = nullptr;
    hipError_t e = step_sync_ptr(&p);
    if (e != hipSuccess)
        return e;
    int v = 0;
    e = hipMemcpy(&v, p + SY_STATUS * SY_STRIDE, sizeof(int), hipMemcpyDeviceToHost);
    if (e != hipSuccess)
        return e;
    if (clear && v) {
        // a wait that gave up leaves the counters in an unknown state: start the next launch from zero
        static const int zero[SY_SLOTS * SY_STRIDE] = {};
        e = hipMemcpy(p, zero, sizeof(zero), hipMemcpyHostToDevice);
        if (e != hipSuccess)
            return e;
    }
    *status = v;
    return hipSuccess;
}

hipError_t launch_prefill_step(const float *logits, const float *bias, const uint16_t *x, int T, int H, int E, int Ec,
                               int K, int quant_mode, int cap, bool kmajor, bool skip_unrouted, int32_t *topk_idx,
                               float *topk_w, int32_t *counts, int32_t *pref, int32_t *chunk_rank,
                               int32_t *send_offset, int32_t *recv_count, int64_t *tokens_per_expert,
                               void *expand_x, float *scales, int32_t *expand_idx, int32_t *inv, hipStream_t s)
{
    if (T < 1 || E > 16 * ROUTE_MAX_PER_LANE || K > 16 || Ec < 1 || Ec > E || H > 7 * 1024 || (H & 15))
        return hipErrorInvalidValue;
    if (quant_mode != QUANT_NONE && quant_mode != QUANT_FP8_BLOCK)
        return hipErrorNotSupported;
    if (quant_mode == QUANT_FP8_BLOCK && (H & 127))
        return hipErrorInvalidValue;
    int *sync = nullptr;
    hipError_t e = step_sync_ptr(&sync);
    if (e != hipSuccess)
        return e;
    StepArgs a{};
    a.logits = logits;
    a.bias = bias;
    a.x = x;
    a.T = T;
    a.H = H;
    a.E = E;
    a.Ec = Ec;
    a.K = K;
    a.cap = cap;
    a.nchunk = (H + 1023) / 1024;
    a.kmajor = kmajor ? 1 : 0;
    a.skip_unrouted = skip_unrouted ? 1 : 0;
    a.topk_idx = topk_idx;
    a.topk_w = topk_w;
    a.counts = counts;
    a.pref = pref;
    a.chunk_rank = chunk_rank;
    a.send_offset = send_offset;
    a.recv_count = recv_count;
    a.tokens_per_expert = tokens_per_expert;
    a.expand_x = (uint8_t *)expand_x;
    a.scales = scales;
    a.expand_idx = expand_idx;
    a.inv = inv;
    a.nroute = (T + ROUTE_WAVES * 4 - 1) / (ROUTE_WAVES * 4);
    a.nscan = (Ec + 3) / 4;
    a.ndisp_waves = T * a.nchunk;
    const bool all_in_one = step_fused_mode() == 2;
    a.ndisp_blocks = all_in_one ? std::min((a.ndisp_waves + 3) / 4, STEP_MAX_DISP_BLOCKS) : 0;
    a.sync = sync;
    a.extra = g_step_unreach.load(std::memory_order_relaxed);
    const long long tk = g_step_ticks.load(std::memory_order_relaxed);
    a.ticks = tk > 0 ? tk : 200000000LL;  // 2 s of the 100 MHz constant clock
    const unsigned grid = (unsigned)(a.nroute + a.nscan + a.ndisp_blocks);
    const int per = (E + 15) >> 4;
#define STEP_CASE(P)                                                                                                \
    do {                                                                                                            \
        if (quant_mode == QUANT_FP8_BLOCK)                                                                          \
            hipLaunchKernelGGL((prefill_step_kernel<P, QUANT_FP8_BLOCK>), dim3(grid), dim3(256), 0, s, a);          \
        else                                                                                                        \
            hipLaunchKernelGGL((prefill_step_kernel<P, QUANT_NONE>), dim3(grid), dim3(256), 0, s, a);               \
    } while (0)
    if (per <= 1)
        STEP_CASE(1);
    else if (per <= 2)
        STEP_CASE(2);
    else if (per <= 4)
        STEP_CASE(4);
    else if (per <= 8)
        STEP_CASE(8);
    else if (per <= 16)
        STEP_CASE(16);
    else
        STEP_CASE(32);
#undef STEP_CASE
    e = hipGetLastError();
    if (e != hipSuccess || all_in_one)
        return e;
    return launch_dispatch(x, topk_idx, send_offset, nullptr, T, H, K, Ec, 0, cap, quant_mode, expand_x, scales,
                           expand_idx, s, inv, nullptr, kmajor, counts, ROUTE_WAVES * 4, chunk_rank, skip_unrouted);
}

}  // namespace cam
