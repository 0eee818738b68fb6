// camhipFusedDeepMoe: the decode entry of CAM (aclnnFusedDeepMoe,
// fused_deep_moe/op_api/aclnn_fused_deep_moe.h:19-50; kernel
// fused_deep_moe.h:355-448) on one GPU, composed from the path's kernels:
//   prepare ids (x_active_mask, local expert range) -> layout -> count
//   exchange -> quantised dispatch -> GMM1+SwiGLU -> GMM2 -> combine,
//   plus the optional shared expert on all tokens.  At decode sizes
//   (batch*topk <= 2048, bf16 or fp8) the first four stages are one launch
//   (every block computes the layout in LDS), dispatch writes the combine's
//   row map, and GMM1 and GMM2 run as one chained launch (each GMM2 tile waits
//   for the GMM1 tiles of its rows): three launches in all.  int8 and
//   batch*topk <= 8192: the first three stages are one single-block launch.
// Every intermediate lives in the caller's workspace and every size is fixed
// by (batch, topk): no host synchronisation and no allocation, so the call can
// be captured in a HIP graph (the reference's fused op is its graph-capturable
// decode path, doc/en/cam/CAM API Guide.md:212).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <functional>
#include <new>
#include <string>

#include "../../include/camhip.h"
#include "gmm.h"
#include "launchers.h"

namespace cam {
camhipStatus api_fail(camhipStatus code, const char *fmt, ...);
camhipStatus api_make_executor(uint64_t ws_bytes, std::function<hipError_t(void *, hipStream_t)> fn,
                               uint64_t *workspaceSize, camhipExecutor **executor);
camhipStatus api_run_executor(const char *op, void *workspace, uint64_t workspaceSize, camhipExecutor *ex,
                              void *stream);
}  // namespace cam

namespace {

struct Carve {
    uint64_t off = 0;
    uint64_t take(uint64_t bytes)
    {
        const uint64_t o = off;
        off += (bytes + 255) & ~(uint64_t)255;
        return o;
    }
};

struct FusedLayout {
    uint64_t ids, layout_ws, counts, send_off, recv_cnt, total, sti, ex, xs, eidx, h, hs, y, inv, hf, amax, ready;
    uint64_t sh_x, sh_xs, sh_h, sh_hs, sh_gl, sh_hf, sh_amax;
    uint64_t bytes;
};

// Scale bytes per row of `cols` elements: fp8 one float per 128, int8 one per row, bf16 none.
static uint64_t scale_bytes(int dt, uint64_t cols)
{
    return dt == cam::DT_FP8 ? cols / 128 * 4 : dt == cam::DT_INT8 ? 4 : 0;
}

FusedLayout plan_fused(int T, int H, int K, int L, int I, int Ish, int dt, bool shared)
{
    Carve c;
    FusedLayout f{};
    const uint64_t N = (uint64_t)T * K;
    const uint64_t esz = dt == cam::DT_BF16 ? 2 : 1;
    const bool int8 = dt == cam::DT_INT8;
    f.ids = c.take(4 * N);
    f.layout_ws = c.take(cam::layout_workspace_bytes(T, K, L, 1));
    f.counts = c.take(4 * (uint64_t)L);
    f.send_off = c.take(4 * (uint64_t)L);
    f.recv_cnt = c.take(4 * (uint64_t)L);
    f.total = c.take(4);
    f.sti = c.take(4 * N);
    f.ex = c.take(N * H * esz);
    f.xs = c.take(N * scale_bytes(dt, H));
    f.eidx = c.take(12 * N);
    f.h = c.take(N * I * esz);
    f.hs = c.take(N * scale_bytes(dt, I));
    f.y = c.take(N * H * 2);
    f.inv = c.take(4 * N);
    f.hf = c.take(int8 ? N * I * 4 : 0);  // int8: fp32 h and its row maxima before the requantisation
    f.amax = c.take(int8 ? N * (I / cam::GMM_AMAX_COLS) * 4 : 0);  // partial row maxima of h
    f.ready = c.take(int8 ? 0 : 4 * (uint64_t)cam::gmm_chain_counters((int)N, L));  // chained GEMMs' counters
    if (shared) {
        f.sh_x = c.take((uint64_t)T * H * esz);
        f.sh_xs = c.take((uint64_t)T * scale_bytes(dt, H));
        f.sh_h = c.take((uint64_t)T * Ish * esz);
        f.sh_hs = c.take((uint64_t)T * scale_bytes(dt, Ish));
        f.sh_gl = c.take(8);
        f.sh_hf = c.take(int8 ? (uint64_t)T * Ish * 4 : 0);
        f.sh_amax = c.take(int8 ? (uint64_t)T * (Ish / cam::GMM_AMAX_COLS) * 4 : 0);
    }
    f.bytes = c.off;
    return f;
}

#define F_CHECK(cond, ...)                                                                                          \
    do {                                                                                                            \
        if (!(cond))                                                                                                \
            return cam::api_fail(CAMHIP_ERROR_INVALID_PARAM, __VA_ARGS__);                                          \
    } while (0)
#define F_PTR(p)                                                                                                    \
    do {                                                                                                            \
        if ((p) == nullptr)                                                                                         \
            return cam::api_fail(CAMHIP_ERROR_NULLPTR, "fused_deep_moe: %s must not be NULL", #p);                  \
    } while (0)

#define HIP_TRY(x)                                                                                                  \
    do {                                                                                                            \
        hipError_t e_ = (x);                                                                                        \
        if (e_ != hipSuccess)                                                                                       \
            return e_;                                                                                              \
    } while (0)

}  // namespace

extern "C" {

camhipStatus camhipFusedDeepMoeGetWorkspaceSize(
    const uint16_t *x, const int32_t *expertIds, const void *gmm1Weight, const float *gmm1WeightScale,
    const void *gmm2Weight, const float *gmm2WeightScale, const float *expertScales, const void *shareGmm1Weight,
    const float *shareGmm1WeightScale, const void *shareGmm2Weight, const float *shareGmm2WeightScale,
    const float *expertSmoothScales, const float *shareSmoothScales, const uint8_t *xActiveMask, int64_t batchSize,
    int64_t hidden, int64_t topK, int64_t gmm1HiddenSize, int64_t shareGmm1HiddenSize, int64_t weightDtype,
    int64_t epRankSize, int64_t epRankId, int64_t moeExpertNum, int64_t quantMode, int64_t globalBs,
    uint16_t *output, uint16_t *shareOutput, int64_t *expertTokenNums, uint64_t *workspaceSize,
    camhipExecutor **executor)
{
    F_CHECK(epRankSize == 1 && epRankId == 0,
            "fused_deep_moe: this build runs one EP rank per GPU (ep_rank_size %lld, ep_rank_id %lld; need 1, 0)",
            (long long)epRankSize, (long long)epRankId);
    F_CHECK(batchSize >= 0 && batchSize <= 4096, "fused_deep_moe: batch size %lld out of [0,4096]",
            (long long)batchSize);
    F_CHECK(topK >= 1 && topK <= 12, "fused_deep_moe: topk %lld out of [1,12]", (long long)topK);
    F_CHECK(moeExpertNum >= 1 && moeExpertNum <= 512 && topK <= moeExpertNum,
            "fused_deep_moe: moe_expert_num %lld out of [topk,512]", (long long)moeExpertNum);
    // the reference's fused tiling accepts token lengths from 512 (fused_deep_moe_tiling.cpp:66-67)
    F_CHECK(hidden >= 512 && hidden <= 7168 && hidden % 256 == 0,
            "fused_deep_moe: hidden %lld must be in [512,7168] and a multiple of 256", (long long)hidden);
    F_CHECK(gmm1HiddenSize >= 256 && gmm1HiddenSize % 256 == 0,
            "fused_deep_moe: gmm1 hidden size (2I) %lld must be a multiple of 256", (long long)gmm1HiddenSize);
    // separated mode (the reference's per-expert tensor lists, dynamic EPLB): the four routed-expert weight
    // arguments are device arrays of L pointers
    const bool wlist = (weightDtype & CAMHIP_WEIGHT_LIST) != 0;
    weightDtype &= ~(int64_t)CAMHIP_WEIGHT_LIST;
    F_CHECK(weightDtype == CAMHIP_DTYPE_BF16 || weightDtype == CAMHIP_DTYPE_INT8 || weightDtype == CAMHIP_DTYPE_FP8,
            "fused_deep_moe: weight dtype %lld not supported (bf16, int8 or fp8 e4m3fn)", (long long)weightDtype);
    F_CHECK(quantMode == 0, "fused_deep_moe: quant_mode is reserved and must be 0 (got %lld)", (long long)quantMode);
    F_CHECK(globalBs >= 0 && globalBs % epRankSize == 0, "fused_deep_moe: global_bs %lld invalid",
            (long long)globalBs);
    F_CHECK(weightDtype == CAMHIP_DTYPE_INT8 || (expertSmoothScales == nullptr && shareSmoothScales == nullptr),
            "fused_deep_moe: smooth-quant scales need int8 weights");
    const bool shared = shareGmm1Weight != nullptr;
    F_CHECK(shared == (shareGmm2Weight != nullptr),
            "fused_deep_moe: shared-expert weights must be given together");
    if (!shared)  // the reference's test passes share_smooth_scales with or without a shared expert
        shareSmoothScales = nullptr;
    const bool quantised = weightDtype != CAMHIP_DTYPE_BF16;
    {
        // the grouped GEMMs address an operand with 32-bit byte offsets: one expert's weights, the dispatched
        // rows and h stay under 4 GiB
        const int64_t esz = weightDtype == CAMHIP_DTYPE_BF16 ? 2 : 1, lim = (int64_t)1 << 32;
        const int64_t rows = batchSize * topK, i2 = std::max(gmm1HiddenSize, shared ? shareGmm1HiddenSize : 0);
        F_CHECK(i2 * hidden * esz < lim && rows * hidden * esz < lim && rows * (i2 / 2) * esz < lim,
                "fused_deep_moe: an expert's weights or the dispatched rows exceed 4 GiB (gmm1 hidden size %lld)",
                (long long)i2);
    }
    if (shared) {
        F_CHECK(shareGmm1HiddenSize >= 256 && shareGmm1HiddenSize % 256 == 0,
                "fused_deep_moe: share gmm1 hidden size %lld must be a multiple of 256",
                (long long)shareGmm1HiddenSize);
        F_PTR(shareOutput);
        if (quantised) {
            F_PTR(shareGmm1WeightScale);
            F_PTR(shareGmm2WeightScale);
        }
    }
    F_PTR(gmm1Weight);
    F_PTR(gmm2Weight);
    F_PTR(expertTokenNums);
    if (quantised) {
        F_PTR(gmm1WeightScale);
        F_PTR(gmm2WeightScale);
    }
    if (batchSize > 0) {
        F_PTR(x);
        F_PTR(expertIds);
        F_PTR(expertScales);
        F_PTR(output);
    }
    F_CHECK(workspaceSize != nullptr && executor != nullptr, "fused_deep_moe: NULL workspace size or executor");

    const int T = (int)batchSize, H = (int)hidden, K = (int)topK, L = (int)(moeExpertNum / epRankSize);
    const int I = (int)(gmm1HiddenSize / 2), Ish = (int)(shareGmm1HiddenSize / 2);
    const int dt = (int)weightDtype;  // CAMHIP_DTYPE_* equal cam::DT_*
    const bool int8 = dt == cam::DT_INT8;
    const FusedLayout f = plan_fused(T, H, K, L, I, shared ? Ish : 0, dt, shared);
    const int N = T * K;
    const int q = dt == cam::DT_FP8 ? cam::QUANT_FP8_BLOCK : int8 ? cam::QUANT_INT8_FUSED : cam::QUANT_NONE;
    const int epi1 = dt == cam::DT_FP8 ? cam::EPI_SWIGLU_FP8 : int8 ? cam::EPI_SWIGLU_F32AMAX : cam::EPI_SWIGLU_BF16;
    // GMM1 + SwiGLU: int8 writes fp32 h and row maxima, then requantises per token
    auto gmm1 = [=](cam::GmmArgs a, float *hf, float *amax, hipStream_t s) -> hipError_t {
        if (!int8)
            return cam::launch_gmm(a, dt, epi1, s);
        int8_t *hq = (int8_t *)a.C;
        float *hs = a.Cs;
        a.C = (uint8_t *)hf;
        a.Cs = amax;
        HIP_TRY(cam::launch_gmm(a, dt, epi1, s));
        return cam::launch_quant_rows_int8(hf, amax, a.group_list, a.L, a.M, a.N / 2, hq, hs, s);
    };

    auto fn = [=](void *wsv, hipStream_t s) -> hipError_t {
        uint8_t *ws = (uint8_t *)wsv;
        auto P = [&](uint64_t off) { return (void *)(ws + off); };
        int32_t *ids = (int32_t *)P(f.ids);
        int32_t *counts = (int32_t *)P(f.counts), *send_off = (int32_t *)P(f.send_off);
        int32_t *recv_cnt = (int32_t *)P(f.recv_cnt);
        if (T == 0) {  // no tokens: no expert receives any
            return cam::launch_fill_i64(expertTokenNums, 0, L, s);
        }
        cam::GmmArgs g1{(const uint8_t *)P(f.ex), (const float *)P(f.xs), expertTokenNums, L, N, H, 2 * I,
                        (const uint8_t *)gmm1Weight, gmm1WeightScale, (uint8_t *)P(f.h), (float *)P(f.hs)};
        cam::GmmArgs g2{(const uint8_t *)P(f.h), (const float *)P(f.hs), expertTokenNums, L, N, I, H,
                        (const uint8_t *)gmm2Weight, gmm2WeightScale, (uint8_t *)P(f.y), nullptr};
        if (wlist) {
            g1.Wl = (const uint8_t *const *)gmm1Weight;
            g1.Wsl = (const float *const *)gmm1WeightScale;
            g2.Wl = (const uint8_t *const *)gmm2Weight;
            g2.Wsl = (const float *const *)gmm2WeightScale;
        }
        // GMM1 -> GMM2 as one launch where a chained kernel exists; its readiness counters start at zero
        const bool chained = cam::gmm_chain_supported(g1, g2, dt);
        int32_t *ready = (int32_t *)P(f.ready);
        const int nready = chained ? cam::gmm_chain_counters(N, L) : 0;
        // decode sizes with bf16 or fp8 rows: id preparation, layout, count exchange and the dispatch in one
        // launch (which also clears the counters)
        const bool one_launch = !int8 && cam::dispatch_decode_fits(T, K, L);
        if (one_launch) {
            HIP_TRY(cam::launch_dispatch_decode(expertIds, xActiveMask, x, T, H, K, L, N, q, P(f.ex), (float *)P(f.xs),
                                                (int32_t *)P(f.eidx), (int32_t *)P(f.inv), true, counts, send_off,
                                                recv_cnt, (int32_t *)P(f.total), expertTokenNums, s, ready, nready));
        } else if (N <= 8192) {
            // decode sizes: id preparation, layout and count exchange in one launch (which also clears the
            // counters)
            HIP_TRY(cam::launch_layout_small(expertIds, xActiveMask, T, K, L, ids, counts, (int32_t *)P(f.sti),
                                             send_off, recv_cnt, (int32_t *)P(f.total), expertTokenNums, s, ready,
                                             nready));
        } else {
            if (chained)
                HIP_TRY(cam::launch_fill_i32(ready, 0, nready, s));
            HIP_TRY(cam::launch_prepare_ids(expertIds, xActiveMask, T, K, 0, L, ids, s));
            HIP_TRY(cam::launch_layout_i32(ids, T, K, L, counts, (int32_t *)P(f.sti), P(f.layout_ws), s));
            HIP_TRY(cam::launch_notify(counts, L, T, send_off, (int32_t *)P(f.total), recv_cnt, nullptr, nullptr,
                                       expertTokenNums, L, s));
        }
        // dispatch also writes the combine's row map (inv), so the combine is a single gather; fp8 block
        // scales come out k-major, the layout GMM1 reads
        if (!one_launch)
            HIP_TRY(cam::launch_dispatch(x, ids, send_off, (int32_t *)P(f.sti), T, H, K, L, 0, N, q, P(f.ex),
                                         (float *)P(f.xs), (int32_t *)P(f.eidx), s, (int32_t *)P(f.inv),
                                         expertSmoothScales, true));
        if (chained) {
            HIP_TRY(cam::launch_gmm_chain(g1, g2, dt, ready, s));
        } else {
            HIP_TRY(gmm1(g1, (float *)P(f.hf), (float *)P(f.amax), s));
            HIP_TRY(cam::launch_gmm(g2, dt, cam::EPI_PLAIN, s));
        }
        HIP_TRY(cam::launch_combine_gather((const uint16_t *)P(f.y), (const int32_t *)P(f.eidx), N,
                                           recv_cnt + (L - 1), expertScales, T, K, H, output,
                                           (const int32_t *)P(f.inv), s));
        if (shared) {
            // shared expert on every token: x quantised in token order, one group of T rows
            int64_t *gl = (int64_t *)P(f.sh_gl);
            HIP_TRY(cam::launch_fill_i64(gl, T, 1, s));
            const void *sx = x;
            const float *sxs = nullptr;
            if (dt != cam::DT_BF16) {
                HIP_TRY(cam::launch_dispatch(x, nullptr, nullptr, nullptr, T, H, 1, 1, 0, T, q, P(f.sh_x),
                                             (float *)P(f.sh_xs), nullptr, s, nullptr, shareSmoothScales, true));
                sx = P(f.sh_x);
                sxs = (const float *)P(f.sh_xs);
            }
            cam::GmmArgs s1{(const uint8_t *)sx, sxs, gl, 1, T, H, 2 * Ish, (const uint8_t *)shareGmm1Weight,
                            shareGmm1WeightScale, (uint8_t *)P(f.sh_h), (float *)P(f.sh_hs)};
            HIP_TRY(gmm1(s1, (float *)P(f.sh_hf), (float *)P(f.sh_amax), s));
            cam::GmmArgs s2{(const uint8_t *)P(f.sh_h), (const float *)P(f.sh_hs), gl, 1, T, Ish, H,
                            (const uint8_t *)shareGmm2Weight, shareGmm2WeightScale, (uint8_t *)shareOutput,
                            nullptr};
            HIP_TRY(cam::launch_gmm(s2, dt, cam::EPI_PLAIN, s));
        }
        return hipSuccess;
    };
    return cam::api_make_executor(f.bytes, fn, workspaceSize, executor);
}

camhipStatus camhipFusedDeepMoe(void *workspace, uint64_t workspaceSize, camhipExecutor *executor, void *stream)
{
    return cam::api_run_executor("fused_deep_moe", workspace, workspaceSize, executor, stream);
}

}  // extern "C"
