// Two-phase C ABI (include/camhip.h): argument validation, workspace sizing,
// executor lifetime and error reporting.  Mirrors the aclnn pattern of the
// reference (op_api/aclnn_*.h; status + message as in
// pybind/pytorch_extension/pytorch_npu_helper.hpp:585,599 and the tiling
// range checks, e.g. dispatch_layout_tiling.cpp:98-122).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <functional>
#include <new>
#include <string>

#include "../../include/camhip.h"
#include "gmm.h"
#include "launchers.h"

static_assert(CAMHIP_COMBINE_NOALLOC_MAX_SLOTS == cam::COMBINE_NOALLOC_MAX_SLOTS, "scratch size of the header");

struct camhipExecutor {
    uint64_t workspace_bytes = 0;
    std::function<hipError_t(void *ws, hipStream_t s)> launch;
};

namespace {

thread_local std::string g_last_error;

camhipStatus fail(camhipStatus code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

#define CHECK_PARAM(cond, ...)                                                                                      \
    do {                                                                                                            \
        if (!(cond))                                                                                                \
            return fail(CAMHIP_ERROR_INVALID_PARAM, __VA_ARGS__);                                                   \
    } while (0)
#define CHECK_PTR(p)                                                                                                \
    do {                                                                                                            \
        if ((p) == nullptr)                                                                                         \
            return fail(CAMHIP_ERROR_NULLPTR, "%s: %s must not be NULL", __func__, #p);                             \
    } while (0)

camhipStatus make_executor(uint64_t ws_bytes, std::function<hipError_t(void *, hipStream_t)> fn,
                           uint64_t *workspaceSize, camhipExecutor **executor)
{
    CHECK_PTR(workspaceSize);
    CHECK_PTR(executor);
    camhipExecutor *ex = new (std::nothrow) camhipExecutor;
    if (!ex)
        return fail(CAMHIP_ERROR_RUNTIME, "out of host memory creating an executor");
    ex->workspace_bytes = ws_bytes;
    ex->launch = std::move(fn);
    *workspaceSize = ws_bytes;
    *executor = ex;
    g_last_error.clear();
    return CAMHIP_SUCCESS;
}

camhipStatus run_executor(const char *op, void *workspace, uint64_t workspaceSize, camhipExecutor *ex, void *stream)
{
    if (!ex)
        return fail(CAMHIP_ERROR_NULLPTR, "%s: executor is NULL", op);
    camhipStatus st = CAMHIP_SUCCESS;
    if (workspaceSize < ex->workspace_bytes || (ex->workspace_bytes > 0 && workspace == nullptr)) {
        st = fail(CAMHIP_ERROR_WORKSPACE, "%s: workspace of %llu bytes given, %llu needed", op,
                  (unsigned long long)workspaceSize, (unsigned long long)ex->workspace_bytes);
    } else {
        hipError_t err = ex->launch(workspace, (hipStream_t)stream);
        if (err != hipSuccess)
            st = fail(CAMHIP_ERROR_RUNTIME, "%s: launch failed: %s", op, hipGetErrorString(err));
        else
            g_last_error.clear();
    }
    delete ex;
    return st;
}

}  // namespace

namespace cam {
// shared with fused_api.cpp
camhipStatus api_fail(camhipStatus code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}
camhipStatus api_make_executor(uint64_t ws_bytes, std::function<hipError_t(void *, hipStream_t)> fn,
                               uint64_t *workspaceSize, camhipExecutor **executor)
{
    return make_executor(ws_bytes, std::move(fn), workspaceSize, executor);
}
camhipStatus api_run_executor(const char *op, void *workspace, uint64_t workspaceSize, camhipExecutor *ex,
                              void *stream)
{
    return run_executor(op, workspace, workspaceSize, ex, stream);
}
}  // namespace cam

namespace {

constexpr int64_t kMaxTokens = 65536;
constexpr int64_t kMaxExperts = 512;
constexpr int64_t kMaxRanks = 384;
constexpr int64_t kMaxTopk = 16;
constexpr int64_t kMinHidden = 1024;
constexpr int64_t kMaxHidden = 7168;

}  // namespace

extern "C" {

const char *camhipGetLastErrorMsg(void) { return g_last_error.c_str(); }
const char *camhipGetVersion(void) { return "camhip 0.1.0 gfx950"; }
void camhipReleaseExecutor(camhipExecutor *executor) { delete executor; }

// ---------------------------------------------------------------- routing
camhipStatus camhipMoeRouteGetWorkspaceSize(const float *logits, const float *bias, int64_t numTokens,
                                            int64_t numExperts, int64_t topK, int32_t *topkIdx, float *topkWeights,
                                            int64_t *topkIdxInt64, uint64_t *workspaceSize,
                                            camhipExecutor **executor)
{
    CHECK_PARAM(numTokens >= 0 && numTokens <= kMaxTokens, "moe_route: numTokens %lld out of [0,%lld]",
                (long long)numTokens, (long long)kMaxTokens);
    CHECK_PARAM(numExperts >= 1 && numExperts <= kMaxExperts, "moe_route: numExperts %lld out of [1,%lld]",
                (long long)numExperts, (long long)kMaxExperts);
    CHECK_PARAM(topK >= 1 && topK <= kMaxTopk && topK <= numExperts, "moe_route: topK %lld out of [1,min(16,E)]",
                (long long)topK);
    if (numTokens > 0) {
        CHECK_PTR(logits);
        CHECK_PTR(topkIdx);
        CHECK_PTR(topkWeights);
    }
    const int T = (int)numTokens, E = (int)numExperts, K = (int)topK;
    return make_executor(
        0,
        [=](void *, hipStream_t s) {
            return cam::launch_route(logits, bias, T, E, K, topkIdx, topkWeights, s, topkIdxInt64);
        },
        workspaceSize, executor);
}

camhipStatus camhipMoeRoute(void *workspace, uint64_t workspaceSize, camhipExecutor *executor, void *stream)
{
    return run_executor("moe_route", workspace, workspaceSize, executor, stream);
}

// ---------------------------------------------------------------- layout
camhipStatus camhipDispatchLayoutGetWorkspaceSize(const int64_t *topkIdx, int64_t numTokens, int64_t numRanks,
                                                  int64_t numExperts, int64_t numTopk, int32_t *numTokensPerRank,
                                                  int32_t *numTokensPerExpert, int32_t *isTokenInRank,
                                                  int32_t *sendTokenIdxSmall, uint64_t *workspaceSize,
                                                  camhipExecutor **executor)
{
    CHECK_PARAM(numTokens >= 0 && numTokens <= kMaxTokens, "dispatch_layout: numTokens %lld out of [0,%lld]",
                (long long)numTokens, (long long)kMaxTokens);
    CHECK_PARAM(numRanks >= 1 && numRanks <= kMaxRanks, "dispatch_layout: numRanks %lld out of [1,%lld]",
                (long long)numRanks, (long long)kMaxRanks);
    CHECK_PARAM(numExperts >= 1 && numExperts <= kMaxExperts, "dispatch_layout: numExperts %lld out of [1,%lld]",
                (long long)numExperts, (long long)kMaxExperts);
    CHECK_PARAM(numExperts % numRanks == 0, "dispatch_layout: numExperts %lld not divisible by numRanks %lld",
                (long long)numExperts, (long long)numRanks);
    CHECK_PARAM(numTopk >= 1 && numTopk <= kMaxTopk, "dispatch_layout: numTopk %lld out of [1,%lld]",
                (long long)numTopk, (long long)kMaxTopk);
    CHECK_PTR(numTokensPerExpert);
    if (numTokens > 0) {
        CHECK_PTR(topkIdx);
        CHECK_PTR(sendTokenIdxSmall);
    }
    const int T = (int)numTokens, K = (int)numTopk, E = (int)numExperts, R = (int)numRanks;
    const uint64_t ws = cam::layout_workspace_bytes(T, K, E, R);
    return make_executor(
        ws,
        [=](void *w, hipStream_t s) {
            return cam::launch_layout(topkIdx, T, K, E, R, numTokensPerRank, numTokensPerExpert, isTokenInRank,
                                      sendTokenIdxSmall, w, s);
        },
        workspaceSize, executor);
}

camhipStatus camhipDispatchLayout(void *workspace, uint64_t workspaceSize, camhipExecutor *executor, void *stream)
{
    return run_executor("dispatch_layout", workspace, workspaceSize, executor, stream);
}

// ---------------------------------------------------------------- notify
camhipStatus camhipNotifyDispatchGetWorkspaceSize(const int32_t *tokenPerExpertData, int64_t numExperts,
                                                  int64_t numTokens, int64_t rankSize, int64_t rankId,
                                                  int32_t *sendDataOffset, int32_t *totalRecvTokens,
                                                  int32_t *recvCount, int32_t *recvOffset, int32_t *maxBs,
                                                  int64_t *recvTokensPerExpert, uint64_t *workspaceSize,
                                                  camhipExecutor **executor)
{
    CHECK_PARAM(rankSize == 1 && rankId == 0,
                "notify_dispatch: this build runs one EP rank per GPU (rankSize %lld, rankId %lld; need 1, 0)",
                (long long)rankSize, (long long)rankId);
    CHECK_PARAM(numExperts >= 1 && numExperts <= kMaxExperts, "notify_dispatch: numExperts %lld out of [1,%lld]",
                (long long)numExperts, (long long)kMaxExperts);
    CHECK_PARAM(numTokens >= 0 && numTokens <= kMaxTokens, "notify_dispatch: numTokens %lld out of range",
                (long long)numTokens);
    CHECK_PTR(tokenPerExpertData);
    CHECK_PTR(sendDataOffset);
    const int E = (int)numExperts, T = (int)numTokens, L = (int)(numExperts / rankSize);
    return make_executor(
        0,
        [=](void *, hipStream_t s) {
            return cam::launch_notify(tokenPerExpertData, E, T, sendDataOffset, totalRecvTokens, recvCount,
                                      recvOffset, maxBs, recvTokensPerExpert, L, s);
        },
        workspaceSize, executor);
}

camhipStatus camhipNotifyDispatch(void *workspace, uint64_t workspaceSize, camhipExecutor *executor, void *stream)
{
    return run_executor("notify_dispatch", workspace, workspaceSize, executor, stream);
}

// ---------------------------------------------------------------- dispatch
camhipStatus camhipMoeDispatchNormalGetWorkspaceSize(const uint16_t *x, const int32_t *topkIdx,
                                                     const int32_t *sendOffset, const int32_t *sendTokenIdx,
                                                     const int32_t *recvOffset, const int32_t *recvCount,
                                                     int64_t numTokens, int64_t hidden, int64_t numTopk,
                                                     int64_t epWorldSize, int64_t epRankId, int64_t moeExpertNum,
                                                     int64_t quantMode, int64_t recvRowsCapacity, void *recvX,
                                                     float *recvXScales, int32_t *assistInfoForCombine,
                                                     int32_t *waitRecvCostStats, uint64_t *workspaceSize,
                                                     camhipExecutor **executor)
{
    (void)recvOffset;
    (void)recvCount;
    CHECK_PARAM(epWorldSize == 1 && epRankId == 0,
                "moe_dispatch: this build runs one EP rank per GPU (epWorldSize %lld, epRankId %lld; need 1, 0)",
                (long long)epWorldSize, (long long)epRankId);
    CHECK_PARAM(numTokens >= 0 && numTokens <= kMaxTokens, "moe_dispatch: numTokens %lld out of range",
                (long long)numTokens);
    CHECK_PARAM(hidden >= kMinHidden && hidden <= kMaxHidden && hidden % 16 == 0,
                "moe_dispatch: hidden %lld must be in [%lld,%lld] and a multiple of 16", (long long)hidden,
                (long long)kMinHidden, (long long)kMaxHidden);
    CHECK_PARAM(numTopk >= 1 && numTopk <= kMaxTopk, "moe_dispatch: numTopk %lld out of [1,%lld]",
                (long long)numTopk, (long long)kMaxTopk);
    CHECK_PARAM(moeExpertNum >= 1 && moeExpertNum <= kMaxExperts, "moe_dispatch: moeExpertNum %lld out of range",
                (long long)moeExpertNum);
    CHECK_PARAM(quantMode == CAMHIP_QUANT_NONE || quantMode == CAMHIP_QUANT_INT8_TOKEN ||
                    quantMode == CAMHIP_QUANT_FP8_BLOCK || quantMode == CAMHIP_QUANT_FP8_BLOCK_KMAJOR,
                "moe_dispatch: quantMode %lld not supported (0, 2, 3 or 5)", (long long)quantMode);
    const bool kmajor = quantMode == CAMHIP_QUANT_FP8_BLOCK_KMAJOR;
    if (kmajor)
        quantMode = CAMHIP_QUANT_FP8_BLOCK;
    CHECK_PARAM(quantMode != CAMHIP_QUANT_FP8_BLOCK || hidden % 128 == 0,
                "moe_dispatch: fp8 1x128 quantisation needs hidden %% 128 == 0 (hidden %lld)", (long long)hidden);
    CHECK_PARAM(recvRowsCapacity >= 0, "moe_dispatch: negative recvRowsCapacity");
    if (numTokens > 0) {
        CHECK_PTR(x);
        CHECK_PTR(topkIdx);
        CHECK_PTR(sendOffset);
        CHECK_PTR(sendTokenIdx);
        CHECK_PTR(recvX);
        CHECK_PTR(assistInfoForCombine);
        if (quantMode != CAMHIP_QUANT_NONE)
            CHECK_PTR(recvXScales);
    }
    const int T = (int)numTokens, H = (int)hidden, K = (int)numTopk, E = (int)moeExpertNum, q = (int)quantMode;
    const int rank = (int)epRankId;
    const int cap = recvRowsCapacity > 0x7fffffff ? 0x7fffffff : (int)recvRowsCapacity;
    // diagnose output: [epWorldSize] int32, microseconds of the dispatch phase per source rank, accumulated
    int32_t *stats = waitRecvCostStats;
    return make_executor(
        stats ? sizeof(uint64_t) : 0,
        [=](void *w, hipStream_t s) {
            if (stats) {
                hipError_t e = cam::launch_phase_begin((uint64_t *)w, s);
                if (e != hipSuccess)
                    return e;
            }
            hipError_t e = cam::launch_dispatch(x, topkIdx, sendOffset, sendTokenIdx, T, H, K, E, rank, cap, q, recvX,
                                                recvXScales, assistInfoForCombine, s, nullptr, nullptr, kmajor);
            if (e != hipSuccess || !stats)
                return e;
            return cam::launch_phase_end((const uint64_t *)w, stats, rank, s);
        },
        workspaceSize, executor);
}

camhipStatus camhipMoeDispatchNormal(void *workspace, uint64_t workspaceSize, camhipExecutor *executor, void *stream)
{
    return run_executor("moe_dispatch", workspace, workspaceSize, executor, stream);
}

// ---------------------------------------------------------------- combine
static camhipStatus check_combine(const uint16_t *recvX, const int32_t *tokenSrcInfo, int64_t numRecvRows,
                                  const float *recvTopkWeights, int64_t numTokens, int64_t numTopk, int64_t hidden,
                                  int64_t epWorldSize, int64_t epRankId, int64_t moeExpertNum, uint16_t *out)
{
    CHECK_PARAM(epWorldSize == 1 && epRankId == 0,
                "moe_combine: this build runs one EP rank per GPU (epWorldSize %lld, epRankId %lld; need 1, 0)",
                (long long)epWorldSize, (long long)epRankId);
    CHECK_PARAM(numTokens >= 0 && numTokens <= kMaxTokens, "moe_combine: numTokens %lld out of range",
                (long long)numTokens);
    CHECK_PARAM(numRecvRows >= 0 && numRecvRows <= numTokens * 16 + 1,
                "moe_combine: numRecvRows %lld out of range", (long long)numRecvRows);
    CHECK_PARAM(hidden >= kMinHidden && hidden <= kMaxHidden && hidden % 16 == 0,
                "moe_combine: hidden %lld must be in [%lld,%lld] and a multiple of 16", (long long)hidden,
                (long long)kMinHidden, (long long)kMaxHidden);
    CHECK_PARAM(numTopk >= 1 && numTopk <= kMaxTopk, "moe_combine: numTopk %lld out of [1,%lld]", (long long)numTopk,
                (long long)kMaxTopk);
    CHECK_PARAM(moeExpertNum >= 1 && moeExpertNum <= kMaxExperts, "moe_combine: moeExpertNum %lld out of range",
                (long long)moeExpertNum);
    if (numTokens > 0) {
        CHECK_PTR(recvTopkWeights);
        CHECK_PTR(out);
        if (numRecvRows > 0) {
            CHECK_PTR(recvX);
            CHECK_PTR(tokenSrcInfo);
        }
    }
    return CAMHIP_SUCCESS;
}

camhipStatus camhipMoeCombineNormalGetWorkspaceSize(const uint16_t *recvX, const int32_t *tokenSrcInfo,
                                                    int64_t numRecvRows, const int32_t *epRecvCounts,
                                                    const float *recvTopkWeights, int64_t numTokens, int64_t numTopk,
                                                    int64_t hidden, int64_t epWorldSize, int64_t epRankId,
                                                    int64_t moeExpertNum, uint16_t *out, int32_t *sendCostStats,
                                                    uint64_t *workspaceSize, camhipExecutor **executor)
{
    camhipStatus st = check_combine(recvX, tokenSrcInfo, numRecvRows, recvTopkWeights, numTokens, numTopk, hidden,
                                    epWorldSize, epRankId, moeExpertNum, out);
    if (st != CAMHIP_SUCCESS)
        return st;
    const int N = (int)numRecvRows, T = (int)numTokens, K = (int)numTopk, H = (int)hidden;
    const int32_t *last = epRecvCounts ? epRecvCounts + (moeExpertNum - 1) : nullptr;
    // workspace: the row map [T*K] int32, then (diagnose output requested) the phase's start stamp
    const uint64_t map_bytes = (sizeof(int32_t) * (uint64_t)T * K + 7) & ~(uint64_t)7;
    int32_t *stats = sendCostStats;
    const int rank = (int)epRankId;
    return make_executor(
        map_bytes + (stats ? sizeof(uint64_t) : 0),
        [=](void *w, hipStream_t s) {
            uint64_t *stamp = (uint64_t *)((uint8_t *)w + map_bytes);
            if (stats) {
                hipError_t e = cam::launch_phase_begin(stamp, s);
                if (e != hipSuccess)
                    return e;
            }
            hipError_t e =
                cam::launch_combine(recvX, tokenSrcInfo, N, last, recvTopkWeights, T, K, H, out, (int32_t *)w, s);
            if (e != hipSuccess || !stats)
                return e;
            return cam::launch_phase_end(stamp, stats, rank, s);
        },
        workspaceSize, executor);
}

camhipStatus camhipMoeCombineNormal(void *workspace, uint64_t workspaceSize, camhipExecutor *executor, void *stream)
{
    return run_executor("moe_combine", workspace, workspaceSize, executor, stream);
}

// ---------------------------------------------------------------- prefill step (extension)
camhipStatus camhipMoePrefillDispatchGetWorkspaceSize(const float *logits, const float *bias, const uint16_t *x,
                                                      int64_t numTokens, int64_t hidden, int64_t numExperts,
                                                      int64_t localExperts, int64_t topK, int64_t quantMode,
                                                      int64_t recvRowsCapacity, int32_t *topkIdx, float *topkWeights,
                                                      void *recvX, float *recvXScales, int32_t *expandIdx,
                                                      int32_t *recvCount, int64_t *recvTokensPerExpert,
                                                      int32_t *combineRowMap, uint64_t *workspaceSize,
                                                      camhipExecutor **executor)
{
    CHECK_PARAM(numTokens >= 1 && numTokens <= kMaxTokens, "moe_prefill_dispatch: numTokens %lld out of [1,%lld]",
                (long long)numTokens, (long long)kMaxTokens);
    CHECK_PARAM(numExperts >= 1 && numExperts <= kMaxExperts, "moe_prefill_dispatch: numExperts %lld out of range",
                (long long)numExperts);
    CHECK_PARAM(localExperts >= 1 && localExperts <= numExperts,
                "moe_prefill_dispatch: localExperts %lld out of [1, numExperts]", (long long)localExperts);
    CHECK_PARAM(topK >= 1 && topK <= kMaxTopk && topK <= numExperts, "moe_prefill_dispatch: topK %lld out of range",
                (long long)topK);
    CHECK_PARAM(hidden >= kMinHidden && hidden <= kMaxHidden && hidden % 16 == 0,
                "moe_prefill_dispatch: hidden %lld must be in [%lld,%lld] and a multiple of 16", (long long)hidden,
                (long long)kMinHidden, (long long)kMaxHidden);
    CHECK_PARAM(quantMode == CAMHIP_QUANT_NONE || quantMode == CAMHIP_QUANT_INT8_TOKEN ||
                    quantMode == CAMHIP_QUANT_FP8_BLOCK || quantMode == CAMHIP_QUANT_FP8_BLOCK_KMAJOR,
                "moe_prefill_dispatch: quantMode %lld not supported (0, 2, 3 or 5)", (long long)quantMode);
    const bool kmajor = quantMode == CAMHIP_QUANT_FP8_BLOCK_KMAJOR;
    const int q = kmajor ? CAMHIP_QUANT_FP8_BLOCK : (int)quantMode;
    CHECK_PARAM(q != CAMHIP_QUANT_FP8_BLOCK || hidden % 128 == 0,
                "moe_prefill_dispatch: fp8 1x128 quantisation needs hidden %% 128 == 0 (hidden %lld)",
                (long long)hidden);
    CHECK_PARAM(recvRowsCapacity >= 1 && recvRowsCapacity <= numTokens * topK,
                "moe_prefill_dispatch: recvRowsCapacity %lld out of [1, numTokens * topK]",
                (long long)recvRowsCapacity);
    CHECK_PTR(logits);
    CHECK_PTR(x);
    CHECK_PTR(topkIdx);
    CHECK_PTR(topkWeights);
    CHECK_PTR(recvX);
    CHECK_PTR(expandIdx);
    CHECK_PTR(recvCount);
    CHECK_PTR(recvTokensPerExpert);
    CHECK_PTR(combineRowMap);
    if (q != CAMHIP_QUANT_NONE)
        CHECK_PTR(recvXScales);
    const int T = (int)numTokens, H = (int)hidden, E = (int)numExperts, L = (int)localExperts, K = (int)topK;
    const int cap = (int)recvRowsCapacity;
    const int tpc = cam::route_tokens_per_block();
    const int nc = (T + tpc - 1) / tpc;
    // workspace: chunk counts -> chunk bases [L][nc], chunk prefixes over the experts [L][nc], send offsets [L],
    // the in-chunk ranks [T][K]
    const uint64_t counts_bytes = ((uint64_t)L * nc * sizeof(int32_t) + 255) & ~(uint64_t)255;
    const uint64_t vec_bytes = ((uint64_t)L * sizeof(int32_t) + 255) & ~(uint64_t)255;
    const uint64_t rank_off = 2 * counts_bytes + vec_bytes;
    const uint64_t ws = rank_off + (uint64_t)T * K * sizeof(int32_t);
    return make_executor(
        ws,
        [=](void *w, hipStream_t s) {
            int32_t *counts = (int32_t *)w;
            int32_t *pref = (int32_t *)((uint8_t *)w + counts_bytes);
            int32_t *send_off = (int32_t *)((uint8_t *)w + 2 * counts_bytes);
            int32_t *chunk_rank = (int32_t *)((uint8_t *)w + rank_off);
            hipError_t e = cam::launch_route_hist(logits, bias, T, E, K, L, topkIdx, topkWeights, counts, pref,
                                                  chunk_rank, s);
            if (e != hipSuccess)
                return e;
            e = cam::launch_scan_notify(L, nc, counts, pref, send_off, recvCount, recvTokensPerExpert, s);
            if (e != hipSuccess)
                return e;
            return cam::launch_dispatch(x, topkIdx, send_off, nullptr, T, H, K, L, 0, cap, q, recvX, recvXScales,
                                        expandIdx, s, combineRowMap, nullptr, kmajor, counts, tpc, chunk_rank, L < E);
        },
        workspaceSize, executor);
}

camhipStatus camhipMoePrefillDispatch(void *workspace, uint64_t workspaceSize, camhipExecutor *executor, void *stream)
{
    return run_executor("moe_prefill_dispatch", workspace, workspaceSize, executor, stream);
}

camhipStatus camhipMoePrefillCombineGetWorkspaceSize(const uint16_t *y, const int32_t *expandIdx,
                                                     const int32_t *combineRowMap, const int32_t *recvCount,
                                                     const float *topkWeights, int64_t numTokens, int64_t topK,
                                                     int64_t hidden, int64_t localExperts, int64_t recvRowsCapacity,
                                                     uint16_t *out, uint64_t *workspaceSize,
                                                     camhipExecutor **executor)
{
    CHECK_PARAM(numTokens >= 1 && numTokens <= kMaxTokens, "moe_prefill_combine: numTokens %lld out of [1,%lld]",
                (long long)numTokens, (long long)kMaxTokens);
    CHECK_PARAM(topK >= 1 && topK <= kMaxTopk, "moe_prefill_combine: topK %lld out of range", (long long)topK);
    CHECK_PARAM(hidden >= kMinHidden && hidden <= kMaxHidden && hidden % 16 == 0,
                "moe_prefill_combine: hidden %lld must be in [%lld,%lld] and a multiple of 16", (long long)hidden,
                (long long)kMinHidden, (long long)kMaxHidden);
    CHECK_PARAM(localExperts >= 1 && localExperts <= kMaxExperts, "moe_prefill_combine: localExperts out of range");
    CHECK_PARAM(recvRowsCapacity >= 1 && recvRowsCapacity <= numTokens * topK,
                "moe_prefill_combine: recvRowsCapacity %lld out of [1, numTokens * topK]",
                (long long)recvRowsCapacity);
    CHECK_PTR(y);
    CHECK_PTR(expandIdx);
    CHECK_PTR(combineRowMap);
    CHECK_PTR(recvCount);
    CHECK_PTR(topkWeights);
    CHECK_PTR(out);
    const int T = (int)numTokens, K = (int)topK, H = (int)hidden, N = (int)recvRowsCapacity;
    const int32_t *last = recvCount + (localExperts - 1);
    return make_executor(
        0,
        [=](void *, hipStream_t s) {
            return cam::launch_combine_gather(y, expandIdx, N, last, topkWeights, T, K, H, out, combineRowMap, s);
        },
        workspaceSize, executor);
}

camhipStatus camhipMoePrefillCombine(void *workspace, uint64_t workspaceSize, camhipExecutor *executor, void *stream)
{
    return run_executor("moe_prefill_combine", workspace, workspaceSize, executor, stream);
}

camhipStatus camhipMoeCombineNormalNoAlloc(const uint16_t *recvX, const int32_t *tokenSrcInfo, int64_t numRecvRows,
                                           const int32_t *epRecvCounts, const float *recvTopkWeights, int64_t numTokens,
                                           int64_t numTopk, int64_t hidden, int64_t epWorldSize, int64_t epRankId,
                                           int64_t moeExpertNum, uint16_t *out, int32_t *sendCostStats, void *stream)
{
    camhipStatus st = check_combine(recvX, tokenSrcInfo, numRecvRows, recvTopkWeights, numTokens, numTopk, hidden,
                                    epWorldSize, epRankId, moeExpertNum, out);
    if (st != CAMHIP_SUCCESS)
        return st;
    CHECK_PARAM(numTokens * numTopk <= CAMHIP_COMBINE_NOALLOC_MAX_SLOTS,
                "moe_combine_noalloc: numTokens * numTopk = %lld exceeds the static scratch of %lld row slots",
                (long long)(numTokens * numTopk), (long long)CAMHIP_COMBINE_NOALLOC_MAX_SLOTS);
    const int32_t *last = epRecvCounts ? epRecvCounts + (moeExpertNum - 1) : nullptr;
    hipError_t e = cam::launch_combine_noalloc(recvX, tokenSrcInfo, (int)numRecvRows, last, recvTopkWeights,
                                               (int)numTokens, (int)numTopk, (int)hidden, out, sendCostStats,
                                               (int)epRankId, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(CAMHIP_ERROR_RUNTIME, "moe_combine_noalloc: launch failed: %s", hipGetErrorString(e));
    g_last_error.clear();
    return CAMHIP_SUCCESS;
}

// ---------------------------------------------------------------- grouped GEMMs
static camhipStatus check_gmm(const char *op, const void *x, const float *xScale, const int64_t *groupList,
                              int64_t numGroups, int64_t m, int64_t k, int64_t n, const void *weight,
                              const float *weightScale, int64_t dtype, bool swiglu)
{
    CHECK_PARAM(dtype == CAMHIP_DTYPE_BF16 || dtype == CAMHIP_DTYPE_INT8 || dtype == CAMHIP_DTYPE_FP8,
                "%s: dtype %lld not supported (0, 2 or 3)", op, (long long)dtype);
    CHECK_PARAM(numGroups >= 1 && numGroups <= 512, "%s: numGroups %lld out of [1,512]", op, (long long)numGroups);
    CHECK_PARAM(m >= 1 && m <= (1 << 24), "%s: m %lld out of range", op, (long long)m);
    const int64_t esz = dtype == CAMHIP_DTYPE_BF16 ? 2 : 1;
    CHECK_PARAM(k >= 128 / esz && (k * esz) % 128 == 0, "%s: k %lld must be a multiple of %lld", op, (long long)k,
                (long long)(128 / esz));
    if (swiglu)
        CHECK_PARAM(n >= 256 && n % 256 == 0, "%s: n = 2I = %lld needs I a multiple of 128", op, (long long)n);
    else
        CHECK_PARAM(n >= 256 && n % 256 == 0, "%s: n %lld must be a multiple of 256", op, (long long)n);
    CHECK_PARAM(m * k * esz < (int64_t)1 << 32 && n * k * esz < (int64_t)1 << 32,
                "%s: x or one group's weight exceeds 4 GiB", op);
    CHECK_PTR(x);
    CHECK_PTR(groupList);
    CHECK_PTR(weight);
    if (dtype != CAMHIP_DTYPE_BF16) {
        CHECK_PTR(xScale);
        CHECK_PTR(weightScale);
    }
    return CAMHIP_SUCCESS;
}

// fp8 activation scales reach the kernels k-major ([k/128, m]: one k-step's scales of consecutive rows
// contiguous); row-major scales ([m, k/128], xScaleLayout 0) are transposed into the workspace first.
static camhipStatus gmm_executor(const char *op, cam::GmmArgs a, int dt, int epi, int64_t xScaleLayout,
                                 uint64_t *workspaceSize, camhipExecutor **executor)
{
    CHECK_PARAM(xScaleLayout == 0 || xScaleLayout == 1, "%s: xScaleLayout %lld must be 0 (row-major) or 1 (k-major)",
                op, (long long)xScaleLayout);
    if (dt != cam::DT_FP8 || xScaleLayout == 1)
        return make_executor(
            0, [=](void *, hipStream_t s) { return cam::launch_gmm(a, dt, epi, s); }, workspaceSize, executor);
    const int nb = a.K / 128;
    const uint64_t ws = (uint64_t)a.M * nb * sizeof(float);
    return make_executor(
        ws,
        [=](void *w, hipStream_t s) {
            cam::GmmArgs b = a;
            hipError_t e = cam::launch_scales_to_kmajor(a.As, a.group_list, a.L, a.M, nb, (float *)w, s);
            if (e != hipSuccess)
                return e;
            b.As = (const float *)w;
            return cam::launch_gmm(b, dt, epi, s);
        },
        workspaceSize, executor);
}

camhipStatus camhipGroupedMatmulSwigluGetWorkspaceSize(const void *x, const float *xScale, const int64_t *groupList,
                                                       int64_t numGroups, int64_t m, int64_t k, int64_t n,
                                                       const void *weight, const float *weightScale, int64_t dtype,
                                                       int64_t xScaleLayout, int64_t outQuant, void *h, float *hScale,
                                                       uint64_t *workspaceSize, camhipExecutor **executor)
{
    camhipStatus st = check_gmm("grouped_matmul_swiglu", x, xScale, groupList, numGroups, m, k, n, weight,
                                weightScale, dtype, true);
    if (st != CAMHIP_SUCCESS)
        return st;
    CHECK_PTR(h);
    if (dtype == CAMHIP_DTYPE_INT8) {
        // int32 GEMM, fp32 h and its partial row maxima (one per 32 h-columns) in the workspace, then the
        // per-token int8 requantisation
        CHECK_PARAM(outQuant == CAMHIP_QUANT_INT8_TOKEN, "grouped_matmul_swiglu: int8 inputs need outQuant 2 (got %lld)",
                    (long long)outQuant);
        CHECK_PTR(hScale);
        const uint64_t h_off = 0, amax_off = ((uint64_t)m * (n / 2) * 4 + 255) & ~(uint64_t)255;
        const uint64_t ws_bytes = amax_off + (uint64_t)m * (n / 2 / cam::GMM_AMAX_COLS) * 4;
        const int L = (int)numGroups, M = (int)m, I = (int)(n / 2);
        const cam::GmmArgs base{(const uint8_t *)x, xScale, groupList, L, M, (int)k, (int)n,
                                (const uint8_t *)weight, weightScale, nullptr, nullptr};
        return make_executor(
            ws_bytes,
            [=](void *ws, hipStream_t s) {
                cam::GmmArgs a = base;
                float *hf = (float *)((uint8_t *)ws + h_off), *amax = (float *)((uint8_t *)ws + amax_off);
                a.C = (uint8_t *)hf;
                a.Cs = amax;
                hipError_t e = cam::launch_gmm(a, cam::DT_INT8, cam::EPI_SWIGLU_F32AMAX, s);
                if (e != hipSuccess)
                    return e;
                return cam::launch_quant_rows_int8(hf, amax, groupList, L, M, I, (int8_t *)h, hScale, s);
            },
            workspaceSize, executor);
    }
    CHECK_PARAM(outQuant == CAMHIP_QUANT_NONE || outQuant == CAMHIP_QUANT_FP8_BLOCK,
                "grouped_matmul_swiglu: outQuant %lld not supported (0 or 3)", (long long)outQuant);
    if (outQuant == CAMHIP_QUANT_FP8_BLOCK)
        CHECK_PTR(hScale);
    cam::GmmArgs a{(const uint8_t *)x, xScale, groupList, (int)numGroups, (int)m, (int)k, (int)n,
                   (const uint8_t *)weight, weightScale, (uint8_t *)h, hScale};
    const int dt = (int)dtype;
    const int epi = outQuant == CAMHIP_QUANT_FP8_BLOCK ? cam::EPI_SWIGLU_FP8 : cam::EPI_SWIGLU_BF16;
    if (dt == cam::DT_BF16 && epi == cam::EPI_SWIGLU_FP8)
        return fail(CAMHIP_ERROR_INVALID_PARAM, "grouped_matmul_swiglu: fp8 h needs fp8 inputs");
    return gmm_executor("grouped_matmul_swiglu", a, dt, epi, xScaleLayout, workspaceSize, executor);
}

camhipStatus camhipGroupedMatmulSwiglu(void *workspace, uint64_t workspaceSize, camhipExecutor *executor, void *stream)
{
    return run_executor("grouped_matmul_swiglu", workspace, workspaceSize, executor, stream);
}

camhipStatus camhipGroupedMatmulGetWorkspaceSize(const void *x, const float *xScale, const int64_t *groupList,
                                                 int64_t numGroups, int64_t m, int64_t k, int64_t n,
                                                 const void *weight, const float *weightScale, int64_t dtype,
                                                 int64_t xScaleLayout, uint16_t *out, uint64_t *workspaceSize,
                                                 camhipExecutor **executor)
{
    camhipStatus st = check_gmm("grouped_matmul", x, xScale, groupList, numGroups, m, k, n, weight, weightScale,
                                dtype, false);
    if (st != CAMHIP_SUCCESS)
        return st;
    CHECK_PTR(out);
    cam::GmmArgs a{(const uint8_t *)x, xScale, groupList, (int)numGroups, (int)m, (int)k, (int)n,
                   (const uint8_t *)weight, weightScale, (uint8_t *)out, nullptr};
    return gmm_executor("grouped_matmul", a, (int)dtype, cam::EPI_PLAIN, xScaleLayout, workspaceSize, executor);
}

camhipStatus camhipGroupedMatmul(void *workspace, uint64_t workspaceSize, camhipExecutor *executor, void *stream)
{
    return run_executor("grouped_matmul", workspace, workspaceSize, executor, stream);
}

// ---------------------------------------------------------------- experts: GMM1 + SwiGLU -> GMM2
camhipStatus camhipMoeExpertsGetWorkspaceSize(const void *x, const float *xScale, const int64_t *groupList,
                                              int64_t numGroups, int64_t m, int64_t hidden, int64_t gmm1HiddenSize,
                                              const void *gmm1Weight, const float *gmm1WeightScale,
                                              const void *gmm2Weight, const float *gmm2WeightScale, int64_t dtype,
                                              int64_t xScaleLayout, void *h, float *hScale, uint16_t *out,
                                              uint64_t *workspaceSize, camhipExecutor **executor)
{
    CHECK_PARAM(dtype == CAMHIP_DTYPE_BF16 || dtype == CAMHIP_DTYPE_FP8,
                "moe_experts: dtype %lld not supported (0 bf16 or 3 fp8; int8 runs the two grouped-matmul calls)",
                (long long)dtype);
    camhipStatus st = check_gmm("moe_experts", x, xScale, groupList, numGroups, m, hidden, gmm1HiddenSize,
                                gmm1Weight, gmm1WeightScale, dtype, true);
    if (st != CAMHIP_SUCCESS)
        return st;
    st = check_gmm("moe_experts", h, dtype == CAMHIP_DTYPE_FP8 ? hScale : nullptr, groupList, numGroups, m,
                   gmm1HiddenSize / 2, hidden, gmm2Weight, gmm2WeightScale, dtype, false);
    if (dtype == CAMHIP_DTYPE_BF16 && st == CAMHIP_SUCCESS)
        CHECK_PTR(h);
    if (st != CAMHIP_SUCCESS)
        return st;
    CHECK_PTR(out);
    CHECK_PARAM(xScaleLayout == 0 || xScaleLayout == 1, "moe_experts: xScaleLayout %lld must be 0 or 1",
                (long long)xScaleLayout);
    const int L = (int)numGroups, M = (int)m, H = (int)hidden, N1 = (int)gmm1HiddenSize, dt = (int)dtype;
    const int epi1 = dt == cam::DT_FP8 ? cam::EPI_SWIGLU_FP8 : cam::EPI_SWIGLU_BF16;
    const cam::GmmArgs g1{(const uint8_t *)x, xScale, groupList, L, M, H, N1, (const uint8_t *)gmm1Weight,
                          gmm1WeightScale, (uint8_t *)h, hScale};
    const cam::GmmArgs g2{(const uint8_t *)h, dt == cam::DT_FP8 ? hScale : nullptr, groupList, L, M, N1 / 2, H,
                          (const uint8_t *)gmm2Weight, gmm2WeightScale, (uint8_t *)out, nullptr};
    const bool chained = cam::gmm_chain_supported(g1, g2, dt);
    // workspace: the readiness counters (chained), then the k-major copy of row-major fp8 scales
    const uint64_t ready_bytes = chained ? ((uint64_t)cam::gmm_chain_counters(M, L) * 4 + 255) & ~(uint64_t)255 : 0;
    const bool transpose = dt == cam::DT_FP8 && xScaleLayout == 0;
    const int nb = H / 128;
    const uint64_t ws = ready_bytes + (transpose ? (uint64_t)M * nb * 4 : 0);
    return make_executor(
        ws,
        [=](void *w, hipStream_t s) {
            cam::GmmArgs a = g1;
            hipError_t e = hipSuccess;
            if (transpose) {
                float *ks = (float *)((uint8_t *)w + ready_bytes);
                e = cam::launch_scales_to_kmajor(g1.As, groupList, L, M, nb, ks, s);
                if (e != hipSuccess)
                    return e;
                a.As = ks;
            }
            if (!chained) {
                e = cam::launch_gmm(a, dt, epi1, s);
                return e != hipSuccess ? e : cam::launch_gmm(g2, dt, cam::EPI_PLAIN, s);
            }
            int32_t *ready = (int32_t *)w;
            e = cam::launch_fill_i32(ready, 0, cam::gmm_chain_counters(M, L), s);
            return e != hipSuccess ? e : cam::launch_gmm_chain(a, g2, dt, ready, s);
        },
        workspaceSize, executor);
}

camhipStatus camhipMoeExperts(void *workspace, uint64_t workspaceSize, camhipExecutor *executor, void *stream)
{
    return run_executor("moe_experts", workspace, workspaceSize, executor, stream);
}

camhipStatus camhipGetSyncStatus(int32_t *status, int32_t clear)
{
    CHECK_PTR(status);
    int v = 0;
    hipError_t e = cam::sync_status_read(&v, clear != 0);
    if (e != hipSuccess)
        return fail(CAMHIP_ERROR_RUNTIME, "get_sync_status: %s", hipGetErrorString(e));
    *status = v;
    g_last_error.clear();
    return CAMHIP_SUCCESS;
}

void camhipDebugSetSyncWait(int64_t waitTicks, int32_t unreachable)
{
    cam::sync_debug_set(waitTicks, unreachable);
}

}  // extern "C"
