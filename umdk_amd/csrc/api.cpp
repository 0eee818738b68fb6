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
#include "launchers.h"

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
                                            uint64_t *workspaceSize, camhipExecutor **executor)
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
        0, [=](void *, hipStream_t s) { return cam::launch_route(logits, bias, T, E, K, topkIdx, topkWeights, s); },
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
                                                     uint64_t *workspaceSize, camhipExecutor **executor)
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
                    quantMode == CAMHIP_QUANT_FP8_BLOCK,
                "moe_dispatch: quantMode %lld not supported (0, 2 or 3)", (long long)quantMode);
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
    return make_executor(
        0,
        [=](void *, hipStream_t s) {
            return cam::launch_dispatch(x, topkIdx, sendOffset, sendTokenIdx, T, H, K, E, rank, cap, q, recvX, recvXScales,
                                        assistInfoForCombine, s);
        },
        workspaceSize, executor);
}

camhipStatus camhipMoeDispatchNormal(void *workspace, uint64_t workspaceSize, camhipExecutor *executor, void *stream)
{
    return run_executor("moe_dispatch", workspace, workspaceSize, executor, stream);
}

// ---------------------------------------------------------------- combine
camhipStatus camhipMoeCombineNormalGetWorkspaceSize(const uint16_t *recvX, const int32_t *tokenSrcInfo,
                                                    int64_t numRecvRows, const int32_t *epRecvCounts,
                                                    const float *recvTopkWeights, int64_t numTokens, int64_t numTopk,
                                                    int64_t hidden, int64_t epWorldSize, int64_t epRankId,
                                                    int64_t moeExpertNum, uint16_t *out, uint64_t *workspaceSize,
                                                    camhipExecutor **executor)
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
    const int N = (int)numRecvRows, T = (int)numTokens, K = (int)numTopk, H = (int)hidden;
    const int32_t *last = epRecvCounts ? epRecvCounts + (moeExpertNum - 1) : nullptr;
    const uint64_t ws = sizeof(int32_t) * (uint64_t)T * K;
    return make_executor(
        ws,
        [=](void *w, hipStream_t s) {
            return cam::launch_combine(recvX, tokenSrcInfo, N, last, recvTopkWeights, T, K, H, out, (int32_t *)w, s);
        },
        workspaceSize, executor);
}

camhipStatus camhipMoeCombineNormal(void *workspace, uint64_t workspaceSize, camhipExecutor *executor, void *stream)
{
    return run_executor("moe_combine", workspace, workspaceSize, executor, stream);
}

}  // extern "C"
