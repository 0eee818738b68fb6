/*
 * camhip.h -- C ABI of the MI355X (gfx950) CAM MoE hot path.
 *
 * Drop-in for the aclnn two-phase interface of UMDK CAM
 * (src/cam/comm_operator/ascend_kernels/<op>/op_api/aclnn_<op>.h):
 *
 *   status = camhipXxxGetWorkspaceSize(inputs..., attrs..., outputs...,
 *                                      &workspaceSize, &executor);
 *   status = camhipXxx(workspace, workspaceSize, executor, stream);
 *
 * Tensors are plain device pointers with explicit sizes; the caller owns
 * every input, output and workspace buffer.  The executor is owned by the
 * library and freed by the second call, whether it launches or fails.
 * Launches are asynchronous and ordered on `stream` (a hipStream_t, NULL for
 * the default stream).  No call synchronises with the host or allocates
 * device memory.  Calls that share a workspace must not overlap.
 *
 * Every function returns CAMHIP_SUCCESS (0) or an error code; the message of
 * the last error on the calling thread is camhipGetLastErrorMsg().
 *
 * Layouts: bf16 tensors are uint16 bit patterns, fp8 tensors are OCP e4m3fn
 * byte codes, all row-major and contiguous unless stated.
 *
 * This build runs one EP rank on one GPU: epWorldSize/rankSize must be 1 for
 * the dispatch, notify and combine calls (the reference requires 2..384 ranks,
 * moe_dispatch_prefill.cpp:63, and exchanges rows between ranks).
 */
#ifndef CAMHIP_H
#define CAMHIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CAMHIP_API __attribute__((visibility("default")))

typedef int camhipStatus;
#define CAMHIP_SUCCESS 0
#define CAMHIP_ERROR_INVALID_PARAM 161001 /* same code aclnn uses for ACLNN_ERR_PARAM_INVALID */
#define CAMHIP_ERROR_NULLPTR 161002
#define CAMHIP_ERROR_RUNTIME 361001       /* a HIP launch failed */
#define CAMHIP_ERROR_WORKSPACE 161003     /* workspace smaller than requested */

typedef struct camhipExecutor camhipExecutor;

/* Quantisation of dispatched rows (quantMode attribute of aclnnMoeDispatchNormal). */
#define CAMHIP_QUANT_NONE 0        /* bf16 rows, scales untouched */
#define CAMHIP_QUANT_INT8_TOKEN 2  /* int8, one fp32 scale per row (reference use_quant=True) */
#define CAMHIP_QUANT_FP8_BLOCK 3   /* fp8 e4m3fn, one fp32 scale per 1x128 block (extension) */
/* the same fp8 rows with the block scales written k-major, [hidden/128, recvRowsCapacity]: the layout the
 * grouped GEMMs read (xScaleLayout 1), so no transpose runs between dispatch and GMM1 (extension) */
#define CAMHIP_QUANT_FP8_BLOCK_KMAJOR 5

CAMHIP_API const char *camhipGetLastErrorMsg(void);
CAMHIP_API const char *camhipGetVersion(void);
/* Frees an executor that will not be launched (aclnn has no counterpart: its
 * executors are consumed by the launch call, as camhip's are). */
CAMHIP_API void camhipReleaseExecutor(camhipExecutor *executor);

/* ------------------------------------------------------------------ routing
 * No reference counterpart (CAM callers compute topk_idx themselves,
 * src/cam/examples/moe_dispatch_combine_prefill_sample.py:87-93).
 * logits [numTokens, numExperts] fp32, bias [numExperts] fp32 or NULL.
 * topkIdx[t,k]: the k-th largest logit+bias (ties -> lower expert id).
 * topkWeights[t,k] = softmax(logits[t])[topkIdx[t,k]] renormalised over the K picks.
 * topkIdxInt64 (optional, may be NULL): the same ids as int64, the input type of
 * camhipDispatchLayout (aclnnDispatchLayout takes int64 topk_idx).
 * Limits: 1 <= topK <= 16, topK <= numExperts <= 512. */
CAMHIP_API camhipStatus camhipMoeRouteGetWorkspaceSize(const float *logits, const float *bias, int64_t numTokens,
                                                       int64_t numExperts, int64_t topK, int32_t *topkIdx,
                                                       float *topkWeights, int64_t *topkIdxInt64,
                                                       uint64_t *workspaceSize, camhipExecutor **executor);
CAMHIP_API camhipStatus camhipMoeRoute(void *workspace, uint64_t workspaceSize, camhipExecutor *executor,
                                       void *stream);

/* ------------------------------------------------------------------ layout
 * Replaces aclnnDispatchLayoutGetWorkspaceSize / aclnnDispatchLayout
 * (dispatch_layout/op_api/aclnn_dispatch_layout.h:33-46; kernel
 * dispatch_layout.h:83-166).  topkIdx [numTokens, numTopk] int64.
 * Outputs: numTokensPerRank [numRanks] (may be NULL), numTokensPerExpert
 * [numExperts], isTokenInRank [numTokens, numRanks] (may be NULL),
 * sendTokenIdxSmall [numTokens, numTopk] = stable rank of (t,k) within its
 * expert.  The reference's notifySendData scratch lives in the workspace.
 * Expert ids outside [0,numExperts) are not routed (sendTokenIdx = -1).
 * Limits (dispatch_layout_tiling.cpp:55-65,98-122): numRanks in [1,384],
 * numExperts in [1,512] and divisible by numRanks, numTopk in [1,16],
 * numTokens in [0,65536] (the reference stops at 8000). */
CAMHIP_API camhipStatus camhipDispatchLayoutGetWorkspaceSize(const int64_t *topkIdx, int64_t numTokens,
                                                             int64_t numRanks, int64_t numExperts, int64_t numTopk,
                                                             int32_t *numTokensPerRank, int32_t *numTokensPerExpert,
                                                             int32_t *isTokenInRank, int32_t *sendTokenIdxSmall,
                                                             uint64_t *workspaceSize, camhipExecutor **executor);
CAMHIP_API camhipStatus camhipDispatchLayout(void *workspace, uint64_t workspaceSize, camhipExecutor *executor,
                                             void *stream);

/* ------------------------------------------------------------------ notify
 * Replaces aclnnNotifyDispatch (notify_dispatch/op_api/aclnn_notify_dispatch.h:19-27;
 * kernel notify_dispatch.h:129-160, 306-412) for a single rank.
 * tokenPerExpertData [numExperts] int32 -> sendDataOffset [numExperts]
 * (exclusive prefix), totalRecvTokens [1], recvCount [numExperts] (inclusive
 * prefix, expert-major), recvOffset [numExperts], maxBs [1] = numTokens,
 * recvTokensPerExpert [numExperts/rankSize] int64.  Optional outputs may be
 * NULL except sendDataOffset. */
CAMHIP_API camhipStatus camhipNotifyDispatchGetWorkspaceSize(const int32_t *tokenPerExpertData, int64_t numExperts,
                                                             int64_t numTokens, int64_t rankSize, int64_t rankId,
                                                             int32_t *sendDataOffset, int32_t *totalRecvTokens,
                                                             int32_t *recvCount, int32_t *recvOffset, int32_t *maxBs,
                                                             int64_t *recvTokensPerExpert, uint64_t *workspaceSize,
                                                             camhipExecutor **executor);
CAMHIP_API camhipStatus camhipNotifyDispatch(void *workspace, uint64_t workspaceSize, camhipExecutor *executor,
                                             void *stream);

/* ------------------------------------------------------------------ dispatch
 * Replaces aclnnMoeDispatchNormal (moe_dispatch_normal/op_api/aclnn_moe_dispatch_normal.h:19-27;
 * kernel moe_dispatch_normal.h:295-410, 545-591).
 * x [numTokens, hidden] bf16, topkIdx/sendTokenIdx [numTokens, numTopk] int32,
 * sendOffset [moeExpertNum].  recvOffset/recvCount are accepted for signature
 * parity and unused with one rank (may be NULL).
 * Output row of (t,k) = sendOffset[e] + sendTokenIdx[t,k]; rows must fit in
 * recvRowsCapacity.  recvX [rows, hidden]: bf16 (quantMode 0), int8 (2) or
 * fp8 e4m3fn (3, 5).  recvXScales: untouched (0), [rows] (2), [rows, hidden/128] (3),
 * [hidden/128, recvRowsCapacity] (5: element (row, b) at b * recvRowsCapacity + row).
 * assistInfoForCombine [rows, 3] int32 = (epRankId, t, k).
 * waitRecvCostStats (diagnose output, may be NULL): [epWorldSize] int32, per
 * source rank the microseconds the dispatch spent on that rank's rows,
 * accumulated across calls (moe_dispatch_normal.h:489-529); with one rank,
 * entry 0 gains the dispatch phase's time on the stream.
 * Limits (moe_dispatch_normal_tiling.cpp:72-94): hidden in [1024,7168] and a
 * multiple of 16 (of 128 for quantMode 3 and 5), numTopk in [1,16], moeExpertNum
 * in [1,512], epWorldSize == 1. */
CAMHIP_API camhipStatus camhipMoeDispatchNormalGetWorkspaceSize(
    const uint16_t *x, const int32_t *topkIdx, const int32_t *sendOffset, const int32_t *sendTokenIdx,
    const int32_t *recvOffset, const int32_t *recvCount, int64_t numTokens, int64_t hidden, int64_t numTopk,
    int64_t epWorldSize, int64_t epRankId, int64_t moeExpertNum, int64_t quantMode, int64_t recvRowsCapacity,
    void *recvX, float *recvXScales, int32_t *assistInfoForCombine, int32_t *waitRecvCostStats,
    uint64_t *workspaceSize, camhipExecutor **executor);
CAMHIP_API camhipStatus camhipMoeDispatchNormal(void *workspace, uint64_t workspaceSize, camhipExecutor *executor,
                                                void *stream);

/* ------------------------------------------------------------------ combine
 * Replaces aclnnMoeCombineNormal (moe_combine_normal/op_api/aclnn_moe_combine_normal.h:19-27;
 * kernel moe_combine_normal.h:223-412).
 * recvX [numRecvRows, hidden] bf16 expert outputs in dispatch order,
 * tokenSrcInfo [numRecvRows, 3] = (rank, t, k) from dispatch, epRecvCounts
 * [moeExpertNum] (its last entry bounds the rows used; may be NULL),
 * recvTopkWeights [numTokens, numTopk] fp32 -> out [numTokens, hidden] bf16:
 * out[t] = bf16_rne(sum_k float(row(t,k)) * w[t,k]), fp32, k ascending, no FMA.
 * (t,k) slots that received no row contribute nothing.
 * sendCostStats (diagnose output, may be NULL): [epWorldSize] int32, microseconds
 * per destination rank, accumulated (moe_combine_normal.h:197); entry 0 gains
 * the combine phase's time on the stream.
 * Limits: hidden in [1024,7168] and a multiple of 16, numTopk in [1,16],
 * epWorldSize == 1. */
CAMHIP_API camhipStatus camhipMoeCombineNormalGetWorkspaceSize(
    const uint16_t *recvX, const int32_t *tokenSrcInfo, int64_t numRecvRows, const int32_t *epRecvCounts,
    const float *recvTopkWeights, int64_t numTokens, int64_t numTopk, int64_t hidden, int64_t epWorldSize,
    int64_t epRankId, int64_t moeExpertNum, uint16_t *out, int32_t *sendCostStats, uint64_t *workspaceSize,
    camhipExecutor **executor);
CAMHIP_API camhipStatus camhipMoeCombineNormal(void *workspace, uint64_t workspaceSize, camhipExecutor *executor,
                                               void *stream);

/* ------------------------------------------------------------------ prefill step (extension)
 * No reference counterpart: the route -> layout -> count exchange -> dispatch -> combine chain of one EP rank
 * in four launches instead of eight, for runners that own the whole step (umdk_amd.plan).  The results are
 * those of the reference-shaped calls above, bit for bit:
 *   camhipMoePrefillDispatch: camhipMoeRoute over numExperts experts, then, over the localExperts experts
 *   0..localExperts-1 (other ids are not routed on this rank), the layout, count exchange and
 *   camhipMoeDispatchNormal.  The per-expert rank of each (t,k) is not materialised (send_token_idx): the
 *   routing writes per-chunk expert histograms, a scan turns them into chunk bases and runs the count
 *   exchange, and the dispatch ranks each entry inside its chunk (three launches).  Outputs: topkIdx/topkWeights [numTokens, topK],
 *   recvX and recvXScales as the dispatch call's quantMode (0, 2, 3, 5), expandIdx [rows, 3], recvCount
 *   [localExperts] (inclusive prefix), recvTokensPerExpert [localExperts] int64, and combineRowMap
 *   [numTokens, topK] = the row of (t,k), or -1, which replaces the combine's own scatter pass.
 *   camhipMoePrefillCombine: camhipMoeCombineNormal on those outputs (y [rows, hidden] bf16 expert outputs in
 *   dispatch order), reading combineRowMap instead of building it.  Its localExperts and recvRowsCapacity must
 *   be the values of the camhipMoePrefillDispatch call that produced the outputs (recvCount[localExperts - 1]
 *   is the row total; y and expandIdx hold recvRowsCapacity rows): the call cannot check buffer sizes.
 * Limits: numTokens in [1,65536], topK <= 16, localExperts <= numExperts <= 512, recvRowsCapacity in
 * [1, numTokens * topK]. */
CAMHIP_API camhipStatus camhipMoePrefillDispatchGetWorkspaceSize(
    const float *logits, const float *bias, const uint16_t *x, int64_t numTokens, int64_t hidden, int64_t numExperts,
    int64_t localExperts, int64_t topK, int64_t quantMode, int64_t recvRowsCapacity, int32_t *topkIdx,
    float *topkWeights, void *recvX, float *recvXScales, int32_t *expandIdx, int32_t *recvCount,
    int64_t *recvTokensPerExpert, int32_t *combineRowMap, uint64_t *workspaceSize, camhipExecutor **executor);
CAMHIP_API camhipStatus camhipMoePrefillDispatch(void *workspace, uint64_t workspaceSize, camhipExecutor *executor,
                                                 void *stream);
CAMHIP_API camhipStatus camhipMoePrefillCombineGetWorkspaceSize(
    const uint16_t *y, const int32_t *expandIdx, const int32_t *combineRowMap, const int32_t *recvCount,
    const float *topkWeights, int64_t numTokens, int64_t topK, int64_t hidden, int64_t localExperts,
    int64_t recvRowsCapacity, uint16_t *out, uint64_t *workspaceSize, camhipExecutor **executor);
CAMHIP_API camhipStatus camhipMoePrefillCombine(void *workspace, uint64_t workspaceSize, camhipExecutor *executor,
                                                void *stream);

/* Allocation-free combine.  No reference counterpart: for callers that cannot allocate or pass a
 * workspace (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The same arguments and results as camhipMoeCombineNormalGetWorkspaceSize + camhipMoeCombineNormal in
 * one call; the row map lives in a static per-device scratch array of the library (1 MiB + 256 B per
 * GPU, held until the process ends), so numTokens * numTopk must not exceed
 * CAMHIP_COMBINE_NOALLOC_MAX_SLOTS (CAMHIP_ERROR_INVALID_PARAM otherwise).  Every call on a GPU shares
 * that scratch: calls that overlap on one GPU (other streams, other threads) race and must be
 * serialised by the caller.  No hipMalloc, hipFree or allocating library call is made.  The scratch's
 * device address is looked up once per device and kept for the process: after hipDeviceReset (or anything
 * else that unloads the library's code objects) the entry point must not be called again in that process. */
#define CAMHIP_COMBINE_NOALLOC_MAX_SLOTS (1L << 18)
CAMHIP_API camhipStatus camhipMoeCombineNormalNoAlloc(const uint16_t *recvX, const int32_t *tokenSrcInfo,
                                                      int64_t numRecvRows, const int32_t *epRecvCounts,
                                                      const float *recvTopkWeights, int64_t numTokens,
                                                      int64_t numTopk, int64_t hidden, int64_t epWorldSize,
                                                      int64_t epRankId, int64_t moeExpertNum, uint16_t *out,
                                                      int32_t *sendCostStats, void *stream);

/* ------------------------------------------------------------------ grouped expert GEMMs
 * The GMM1 / SwiGLU / GMM2 stages of fused_deep_moe as standalone calls
 * (fused_deep_moe.h:56-238; kernels
 * grouped_matmul_slice_m_per_token_dequant_swiglu_quant_multistage_workspace.h:299-455 and
 * grouped_matmul_slice_m_per_token_dequant_multistage_workspace.h:141-292).  The
 * reference computes them in int8 with per-channel weight and per-token
 * activation scales; these take that int8 mode, bf16, or fp8 e4m3fn with
 * DeepSeek-style block scales.
 * x [m, k]: rows in dispatch order; expert g owns groupList[g] consecutive
 * rows starting at the sum of the earlier counts (groupList is int64 on the
 * device, as recvTokensPerExpert / expert_token_nums).  Rows past the sum are
 * neither read for output nor written.
 * weight [numGroups, n, k] with k contiguous (the transpose of the reference's
 * logical [L, k, n] layout).  dtype: CAMHIP_DTYPE_BF16, CAMHIP_DTYPE_INT8 or
 * CAMHIP_DTYPE_FP8; for fp8, xScale [m, k/128] and weightScale
 * [numGroups, n/128, k/128] fp32 (dequantised value = code * scale),
 * accumulation fp32.  xScaleLayout (fp8 only; 0 for bf16 and int8) says how
 * xScale is stored: 0 row-major [m, k/128] (as the dispatch writes it; the op
 * then transposes it into its workspace, m*(k/128)*4 bytes), 1 k-major
 * [k/128, m] (element (row, b) at b*m + row; read directly, no workspace); for int8, xScale [m] per token and weightScale
 * [numGroups, n] per output channel, exact int32 accumulation and
 * value = ((float)acc * weightScale[n]) * xScale[m]
 * (block_epilogue_per_token_dequant.hpp:338-361). */
#define CAMHIP_DTYPE_BF16 0
#define CAMHIP_DTYPE_INT8 2
#define CAMHIP_DTYPE_FP8 3
/* OR'ed into camhipFusedDeepMoe's weightDtype: separated weights, the reference's per-expert
 * tensor lists (pybind/fused_deep_moe.cpp:33-36, TensorList gmm1Weight ...; dynamic EPLB,
 * test_fused_deep_moe.py:256-269).  gmm1Weight, gmm1WeightScale, gmm2Weight and
 * gmm2WeightScale then each point to a device array of L device pointers, entry e being
 * expert e's [n, k] weight (k contiguous) or its scales ([n/128, k/128] fp8, [n] int8). */
#define CAMHIP_WEIGHT_LIST 0x100

/* GMM1 + SwiGLU: n = 2I, weight rows [0,I) gate, [I,2I) up;
 * h[m, I] = silu(x W_gate^T) * (x W_up^T), silu(g) = g / (1 + exp(-g))
 * (block_epilogue_per_token_dequant_swiglu.h:256-286).
 * outQuant CAMHIP_QUANT_NONE: h bf16; CAMHIP_QUANT_FP8_BLOCK: h fp8 e4m3fn with
 * hScale stored k-major [I/128, m] (ready for GMM2 with xScaleLayout 1),
 * quantised per 1x128 block like the dispatch quantiser.
 * int8 inputs require outQuant CAMHIP_QUANT_INT8_TOKEN: h int8 [m, I] with
 * hScale [m], requantised per token over the whole row,
 * q = rint((h * 127) * (1/amax)), scale = amax * (1/127)
 * (post_swiglu_dynamic_quant.h:164-231); this mode needs a workspace of
 * m*I*4 + m*(I/32)*4 bytes (fp32 h and its partial row maxima); fp8 with row-major xScale
 * needs the transposed scales' workspace; the others none.
 * Limits: 1 <= numGroups <= 512, k a multiple of 64 (bf16) / 128 (fp8, int8),
 * I a multiple of 128, m*k and n*k bytes below 4 GiB. */
CAMHIP_API camhipStatus camhipGroupedMatmulSwigluGetWorkspaceSize(
    const void *x, const float *xScale, const int64_t *groupList, int64_t numGroups, int64_t m, int64_t k, int64_t n,
    const void *weight, const float *weightScale, int64_t dtype, int64_t xScaleLayout, int64_t outQuant, void *h,
    float *hScale, uint64_t *workspaceSize, camhipExecutor **executor);
CAMHIP_API camhipStatus camhipGroupedMatmulSwiglu(void *workspace, uint64_t workspaceSize, camhipExecutor *executor,
                                                  void *stream);

/* GMM2: out[m, n] = bf16(x W^T) per group (block_epilogue_per_token_dequant.hpp:338-361).
 * Limits as above, with n a multiple of 256. */
CAMHIP_API camhipStatus camhipGroupedMatmulGetWorkspaceSize(const void *x, const float *xScale,
                                                            const int64_t *groupList, int64_t numGroups, int64_t m,
                                                            int64_t k, int64_t n, const void *weight,
                                                            const float *weightScale, int64_t dtype,
                                                            int64_t xScaleLayout, uint16_t *out,
                                                            uint64_t *workspaceSize, camhipExecutor **executor);
CAMHIP_API camhipStatus camhipGroupedMatmul(void *workspace, uint64_t workspaceSize, camhipExecutor *executor,
                                            void *stream);

/* Both expert GEMMs of a layer in one call (extension, no reference counterpart; the reference runs them
 * as two workspace-linked stages inside its fused op, grouped_matmul_slice_m_per_token_dequant_swiglu_quant_
 * multistage_workspace.h:386-401 waiting per group on the first stage's flags): GMM1 + SwiGLU exactly as
 * camhipGroupedMatmulSwiglu with n = gmm1HiddenSize (fp8: h requantised to fp8 1x128, hScale k-major
 * [I/128, m]; bf16: h bf16), then GMM2 exactly as camhipGroupedMatmul on h -> out [m, hidden] bf16.  The
 * results are bit-identical to those two calls.  Where a chained kernel exists (decode-sized groups, at most
 * 48 rows per group on average) the two run as one launch in which each GMM2 tile waits for the GMM1 tiles
 * of its rows; the workspace then holds the readiness counters, cleared by this call.  dtype 0 (bf16) or
 * 3 (fp8); int8 is not accepted (use the two calls).  If a wait in the chained launch outlasts its bound
 * (2 s, which only a GPU shared with other work that keeps blocks of the launch from running could cause),
 * the launch ends with unspecified outputs and sets the device's sync status (camhipGetSyncStatus). */
CAMHIP_API camhipStatus camhipMoeExpertsGetWorkspaceSize(const void *x, const float *xScale,
                                                         const int64_t *groupList, int64_t numGroups, int64_t m,
                                                         int64_t hidden, int64_t gmm1HiddenSize,
                                                         const void *gmm1Weight, const float *gmm1WeightScale,
                                                         const void *gmm2Weight, const float *gmm2WeightScale,
                                                         int64_t dtype, int64_t xScaleLayout, void *h, float *hScale,
                                                         uint16_t *out, uint64_t *workspaceSize,
                                                         camhipExecutor **executor);
CAMHIP_API camhipStatus camhipMoeExperts(void *workspace, uint64_t workspaceSize, camhipExecutor *executor,
                                         void *stream);

/* Sync status of the current device's chained GEMM launches (camhipMoeExperts, camhipFusedDeepMoe), an
 * extension with no reference counterpart: *status = 0, or nonzero once a readiness wait gave up (sticky;
 * clear != 0 resets it).  A wait only gives up when blocks of its launch cannot run (a GPU shared with other
 * work that holds the compute units); the launch's outputs are then unspecified.  Synchronous: call it after
 * the launches have completed. */
CAMHIP_API camhipStatus camhipGetSyncStatus(int32_t *status, int32_t clear);
/* Test hook (extension): waitTicks > 0 sets the chained launches' wait bound in 100 MHz constant-clock
 * ticks (<= 0 restores 2 s); unreachable != 0 makes every wait unreachable, so that each one gives up at
 * the bound.  Applies to launches issued after the call, from any thread. */
CAMHIP_API void camhipDebugSetSyncWait(int64_t waitTicks, int32_t unreachable);

/* ------------------------------------------------------------------ fused decode entry
 * Replaces aclnnFusedDeepMoe (fused_deep_moe/op_api/aclnn_fused_deep_moe.h:19-50;
 * binding pybind/fused_deep_moe.cpp:30-83): dispatch + GMM1 + SwiGLU + GMM2 +
 * combine (+ optional shared expert) in one stream-ordered call with fixed-size
 * outputs and no host synchronisation, so it can be captured in a HIP graph.
 * x [batchSize, hidden] bf16; expertIds [batchSize, topK] int32 in
 * [-1, moeExpertNum) (-1: placeholder, not routed); expertScales [batchSize, topK]
 * fp32 combine weights; xActiveMask [batchSize] bool (1 byte, true prefix) or NULL.
 * Weights in coupled mode (or separated: CAMHIP_WEIGHT_LIST) with the reduction dimension contiguous:
 * gmm1Weight [L, gmm1HiddenSize, hidden] (rows [0,I) gate, [I,2I) up),
 * gmm2Weight [L, hidden, gmm1HiddenSize/2]; weightDtype CAMHIP_DTYPE_BF16,
 * CAMHIP_DTYPE_FP8 with block scales [L, n/128, k/128] (activations are then
 * quantised to fp8 1x128 on the fly), or CAMHIP_DTYPE_INT8, the reference's
 * own mode: per-channel scales gmm1WeightScale [L, gmm1HiddenSize] and
 * gmm2WeightScale [L, hidden], x quantised per token (s = 127/amax after the
 * optional smooth scales expertSmoothScales [moeExpertNum, hidden] of the
 * destination expert), h requantised per token between the GEMMs.  Smooth
 * scales are accepted in int8 mode only (NULL otherwise).
 * Shared expert (optional, all four given together): shareGmm1Weight
 * [shareGmm1HiddenSize, hidden], shareGmm2Weight [hidden, shareGmm1HiddenSize/2]
 * (+ scales [n/128, k/128] for fp8, [n] for int8; int8 also takes
 * shareSmoothScales [hidden]) -> shareOutput [batchSize, hidden] bf16.
 * Outputs: output [batchSize, hidden] bf16; expertTokenNums [L] int64 (rows per
 * local expert).  L = moeExpertNum / epRankSize; epRankSize must be 1 here.
 * quantMode is reserved (0), as in the reference.  Limits
 * (fused_deep_moe_tiling.cpp:59-75, widened where the GPU allows): batchSize
 * <= 4096, topK <= 12, hidden in [512,7168] and % 256 == 0 (the reference fused tiling's smallest token length is 512), gmm1HiddenSize % 256 == 0. */
CAMHIP_API camhipStatus camhipFusedDeepMoeGetWorkspaceSize(
    const uint16_t *x, const int32_t *expertIds, const void *gmm1Weight, const float *gmm1WeightScale,
    const void *gmm2Weight, const float *gmm2WeightScale, const float *expertScales, const void *shareGmm1Weight,
    const float *shareGmm1WeightScale, const void *shareGmm2Weight, const float *shareGmm2WeightScale,
    const float *expertSmoothScales, const float *shareSmoothScales, const uint8_t *xActiveMask, int64_t batchSize,
    int64_t hidden, int64_t topK, int64_t gmm1HiddenSize, int64_t shareGmm1HiddenSize, int64_t weightDtype,
    int64_t epRankSize, int64_t epRankId, int64_t moeExpertNum, int64_t quantMode, int64_t globalBs,
    uint16_t *output, uint16_t *shareOutput, int64_t *expertTokenNums, uint64_t *workspaceSize,
    camhipExecutor **executor);
CAMHIP_API camhipStatus camhipFusedDeepMoe(void *workspace, uint64_t workspaceSize, camhipExecutor *executor,
                                           void *stream);

#ifdef __cplusplus
}
#endif
#endif /* CAMHIP_H */
