/*
 * cam_oracle.c -- CPU restatement of the CAM MoE hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP path is compared
 * against; it is imported only by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py.  The product library (umdk_amd/) never links,
 * loads or calls it, and there is no CPU fallback built on it.
 *
 * Reference files each function restates (paths relative to the reference's
 * src/cam/comm_operator/ascend_kernels/):
 *   orc_route              -- no reference kernel (callers pass topk_idx; see
 *                             src/cam/examples/moe_dispatch_combine_prefill_sample.py:87-93).
 *                             Spec: top-K of logit+bias, ties to the lower
 *                             index; gates = softmax(logits) at the selected
 *                             experts, renormalised over the K selected.
 *   orc_dispatch_layout    -- dispatch_layout/op_kernel/dispatch_layout.h:112-161
 *   orc_notify_dispatch    -- notify_dispatch/op_kernel/notify_dispatch.h:143-152,
 *                             340-360, 389-412 (single rank: src_rank dimension is 1)
 *   orc_dispatch           -- moe_dispatch_normal/op_kernel/moe_dispatch_normal.h:381-398
 *                             (row placement), :335-344 (triple), :545-591 (copy out),
 *                             :295-332 (int8 per-token quant, quant_mode 2).
 *                             quant_mode 3 (fp8 e4m3fn, 1x128 blocks) has no
 *                             reference counterpart; it follows the published
 *                             DeepSeek-V3 / DeepGEMM per_token_cast_to_fp8 recipe:
 *                             amax per 128 block clamped to >= 1e-4,
 *                             q = e4m3fn_rne(x * (448/amax)), scale = amax/448.
 *   orc_combine            -- moe_combine_normal/op_kernel/moe_combine_normal.h:343-377
 *                             and fused_deep_moe/.../cam_moe_distribute_combine.h:654-716
 *                             (fp32 accumulate in k order, multiply then add,
 *                             bf16 RINT, entries with expert < 0 skipped).
 *   orc_gmm1_swiglu_*      -- fused_deep_moe/op_kernel/fused_deep_moe/epilogue/block/
 *                             block_epilogue_per_token_dequant_swiglu.h:256-286
 *                             (left half = gate through silu, right half = up),
 *                             post_swiglu_dynamic_quant.h:164-231 (requant of h).
 *   orc_gmm2_*             -- block_epilogue_per_token_dequant.hpp:338-361
 *   orc_dispatch_int8_fused -- fused_deep_moe/.../raw_distributed/cam_moe_distribute_dispatch.h:640-681
 *   orc_*_int8, orc_quant_rows_int8 -- the reference's own int8 W8A8 numerics (see their comment)
 *
 * Build with -ffp-contract=off: the combine and the quantisers are specified
 * as separate fp32 multiply and add steps, never a fused multiply-add.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

/* ---------------------------------------------------------------- numerics */

static inline float bf16_to_f32(uint16_t h)
{
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* fp32 -> bf16, round to nearest even; NaN becomes a quiet NaN. */
static inline uint16_t f32_to_bf16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* OCP FP8 E4M3FN decode: bias 7, no infinities, 0x7f/0xff are NaN. */
static inline float e4m3_to_f32(uint8_t c)
{
    int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
    float v;
    if (e == 15 && m == 7)
        return NAN;
    if (e == 0)
        v = ldexpf((float)m, -9);            /* subnormal: m/8 * 2^-6 */
    else
        v = ldexpf((float)(8 + m), e - 10);  /* (1+m/8) * 2^(e-7) */
    return s ? -v : v;
}

/* OCP FP8 E4M3FN encode, round to nearest even, saturating at +-448.
 * Encodings are monotone in magnitude, so the rounded quotient
 * a / 2^(e-3) carries into the exponent field on its own. */
static inline uint8_t f32_to_e4m3(float x)
{
    uint8_t sign = signbit(x) ? 0x80 : 0x00;
    float a = fabsf(x);
    if (isnan(x))
        return 0x7f;
    if (a >= 448.0f)
        return sign | 0x7e;
    int code;
    if (a < 0x1p-6f) {
        code = (int)rintf(a * 0x1p9f);        /* subnormal grid step 2^-9 */
    } else {
        int e;
        frexpf(a, &e);                          /* a = f * 2^e, f in [0.5,1) */
        e -= 1;                                 /* a in [2^e, 2^(e+1)) */
        code = ((e + 7) << 3) + (int)rintf(ldexpf(a, 3 - e)) - 8;
    }
    if (code > 0x7e)
        code = 0x7e;
    return sign | (uint8_t)code;
}

ORC_API uint8_t orc_f32_to_e4m3(float x) { return f32_to_e4m3(x); }
ORC_API float orc_e4m3_to_f32(uint8_t c) { return e4m3_to_f32(c); }
ORC_API uint16_t orc_f32_to_bf16(float x) { return f32_to_bf16(x); }

/* Threads the token-parallel loops (route, dispatch, combine) use: OpenMP's team size (1 without
 * OpenMP).  Every token's arithmetic is the same whatever the thread count. */
ORC_API int orc_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static inline float silu(float g) { return g / (1.0f + expf(-g)); }

/* ------------------------------------------------------------------ R0 */

/* logits [T,E] f32, bias [E] or NULL -> topk_idx [T,K] int32, topk_w [T,K] f32 */
ORC_API void orc_route(const float *logits, const float *bias, int T, int E, int K,
                       int32_t *topk_idx, float *topk_w)
{
#pragma omp parallel
    {
    char *taken = (char *)malloc((size_t)E);
#pragma omp for schedule(static)
    for (int t = 0; t < T; ++t) {
        const float *l = logits + (size_t)t * E;
        memset(taken, 0, (size_t)E);
        float mx = -INFINITY;
        for (int e = 0; e < E; ++e)
            mx = l[e] > mx ? l[e] : mx;
        float ex[64];
        float denom = 0.0f;
        for (int k = 0; k < K; ++k) {
            int best = -1;
            float bs = 0.0f;
            for (int e = 0; e < E; ++e) {
                if (taken[e])
                    continue;
                float s = bias ? l[e] + bias[e] : l[e];
                if (best < 0 || s > bs) {   /* strict '>' keeps the lower index on ties */
                    best = e;
                    bs = s;
                }
            }
            taken[best] = 1;
            topk_idx[(size_t)t * K + k] = best;
            ex[k] = expf(l[best] - mx);
        }
        for (int k = 0; k < K; ++k)
            denom += ex[k];
        for (int k = 0; k < K; ++k)
            topk_w[(size_t)t * K + k] = ex[k] / denom;
    }
    free(taken);
    }
}

/* ------------------------------------------------------------------ D1 */

/* Stable rank of every (t,k) within its expert, histograms per expert and per
 * rank, and the token->rank membership table.  Expert ids outside [0,E) are
 * not routed: they get send_token_idx = -1 and count nowhere. */
ORC_API void orc_dispatch_layout(const int64_t *topk_idx, int T, int K, int E, int R,
                                 int32_t *num_tokens_per_rank, int32_t *num_tokens_per_expert,
                                 int32_t *is_token_in_rank, int32_t *send_token_idx)
{
    int per_rank = E / R;
    memset(num_tokens_per_expert, 0, sizeof(int32_t) * (size_t)E);
    memset(num_tokens_per_rank, 0, sizeof(int32_t) * (size_t)R);
    memset(is_token_in_rank, 0, sizeof(int32_t) * (size_t)T * R);
    for (int t = 0; t < T; ++t) {
        for (int k = 0; k < K; ++k) {
            int64_t e = topk_idx[(size_t)t * K + k];
            if (e < 0 || e >= E) {
                send_token_idx[(size_t)t * K + k] = -1;
                continue;
            }
            send_token_idx[(size_t)t * K + k] = num_tokens_per_expert[e]++;
            int r = (int)(e / per_rank);
            if (!is_token_in_rank[(size_t)t * R + r]) {
                is_token_in_rank[(size_t)t * R + r] = 1;
                num_tokens_per_rank[r]++;
            }
        }
    }
}

/* ------------------------------------------------------------------ D2 */

/* Single rank: send_offset = exclusive prefix of counts, recv_count =
 * inclusive prefix (expert-major, one source rank), recv_tokens_per_expert =
 * counts as int64, total = sum. */
ORC_API void orc_notify_dispatch(const int32_t *counts, int E, int32_t *send_offset,
                                 int32_t *recv_count, int64_t *recv_tokens_per_expert,
                                 int32_t *total_recv)
{
    int32_t run = 0;
    for (int e = 0; e < E; ++e) {
        send_offset[e] = run;
        run += counts[e];
        recv_count[e] = run;
        recv_tokens_per_expert[e] = counts[e];
    }
    *total_recv = run;
}

/* ------------------------------------------------------------- D3 + Q1/Q2 */

enum { ORC_QUANT_NONE = 0, ORC_QUANT_INT8_TOKEN = 2, ORC_QUANT_FP8_BLOCK = 3 };

/* x [T,H] bf16 -> expand_x [N,H] (bf16 | int8 | fp8), scales ([N] | [N,H/128]),
 * expand_idx [N,3] = (src_rank, t, k).  Row of (t,k) = send_offset[e] + send_token_idx[t,k]. */
ORC_API void orc_dispatch(const uint16_t *x, const int32_t *topk_idx, const int32_t *send_offset,
                          const int32_t *send_token_idx, int T, int H, int K, int E, int rank,
                          int quant_mode, void *expand_x, float *scales, int32_t *expand_idx)
{
    int nb = H / 128;
#pragma omp parallel
    {
    float *rowf = (float *)malloc(sizeof(float) * (size_t)H);
    uint8_t *q = (uint8_t *)malloc((size_t)H);
    float *bs = (float *)malloc(sizeof(float) * (size_t)(nb > 0 ? nb : 1));
#pragma omp for schedule(static)
    for (int t = 0; t < T; ++t) {
        const uint16_t *xr = x + (size_t)t * H;
        for (int h = 0; h < H; ++h)
            rowf[h] = bf16_to_f32(xr[h]);
        float tok_scale = 0.0f;
        if (quant_mode == ORC_QUANT_INT8_TOKEN) {
            float amax = 0.0f;
            for (int h = 0; h < H; ++h)
                amax = fabsf(rowf[h]) > amax ? fabsf(rowf[h]) : amax;
            float s = 127.0f / (amax + 1e-12f);
            for (int h = 0; h < H; ++h)
                q[h] = (uint8_t)(int8_t)rintf(rowf[h] * s);
            tok_scale = 1.0f / s;
        } else if (quant_mode == ORC_QUANT_FP8_BLOCK) {
            for (int b = 0; b < nb; ++b) {
                float amax = 0.0f;
                for (int h = b * 128; h < b * 128 + 128; ++h)
                    amax = fabsf(rowf[h]) > amax ? fabsf(rowf[h]) : amax;
                amax = amax > 1e-4f ? amax : 1e-4f;
                float inv = 448.0f / amax;
                for (int h = b * 128; h < b * 128 + 128; ++h)
                    q[h] = f32_to_e4m3(rowf[h] * inv);
                bs[b] = amax / 448.0f;
            }
        }
        for (int k = 0; k < K; ++k) {
            int e = topk_idx[(size_t)t * K + k];
            if (e < 0 || e >= E)
                continue;
            size_t row = (size_t)send_offset[e] + (size_t)send_token_idx[(size_t)t * K + k];
            expand_idx[row * 3 + 0] = rank;
            expand_idx[row * 3 + 1] = t;
            expand_idx[row * 3 + 2] = k;
            if (quant_mode == ORC_QUANT_NONE) {
                memcpy((uint16_t *)expand_x + row * H, xr, sizeof(uint16_t) * (size_t)H);
            } else {
                memcpy((uint8_t *)expand_x + row * H, q, (size_t)H);
                if (quant_mode == ORC_QUANT_INT8_TOKEN)
                    scales[row] = tok_scale;
                else
                    memcpy(scales + row * nb, bs, sizeof(float) * (size_t)nb);
            }
        }
    }
    free(rowf);
    free(q);
    free(bs);
    }
}

/* Fused-op int8 dispatch (fused_deep_moe/.../cam_moe_distribute_dispatch.h:640-681; the shared
 * expert's QuantToken in grouped_matmul_slice_m_per_token_dequant_swiglu_quant_multistage_workspace.h
 * follows the same steps): f = float(x) [* smooth[e, h], e the destination expert], amax = max |f|,
 * s = 127/amax (no epsilon), q = rint(f * s), scale = 1/s.  Each destination row is quantised on its
 * own, since the smooth scales depend on the expert.  A zero row (amax 0) gets q = 0 and scale 0
 * (the reference's 127/0 is undefined there). */
ORC_API void orc_dispatch_int8_fused(const uint16_t *x, const int32_t *topk_idx, const int32_t *send_offset,
                                     const int32_t *send_token_idx, int T, int H, int K, int E, const float *smooth,
                                     int8_t *expand_x, float *scales, int32_t *expand_idx)
{
    float *f = (float *)malloc(sizeof(float) * (size_t)H);
    for (int t = 0; t < T; ++t) {
        for (int k = 0; k < K; ++k) {
            int e = topk_idx[(size_t)t * K + k];
            if (e < 0 || e >= E)
                continue;
            size_t row = (size_t)send_offset[e] + (size_t)send_token_idx[(size_t)t * K + k];
            float amax = 0.0f;
            for (int h = 0; h < H; ++h) {
                f[h] = bf16_to_f32(x[(size_t)t * H + h]);
                if (smooth)
                    f[h] = f[h] * smooth[(size_t)e * H + h];
                amax = fabsf(f[h]) > amax ? fabsf(f[h]) : amax;
            }
            float s = amax > 0.0f ? 127.0f / amax : 0.0f;
            for (int h = 0; h < H; ++h)
                expand_x[row * H + h] = (int8_t)rintf(f[h] * s);
            scales[row] = amax > 0.0f ? 1.0f / s : 0.0f;
            expand_idx[row * 3 + 0] = 0;
            expand_idx[row * 3 + 1] = t;
            expand_idx[row * 3 + 2] = k;
        }
    }
    free(f);
}

/* ------------------------------------------------------------------ C1 */

/* y [N,H] bf16 in dispatch order, expand_idx [N,3], topk_idx/topk_w [T,K]
 * -> out [T,H] bf16.  out[t] = bf16_rne(sum_k y[row(t,k)] * w[t,k]) with the
 * sum in fp32, k ascending, starting from +0. */
ORC_API void orc_combine(const uint16_t *y, const int32_t *expand_idx, int N, const int32_t *topk_idx,
                         const float *topk_w, int T, int K, int E, int H, uint16_t *out)
{
    int32_t *inv = (int32_t *)malloc(sizeof(int32_t) * (size_t)T * K);
    for (size_t i = 0; i < (size_t)T * K; ++i)
        inv[i] = -1;
    for (int r = 0; r < N; ++r) {
        int t = expand_idx[(size_t)r * 3 + 1], k = expand_idx[(size_t)r * 3 + 2];
        if (t >= 0 && t < T && k >= 0 && k < K)
            inv[(size_t)t * K + k] = r;
    }
#pragma omp parallel
    {
    float *acc = (float *)malloc(sizeof(float) * (size_t)H);
#pragma omp for schedule(static)
    for (int t = 0; t < T; ++t) {
        for (int h = 0; h < H; ++h)
            acc[h] = 0.0f;
        for (int k = 0; k < K; ++k) {
            int e = topk_idx[(size_t)t * K + k];
            int r = inv[(size_t)t * K + k];
            if (e < 0 || e >= E || r < 0)
                continue;
            float w = topk_w[(size_t)t * K + k];
            const uint16_t *yr = y + (size_t)r * H;
            for (int h = 0; h < H; ++h) {
                float p = bf16_to_f32(yr[h]) * w;
                acc[h] = acc[h] + p;
            }
        }
        for (int h = 0; h < H; ++h)
            out[(size_t)t * H + h] = f32_to_bf16(acc[h]);
    }
    free(acc);
    }
    free(inv);
}

/* ------------------------------------------------------------ G1..G3 */
/* Grouped GEMMs over ragged expert segments.  Rows of A are in dispatch
 * order: expert e owns rows [off[e], off[e]+cnt[e]).  Weights are stored
 * N-major with K contiguous: W1 [L, 2I, H] (rows 0..I-1 gate, I..2I-1 up),
 * W2 [L, H, I].  Dot products accumulate in double. */

static void seg_offsets(const int64_t *cnt, int L, int64_t *off)
{
    int64_t run = 0;
    for (int e = 0; e < L; ++e) {
        off[e] = run;
        run += cnt[e];
    }
}

/* bf16: h[m,i] = bf16( silu(g) * u ), g/u rounded to fp32 first */
ORC_API void orc_gmm1_swiglu_bf16(const uint16_t *A, const int64_t *cnt, int L, const uint16_t *W1,
                                  int H, int I, uint16_t *hout)
{
    int64_t *off = (int64_t *)malloc(sizeof(int64_t) * (size_t)L);
    seg_offsets(cnt, L, off);
    for (int e = 0; e < L; ++e) {
        const uint16_t *W = W1 + (size_t)e * 2 * I * H;
#pragma omp parallel for schedule(dynamic, 1)
        for (int64_t m = off[e]; m < off[e] + cnt[e]; ++m) {
            float *a = (float *)malloc(sizeof(float) * (size_t)H);
            for (int h = 0; h < H; ++h)
                a[h] = bf16_to_f32(A[(size_t)m * H + h]);
            for (int i = 0; i < I; ++i) {
                const uint16_t *wg = W + (size_t)i * H, *wu = W + (size_t)(I + i) * H;
                double g = 0.0, u = 0.0;
                for (int h = 0; h < H; ++h) {
                    g += (double)a[h] * (double)bf16_to_f32(wg[h]);
                    u += (double)a[h] * (double)bf16_to_f32(wu[h]);
                }
                hout[(size_t)m * I + i] = f32_to_bf16(silu((float)g) * (float)u);
            }
            free(a);
        }
    }
    free(off);
}

ORC_API void orc_gmm2_bf16(const uint16_t *Hin, const int64_t *cnt, int L, const uint16_t *W2, int I,
                           int H, uint16_t *out)
{
    int64_t *off = (int64_t *)malloc(sizeof(int64_t) * (size_t)L);
    seg_offsets(cnt, L, off);
    for (int e = 0; e < L; ++e) {
        const uint16_t *W = W2 + (size_t)e * H * I;
#pragma omp parallel for schedule(dynamic, 1)
        for (int64_t m = off[e]; m < off[e] + cnt[e]; ++m) {
            float *a = (float *)malloc(sizeof(float) * (size_t)I);
            for (int i = 0; i < I; ++i)
                a[i] = bf16_to_f32(Hin[(size_t)m * I + i]);
            for (int n = 0; n < H; ++n) {
                const uint16_t *w = W + (size_t)n * I;
                double s = 0.0;
                for (int i = 0; i < I; ++i)
                    s += (double)a[i] * (double)bf16_to_f32(w[i]);
                out[(size_t)m * H + n] = f32_to_bf16((float)s);
            }
            free(a);
        }
    }
    free(off);
}

/* FP8: A [M,H] e4m3 with As [M,H/128]; W1 [L,2I,H] e4m3 with W1s [L,2I/128,H/128].
 * g,u = sum_k a*w*sa*sw (dequantised operands, double accumulate); h = silu(g)*u
 * in fp32, requantised per 1x128 block of h exactly like the dispatch quantiser. */
ORC_API void orc_gmm1_swiglu_fp8(const uint8_t *A, const float *As, const int64_t *cnt, int L,
                                 const uint8_t *W1, const float *W1s, int H, int I, uint8_t *hq,
                                 float *hs)
{
    int kb = H / 128, nb2 = 2 * I / 128;
    float lut[256];  /* e4m3 decode of every code */
    for (int c = 0; c < 256; ++c)
        lut[c] = e4m3_to_f32((uint8_t)c);
    int64_t *off = (int64_t *)malloc(sizeof(int64_t) * (size_t)L);
    seg_offsets(cnt, L, off);
    for (int e = 0; e < L; ++e) {
        const uint8_t *W = W1 + (size_t)e * 2 * I * H;
        const float *Ws = W1s + (size_t)e * nb2 * kb;
#pragma omp parallel for schedule(dynamic, 1)
        for (int64_t m = off[e]; m < off[e] + cnt[e]; ++m) {
            double *a = (double *)malloc(sizeof(double) * (size_t)H);
            float *hrow = (float *)malloc(sizeof(float) * (size_t)I);
            for (int h = 0; h < H; ++h)
                a[h] = (double)e4m3_to_f32(A[(size_t)m * H + h]) * (double)As[(size_t)m * kb + h / 128];
            for (int i = 0; i < I; ++i) {
                int ng = i, nu = I + i;
                const uint8_t *wg = W + (size_t)ng * H, *wu = W + (size_t)nu * H;
                double g = 0.0, u = 0.0;
                for (int h = 0; h < H; ++h) {
                    g += a[h] * (double)lut[wg[h]] * (double)Ws[(ng / 128) * kb + h / 128];
                    u += a[h] * (double)lut[wu[h]] * (double)Ws[(nu / 128) * kb + h / 128];
                }
                hrow[i] = silu((float)g) * (float)u;
            }
            for (int b = 0; b < I / 128; ++b) {
                float amax = 0.0f;
                for (int i = b * 128; i < b * 128 + 128; ++i)
                    amax = fabsf(hrow[i]) > amax ? fabsf(hrow[i]) : amax;
                amax = amax > 1e-4f ? amax : 1e-4f;
                float inv = 448.0f / amax;
                for (int i = b * 128; i < b * 128 + 128; ++i)
                    hq[(size_t)m * I + i] = f32_to_e4m3(hrow[i] * inv);
                hs[(size_t)m * (I / 128) + b] = amax / 448.0f;
            }
            free(hrow);
            free(a);
        }
    }
    free(off);
}

ORC_API void orc_gmm2_fp8(const uint8_t *Hq, const float *Hs, const int64_t *cnt, int L,
                          const uint8_t *W2, const float *W2s, int I, int H, uint16_t *out)
{
    int kb = I / 128, nbk = H / 128;
    float lut[256];  /* e4m3 decode of every code */
    for (int c = 0; c < 256; ++c)
        lut[c] = e4m3_to_f32((uint8_t)c);
    int64_t *off = (int64_t *)malloc(sizeof(int64_t) * (size_t)L);
    seg_offsets(cnt, L, off);
    for (int e = 0; e < L; ++e) {
        const uint8_t *W = W2 + (size_t)e * H * I;
        const float *Ws = W2s + (size_t)e * nbk * kb;
#pragma omp parallel for schedule(dynamic, 1)
        for (int64_t m = off[e]; m < off[e] + cnt[e]; ++m) {
            double *a = (double *)malloc(sizeof(double) * (size_t)I);
            for (int i = 0; i < I; ++i)
                a[i] = (double)e4m3_to_f32(Hq[(size_t)m * I + i]) * (double)Hs[(size_t)m * kb + i / 128];
            for (int n = 0; n < H; ++n) {
                const uint8_t *w = W + (size_t)n * I;
                double s = 0.0;
                for (int i = 0; i < I; ++i)
                    s += a[i] * (double)lut[w[i]] * (double)Ws[(n / 128) * kb + i / 128];
                out[(size_t)m * H + n] = f32_to_bf16((float)s);
            }
            free(a);
        }
    }
    free(off);
}

/* ------------------------------------------------------------ int8 W8A8 (reference numerics) */
/* The reference's fused path in int8: per-channel weight scales, per-token activation scales.
 * GMM1 epilogue (block_epilogue_per_token_dequant_swiglu.h:256-286):
 *   v = ((float)acc * w_scale[n]) * x_scale[m]; gate half through silu v / (1 + exp(-v)).
 * Post-SwiGLU requant (post_swiglu_dynamic_quant.h:164-231), per token over the whole row:
 *   h = silu(g) * u; amax = max |h|; q = rint((h * 127) * (1 / amax)); scale = amax * (1/127).
 * GMM2 epilogue (block_epilogue_per_token_dequant.hpp:338-361):
 *   out = bf16_rint(((float)acc * w_scale[n]) * h_scale[m]).
 * Integer dot products are exact (int32). */
ORC_API void orc_gmm1_swiglu_int8(const int8_t *A, const float *As, const int64_t *cnt, int L, const int8_t *W1,
                                  const float *W1s, int H, int I, float *hout)
{
    int64_t *off = (int64_t *)malloc(sizeof(int64_t) * (size_t)L);
    seg_offsets(cnt, L, off);
    for (int e = 0; e < L; ++e) {
        const int8_t *W = W1 + (size_t)e * 2 * I * H;
        const float *Ws = W1s + (size_t)e * 2 * I;
        for (int64_t m = off[e]; m < off[e] + cnt[e]; ++m) {
            const int8_t *a = A + (size_t)m * H;
            for (int i = 0; i < I; ++i) {
                const int8_t *wg = W + (size_t)i * H, *wu = W + (size_t)(I + i) * H;
                int32_t g = 0, u = 0;
                for (int h = 0; h < H; ++h) {
                    g += (int32_t)a[h] * (int32_t)wg[h];
                    u += (int32_t)a[h] * (int32_t)wu[h];
                }
                float gf = ((float)g * Ws[i]) * As[m];
                float uf = ((float)u * Ws[I + i]) * As[m];
                gf = gf / (1.0f + expf(-gf));
                hout[(size_t)m * I + i] = gf * uf;
            }
        }
    }
    free(off);
}

ORC_API void orc_quant_rows_int8(const float *h, int M, int I, int8_t *q, float *scale)
{
    for (int m = 0; m < M; ++m) {
        const float *r = h + (size_t)m * I;
        float amax = 0.0f;
        for (int i = 0; i < I; ++i)
            amax = fabsf(r[i]) > amax ? fabsf(r[i]) : amax;
        const float inv = amax > 0.0f ? 1.0f / amax : 0.0f;  /* a zero row: q = 0, scale 0 */
        for (int i = 0; i < I; ++i)
            q[(size_t)m * I + i] = (int8_t)rintf((r[i] * 127.0f) * inv);
        scale[m] = amax * (1.0f / 127.0f);
    }
}

ORC_API void orc_gmm2_int8(const int8_t *Hq, const float *Hs, const int64_t *cnt, int L, const int8_t *W2,
                           const float *W2s, int I, int H, uint16_t *out)
{
    int64_t *off = (int64_t *)malloc(sizeof(int64_t) * (size_t)L);
    seg_offsets(cnt, L, off);
    for (int e = 0; e < L; ++e) {
        const int8_t *W = W2 + (size_t)e * H * I;
        const float *Ws = W2s + (size_t)e * H;
        for (int64_t m = off[e]; m < off[e] + cnt[e]; ++m) {
            const int8_t *a = Hq + (size_t)m * I;
            for (int n = 0; n < H; ++n) {
                const int8_t *w = W + (size_t)n * I;
                int32_t s = 0;
                for (int i = 0; i < I; ++i)
                    s += (int32_t)a[i] * (int32_t)w[i];
                out[(size_t)m * H + n] = f32_to_bf16(((float)s * Ws[n]) * Hs[m]);
            }
        }
    }
    free(off);
}
