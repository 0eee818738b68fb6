// Device bodies of the prefill step's three stages -- routing of a 16-token chunk (R0 + the chunk histograms
// of D1), one expert's chunk scan and count exchange (D1 + D2), one dispatch wave (D3 + Q1) -- used by their
// kernels (route.hip, layout.hip, dispatch.hip).  (Measured: the three stages in one launch, waiting on each
// other through counters, took 65-67 us against 62-63 us for three launches at config 2's shape; a kernel
// boundary gives the same ordering for less.)
#pragma once
#include "cam_device.h"

namespace cam {

// ---------------------------------------------------------------- R0: routing
// A token is handled by a 16-lane row of a wave (four tokens per wave); lane l of the row holds experts l,
// l+16, l+32, ...  Each (score, expert) pair is ordered by the score's bits mapped to an order-preserving
// unsigned integer, then by the lower expert id: each of the K rounds takes the row-wide maximum of the score
// key, then of ~expert over the lanes holding that score, each with four DPP max steps (quad xor 1, quad xor 2,
// half-row mirror, row mirror; no LDS traffic, no branches), and the owning lane retires that expert by zeroing
// its key.  Gates are softmax(logits) at the picks renormalised over the K picks:
// w_k = exp(l_k - max_l) / sum_j exp(l_j - max_l), summed in pick order.
constexpr int ROUTE_WAVES = 4;
constexpr int ROUTE_MAX_PER_LANE = 32;  // E <= 512 over 16 lanes

// dpp_ctrl codes (GCN/CDNA DPP): quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror
constexpr int DPP_QUAD_XOR1 = 0xB1;
constexpr int DPP_QUAD_XOR2 = 0x4E;
constexpr int DPP_HALF_MIRROR = 0x141;
constexpr int DPP_MIRROR = 0x140;

template <int CTRL> __device__ __forceinline__ uint32_t dpp(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL> __device__ __forceinline__ uint32_t umax_step(uint32_t v) { return max(v, dpp<CTRL>(v)); }
template <int CTRL> __device__ __forceinline__ float fmax_step(float v)
{
    return fmaxf(v, __uint_as_float(dpp<CTRL>(__float_as_uint(v))));
}
__device__ __forceinline__ uint32_t order_key(float s)
{
    const uint32_t u = __float_as_uint(s);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Routes chunk `b` of `nb` (tokens [16 b, 16 b + 16)) with the block's 256 threads.  HIST: the chunk is also
// a layout chunk, and the block writes the chunk's histogram of the picked ids below Ec (the local experts),
// chunk_counts[e * nb + b] for every e < Ec, the chunk's exclusive prefix of that histogram over the experts,
// chunk_pref[e * nb + b] (summed over the chunks it is expert e's offset among the received rows, so no later
// step needs every expert's total), and each such pick's rank among the chunk's picks of the same expert in
// (t,k) order, chunk_rank[t * K + k].  A token's K picks are distinct experts, so that rank is the number of
// earlier tokens of the chunk that picked the expert: each expert gets a 16-bit mask of the chunk's tokens that
// picked it (an LDS atomic OR, which no order of the ORs changes), the rank is the popcount of the mask below
// the token, the count that of the whole mask.
template <int PER, bool HIST>
__device__ __forceinline__ void route_block(const float *__restrict__ logits, const float *__restrict__ bias, int T,
                                            int E, int K, int32_t *__restrict__ topk_idx, float *__restrict__ topk_w,
                                            int64_t *__restrict__ topk_idx64, int Ec, int32_t *__restrict__ chunk_counts,
                                            int32_t *__restrict__ chunk_pref, int32_t *__restrict__ chunk_rank, int b,
                                            int nb)
{
    const int lane = threadIdx.x & 63;
    const int l16 = lane & 15;
    const int t = (b * ROUTE_WAVES + (int)(threadIdx.x >> 6)) * 4 + (lane >> 4);
    const bool live = t < T;  // dead rows still run the DPP steps (they read only their own row)
    const float *l = logits + (size_t)(live ? t : 0) * E;
    uint32_t khi[PER];
    float lg[PER], bs[PER];
    // loads first, all unconditional (clamped index) so they are in flight together
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = min(l16 + 16 * j, E - 1);
        lg[j] = l[e];
        bs[j] = bias ? bias[e] : 0.0f;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const bool valid = live && l16 + 16 * j < E;
        // + 0.0f turns -0.0 into +0.0, so the integer key orders zeros as a float compare does
        const float sc = (bias ? lg[j] + bs[j] : lg[j]) + 0.0f;
        mx = valid ? fmaxf(mx, lg[j]) : mx;
        khi[j] = valid ? order_key(sc) : 0u;
    }
    mx = fmax_step<DPP_QUAD_XOR1>(mx);
    mx = fmax_step<DPP_QUAD_XOR2>(mx);
    mx = fmax_step<DPP_HALF_MIRROR>(mx);
    mx = fmax_step<DPP_MIRROR>(mx);

    int my_idx = 0;
#pragma unroll 1
    for (int k = 0; k < K; ++k) {
        // row-wide best score key, then the lowest expert id holding it (picked slots are zeroed):
        // two branch-free 32-bit max reductions instead of one 64-bit one
        uint32_t hi = 0;
#pragma unroll
        for (int j = 0; j < PER; ++j)
            hi = max(hi, khi[j]);
        hi = umax_step<DPP_QUAD_XOR1>(hi);
        hi = umax_step<DPP_QUAD_XOR2>(hi);
        hi = umax_step<DPP_HALF_MIRROR>(hi);
        hi = umax_step<DPP_MIRROR>(hi);
        int jb = PER;  // this lane's lowest slot holding the row maximum (slots ascend in expert id)
#pragma unroll
        for (int j = PER - 1; j >= 0; --j)
            jb = khi[j] == hi ? j : jb;
        uint32_t lo = (hi != 0 && jb < PER) ? ~(uint32_t)(l16 + 16 * jb) : 0u;
        lo = umax_step<DPP_QUAD_XOR1>(lo);
        lo = umax_step<DPP_QUAD_XOR2>(lo);
        lo = umax_step<DPP_HALF_MIRROR>(lo);
        lo = umax_step<DPP_MIRROR>(lo);
        const int best = (int)~lo;
        const int clear = (best & 15) == l16 ? best >> 4 : -1;
#pragma unroll
        for (int j = 0; j < PER; ++j)
            khi[j] = j == clear ? 0u : khi[j];
        if (l16 == k)
            my_idx = best;
    }
    float my_ex = 0.0f;
    if (l16 < K && live)
        my_ex = expf(l[my_idx] - mx);
    float denom = 0.0f;
    for (int k = 0; k < K; ++k)
        denom += __shfl(my_ex, (lane & 48) | k, 64);
    if (l16 < K && live) {
        topk_idx[(size_t)t * K + l16] = my_idx;
        topk_w[(size_t)t * K + l16] = my_ex / denom;
        if (topk_idx64)
            topk_idx64[(size_t)t * K + l16] = my_idx;
    }
    if constexpr (HIST) {
        static_assert(ROUTE_WAVES * 4 <= 32, "a chunk's tokens fit a 32-bit mask");
        __shared__ uint32_t picked[ROUTE_MAX_PER_LANE * 16];  // per expert: the chunk's tokens that picked it
        for (int e = threadIdx.x; e < Ec; e += ROUTE_WAVES * 64)
            picked[e] = 0u;
        __syncthreads();
        const int tl = t - b * ROUTE_WAVES * 4;  // the token's place in the chunk
        const bool local = l16 < K && live && my_idx < Ec;
        if (local)
            atomicOr(&picked[my_idx], 1u << tl);
        __syncthreads();
        if (local)
            chunk_rank[(size_t)t * K + l16] = __popc(picked[my_idx] & ((1u << tl) - 1u));
        // the histogram, and its exclusive prefix over the experts: thread i owns experts [i PE, (i + 1) PE)
        constexpr int NT = ROUTE_WAVES * 64, PE = (ROUTE_MAX_PER_LANE * 16 + NT - 1) / NT;
        __shared__ int32_t wsum[ROUTE_WAVES];
        int cnt[PE], own = 0;
#pragma unroll
        for (int q = 0; q < PE; ++q) {
            const int e = threadIdx.x * PE + q;
            cnt[q] = e < Ec ? __popc(picked[e]) : 0;
            own += cnt[q];
        }
        int incl = own;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int u = __shfl_up(incl, o, 64);
            if (lane >= o)
                incl += u;
        }
        if (lane == 63)
            wsum[threadIdx.x >> 6] = incl;
        __syncthreads();
        int run = incl - own;
        for (int v = 0; v < (int)(threadIdx.x >> 6); ++v)
            run += wsum[v];
#pragma unroll
        for (int q = 0; q < PE; ++q) {
            const int e = threadIdx.x * PE + q;
            if (e < Ec) {
                chunk_counts[(size_t)e * nb + b] = cnt[q];
                chunk_pref[(size_t)e * nb + b] = run;
            }
            run += cnt[q];
        }
    }
}

// ---------------------------------------------------------------- D1 + D2: one expert's chunk scan
// The wave of expert e scans the expert's row of chunk counts in place into exclusive chunk bases and sums
// its row of chunk prefixes (each chunk's count of the lower experts' picks) into its send offset, so every
// expert's count exchange entry is known without a second pass over the totals: send_offset = exclusive,
// recv_count = inclusive prefix over the experts, tokens_per_expert as int64.
__device__ __forceinline__ void scan_expert(int e, int nc, int32_t *__restrict__ counts,
                                            const int32_t *__restrict__ pref, int32_t *__restrict__ send_offset,
                                            int32_t *__restrict__ recv_count, int64_t *__restrict__ tokens_per_expert)
{
    const int lane = threadIdx.x & 63;
    int32_t *row = counts + (size_t)e * nc;
    const int32_t *prow = pref + (size_t)e * nc;
    int32_t pre[4], pp[4];  // the first 256 chunks' counts and prefixes in flight together
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const bool in = u * 64 + lane < nc;
        pre[u] = in ? row[u * 64 + lane] : 0;
        pp[u] = in ? prow[u * 64 + lane] : 0;
    }
    int32_t carry = 0, below = 0;
    for (int c0 = 0; c0 < nc; c0 += 64) {
        const int c = c0 + lane;
        int32_t v = 0, bq = 0;
        if (c0 < 256) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                v = c0 == u * 64 ? pre[u] : v;
                bq = c0 == u * 64 ? pp[u] : bq;
            }
        } else if (c < nc) {
            v = row[c];
            bq = prow[c];
        }
        int32_t incl = v;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int32_t u = __shfl_up(incl, o, 64);
            if (lane >= o)
                incl += u;
        }
        if (c < nc)
            row[c] = carry + incl - v;
        carry += __shfl(incl, 63, 64);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
            bq += __shfl_xor(bq, o, 64);
        below += bq;
    }
    if (lane == 0) {
        send_offset[e] = below;
        recv_count[e] = below + carry;
        tokens_per_expert[e] = carry;
    }
}

// ---------------------------------------------------------------- D1 + D2 of a decode step, in one block
// The whole layout of T*K <= LAYOUT_LDS_MAX_TK picks over E <= LAYOUT_LDS_MAX_E experts, computed by one block
// of NT threads into LDS: the effective id of every pick (-1 when masked or outside [0, E)), its stable rank
// among the picks of its expert in (t,k) order (lanes sharing an expert found with one ballot per bit of the
// id, waves ordered by per-wave counts, windows of NT picks in turn), the count of every expert and its
// exclusive offset (the count exchange of one rank).  The same results as layout_small_kernel.
constexpr int LAYOUT_LDS_MAX_TK = 2048;
constexpr int LAYOUT_LDS_MAX_E = 512;
template <int NT> struct LayoutLds {
    int32_t ids[LAYOUT_LDS_MAX_TK], rank[LAYOUT_LDS_MAX_TK];
    int32_t count[LAYOUT_LDS_MAX_E], off[LAYOUT_LDS_MAX_E];
    int32_t wave_hist[NT / 64][LAYOUT_LDS_MAX_E];
    int32_t wave_sum[NT / 64];
};
template <int NT>
__device__ __forceinline__ void layout_lds(const int32_t *__restrict__ ids, const uint8_t *__restrict__ active, int T,
                                           int K, int E, LayoutLds<NT> &s)
{
    constexpr int NW = NT / 64, NPASS = LAYOUT_LDS_MAX_TK / NT, PE = (LAYOUT_LDS_MAX_E + NT - 1) / NT;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, TK = T * K;
    // every pick's effective id first: unconditional loads (indices clamped to the last pick), all in flight
    // together
    int eff[NPASS], on[NPASS];
#pragma unroll
    for (int q = 0; q < NPASS; ++q) {
        eff[q] = ids[min(q * NT + tid, TK - 1)];
        on[q] = 1;
    }
    if (active) {
#pragma unroll
        for (int q = 0; q < NPASS; ++q)
            on[q] = active[min(q * NT + tid, TK - 1) / K];
    }
#pragma unroll
    for (int q = 0; q < NPASS; ++q) {
        const int id = eff[q];
        eff[q] = q * NT + tid < TK && on[q] != 0 && id >= 0 && id < E ? id : -1;
    }
    for (int e = tid; e < E; e += NT)
        s.count[e] = 0;
    const int nbits = E > 1 ? 32 - __clz(E - 1) : 1;
    const uint64_t lt = lanemask_lt();
#pragma unroll
    for (int q = 0; q < NPASS; ++q) {
        if (q * NT >= TK)
            break;
        for (int j = tid; j < NW * E; j += NT)
            s.wave_hist[j / E][j % E] = 0;
        __syncthreads();
        const int i = q * NT + tid, e = eff[q];
        if (i < TK)
            s.ids[i] = e;
        const bool valid = e >= 0;
        uint64_t peers = __ballot(valid);
        for (int b = 0; b < nbits; ++b) {
            const bool bit = valid && ((e >> b) & 1);
            const uint64_t m = __ballot(bit);
            peers &= bit ? m : ~m;
        }
        const int inrank = __popcll(peers & lt);
        if (valid && inrank == 0)
            s.wave_hist[w][e] = __popcll(peers);
        __syncthreads();
        if (i < TK) {
            int32_t r = -1;
            if (valid) {
                r = s.count[e] + inrank;
                for (int ww = 0; ww < w; ++ww)
                    r += s.wave_hist[ww][e];
            }
            s.rank[i] = r;
        }
        __syncthreads();
        for (int ee = tid; ee < E; ee += NT) {
            int32_t acc = 0;
#pragma unroll
            for (int ww = 0; ww < NW; ++ww)
                acc += s.wave_hist[ww][ee];
            s.count[ee] += acc;
        }
        __syncthreads();
    }
    // exclusive offsets over the experts: thread i owns experts [i PE, (i + 1) PE)
    int cnt[PE], own = 0;
#pragma unroll
    for (int u = 0; u < PE; ++u) {
        const int e = tid * PE + u;
        cnt[u] = e < E ? s.count[e] : 0;
        own += cnt[u];
    }
    int32_t v = own;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int32_t u = __shfl_up(v, o, 64);
        if (lane >= o)
            v += u;
    }
    if (lane == 63)
        s.wave_sum[w] = v;
    __syncthreads();
    int32_t run = v - own;
    for (int ww = 0; ww < w; ++ww)
        run += s.wave_sum[ww];
#pragma unroll
    for (int u = 0; u < PE; ++u) {
        const int e = tid * PE + u;
        if (e < E)
            s.off[e] = run;
        run += cnt[u];
    }
    __syncthreads();
}
// The layout's global outputs (by one block): counts, send offsets, inclusive counts, the total and the int64
// tokens per expert.
template <int NT>
__device__ __forceinline__ void layout_lds_store(const LayoutLds<NT> &s, int E, int32_t *__restrict__ counts,
                                                 int32_t *__restrict__ send_offset, int32_t *__restrict__ recv_count,
                                                 int32_t *__restrict__ total, int64_t *__restrict__ tokens_per_expert)
{
    for (int e = threadIdx.x; e < E; e += NT) {
        const int32_t c = s.count[e], o = s.off[e];
        counts[e] = c;
        send_offset[e] = o;
        recv_count[e] = o + c;
        tokens_per_expert[e] = c;
        if (e == E - 1)
            *total = o + c;
    }
}

// ---------------------------------------------------------------- D3 + Q1: one dispatch wave
// Where the rank of (t,k) within its expert comes from: send_token_idx[t,k] (the layout op's output), or,
// with send_token_idx == nullptr, chunk_base (the prefill step: chunks of `tpc` tokens, chunk_base[e * nc + c]
// = entries of expert e in chunks before c) plus chunk_rank[t,k], the rank inside the chunk (the routing
// kernel's).
struct RankSrc {
    const int32_t *send_token_idx;
    const int32_t *chunk_base;
    const int32_t *chunk_rank;
    int tpc;
};

// Resolves the K destination rows of token t: lane k < K holds row(t,k) or -1.
__device__ __forceinline__ int dispatch_dest(const int32_t *__restrict__ topk_idx,
                                             const int32_t *__restrict__ send_offset, const RankSrc &rs, int t,
                                             int T, int K, int E, int cap, int lane)
{
    int dst = -1;
    if (topk_idx == nullptr)  // identity mode (K = 1): row t of x quantised into row t
        return lane == 0 ? t : -1;
    if (rs.send_token_idx) {
        if (lane < K) {
            const int e = topk_idx[(size_t)t * K + lane];
            if (e >= 0 && e < E)
                dst = send_offset[e] + rs.send_token_idx[(size_t)t * K + lane];
        }
    } else if (lane < K) {
        const int e = topk_idx[(size_t)t * K + lane];
        if (e >= 0 && e < E) {
            const int nc = (T + rs.tpc - 1) / rs.tpc;
            dst = send_offset[e] + rs.chunk_base[(size_t)e * nc + t / rs.tpc] + rs.chunk_rank[(size_t)t * K + lane];
        }
    }
    if (dst >= cap)  // inconsistent counts: never write outside the output
        dst = -1;
    return dst < 0 ? -1 : dst;
}

// The wave of (token t, 1024-column chunk j): bf16 copy (MODE QUANT_NONE = 0) or fp8 1x128 quantisation
// (MODE 3: amax clamped to >= 1e-4, q = e4m3_rne_sat(x * (448/amax)), scale = amax/448; a 128-block is 8
// adjacent lanes, so its amax is a 3-step xor shuffle).  The slice of x is read once (16-byte loads),
// quantised once in registers and written to each of the token's K destination rows with 16-byte stores.
// `ready()` is called between the loads of x and the first read of the routing results (a hook for a kernel
// that waits there for earlier stages of the same launch; a no-op in the dispatch kernel).  skip_unrouted: a token none of whose
// picks is below E reads nothing and only writes its row-map entries (`ready()` comes first then).
template <int MODE, typename Ready>
__device__ __forceinline__ void dispatch_wave(const uint16_t *__restrict__ x, const int32_t *__restrict__ topk_idx,
                                              const int32_t *__restrict__ send_offset, const RankSrc &rs, int t,
                                              int j, int T, int H, int K, int E, int rank, int cap,
                                              uint8_t *__restrict__ expand_x, float *__restrict__ scales,
                                              int32_t *__restrict__ expand_idx, int32_t *__restrict__ inv_out,
                                              int kmajor, int skip_unrouted, Ready ready)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    bool waited = false;
    // skip_unrouted (a rank holding some of the experts): a token none of whose picks is an expert of this rank
    // reads nothing, only its row-map entries are written (config 4, 32 of 256 experts local: 40% of the
    // tokens, the layer 2-3 us faster; with every expert local the check measured 0.7 us slower per step)
    if (skip_unrouted && topk_idx) {
        ready();
        waited = true;
        const int e0 = lane < K ? topk_idx[(size_t)t * K + lane] : -1;
        if (__ballot(e0 >= 0 && e0 < E) == 0) {
            if (inv_out && j == 0 && lane < K)
                inv_out[(size_t)t * K + lane] = -1;
            return;
        }
    }
    // the slice of x is requested first, so its loads are in flight while the destination rows resolve
    if constexpr (MODE == 0) {
        // lane l copies columns [1024 j + 8 l, +8) and [1024 j + 512 + 8 l, +8): each 16-byte
        // store instruction of the wave writes one contiguous kilobyte
        const int col = j * 1024 + lane * 8;
        const bool act = col < H, act1 = col + 512 < H;
        u32x4 raw0 = u32x4{0, 0, 0, 0}, raw1 = u32x4{0, 0, 0, 0};
        if (act) {
            raw0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(x + (size_t)t * H + col));
            if (act1)
                raw1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(x + (size_t)t * H + col + 512));
        }
        if (!waited)
            ready();
        const int dst = dispatch_dest(topk_idx, send_offset, rs, t, T, K, E, cap, lane);
        if (inv_out && j == 0 && lane < K)  // the combine's row map, so it needs no scatter pass
            inv_out[(size_t)t * K + lane] = dst;
        for (int k = 0; k < K; ++k) {
            const int row = __shfl(dst, k, 64);
            if (row < 0)
                continue;
            if (act) {
                uint16_t *out = reinterpret_cast<uint16_t *>(expand_x) + (size_t)row * H + col;
                *reinterpret_cast<u32x4 *>(out) = raw0;
                if (act1)
                    *reinterpret_cast<u32x4 *>(out + 512) = raw1;
            }
            if (j == 0 && lane == 0 && expand_idx) {
                expand_idx[(size_t)row * 3 + 0] = rank;
                expand_idx[(size_t)row * 3 + 1] = t;
                expand_idx[(size_t)row * 3 + 2] = k;
            }
        }
    } else {
        // lane l quantises columns [1024 j + 16 l, +16): one 16-byte fp8 store per row.  Cached loads of x
        // and streaming (nontemporal) stores of the rows: measured 5% faster on the DSV3 rank shape than the
        // reverse (nontemporal loads, cached stores), and 11% faster than cached loads and stores.
        const int col = j * 1024 + lane * 16;
        const bool act = col < H;
        u32x4 raw0 = u32x4{0, 0, 0, 0}, raw1 = u32x4{0, 0, 0, 0};
        if (act) {
            const u32x4 *src = reinterpret_cast<const u32x4 *>(x + (size_t)t * H + col);
            raw0 = src[0];
            raw1 = src[1];
        }
        if (!waited)
            ready();
        const int dst = dispatch_dest(topk_idx, send_offset, rs, t, T, K, E, cap, lane);
        if (inv_out && j == 0 && lane < K)  // the combine's row map, so it needs no scatter pass
            inv_out[(size_t)t * K + lane] = dst;
        float f[16];
        unpack_bf16x8(raw0, f);
        unpack_bf16x8(raw1, f + 8);
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i)
            amax = fmaxf(amax, fabsf(f[i]));
        amax = fmaxf(group_max<8>(amax), 1e-4f);  // a 128-block is 8 adjacent lanes
        const float inv = 448.0f / amax;
        const float bscale = amax / 448.0f;
        u32x4 q;
#pragma unroll
        for (int w = 0; w < 4; ++w)
            q[w] = f32x4_to_e4m3(f[4 * w] * inv, f[4 * w + 1] * inv, f[4 * w + 2] * inv, f[4 * w + 3] * inv);
        const int nb = H >> 7;
        for (int k = 0; k < K; ++k) {
            const int row = __shfl(dst, k, 64);
            if (row < 0)
                continue;
            if (act) {
                __builtin_nontemporal_store(q, reinterpret_cast<u32x4 *>(expand_x + (size_t)row * H + col));
                if ((lane & 7) == 0)
                    scales[kmajor ? (size_t)(col >> 7) * cap + row : (size_t)row * nb + (col >> 7)] = bscale;
            }
            if (j == 0 && lane == 0 && expand_idx) {
                expand_idx[(size_t)row * 3 + 0] = rank;
                expand_idx[(size_t)row * 3 + 1] = t;
                expand_idx[(size_t)row * 3 + 2] = k;
            }
        }
    }
}

}  // namespace cam
