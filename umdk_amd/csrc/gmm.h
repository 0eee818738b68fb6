// Grouped expert GEMM launcher (gmm.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cam {

enum GmmDtype { DT_BF16 = 0, DT_INT8 = 2, DT_FP8 = 3 };
// EPI_SWIGLU_F32AMAX (int8 only): h in fp32 [M, N/2] and partial row maxima of |h| in Cs [M, N/2/32]: slot
// c of row m holds max |h| over h-columns [32 c, 32 c + 32), written once by the wave that computed them
// (float bits, combined across tiles by atomic max; the launcher clears it first), for the per-token
// int8 requantisation that follows (launch_quant_rows_int8).
enum GmmEpilogue { EPI_PLAIN = 0, EPI_SWIGLU_BF16 = 1, EPI_SWIGLU_FP8 = 2, EPI_SWIGLU_F32AMAX = 3 };

struct GmmArgs {
    const uint8_t *A;           // [M, K] activations in dispatch order (bf16 or fp8 bytes)
    const float *As;            // fp8: [K/128, M] activation block scales (k-major); int8: [M] per-token scales
    const int64_t *group_list;  // [L] rows per local expert (device)
    int L;                      // local experts
    int M;                      // rows allocated in A and the output
    int K;                      // reduction length (elements)
    int N;                      // W rows per expert (2I for SwiGLU, H for the plain GEMM)
    const uint8_t *W;           // [L, N, K]
    const float *Ws;            // fp8: [L, N/128, K/128]; int8: [L, N] per-channel scales
    uint8_t *C;                 // plain: bf16 [M, N]; SwiGLU: h [M, N/2] (bf16, fp8 or fp32)
    float *Cs;                  // SwiGLU fp8: [N/256, M] h block scales (k-major); SwiGLU fp32: [M] row max |h|
    int allow256 = 1;           // set by the launcher: the 256-row tile may be picked on the device
    // Separated weights (optional): device arrays of L pointers, expert e's [N, K] weight and its scales
    // ([N/128, K/128] fp8, [N] int8); when set, W and Ws are not read.
    const uint8_t *const *Wl = nullptr;
    const float *const *Wsl = nullptr;
};

hipError_t launch_gmm(const GmmArgs &a, int dt, int epi, hipStream_t s);

// GMM1 + SwiGLU and GMM2 in one persistent launch (fp8 with fp8 h, or bf16): every block runs its GMM1 tiles,
// then its GMM2 tiles.  A GMM1 tile of (expert e, M-tile m) stores its h rows with agent-coherent stores and,
// once they have completed, adds 1 to ready[m]; a GMM2 tile of m starts its DMAs only after ready[m] has
// reached I/128 (every GMM1 tile of those rows).  ready holds gmm_chain_counters(M, L) zeroed ints (the
// caller clears them before the launch).  A wait that does not complete within the wait bound gives up, sets
// the device's sync status (sync_status_*) and the launch ends normally with unspecified outputs.
// hipErrorNotSupported: this combination (int8, or GEMMs that would pick different row tiles) has no chained
// kernel; run launch_gmm twice instead.  g1.C / g1.Cs are h and its k-major scales, g2.A / g2.As the same.
int gmm_chain_counters(int M, int L);
bool gmm_chain_supported(const GmmArgs &g1, const GmmArgs &g2, int dt);
hipError_t launch_gmm_chain(const GmmArgs &g1, const GmmArgs &g2, int dt, int *ready, hipStream_t s);
// Device sync status of the chained launches: nonzero once a readiness wait has given up (sticky until
// cleared).  Synchronous: reads (and optionally clears) the current device's status word.
hipError_t sync_status_read(int *status, bool clear);
// Test hooks: the wait bound in constant-clock ticks (<= 0: the default, 2 s) and an unreachable target
// (every wait gives up at the bound).
void sync_debug_set(long long wait_ticks, int unreachable);
// fp8 activation scales [M, nb] row-major -> [nb, M] k-major (the layout the GEMMs read: one k-step's
// scales of consecutive rows are contiguous), rows [0, sum(group_list)) only.
hipError_t launch_scales_to_kmajor(const float *src, const int64_t *group_list, int L, int M, int nb, float *dst,
                                   hipStream_t s);
// Per-token int8 requantisation of the fp32 h written by EPI_SWIGLU_F32AMAX, rows [0, sum(group_list)):
// amax = max of the row's I/32 partial maxima, q = rint((h * 127) * (1 / amax)), scale = amax * (1/127);
// rows with amax 0 get q = 0, scale 0.
constexpr int GMM_AMAX_COLS = 32;  // h-columns per partial row maximum
hipError_t launch_quant_rows_int8(const float *h, const float *amax, const int64_t *group_list, int L, int M, int I,
                                  int8_t *q, float *scale, hipStream_t s);

}  // namespace cam
