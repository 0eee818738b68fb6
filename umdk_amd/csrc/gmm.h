// Grouped expert GEMM launcher (gmm.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cam {

enum GmmDtype { DT_BF16 = 0, DT_FP8 = 3 };
enum GmmEpilogue { EPI_PLAIN = 0, EPI_SWIGLU_BF16 = 1, EPI_SWIGLU_FP8 = 2 };

struct GmmArgs {
    const uint8_t *A;           // [M, K] activations in dispatch order (bf16 or fp8 bytes)
    const float *As;            // fp8: [M, K/128] activation block scales
    const int64_t *group_list;  // [L] rows per local expert (device)
    int L;                      // local experts
    int M;                      // rows allocated in A and the output
    int K;                      // reduction length (elements)
    int N;                      // W rows per expert (2I for SwiGLU, H for the plain GEMM)
    const uint8_t *W;           // [L, N, K]
    const float *Ws;            // fp8: [L, N/128, K/128]
    uint8_t *C;                 // plain: bf16 [M, N]; SwiGLU: h [M, N/2] (bf16 or fp8)
    float *Cs;                  // SwiGLU fp8: [M, N/256] h block scales
    int allow256 = 1;           // set by the launcher: the 256-row tile may be picked on the device
};

size_t gmm_lds_bytes();
hipError_t launch_gmm(const GmmArgs &a, int dt, int epi, hipStream_t s);

}  // namespace cam
