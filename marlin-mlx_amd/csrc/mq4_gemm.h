// Host-side interface of the large-M Q4 GEMM (mq4_gemm.hip), used by the C
// entry points of mq4_gemv.hip when M is at least kGemmMinM.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mq4_device.h"

namespace mq4 {

// Rows of x from which the entry points use the MFMA GEMM instead of the
// dot2 GEMV (which re-reads the weights once per chunk of 4 rows).
constexpr int kGemmMinM = 33;

enum GemmEpilogue { GEMM_STORE = 0, GEMM_STORE_F32 = 1, GEMM_RESIDUAL = 2, GEMM_SWIGLU = 3 };

struct GemmArgs {
    const uint16_t* x;       // [M, K] bf16
    int M, N, K;
    QMat A, B;               // B: up projection of the fused SwiGLU
    void* y;                 // [M, N] bf16 (float for GEMM_STORE_F32)
    const uint16_t* res;     // GEMM_RESIDUAL: [M, N]
    const uint16_t* norm_w;  // fused (1 + w) RMSNorm of x: [K] bf16, 16-byte aligned
    float eps;
};

// Enqueue Y = epilogue(X . W^T) on `st` (X = rms_norm(x) with norm, for the
// GEMM_STORE and GEMM_SWIGLU epilogues); 0, or -1 for an unsupported pair.
int launch_q4_gemm(const GemmArgs& a, int epi, bool norm, hipStream_t st);

}  // namespace mq4
