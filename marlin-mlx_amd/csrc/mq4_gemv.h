// Host-side interface shared by the small-M kernel families: the dot2 GEMV
// (mq4_gemv.hip) and the MFMA batched-decode GEMV (mq4_mfma.hip).  The C
// entry points of mq4_gemv.hip pick the family from M.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mq4_device.h"

namespace mq4 {

enum Epilogue {
    EPI_STORE = 0,
    EPI_RESIDUAL = 1,
    EPI_SWIGLU = 2,
    EPI_ARGMAX = 3,
    EPI_STORE_F32 = 4,
    EPI_PARTIAL = 5,   // MFMA GEMV, K split over blockIdx.y: fp32 sum of the block's part to y[part][M][N]
};

constexpr int kPartialStride = 4096;     // max blocks of an argmax launch

struct GemvParams {
    const uint16_t* x;       // [m_valid, K]
    int m_valid;
    int N, K;
    QMat A, B;               // B: up projection of the fused gate/up kernel
    uint16_t* y;             // [m_valid, N] (float for EPI_STORE_F32; may be null for ARGMAX)
    const uint16_t* res;     // EPI_RESIDUAL: [m_valid, N]
    const uint16_t* norm_w;  // NORM: [K] (1 + w) RMSNorm weight
    float eps;
    uint64_t* partial;       // EPI_ARGMAX: [m_valid, kPartialStride] per-block best keys
    uint32_t* idx;           // EPI_ARGMAX: [m_valid]
};

// Rows of x from which the entry points use the MFMA batched-decode GEMV
// (every weight byte read once for up to kMfmaMaxM rows) instead of the dot2
// GEMV, which reads the weights once per chunk of 4 rows and is faster up to
// 4 rows (measured on MI355X at the model's shapes); the MFMA GEMM takes over
// from kGemmMinM (mq4_gemm.h).
constexpr int kMfmaMinM = 5;
constexpr int kMfmaMaxM = 32;

// Enqueue the MFMA GEMV for 1 <= a.m_valid <= kMfmaMaxM; returns 0, or -1 if
// this K / epilogue combination is not provided (the caller then uses the
// dot2 GEMV).
int launch_q4_mfma_gemv(const GemvParams& a, int epi, bool norm, hipStream_t st);

// The down product of a small-M MLP with its K range split over two blocks
// per 16-row tile (each block half the activations, all CUs busy): enqueues
// the fp32 sums of the two K parts into part [2][M][N] and returns 0, or -1
// when the product is not one the 12-wave MFMA GEMV would run (64 < K/64 <=
// 96, M <= kMfmaMaxM).  Each part is the in-block sum of 6 waves in wave
// order; launch_combine2_residual adds the two parts, which is exactly the
// 12-wave kernel's reduction, so the result is bit-identical to it.
int launch_q4_mfma_gemv_split2(const GemvParams& a, float* part, hipStream_t st);

// y = bf16(bf16(res) + round_bf16(part[0] + part[1])) over M x N values (the
// residual epilogue of the MFMA GEMV applied to the two K parts).
void launch_combine2_residual(const float* part, int M, int N, const uint16_t* res, uint16_t* y, hipStream_t st);

// The lm_head + argmax (EPI_ARGMAX, K = 2048, 1 <= m_valid <= kMfmaMaxM)
// with a ring of weight tiles in flight per CU (mq4_lmring.hip): for 1-2
// rows the dot2 GEMV's arithmetic, from 3 rows the MFMA GEMV's, each
// bit-identical to that kernel's logits and tokens.  Enqueues it and the
// argmax finalize and returns 0, or -1 for shapes and alignments it does not
// take (x, wq and the norm weight 16-byte, scales and biases 4-byte aligned).
int launch_lm_ring(const GemvParams& a, bool norm, hipStream_t st);

// idx[m] = argmax of the per-block keys partial[m * kPartialStride + 0 .. count).
void launch_argmax_finalize(const uint64_t* partial, int count, int M, uint32_t* idx, hipStream_t st);

// Compute units of the current device (cached).
int num_cus();

}  // namespace mq4
