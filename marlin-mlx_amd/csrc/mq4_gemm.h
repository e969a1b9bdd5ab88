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
    // Non-null: x is already in the MFMA operand order (every 8-element chunk
    // as (x0, x4, x1, x5, x2, x6, x3, x7), as launch_pair_rows writes it) and
    // xsum[g * M + m] is the fp32 sum of group g of row m (group-major).
    const float* xsum;
    // GEMM_SWIGLU, non-null (with K/64 even, N % 64 == 0): y is written in
    // that same operand order and ysum[g * M + m] = the fp32 sum of group g
    // of row m of y, ready to be the x / xsum of the next product.
    float* ysum;
};

// Enqueue Y = epilogue(X . W^T) on `st` (X = rms_norm(x) with norm, for the
// GEMM_STORE and GEMM_SWIGLU epilogues); 0, or -1 for an unsupported pair
// (a.xsum set: no fused norm, K/64 even, scale/bias rows 4-byte aligned).
int launch_q4_gemm(const GemmArgs& a, int epi, bool norm, hipStream_t st);

// The fp16-weight GEMM (mq4_gemm16.hip): x holds fp16 activations in the
// operand order of launch_pair_rows16, row m scaled by 1 / (xscale[m] *
// ascale) (xscale null: 1; ascale 0: 1), and the product of row m is
// multiplied back by xscale[m] * ascale (powers of two).  Epilogues
// GEMM_RESIDUAL and GEMM_SWIGLU as GemmArgs, plus:
//  * GEMM_SWIGLU with yscale != 0: y = fp16(h * yscale) in the operand order
//    (h the bf16 SwiGLU value; saturated at +-65504), no ysum; with
//    yscale == 0 and ysum: the bf16 paired h and its group sums (N % 128 ==
//    0), as GemmArgs.
struct Gemm16Args {
    const uint16_t* x;       // [M, K] fp16, operand order
    const float* xscale;     // [M] powers of two, or null
    int M, N, K;
    QMat A, B;
    void* y;
    const uint16_t* res;
    float* ysum;
    float ascale;            // a power of two, or 0 (1)
    float yscale;            // GEMM_SWIGLU: fp16 output scale, or 0 (bf16 output)
    // GEMM_RESIDUAL in 1 < ksplit <= 4 K parts (K / 64 a multiple of 8 ksplit):
    // part[k][M][N] fp32 (16-byte aligned, N % 4 == 0), then a second kernel
    // adds the parts in order and the residual (res and y 8-byte aligned)
    int ksplit;
    float* part;
    // GEMM_RESIDUAL: nonzero for blocks of 128 weight columns (one 32-column
    // MFMA tile per wave, three blocks per CU) instead of 256; the same bits
    int narrow;
    // GEMM_SWIGLU: the 4096-entry SiLU table of silu_lut_entry (16-byte
    // aligned; launch_pair_rows16 writes it)
    const uint16_t* silu_lut;
};

// Enqueue the fp16-weight GEMM (GEMM_SWIGLU or GEMM_RESIDUAL, the products of
// mq4_mlp_residual); 0, or -1 for another epilogue or shapes it does not take
// (K % 512 != 0, scales or biases not 16-byte aligned, byte offsets past 32
// bits).
int launch_q4_gemm16(const Gemm16Args& a, int epi, hipStream_t st);

// xp = fp16(x / xscale[m]) (norm_w null) or fp16(bf16(x * rsqrt(mean(x^2) +
// eps) * (1 + norm_w)) / xscale[m]) in the operand order (the bits of
// mq4_rms_norm before the conversion), with xscale[m] = 2^e, e >= 0 the
// smallest that keeps the row below 2^15.  K % 512 == 0; x, xp, norm_w
// 16-byte aligned.  silu_lut non-null: the same launch also writes the
// SiLU table of GEMM_SWIGLU (SILU_LUT_N entries).
int launch_pair_rows16(const uint16_t* x, int M, int K, const uint16_t* norm_w, float eps, uint16_t* xp,
                       float* xscale, uint16_t* silu_lut, hipStream_t st);

// xp = x (norm_w null) or bf16(x * rsqrt(mean(x^2) + eps) * (1 + norm_w)),
// the bits of mq4_rms_norm, with every 8-element chunk of a row in the
// pair order above, and xs[g * M + m] = the fp32 sum of group g of row m
// of xp (group-major).  K % 512 == 0; x, xp, norm_w 16-byte aligned.
int launch_pair_rows(const uint16_t* x, int M, int K, const uint16_t* norm_w, float eps, uint16_t* xp, float* xs,
                     hipStream_t st);

}  // namespace mq4
