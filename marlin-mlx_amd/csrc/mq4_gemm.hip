// Prefill-shaped (large M) MLX-affine Q4 GEMM for gfx950: bf16 MFMA with the
// weight tiles dequantized into LDS.
//
// Replaces mx::quantized_matmul(x, w, s, b, transpose=true, 64, 4) for the
// prompt-processing call sites: qmatmul (src/model/marlin.cpp:18-25) inside
// mlp_forward (:31-35) when the hidden state holds all S prompt tokens
// (src/core/engine.cpp:64, S ~ 2,000 for a 10-frame video turn), with the
// swiglu (:27-29) and residual (:142) fused into the epilogue.
//
//   Y[M, N] = X[M, K] . W[N, K]^T,  W[n, k] = s[n, k/64] * q[n, k] + b[n, k/64]
//
// Work decomposition:
//  * A 256-thread block computes a 128 x 128 tile of Y (two 128 x 128 tiles,
//    gate and up, for the fused SwiGLU); each wave a 64 x 64 quarter as 2 x 2
//    v_mfma_f32_32x32x16_bf16 tiles with fp32 accumulators.
//  * The K loop steps one quantization group (64) at a time.  Per step every
//    thread loads 16 bytes of packed weights (32 nibbles of one row, one
//    scale and bias) and 64 bytes of activations, for the next step while the
//    current one is multiplied (register prefetch, one LDS buffer).
//  * Staging: each weight is dequantized once per tile in fp32,
//    w = fma(s, q, b), from the nibble pair (q_p, q_{p+4}) that one
//    v_and_or_b32 yields as bf16 (128 + q), and split into two bf16 parts,
//    hi = bf16(w) and lo = bf16(w - hi) (w - hi is exact in fp32): the MFMA
//    runs x.hi + x.lo, so the products carry ~2^-17 relative error instead of
//    the 2^-9 of a single bf16 weight (whose accumulated error reaches the
//    1e-2-of-RMS bound over the millions of outputs of a prefill GEMM).  The
//    activations are written in the same within-chunk order (x_p, x_{p+4}),
//    so the MFMA sums the same products over a permuted k: both operands are
//    read as 8 consecutive LDS bf16 per lane, exactly the MFMA operand layout
//    (lane l holds row l % 32, k (l / 32) * 8 .. + 7).
//  * LDS rows are padded to 72 bf16 (144 bytes) against bank conflicts.
#include "mq4_device.h"
#include "mq4_gemm.h"
#include "mq4_host.h"

namespace mq4 {

namespace gemm {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kThreads = 256;
constexpr int LDS_STRIDE = BK + 8;      // bf16 per LDS row

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// 8 bf16 in natural order -> the within-chunk order (v0, v4, v1, v5, v2, v6, v3, v7)
__device__ __forceinline__ uint4 permute_chunk(const uint4& a) {
    return make_uint4((a.x & 0xffffu) | (a.z << 16), (a.x >> 16) | (a.z & 0xffff0000u), (a.y & 0xffffu) | (a.w << 16),
                      (a.y >> 16) | (a.w & 0xffff0000u));
}

// One packed word (8 nibbles of a row) -> its 8 dequantized weights in the
// within-chunk order, pair P = (w_P, w_{P+4}), as bf16 hi and lo parts.
__device__ __forceinline__ void dequant_word(uint32_t word, float s, float b, uint4& hi, uint4& lo) {
#pragma clang fp contract(off)
    uint32_t h[4], l[4];
#pragma unroll
    for (int P = 0; P < 4; ++P) {
        const uint32_t pr = P == 0 ? nib_pair_bf16<0>(word)
                                   : P == 1 ? nib_pair_bf16<1>(word) : P == 2 ? nib_pair_bf16<2>(word) : nib_pair_bf16<3>(word);
        const float w0 = __builtin_fmaf(s, bf16_to_f32(pr & 0xffffu) - 128.0f, b);   // q exact
        const float w1 = __builtin_fmaf(s, bf16_to_f32(pr >> 16) - 128.0f, b);
        h[P] = f32x2_to_bf16x2(w0, w1);
        l[P] = f32x2_to_bf16x2(w0 - bf16_to_f32(h[P] & 0xffffu), w1 - bf16_to_f32(h[P] >> 16));
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}

template <int EPI>
__global__ __launch_bounds__(kThreads, EPI == GEMM_SWIGLU ? 1 : 2) void q4_gemm_kernel(GemmArgs p) {
    constexpr int NMAT = EPI == GEMM_SWIGLU ? 2 : 1;
    __shared__ __align__(16) uint16_t As[BM * LDS_STRIDE];
    __shared__ __align__(16) uint16_t Bs[NMAT][2][BN * LDS_STRIDE];   // [matrix][hi, lo]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;           // 2 x 2 waves of 64 x 64
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int M = p.M, N = p.N, K = p.K;
    const int KT = K / BK, G = K / 64;

    // staging roles: thread t stages row t/2, half t%2 (32 of the 64 k) of
    // both the activation tile and the weight tile(s)
    const int sr = tid >> 1, sh = tid & 1;
    const int xrow = (m0 + sr) < M ? (m0 + sr) : (M - 1);       // clamped: loads stay in bounds
    const int wrow = (n0 + sr) < N ? (n0 + sr) : (N - 1);
    const uint4* xsrc = reinterpret_cast<const uint4*>(p.x + (int64_t)xrow * K) + sh * 4;
    const QMat* mats[2] = {&p.A, &p.B};

    uint4 xr[4];
    uint4 wr[NMAT];
    uint32_t sv[NMAT], bv[NMAT];
    auto gload = [&](int kt) {
#pragma unroll
        for (int c = 0; c < 4; ++c) xr[c] = xsrc[kt * (BK / 8) + c];
#pragma unroll
        for (int t = 0; t < NMAT; ++t) {
            const QMat& Q = *mats[t];
            wr[t] = load_nt_u4(reinterpret_cast<const uint4*>(Q.wq + (int64_t)wrow * (K / 8)) + kt * 2 + sh);
            sv[t] = Q.s[(int64_t)wrow * G + kt];
            bv[t] = Q.b[(int64_t)wrow * G + kt];
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int c = 0; c < 4; ++c)
            *reinterpret_cast<uint4*>(&As[sr * LDS_STRIDE + sh * 32 + c * 8]) = permute_chunk(xr[c]);
#pragma unroll
        for (int t = 0; t < NMAT; ++t) {
            const float s = bf16_to_f32(sv[t]), b = bf16_to_f32(bv[t]);
            const uint32_t wd[4] = {wr[t].x, wr[t].y, wr[t].z, wr[t].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint4 hi, lo;
                dequant_word(wd[j], s, b, hi, lo);
                *reinterpret_cast<uint4*>(&Bs[t][0][sr * LDS_STRIDE + sh * 32 + j * 8]) = hi;
                *reinterpret_cast<uint4*>(&Bs[t][1][sr * LDS_STRIDE + sh * 32 + j * 8]) = lo;
            }
        }
    };

    f32x16_t acc[NMAT][2][2];
#pragma unroll
    for (int t = 0; t < NMAT; ++t)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[t][i][j][e] = 0.0f;

    gload(0);
    stage();
    __syncthreads();
    const int arow = wm * 64 + (lane & 31), brow = wn * 64 + (lane & 31), koff = (lane >> 5) * 8;
    for (int kt = 0; kt < KT; ++kt) {
        if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            bf16x8_t a[2], bm[NMAT][2][2];   // [matrix][hi, lo][column tile]
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const bf16x8_t*>(&As[(arow + i * 32) * LDS_STRIDE + ks * 16 + koff]);
#pragma unroll
            for (int t = 0; t < NMAT; ++t)
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        bm[t][h][j] =
                            *reinterpret_cast<const bf16x8_t*>(&Bs[t][h][(brow + j * 32) * LDS_STRIDE + ks * 16 + koff]);
#pragma unroll
            for (int t = 0; t < NMAT; ++t)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        acc[t][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bm[t][0][j], acc[t][i][j], 0, 0, 0);
                        acc[t][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bm[t][1][j], acc[t][i][j], 0, 0, 0);
                    }
        }
        if (kt + 1 < KT) {
            __syncthreads();
            stage();
            __syncthreads();
        }
    }

    // ---- epilogue: lane l of a 32 x 32 tile holds rows (e/4)*8 + (l/32)*4 + e%4, column l%32 ----
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn * 64 + j * 32 + (lane & 31);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * 64 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
                if (row >= M || col >= N) continue;
                const int64_t o = (int64_t)row * N + col;
                const float v = acc[0][i][j][e];
                if (EPI == GEMM_STORE) {
                    reinterpret_cast<uint16_t*>(p.y)[o] = (uint16_t)f32_to_bf16(v);
                } else if (EPI == GEMM_STORE_F32) {
                    reinterpret_cast<float*>(p.y)[o] = v;
                } else if (EPI == GEMM_RESIDUAL) {
                    reinterpret_cast<uint16_t*>(p.y)[o] =
                        (uint16_t)f32_to_bf16(bf16_to_f32(p.res[o]) + round_bf16(v));
                } else {
                    reinterpret_cast<uint16_t*>(p.y)[o] = (uint16_t)swiglu_bf16(v, acc[NMAT - 1][i][j][e]);
                }
            }
        }
}

}  // namespace gemm

int launch_q4_gemm(const GemmArgs& a, int epi, hipStream_t st) {
    const dim3 grid((unsigned)((a.N + gemm::BN - 1) / gemm::BN), (unsigned)((a.M + gemm::BM - 1) / gemm::BM));
    switch (epi) {
        case GEMM_STORE: hipLaunchKernelGGL(gemm::q4_gemm_kernel<GEMM_STORE>, grid, dim3(gemm::kThreads), 0, st, a); break;
        case GEMM_STORE_F32:
            hipLaunchKernelGGL(gemm::q4_gemm_kernel<GEMM_STORE_F32>, grid, dim3(gemm::kThreads), 0, st, a);
            break;
        case GEMM_RESIDUAL:
            hipLaunchKernelGGL(gemm::q4_gemm_kernel<GEMM_RESIDUAL>, grid, dim3(gemm::kThreads), 0, st, a);
            break;
        case GEMM_SWIGLU:
            hipLaunchKernelGGL(gemm::q4_gemm_kernel<GEMM_SWIGLU>, grid, dim3(gemm::kThreads), 0, st, a);
            break;
        default: return -1;
    }
    return 0;
}

}  // namespace mq4
