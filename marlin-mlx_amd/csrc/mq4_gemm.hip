// Prefill-shaped (large M) MLX-affine Q4 GEMM for gfx950: bf16 MFMA on the
// exact nibbles, the affine scale and offset applied per group in fp32.
//
// Replaces mx::quantized_matmul(x, w, s, b, transpose=true, 64, 4) for the
// prompt-processing call sites: qmatmul (src/model/marlin.cpp:18-25) inside
// mlp_forward (:31-35) when the hidden state holds all S prompt tokens
// (src/core/engine.cpp:64, S ~ 2,000 for a 10-frame video turn), with the
// rms_norm in front (:141, :12-16), the swiglu (:27-29) and the residual
// (:142) fused in.
//
//   Y[M, N] = X[M, K] . W[N, K]^T,  W[n, k] = s[n, g] * q[n, k] + b[n, g],  g = k / 64
//
// Per group g the MFMA forms D[m, n] = sum_{k in g} x[m, k] * (128 + q[n, k])
// with both operands exact in bf16 (128 + q is an 8-bit integer, one
// v_and_or_b32 from two nibbles) and exact products, and the group is folded
// into the fp32 accumulator as
//   acc += s * D + (b - 128 s) * X[m, g],   X[m, g] = sum_{k in g} x[m, k],
// so each weight is used once, untransformed, and the only rounding is the
// fp32 accumulation (the affine form the GEMV kernels use per 32-element slice).
//
// Work decomposition:
//  * A 256-thread block computes 128 rows x 128 weight columns (one matrix,
//    128 output columns; or gate and up, 64 output columns each, for the
//    fused SwiGLU); each wave 64 rows x 64 weight columns as 2 x 2
//    v_mfma_f32_32x32x16_bf16 tiles, with a per-group accumulator D beside
//    the running fp32 result.
//  * Weights go straight from global memory to registers in the MFMA operand
//    layout: lane l of a tile holds weight row l % 32 and, per group, the four
//    packed words of its k-half l / 32 (one 16-byte load).  MFMA step ks uses
//    word ks of each half, so the k-slots of step ks are the 8-element chunks
//    ks and 4 + ks of the group; the sum over the group is the same.
//  * Activations go through LDS, double-buffered, one barrier per group: each
//    thread stages 32 values of one row (register prefetch one group ahead),
//    writing them in the nibble-pair order (x_p, x_{p+4}) of the weights and
//    their sum X.  With the fused RMSNorm each staging thread first reads its
//    half of the row once for the sum of squares (the pair of threads of a
//    row combine their halves), then stages bf16(x * r * (1 + w)) with the
//    same per-element formula as the separate norm kernel, so the operand
//    holds the bf16 values the reference's rms_norm produces.  (Scaling the
//    result by r after the product instead would move that rounding: about one
//    bf16 ulp of the pre-activation, which the SwiGLU amplifies at its largest
//    outputs.)
//  * XCD-aware block order: when the column blocks divide evenly over the 8
//    XCDs, each XCD takes a fixed eighth of the column blocks for every row
//    block, so its weights stay in its own L2 across the row blocks.
//  * LDS rows are padded to 72 bf16 (144 bytes) against bank conflicts.
#include <type_traits>

#include "mq4_device.h"
#include "mq4_gemm.h"
#include "mq4_gemv.h"
#include "mq4_host.h"

namespace mq4 {

namespace gemm {

constexpr int BM = 128;
constexpr int kThreads = 256;
constexpr int LDS_STRIDE = 72;          // bf16 per LDS row (64 activations + 8 pad)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// This file is built with MFMA results and accumulators in VGPRs
// (-amdgpu-mfma-vgpr-form), so the per-group fold reads the MFMA result D
// directly on the VALU.  The compiler pads each v_mfma_f32_32x32x16_bf16 ->
// VALU read with 11 wait states, which measured too few on gfx950 (the sums
// came out wrong); 24 more, once per group between the group's last MFMA and
// its fold, give the right sums at no measurable cost.  The scheduling
// barriers keep the padding between the two.
__device__ __forceinline__ void mfma_result_pad() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
    __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ bf16x8_t weight_operand(uint32_t word) {
    const uint4 q = make_uint4(nib_pair_bf16<0>(word), nib_pair_bf16<1>(word), nib_pair_bf16<2>(word),
                               nib_pair_bf16<3>(word));
    return __builtin_bit_cast(bf16x8_t, q);
}

// weight_operand with the mask (SGPR) and exponent bits (VGPR) held by the
// caller: one v_and_or_b32 per nibble pair plus a shift for pairs 1-3.
__device__ __forceinline__ uint32_t nib_pair_k(uint32_t s, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(s), "s"(m), "v"(c));
    return r;
}
__device__ __forceinline__ bf16x8_t weight_operand_k(uint32_t word, uint32_t m, uint32_t c) {
    const uint4 q = make_uint4(nib_pair_k(word, m, c), nib_pair_k(word >> 4, m, c), nib_pair_k(word >> 8, m, c),
                               nib_pair_k(word >> 12, m, c));
    return __builtin_bit_cast(bf16x8_t, q);
}

__device__ __forceinline__ uint32_t word_of(const uint4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

template <int EPI, bool NORM>
__global__ __launch_bounds__(kThreads, 2) void q4_gemm_kernel(GemmArgs p) {
#pragma clang fp contract(off)
    constexpr int NMAT = EPI == GEMM_SWIGLU ? 2 : 1;
    constexpr int BN = 128 / NMAT;                      // output columns per block
    __shared__ __align__(16) uint16_t As[2][BM * LDS_STRIDE];
    __shared__ __align__(16) float Xs[2][BM];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;            // 2 x 2 waves of 64 rows x 64 weight columns
    const int M = p.M, N = p.N, K = p.K, G = K / 64;

    // block -> (column block, row block)
    const int NB = (N + BN - 1) / BN, MB = (M + BM - 1) / BM;
    int nb, mb;
    {
        const int b = blockIdx.x;
        if ((NB & 7) == 0) {
            const int per = NB >> 3, s = b >> 3;
            nb = (s % per) * 8 + (b & 7);
            mb = s / per;
        } else {
            nb = b % NB;
            mb = b / NB;
        }
    }
    const int n0 = nb * BN, m0 = mb * BM;
    (void)MB;

    // ---- activation staging: thread t holds row t/2, k-half t%2 of each group ----
    const int sr = tid >> 1, sh = tid & 1;
    const int xrow = (m0 + sr) < M ? (m0 + sr) : (M - 1);       // clamped: loads stay in bounds
    const uint4* xsrc = reinterpret_cast<const uint4*>(p.x + (int64_t)xrow * K) + sh * 4;
    const uint4* nwsrc = reinterpret_cast<const uint4*>(NORM ? p.norm_w : p.x) + sh * 4;

    // ---- weight operand: tile j, lane l -> weight row, k-half h = l / 32 ----
    const int h = lane >> 5, col = lane & 31;
    const uint4* bsrc[2];
    const uint16_t* ssrc[2];
    const uint16_t* bbsrc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const QMat& Q = (NMAT == 2 && j == 1) ? p.B : p.A;
        int wrow = NMAT == 2 ? n0 + wn * 32 + col : n0 + wn * 64 + j * 32 + col;
        wrow = wrow < N ? wrow : N - 1;
        bsrc[j] = reinterpret_cast<const uint4*>(Q.wq + (int64_t)wrow * (K / 8)) + h;   // + 2g per group
        ssrc[j] = Q.s + (int64_t)wrow * G;
        bbsrc[j] = Q.b + (int64_t)wrow * G;
    }

    uint4 xr[4], nr[4];
    uint4 wnext[2], wcur[2];
    uint32_t snext[2], bnext[2], scur[2], bcur[2];
    auto gload = [&](int g) {
#pragma unroll
        for (int c = 0; c < 4; ++c) xr[c] = xsrc[g * 8 + c];
        if (NORM) {
#pragma unroll
            for (int c = 0; c < 4; ++c) nr[c] = nwsrc[g * 8 + c];
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            wnext[j] = load_nt_u4(bsrc[j] + 2 * g);
            snext[j] = ssrc[j][g];
            bnext[j] = bbsrc[j][g];
        }
    };
    float rrow = 0.0f;                                  // 1 / rms of the staged row (fused norm)
    if (NORM) {
        float ss = 0.0f;
#pragma unroll 4
        for (int c = 0; c < 4 * G; ++c) {
            const uint4 v = xsrc[(c >> 2) * 8 + (c & 3)];
            ss = sumsq_word(ss, v.x);
            ss = sumsq_word(ss, v.y);
            ss = sumsq_word(ss, v.z);
            ss = sumsq_word(ss, v.w);
        }
        rrow = rms_inv(ss + __shfl_xor(ss, 1), K, p.eps);
    }
    auto stage = [&](int buf) {
        float xsum = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            uint4 a = xr[c];
            if (NORM)
                a = make_uint4(norm_word(a.x, nr[c].x, rrow), norm_word(a.y, nr[c].y, rrow),
                               norm_word(a.z, nr[c].z, rrow), norm_word(a.w, nr[c].w, rrow));
            uint32_t pr[4];
            xsum = pair_chunk(a, pr, xsum);
            *reinterpret_cast<uint4*>(&As[buf][sr * LDS_STRIDE + sh * 32 + c * 8]) =
                make_uint4(pr[0], pr[1], pr[2], pr[3]);
        }
        xsum += __shfl_xor(xsum, 1);                    // both halves of the row
        if (sh == 0) Xs[buf][sr] = xsum;
    };

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    const f32x16_t zero = acc[0][0];

    gload(0);
    stage(0);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        wcur[j] = wnext[j];
        scur[j] = snext[j];
        bcur[j] = bnext[j];
    }
    __syncthreads();
    const int arow = wm * 64 + col;
    for (int g = 0; g < G; ++g) {
        const int buf = g & 1;
        if (g + 1 < G) gload(g + 1);
        f32x16_t D[2][2];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            bf16x8_t a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const bf16x8_t*>(&As[buf][(arow + i * 32) * LDS_STRIDE + (4 * h + ks) * 8]);
#pragma unroll
            for (int j = 0; j < 2; ++j) b[j] = weight_operand(word_of(wcur[j], ks));
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    D[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], ks == 0 ? zero : D[i][j], 0, 0, 0);
        }
        mfma_result_pad();
        // fold the group: acc += s * D + (b - 128 s) * X
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float s = bf16_to_f32(scur[j]);
            const float c = affine_c(s, bcur[j]);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 X = *reinterpret_cast<const float4*>(&Xs[buf][wm * 64 + i * 32 + q * 8 + h * 4]);
                    const float xv[4] = {X.x, X.y, X.z, X.w};
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int e = q * 4 + r;
                        acc[i][j][e] = __builtin_fmaf(s, D[i][j][e], __builtin_fmaf(c, xv[r], acc[i][j][e]));
                    }
                }
            }
        }
        if (g + 1 < G) {
            stage(buf ^ 1);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                wcur[j] = wnext[j];
                scur[j] = snext[j];
                bcur[j] = bnext[j];
            }
        }
        __syncthreads();
    }

    // ---- epilogue: lane l of a 32 x 32 tile holds rows (e/4)*8 + (l/32)*4 + e%4, column l%32 ----
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < (NMAT == 2 ? 1 : 2); ++j) {
            const int cn = NMAT == 2 ? n0 + wn * 32 + col : n0 + wn * 64 + j * 32 + col;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int rl = wm * 64 + i * 32 + (e >> 2) * 8 + h * 4 + (e & 3);
                const int row = m0 + rl;
                if (row >= M || cn >= N) continue;
                const int64_t o = (int64_t)row * N + cn;
                const float v = acc[i][j][e];
                if (EPI == GEMM_STORE) {
                    reinterpret_cast<uint16_t*>(p.y)[o] = (uint16_t)f32_to_bf16(v);
                } else if (EPI == GEMM_STORE_F32) {
                    reinterpret_cast<float*>(p.y)[o] = v;
                } else if (EPI == GEMM_RESIDUAL) {
                    reinterpret_cast<uint16_t*>(p.y)[o] =
                        (uint16_t)f32_to_bf16(bf16_to_f32(p.res[o]) + round_bf16(v));
                } else {
                    reinterpret_cast<uint16_t*>(p.y)[o] = (uint16_t)swiglu_bf16(v, acc[i][1][e]);
                }
            }
        }
}

// ---------------------------------------------------------------------------
// The same product with every operand staged by LDS DMA (global_load_lds)
// through a ring of S = 2 (or 3) stages, for the epilogues without the fused norm.  A block
// is WM x WN waves of 64 rows x 64 weight columns each (BM = 64 WM rows,
// BNW = 64 WN weight columns):
//  * per group, BM x 64 activations (each row's eight 16-byte chunks
//    XOR-swizzled by (row / 2) % 8: with 64 LDS banks the 16 lanes of one
//    ds_read_b128 phase, 16 consecutive rows at one chunk, cover all banks
//    once), BNW x 32 bytes of packed weights (stored k-half major,
//    [half][row], so a phase reads 256 contiguous bytes) and the rows' scales
//    and biases (a 4-byte DMA per row holding groups g & ~1 and g | 1, so the
//    group count must be even and scales/biases 4-byte aligned; other shapes
//    take the register-staged kernel above), issued two groups ahead of use
//    and waited for with an exact vmcnt (nothing else in the loop touches
//    vector memory);
//  * the DMA targets of all stages must lie in the first 64 KiB of the
//    workgroup's LDS (static_assert below);
//  * barriers carry no memory fence (a fence would wait for the DMA in
//    flight), and each ring stage is a separate LDS object, so the compiler
//    sees that reading one stage does not depend on the DMA into another;
//  * X, the group sums of the activations, come from the MFMA operand
//    fragments already in registers (each lane holds half a row per group,
//    v_dot2 with ones, the other half from lane l ^ 32), and the (b - 128 s) X
//    half of the fold runs on the fp32 MFMA (v_mfma_f32_32x32x2_f32, two
//    groups per instruction: its A operand is X of the lane's row, its B
//    operand the lane's column offset), so the VALU fold is acc += s * D only.
namespace dma {


// LDS DMA of 16 (4) bytes per lane from global src to lds + 16 (4) * lane.
// (Plain functions: inside a kernel template, a direct call of the builtin
// keeps the host pass from emitting the kernel's launch stub.)
__device__ __forceinline__ void lds_dma16(const void* src, void* lds) {
    __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
}
__device__ __forceinline__ void lds_dma4(const void* src, void* lds) {
    __builtin_amdgcn_global_load_lds(src, lds, 4, 0, 0);
}

template <int WM, int WN, bool PRE, int TJ>
struct Stage {
    static constexpr int BM = 64 * WM, BNW = 32 * TJ * WN;
    uint4 a[BM * 8];                      // [row][chunk ^ ((row >> 1) & 7)]
    uint4 b[2 * BNW];                     // [k-half][weight row]
    uint32_t sb[2][BNW];                  // scales, biases: groups (g & ~1, g | 1)
    float xs[PRE ? BM : 1];               // PRE: the rows' group sums X
};

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// v_perm_b32 selectors: (lo half of x, lo half of z) and (hi of x, hi of z)
constexpr uint32_t kPermLo = 0x05040100u, kPermHi = 0x07060302u;

template <int EPI, int WM, int WN, int S, bool PRE, int TJ>
__global__ __launch_bounds__(64 * WM * WN, 2) void q4_gemm_dma_kernel(GemmArgs p) {
#pragma clang fp contract(off)
    constexpr int NMAT = EPI == GEMM_SWIGLU ? 2 : 1;
    // TJ 32-column weight tiles per wave (2: 64 x 64 outputs; 1: 64 x 32,
    // twice the waves for a product too small to give every SIMD two; the
    // fused SwiGLU pairs gate and up tiles, so it takes 2)
    static_assert(TJ == 2 || (TJ == 1 && NMAT == 1), "wave tile");
    constexpr int NW = WM * WN;
    constexpr int TBM = 64 * WM, BNW = 32 * TJ * WN, BN = BNW / NMAT;
    constexpr int A_I = TBM * 8 / (64 * NW);            // activation DMA instructions per wave and group
    // weight and scale/bias tiles: B_TOT instructions per block, issued by the
    // first waves (with S = 2 every step waits for all of a wave's DMA, so
    // the per-wave counts need not match)
    constexpr int B_TOT = 2 * BNW / 64;
    constexpr int B_I = (B_TOT + NW - 1) / NW;          // weight
    constexpr int SB_I = B_I;                           // scale/bias
    static_assert(B_TOT % NW == 0 || S == 2, "uneven DMA split needs the 2-stage ring");
    // PRE: the rows' group sums travel with the tile, 64 rows per DMA
    // instruction, issued by the first TBM / 64 waves (with S = 2 every step
    // waits for all of a wave's DMA, so the counts need not match)
    constexpr int X_I = PRE ? 1 : 0;
    static_assert(!PRE || (S == 2 && TBM / 64 <= NW), "group-sum DMA");
    constexpr int kDmaPerWave = A_I + B_I + SB_I + X_I;
    static_assert(A_I * 64 * NW == TBM * 8, "DMA split");
    typedef Stage<WM, WN, PRE, TJ> St;
    static_assert(S == 2 || S == 3, "ring stages");
    static_assert((size_t)S * sizeof(St) <= 65536, "LDS DMA targets must lie in the first 64 KiB");
    typedef typename std::conditional<S == 3, St, char>::type St2;   // no third stage with S = 2
    __shared__ St st0, st1;
    __shared__ St2 st2;

    const int tid = threadIdx.x, lane = tid & 63;
    // the wave index is uniform: kept in scalar registers, as is everything
    // derived from it below (DMA bases and LDS destinations)
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int h = lane >> 5, col = lane & 31;
    const int M = p.M, N = p.N, K = p.K, G = K / 64;

    const int NB = (N + BN - 1) / BN;
    int nb, mb;
    {
        const int b = blockIdx.x;
        if ((NB & 7) == 0) {
            const int per = NB >> 3, s = b >> 3;
            nb = (s % per) * 8 + (b & 7);
            mb = s / per;
        } else {
            nb = b % NB;
            mb = b / NB;
        }
    }
    const int n0 = nb * BN, m0 = mb * TBM;

    // ---- DMA sources: per instruction a wave-uniform base (scalar
    // registers; group g moves it along K) plus a 32-bit byte offset per
    // lane (the host takes this kernel only when every offset fits) ----
    const char* const xbase = reinterpret_cast<const char*>(p.x);
    uint32_t aoff[A_I];
#pragma unroll
    for (int t = 0; t < A_I; ++t) {
        const int slot = (wave * A_I + t) * 64 + lane;
        const int r = slot >> 3, c = (slot & 7) ^ ((r >> 1) & 7);
        const int row = (m0 + r) < M ? (m0 + r) : (M - 1);
        aoff[t] = (uint32_t)(((int64_t)row * K + c * 8) * 2);
    }
    // weight row r of the block -> matrix and output row; the 64 slots of
    // one DMA instruction lie in one matrix and one k-half
    static_assert(NMAT == 1 || (BNW / 2) % 64 == 0, "one matrix per DMA instruction");
    auto wrow_of = [&](int r) -> int {
        const int n = NMAT == 2 ? n0 + (r % (BNW / 2)) : n0 + r;
        return n < N ? n : N - 1;
    };
    auto mat_of = [&](int r) -> const QMat& { return (NMAT == 2 && r >= BNW / 2) ? p.B : p.A; };
    const char* bbase[B_I];
    uint32_t boff[B_I];
#pragma unroll
    for (int t = 0; t < B_I; ++t) {
        const int q0 = ((wave * B_I + t) % B_TOT) * 64, half = q0 / BNW, r0 = q0 % BNW;
        bbase[t] = reinterpret_cast<const char*>(mat_of(r0).wq) + half * 16;
        boff[t] = (uint32_t)((int64_t)wrow_of(r0 + lane) * (K / 2));
    }
    const char* sbbase[SB_I];
    uint32_t sboff[SB_I];
#pragma unroll
    for (int t = 0; t < SB_I; ++t) {
        const int u0 = ((wave * SB_I + t) % B_TOT) * 64, sel = u0 / BNW, r0 = u0 % BNW;
        sbbase[t] = reinterpret_cast<const char*>(sel ? mat_of(r0).b : mat_of(r0).s);
        sboff[t] = (uint32_t)((int64_t)wrow_of(r0 + lane) * G * 2);
    }
    // PRE: group sum of row m0 + 64 wave + lane, group g (clamped row); the
    // sums are group-major, so one instruction reads 256 contiguous bytes
    const char* const xsbase = reinterpret_cast<const char*>(p.xsum);
    uint32_t xsoff = 0;
    if constexpr (PRE) {
        const int r = m0 + 64 * wave + lane;
        xsoff = (uint32_t)((r < M ? r : M - 1) * 4);
    }
    auto issue = [&](int g, St& st) {
        if constexpr (PRE) {
            if (wave < TBM / 64) lds_dma4(xsbase + (int64_t)g * M * 4 + xsoff, &st.xs[64 * wave]);
        }
#pragma unroll
        for (int t = 0; t < A_I; ++t)
            lds_dma16(xbase + g * 128 + aoff[t], &st.a[(wave * A_I + t) * 64]);
#pragma unroll
        for (int t = 0; t < B_I; ++t)
            if (B_TOT % NW == 0 || wave * B_I + t < B_TOT)
                lds_dma16(bbase[t] + g * 32 + boff[t], &st.b[(wave * B_I + t) * 64]);
#pragma unroll
        for (int t = 0; t < SB_I; ++t)
            if (B_TOT % NW == 0 || wave * SB_I + t < B_TOT)
                lds_dma4(sbbase[t] + (g & ~1) * 2 + sboff[t], &st.sb[0][(wave * SB_I + t) * 64]);
    };

    // ---- compute roles: weight row of tile j for this lane ----
    int wr[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) wr[j] = NMAT == 2 ? j * (BNW / 2) + wn * 32 + col : wn * 32 * TJ + j * 32 + col;
    const uint32_t ONES = 0x3f803f80u;        // bf16 pair (1, 1)
    uint32_t nib_mask, nib_exp;               // the nibble-pair constants, set up once
    asm("s_mov_b32 %0, 0x000f000f" : "=s"(nib_mask));
    asm("v_mov_b32 %0, 0x43004300" : "=v"(nib_exp));

    f32x16_t acc[2][TJ];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    const f32x16_t zero = acc[0][0];
    float xprev[2] = {0.0f, 0.0f}, cprev[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) cprev[j] = 0.0f;

    auto compute = [&](int g, const St& st) {
        uint4 bw[TJ];
        float s[TJ], c[TJ];
        const int sh16 = (g & 1) * 16;
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            bw[j] = st.b[h * BNW + wr[j]];
            s[j] = bf16_to_f32((st.sb[0][wr[j]] >> sh16) & 0xffffu);
            c[j] = affine_c(s[j], (st.sb[1][wr[j]] >> sh16) & 0xffffu);
        }
        f32x16_t D[2][TJ];
        float xs[2] = {0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            bf16x8_t a[2], b[TJ];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = wm * 64 + i * 32 + col, ch = 4 * h + ks;
                const uint4 raw = st.a[r * 8 + (ch ^ ((r >> 1) & 7))];
                if constexpr (PRE) {
                    a[i] = __builtin_bit_cast(bf16x8_t, raw);          // already in pair order
                } else {
                    xs[i] = dot2_bf16(raw.w, ONES, dot2_bf16(raw.z, ONES, dot2_bf16(raw.y, ONES, dot2_bf16(raw.x, ONES, xs[i]))));
                    // nibble-pair order (x0, x4), (x1, x5), (x2, x6), (x3, x7)
                    const uint4 pr = make_uint4(__builtin_amdgcn_perm(raw.z, raw.x, kPermLo),
                                                __builtin_amdgcn_perm(raw.z, raw.x, kPermHi),
                                                __builtin_amdgcn_perm(raw.w, raw.y, kPermLo),
                                                __builtin_amdgcn_perm(raw.w, raw.y, kPermHi));
                    a[i] = __builtin_bit_cast(bf16x8_t, pr);
                }
            }
#pragma unroll
            for (int j = 0; j < TJ; ++j) b[j] = weight_operand_k(word_of(bw[j], ks), nib_mask, nib_exp);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    D[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], ks == 0 ? zero : D[i][j], 0, 0, 0);
        }
        mfma_result_pad();
        float X[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if constexpr (PRE) X[i] = st.xs[wm * 64 + i * 32 + col];
            else X[i] = xs[i] + __shfl_xor(xs[i], 32);
        }
        // acc += s * D (VALU) ...
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = __builtin_fmaf(s[j], D[i][j][e], acc[i][j][e]);
        // ... and + (b - 128 s) X on the fp32 MFMA, two groups per instruction:
        // lanes 0-31 carry the earlier group, lanes 32-63 the later one
        if ((g & 1) == 0 && g + 1 < G) {
#pragma unroll
            for (int i = 0; i < 2; ++i) xprev[i] = X[i];
#pragma unroll
            for (int j = 0; j < TJ; ++j) cprev[j] = c[j];
        } else {
            const bool solo = (g & 1) == 0;          // the last group of an odd count
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j) {
                    const float xa = h ? (solo ? 0.0f : X[i]) : (solo ? X[i] : xprev[i]);
                    const float cb = h ? (solo ? 0.0f : c[j]) : (solo ? c[j] : cprev[j]);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(xa, cb, acc[i][j], 0, 0, 0);
                }
        }
    };
    // Every step issues one group's DMA (past the end: the last group again,
    // into a stage nobody reads), so exactly kDmaPerWave instructions follow
    // group g's in each wave when step g waits, and one unconditional vmcnt
    // serves every step.
    auto step = [&](int g, const St& cur, St& nxt) {
        wait_vmcnt<kDmaPerWave * (S - 2)>();
        lds_barrier();                               // group g is in `cur` for every wave
        issue(g + S - 1 < G ? g + S - 1 : G - 1, nxt);   // into the stage read in step g - 1
        compute(g, cur);
    };

    issue(0, st0);
    if constexpr (S == 3) issue(G > 1 ? 1 : 0, st1);
    // whole rounds of S steps without branches inside (a conditional step
    // would merge DMA states and make the compiler wait for all of them),
    // then the G % S remaining steps
    int g0 = 0;
    if constexpr (S == 3) {
        for (; g0 + S <= G; g0 += S) {
            step(g0, st0, st2);
            step(g0 + 1, st1, st0);
            step(g0 + 2, st2, st1);
        }
        if (g0 < G) step(g0, st0, st2);
        if (g0 + 1 < G) step(g0 + 1, st1, st0);
    } else {
        for (; g0 + S <= G; g0 += S) {
            step(g0, st0, st1);
            step(g0 + 1, st1, st0);
        }
        if (g0 < G) step(g0, st0, st1);
    }
    wait_vmcnt<0>();                                 // no DMA outstanding past the loop

    // ---- epilogue: lane l of a 32 x 32 tile holds rows (e/4)*8 + (l/32)*4 + e%4, column l%32 ----
    // SwiGLU with ysum: the block's BN = 64 output columns are one group of y;
    // y goes out in the operand order (column c of a chunk at 2 (c % 4) + c / 4)
    // and the group sums of its rows through LDS (ring stage 0, free now)
    const bool paired_out = EPI == GEMM_SWIGLU && p.ysum != nullptr;
    uint16_t* tile = reinterpret_cast<uint16_t*>(&st0);          // [TBM][72] bf16
    static_assert(TBM * 72 * 2 <= (int)sizeof(St), "epilogue tile");
    if (paired_out) __syncthreads();                               // every wave is done with the ring
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < (NMAT == 2 ? 1 : TJ); ++j) {
            const int cn = NMAT == 2 ? n0 + wn * 32 + col : n0 + wn * 32 * TJ + j * 32 + col;
            const int cw = paired_out ? ((cn & ~7) | (2 * (cn & 3) + ((cn >> 2) & 1))) : cn;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int rl = wm * 64 + i * 32 + (e >> 2) * 8 + h * 4 + (e & 3);
                const int row = m0 + rl;
                if (EPI == GEMM_SWIGLU) {
                    const uint32_t v = swiglu_bf16(acc[i][0][e], acc[i][1][e]);
                    if (paired_out) tile[rl * 72 + wn * 32 + col] = (uint16_t)v;
                    if (row < M && cn < N) reinterpret_cast<uint16_t*>(p.y)[(int64_t)row * N + cw] = (uint16_t)v;
                    continue;
                }
                if (row >= M || cn >= N) continue;
                const int64_t o = (int64_t)row * N + cn;
                const float v = acc[i][j][e];
                if (EPI == GEMM_STORE) {
                    reinterpret_cast<uint16_t*>(p.y)[o] = (uint16_t)f32_to_bf16(v);
                } else if (EPI == GEMM_STORE_F32) {
                    reinterpret_cast<float*>(p.y)[o] = v;
                } else {
                    reinterpret_cast<uint16_t*>(p.y)[o] =
                        (uint16_t)f32_to_bf16(bf16_to_f32(p.res[o]) + round_bf16(v));
                }
            }
        }
    if (paired_out) {
        __syncthreads();
        // thread t: half t % 2 of row t / 2 of the tile (32 values), summed
        // left to right, then the two halves
        static_assert(64 * NW == 2 * TBM, "two threads per row");
        const int rl = threadIdx.x >> 1, half = threadIdx.x & 1;
        float sum = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint4 v = *reinterpret_cast<const uint4*>(&tile[rl * 72 + half * 32 + c * 8]);
            const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                sum += bf16_to_f32(w4[q] & 0xffffu);
                sum += bf16_to_f32(w4[q] >> 16);
            }
        }
        sum += __shfl_xor(sum, 1);
        if (half == 0 && m0 + rl < M) p.ysum[(int64_t)(n0 >> 6) * M + m0 + rl] = sum;
    }
}

// Blocks of the (WM, WN, TJ) layout for an M x N product.
template <int EPI, int WM, int WN, int TJ>
unsigned blocks_of(int M, int N) {
    constexpr int BN = 32 * TJ * WN / (EPI == GEMM_SWIGLU ? 2 : 1);
    return (unsigned)(((N + BN - 1) / BN) * ((M + 64 * WM - 1) / (64 * WM)));
}

template <int EPI, int WM, int WN, int S, bool PRE, int TJ>
void launch_dma(const GemmArgs& a, hipStream_t st) {
    hipLaunchKernelGGL((q4_gemm_dma_kernel<EPI, WM, WN, S, PRE, TJ>), dim3(blocks_of<EPI, WM, WN, TJ>(a.M, a.N)),
                       dim3(64 * WM * WN), 0, st, a);
}

// The layout used for every shape: 2 x 2 waves, 2 stages.  Measured on
// MI355X at M = 1960 / 2048 / 8192 against 1 x 2, 1 x 4 and 2 x 2 with 3
// stages it is as fast or faster for both the gate/up (N = 6144) and the
// down (N = 2048) products, with the least LDS (41 KB, so two blocks per CU).
template <int EPI>
void launch_dma_auto(const GemmArgs& a, hipStream_t st) {
    if (a.xsum) {
        // paired operands: no activation work per wave, so 64 x 32 wave tiles
        // cost the same VALU per MFMA as 64 x 64; when 64 x 64 would leave one
        // block per CU (the down product at M ~ 2,000: 256 blocks), they
        // double the blocks (126 VGPRs, 4 waves per SIMD): 243-248 against
        // 257-258 us for the whole MLP half at M = 2048
        if constexpr (EPI != GEMM_SWIGLU) {
            if (blocks_of<EPI, 2, 2, 2>(a.M, a.N) <= (unsigned)num_cus()) {
                launch_dma<EPI, 2, 2, 2, true, 1>(a, st);
                return;
            }
        }
        launch_dma<EPI, 2, 2, 2, true, 2>(a, st);
    } else {
        launch_dma<EPI, 2, 2, 2, false, 2>(a, st);
    }
}

}  // namespace dma

template <int EPI, bool NORM>
int launch(const GemmArgs& a, hipStream_t st) {
    constexpr int BN = EPI == GEMM_SWIGLU ? 64 : 128;
    const unsigned blocks = (unsigned)(((a.N + BN - 1) / BN) * ((a.M + BM - 1) / BM));
    // the DMA kernel addresses x and the weights by 32-bit byte offsets
    const bool fits32 = (int64_t)a.M * a.K * 2 <= 0xFFFFFFFFLL && (int64_t)a.N * a.K / 2 <= 0xFFFFFFFFLL;
    const bool dma_ok = fits32 && ((a.K / 64) % 2 == 0) && reinterpret_cast<uintptr_t>(a.A.s) % 4 == 0 &&
                        reinterpret_cast<uintptr_t>(a.A.b) % 4 == 0 &&
                        (EPI != GEMM_SWIGLU ||
                         (reinterpret_cast<uintptr_t>(a.B.s) % 4 == 0 && reinterpret_cast<uintptr_t>(a.B.b) % 4 == 0));
    // paired output (ysum): the DMA kernel's SwiGLU epilogue only
    if (a.ysum && (EPI != GEMM_SWIGLU || NORM || !dma_ok || a.N % 64 != 0)) return -1;
    if (a.xsum || a.ysum) {
        // pre-paired activations: the DMA kernel only
        if (NORM || !dma_ok) return -1;
        dma::launch_dma_auto<EPI>(a, st);
        return 0;
    }
    if (NORM || !dma_ok)
        hipLaunchKernelGGL((q4_gemm_kernel<EPI, NORM>), dim3(blocks), dim3(kThreads), 0, st, a);
    else
        dma::launch_dma_auto<EPI>(a, st);
    return 0;
}

}  // namespace gemm

int launch_q4_gemm(const GemmArgs& a, int epi, bool norm, hipStream_t st) {
    if (norm) {
        switch (epi) {
            case GEMM_STORE: return gemm::launch<GEMM_STORE, true>(a, st);
            case GEMM_SWIGLU: return gemm::launch<GEMM_SWIGLU, true>(a, st);
            default: return -1;
        }
    }
    switch (epi) {
        case GEMM_STORE: return gemm::launch<GEMM_STORE, false>(a, st);
        case GEMM_STORE_F32: return gemm::launch<GEMM_STORE_F32, false>(a, st);
        case GEMM_RESIDUAL: return gemm::launch<GEMM_RESIDUAL, false>(a, st);
        case GEMM_SWIGLU: return gemm::launch<GEMM_SWIGLU, false>(a, st);
        default: return -1;
    }
}

// ---------------------------------------------------------------------------
// Activation pre-pass (launch_pair_rows): one wave per row, lane l takes the
// 8-element chunks l, l + 64, ...; with the norm a first pass forms the
// row's sum of squares (each lane its chunks, then the wave), with the
// per-element formula of mq4_rms_norm.  The 8 chunks of a group are 8
// consecutive lanes: their chunk sums are added over the lane pairs, quads
// and octets.  The sums are stored group-major: xs[g * M + m].
template <bool NORM>
__global__ __launch_bounds__(256) void pair_rows_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                        const uint16_t* __restrict__ nw, float eps,
                                                        uint16_t* __restrict__ xp, float* __restrict__ xs) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;                                  // whole waves
    const int CH = K / 8, G = K / 64;
    const uint4* src = reinterpret_cast<const uint4*>(x + (int64_t)m * K);
    uint4* dst = reinterpret_cast<uint4*>(xp + (int64_t)m * K);
    float r = 0.0f;
    if (NORM) {
        float ss = 0.0f;
        for (int c = lane; c < CH; c += 64) {
            const uint4 v = src[c];
            ss = sumsq_word(ss, v.x);
            ss = sumsq_word(ss, v.y);
            ss = sumsq_word(ss, v.z);
            ss = sumsq_word(ss, v.w);
        }
        r = rms_inv(wave_sum(ss), K, eps);
    }
    for (int c = lane; c < CH; c += 64) {
        uint4 v = src[c];
        if (NORM) {
            const uint4 w = reinterpret_cast<const uint4*>(nw)[c];
            v = make_uint4(norm_word(v.x, w.x, r), norm_word(v.y, w.y, r), norm_word(v.z, w.z, r),
                           norm_word(v.w, w.w, r));
        }
        uint32_t pr[4];
        float sum = pair_chunk(v, pr, 0.0f);
        dst[c] = make_uint4(pr[0], pr[1], pr[2], pr[3]);
        sum += __shfl_xor(sum, 1);
        sum += __shfl_xor(sum, 2);
        sum += __shfl_xor(sum, 4);
        if ((lane & 7) == 0) xs[(int64_t)(c >> 3) * M + m] = sum;
    }
}

int launch_pair_rows(const uint16_t* x, int M, int K, const uint16_t* norm_w, float eps, uint16_t* xp, float* xs,
                     hipStream_t st) {
    if (M < 1 || K % 512 != 0) return -1;
    const unsigned blocks = (unsigned)((M + 3) / 4);
    if (norm_w)
        hipLaunchKernelGGL(pair_rows_kernel<true>, dim3(blocks), dim3(256), 0, st, x, M, K, norm_w, eps, xp, xs);
    else
        hipLaunchKernelGGL(pair_rows_kernel<false>, dim3(blocks), dim3(256), 0, st, x, M, K, norm_w, eps, xp, xs);
    return 0;
}

}  // namespace mq4
