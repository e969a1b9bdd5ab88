// Batched-decode (2 <= M <= 32 token rows) MLX-affine Q4 GEMV on bf16 MFMA,
// gfx950.
//
// Replaces mx::quantized_matmul(x, w, s, b, transpose=true, 64, 4) at the
// decode call sites when M token rows are decoded together (M concurrent
// streams through the decode loop, src/core/engine.cpp:79-94): qmatmul
// (src/model/marlin.cpp:18-25) in mlp_forward (:31-35) and
// MarlinModel::lm_head (:161-169), with the fusions of the dot2 GEMV: the
// (1 + w) rms_norm in front (:12-16, 141, 145), swiglu (:27-29), the residual
// add (:142) and greedy argmax (src/sampling/sampler.cpp:15).
//
// Why MFMA: the product costs 2*M flops per weight.  The dot2 GEMV spends one
// v_dot2 per weight pair per row, so past a couple of rows it runs out of
// VALU issue slots before HBM is saturated (~22 VALU lane-ops per packed word
// are available at 8 TB/s).  The matrix cores have ample headroom: every
// weight byte is read once per call whatever M is, and the VALU work per
// packed word no longer grows with M (nibble unpack plus one fold per group).
//
// Arithmetic: products are exact and sums are fp32.  For one 64-element group
// g of weight row n and activation row m,
//     sum_k x[m,k] (s q_k + b) = s * P' + (b - 128 s) * X,
//     P' = sum_k x[m,k] (128 + q_k),   X = sum_k x[m,k].
// (128 + q) is an exact bf16 (the exponent bits of 128.0 OR-ed over the
// nibble, nib_pair_bf16), so v_mfma_f32_16x16x32_bf16 computes P' from exact
// products with fp32 accumulation; a second MFMA against a matrix of ones
// yields X in every output column.  Per group each output takes two fp32
// FMAs, acc = s * P' + (c * X + acc) with c = b - 128 s (exact in fp32).
//
// MFMA operand layout (16 x 16 x 32: A 16 rows x 32 k, B 32 k x 16 columns):
// lane l = (c, kq), c = l % 16, kq = l / 16, holds row / column c and the
// kq-th block of 8 k of A and B; D[4 kq + i][c] is element i of lane l.  A is
// the activations (rows m = 16 mt + c), B the weights transposed (column n of
// the 16-row weight tile).  Step t (0, 1) of group g uses packed word
// 2 kq + t of row n's group: one 8-byte load per lane per group.  The
// activations of the same 8 k are held in the nibble-pair order
// (k0, k4, k1, k5, k2, k6, k3, k7) that nib_pair_bf16 produces, so the MFMA
// sums the same products over a permuted k.
//
// Work decomposition: a block owns 16-row weight tiles (one per round,
// blockIdx.x + r * gridDim.x) and splits K over its KS waves, GW groups each;
// the KS partial accumulators are summed through LDS in wave order (a fixed
// order, so results are deterministic) and wave 0 runs the epilogue.  With
// XREG the wave's activations (and, for NORM, their normalization) stay in
// registers for all rounds; otherwise they are re-read per group from L2.
#include "mq4_device.h"
#include "mq4_gemv.h"
#include "mq4_host.h"
#include "mq4_mfma_ops.h"

namespace mq4 {

namespace mf {

// One round's weights for this lane: the two packed words of each group
// (words 2 kq, 2 kq + 1 of row n's group), and the bf16 scales and biases of
// the wave's GW groups, two per dword.
template <int GW, int NMAT>
struct WTile {
    uint2 w[NMAT][GW];
    uint32_t s[NMAT][GW / 2], b[NMAT][GW / 2];
};

template <int MT, int GW, int KS, int NMAT, int EPI, bool NORM, bool XREG, bool PF, bool SBV>
__global__ __launch_bounds__(64 * KS) void q4_mfma_gemv_kernel(GemvParams p) {
#pragma clang fp contract(off)
    static_assert(MT == 1 || MT == 2, "one or two 16-row tiles of activations");
    static_assert(!NORM || XREG, "the fused norm keeps the activations in registers");
    static_assert(!(NORM && EPI == EPI_PARTIAL), "the norm needs whole rows, not a K part");
    static_assert(GW % 2 == 0, "scales travel two per dword");
    // the group sums X are recomputed per group and round (two MFMAs against
    // ones): the matrix cores have the headroom, while keeping them in
    // registers (32 VGPRs) lowered occupancy and measured slower
    constexpr bool XS = false;
    const int lane = threadIdx.x & 63, kw = threadIdx.x >> 6;
    const int c16 = lane & 15, kq = lane >> 4;
    const int M = p.m_valid, N = p.N, K = p.K;
    const int G = K >> 6;
    // EPI_PARTIAL: block y of the grid takes waves y * KS .. y * KS + KS - 1
    // of the K range (a 12-wave product as two blocks of 6)
    const int g0 = ((EPI == EPI_PARTIAL ? (int)blockIdx.y * KS : 0) + kw) * GW;
    const bool wave_live = g0 < G;                 // wave-uniform: this wave has groups
    const int tiles = (N + 15) >> 4;
    const int rounds = (tiles + (int)gridDim.x - 1) / (int)gridDim.x;   // block-uniform

    const uint4 ones = make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
    const f32x4_t zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    const QMat* mats[2] = {&p.A, &p.B};

    // Weights of round r (tile blockIdx.x + r * gridDim.x).  Rows past N and
    // groups past G read clamped addresses; their results are never used.
    // With SBV the wave's GW scales (and biases) are one 8- or 16-byte load:
    // the dispatcher guarantees G % GW == 0 and aligned scale/bias rows.
    auto load_tile = [&](int r, WTile<GW, NMAT>& T) {
        const int n = ((int)blockIdx.x + r * (int)gridDim.x) * 16 + c16;
        const int nn = n < N ? n : N - 1;
#pragma unroll
        for (int t = 0; t < NMAT; ++t) {
            const QMat& Q = *mats[t];
#pragma unroll
            for (int gi = 0; gi < GW; ++gi) {
                const int gg = (g0 + gi) < G ? (g0 + gi) : G - 1;
                T.w[t][gi] = *reinterpret_cast<const uint2*>(Q.wq + (int64_t)nn * (K >> 3) + 8 * gg + 2 * kq);
            }
            if constexpr (SBV) {
                const uint16_t* sp = Q.s + (int64_t)nn * G + g0;
                const uint16_t* bp = Q.b + (int64_t)nn * G + g0;
                if constexpr (GW == 8) {
                    const uint4 sv = *reinterpret_cast<const uint4*>(sp), bv = *reinterpret_cast<const uint4*>(bp);
                    T.s[t][0] = sv.x, T.s[t][1] = sv.y, T.s[t][2] = sv.z, T.s[t][3] = sv.w;
                    T.b[t][0] = bv.x, T.b[t][1] = bv.y, T.b[t][2] = bv.z, T.b[t][3] = bv.w;
                } else {
                    static_assert(GW == 4, "vector scale loads for 4 or 8 groups");
                    const uint2 sv = *reinterpret_cast<const uint2*>(sp), bv = *reinterpret_cast<const uint2*>(bp);
                    T.s[t][0] = sv.x, T.s[t][1] = sv.y;
                    T.b[t][0] = bv.x, T.b[t][1] = bv.y;
                }
            } else {
#pragma unroll
                for (int j = 0; j < GW / 2; ++j) {
                    const int ga = (g0 + 2 * j) < G ? (g0 + 2 * j) : G - 1;
                    const int gb = (g0 + 2 * j + 1) < G ? (g0 + 2 * j + 1) : G - 1;
                    T.s[t][j] = (uint32_t)Q.s[(int64_t)nn * G + ga] | ((uint32_t)Q.s[(int64_t)nn * G + gb] << 16);
                    T.b[t][j] = (uint32_t)Q.b[(int64_t)nn * G + ga] | ((uint32_t)Q.b[(int64_t)nn * G + gb] << 16);
                }
            }
        }
    };

    // ---- round 0's weights are in flight before the activations are read ----
    WTile<GW, NMAT> cur;
    if (wave_live && rounds > 0) load_tile(0, cur);

    // activations of this wave's groups, MFMA A layout (see the header); rows
    // m >= M and groups g >= G hold zeros, loads use clamped addresses
    auto load_x = [&](int mt, int g, uint4& a0, uint4& a1) {
        const int m = mt * 16 + c16;
        const bool ok = m < M && g < G;
        const int mm = m < M ? m : M - 1, gg = g < G ? g : G - 1;
        const uint4* src = reinterpret_cast<const uint4*>(p.x + (int64_t)mm * K + 64 * gg + 16 * kq);
        const uint4 v0 = src[0], v1 = src[1];
        a0 = ok ? v0 : make_uint4(0u, 0u, 0u, 0u);
        a1 = ok ? v1 : make_uint4(0u, 0u, 0u, 0u);
    };

    uint4 xa[MT][XREG ? GW : 1][2];
    f32x4_t xs[MT][XS ? GW : 1];                      // group sums X (every column)
    __shared__ float red_ss[KS][32];
    // NORM: the block's copy of the (1 + w) norm weights (K <= kNormMaxK), one
    // 16-byte load per thread issued before the activations and read back
    // from LDS after the block barrier of the sum of squares
    constexpr int kNormMaxK = 2048;
    __shared__ uint4 nw_lds[NORM ? kNormMaxK / 8 : 1];
    uint4 nw_reg[NORM ? (kNormMaxK / 8 + 64 * KS - 1) / (64 * KS) : 1];
    if constexpr (NORM) {
#pragma unroll
        for (int i = 0; i < (int)(sizeof(nw_reg) / sizeof(uint4)); ++i) {
            const int c = (int)threadIdx.x + i * 64 * KS;
            nw_reg[i] = c < (K >> 3) ? reinterpret_cast<const uint4*>(p.norm_w)[c] : make_uint4(0u, 0u, 0u, 0u);
        }
    }
    if constexpr (XREG) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int gi = 0; gi < GW; ++gi) load_x(mt, g0 + gi, xa[mt][gi][0], xa[mt][gi][1]);
        if constexpr (NORM) {
            // sum of squares of each row: this lane's 16 values per group, the
            // four k-blocks of the wave (lanes c, c+16, c+32, c+48), then the
            // KS waves of the block in wave order
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                float s = 0.0f;
#pragma unroll
                for (int gi = 0; gi < GW; ++gi) {
                    sumsq4(s, xa[mt][gi][0]);
                    sumsq4(s, xa[mt][gi][1]);
                }
                s += __shfl_xor(s, 16);
                s += __shfl_xor(s, 32);
                if (kq == 0) red_ss[kw][mt * 16 + c16] = s;
            }
#pragma unroll
            for (int i = 0; i < (int)(sizeof(nw_reg) / sizeof(uint4)); ++i) {
                const int c = (int)threadIdx.x + i * 64 * KS;
                if (c < (K >> 3)) nw_lds[c] = nw_reg[i];
            }
            __syncthreads();
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                float tot = 0.0f;
#pragma unroll
                for (int k = 0; k < KS; ++k) tot += red_ss[k][mt * 16 + c16];
                const float r = rms_inv(tot, K, p.eps);
#pragma unroll
                for (int gi = 0; gi < GW; ++gi) {
                    const int gg = (g0 + gi) < G ? (g0 + gi) : G - 1;
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        const uint4 w = nw_lds[8 * gg + 2 * kq + t], v = xa[mt][gi][t];
                        xa[mt][gi][t] = make_uint4(norm_word(v.x, w.x, r), norm_word(v.y, w.y, r),
                                                   norm_word(v.z, w.z, r), norm_word(v.w, w.w, r));
                    }
                }
            }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int gi = 0; gi < GW; ++gi) {
                xa[mt][gi][0] = pair_order(xa[mt][gi][0]);
                xa[mt][gi][1] = pair_order(xa[mt][gi][1]);
                if constexpr (XS) xs[mt][gi] = mfma16(xa[mt][gi][1], ones, mfma16(xa[mt][gi][0], ones, zero4));
            }
    }

    constexpr int NV = NMAT * MT;                      // accumulators per lane (x4 floats)
    __shared__ f32x4_t red[KS > 1 ? KS - 1 : 1][NV][64];
    uint64_t best[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) best[mt][i] = 0;

    for (int r = 0; r < rounds; ++r) {
        const int n = ((int)blockIdx.x + r * (int)gridDim.x) * 16 + c16;
        const bool n_ok = n < N;
        WTile<GW, NMAT> nxt;
        if (PF && wave_live && r + 1 < rounds) load_tile(r + 1, nxt);   // next round in flight
        f32x4_t acc[NMAT][MT];
#pragma unroll
        for (int t = 0; t < NMAT; ++t)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[t][mt] = zero4;

        if (wave_live) {
#pragma unroll
            for (int gi = 0; gi < GW; ++gi) {
                if (g0 + gi >= G) break;               // wave-uniform
                uint4 a[MT][2];
                f32x4_t X[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    if constexpr (XREG) {
                        a[mt][0] = xa[mt][gi][0];
                        a[mt][1] = xa[mt][gi][1];
                        if constexpr (XS) X[mt] = xs[mt][gi];
                        else X[mt] = mfma16(a[mt][1], ones, mfma16(a[mt][0], ones, zero4));
                    } else {
                        load_x(mt, g0 + gi, a[mt][0], a[mt][1]);
                        a[mt][0] = pair_order(a[mt][0]);
                        a[mt][1] = pair_order(a[mt][1]);
                        X[mt] = mfma16(a[mt][1], ones, mfma16(a[mt][0], ones, zero4));
                    }
                }
#pragma unroll
                for (int t = 0; t < NMAT; ++t) {
                    const uint4 b0 = unpack_word(cur.w[t][gi].x), b1 = unpack_word(cur.w[t][gi].y);
                    const uint32_t sw = cur.s[t][gi >> 1], bw = cur.b[t][gi >> 1];
                    const float s = bf16_to_f32((gi & 1) ? (sw >> 16) : (sw & 0xffffu));
                    const float c = affine_c(s, (gi & 1) ? (bw >> 16) : (bw & 0xffffu));
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const f32x4_t P = mfma16(a[mt][1], b1, mfma16(a[mt][0], b0, zero4));
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            acc[t][mt][i] = __builtin_fmaf(s, P[i], __builtin_fmaf(c, X[mt][i], acc[t][mt][i]));
                    }
                }
            }
        }
        if (r + 1 < rounds && wave_live) {
            if constexpr (PF) cur = nxt;
            else load_tile(r + 1, cur);
        }

        // ---- sum the KS partial accumulators in wave order ----
        if constexpr (KS > 1) {
            if (kw > 0) {
#pragma unroll
                for (int t = 0; t < NMAT; ++t)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) red[kw - 1][t * MT + mt][lane] = acc[t][mt];
            }
            __syncthreads();
            if (kw == 0) {
                // wave order; with 12 waves as two halves, (w0 + .. + w5) +
                // (w6 + .. + w11), which is what the two blocks of the split
                // product (EPI_PARTIAL) and their combine compute
                constexpr int KH = KS == 12 ? 6 : KS;
#pragma unroll
                for (int t = 0; t < NMAT; ++t)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
                        for (int k = 0; k < KH - 1; ++k) {
                            const f32x4_t o = red[k][t * MT + mt][lane];
#pragma unroll
                            for (int i = 0; i < 4; ++i) acc[t][mt][i] += o[i];
                        }
                        if constexpr (KH < KS) {
                            f32x4_t hi = red[KH - 1][t * MT + mt][lane];
#pragma unroll
                            for (int k = KH; k < KS - 1; ++k) {
                                const f32x4_t o = red[k][t * MT + mt][lane];
#pragma unroll
                                for (int i = 0; i < 4; ++i) hi[i] += o[i];
                            }
#pragma unroll
                            for (int i = 0; i < 4; ++i) acc[t][mt][i] += hi[i];
                        }
                    }
            }
            __syncthreads();                           // red is rewritten next round
        }

        // ---- epilogue (wave 0): lane holds rows 16 mt + 4 kq + i of column n ----
        if (kw == 0) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = mt * 16 + 4 * kq + i;
                    if (m >= M || !n_ok) continue;
                    const int64_t o = (int64_t)m * N + n;
                    const float v = acc[0][mt][i];
                    if constexpr (EPI == EPI_STORE) {
                        p.y[o] = (uint16_t)f32_to_bf16(v);
                    } else if constexpr (EPI == EPI_PARTIAL) {
                        reinterpret_cast<float*>(p.y)[(int64_t)blockIdx.y * M * N + o] = v;
                    } else if constexpr (EPI == EPI_STORE_F32) {
                        reinterpret_cast<float*>(p.y)[o] = v;
                    } else if constexpr (EPI == EPI_RESIDUAL) {
                        p.y[o] = (uint16_t)f32_to_bf16(bf16_to_f32(p.res[o]) + round_bf16(v));
                    } else if constexpr (EPI == EPI_SWIGLU) {
                        p.y[o] = (uint16_t)swiglu_bf16(v, acc[NMAT - 1][mt][i]);
                    } else {                           // EPI_ARGMAX
                        const uint32_t lb = f32_to_bf16(v);
                        if (p.y) p.y[o] = (uint16_t)lb;
                        const uint64_t key = argmax_key(lb, (uint32_t)n);
                        best[mt][i] = key > best[mt][i] ? key : best[mt][i];
                    }
                }
        }
    }

    if constexpr (EPI == EPI_ARGMAX) {
        if (kw == 0) {
            // max over the 16 columns held by lanes kq*16 .. kq*16+15
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint64_t b = best[mt][i];
#pragma unroll
                    for (int off = 1; off < 16; off <<= 1) {
                        const uint64_t o = shfl_xor_u64(b, off);
                        b = o > b ? o : b;
                    }
                    const int m = mt * 16 + 4 * kq + i;
                    if (c16 == 0 && m < M) p.partial[(int64_t)m * kPartialStride + blockIdx.x] = b;
                }
        }
    }
}

// y = bf16(bf16(res) + round_bf16(part0 + part1)): the residual epilogue on the
// two K parts of the split product.
__global__ __launch_bounds__(256) void combine2_residual_kernel(const float* part, int64_t n, const uint16_t* res,
                                                               uint16_t* y) {
#pragma clang fp contract(off)
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < n; o += (int64_t)gridDim.x * 256) {
        const float v = part[o] + part[n + o];
        y[o] = (uint16_t)f32_to_bf16(bf16_to_f32(res[o]) + round_bf16(v));
    }
}

}  // namespace mf

namespace {

// Workgroups of `kernel` (64 * KS threads) that one CU holds at once, from the
// runtime's occupancy calculation; cached per kernel instance.
template <int KS>
int resident_per_cu(const void* kernel, int& cache) {
    if (cache == 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, 64 * KS, 0) != hipSuccess || n < 1) n = 1;
        cache = n;
    }
    return cache;
}

template <int MT, int GW, int KS, int NMAT, int EPI, bool NORM, bool XREG, bool PF, bool SBV>
void launch_one(const GemvParams& a, int tiles, hipStream_t st) {
    // The grid never exceeds what the GPU holds at once: a second batch of
    // workgroups would start only as the first drains.  Workgroups loop over
    // tiles (blockIdx.x + r * gridDim.x) instead.
    static int per_cu = 0;
    auto* k = mf::q4_mfma_gemv_kernel<MT, GW, KS, NMAT, EPI, NORM, XREG, PF, SBV>;
    int grid = resident_per_cu<KS>(reinterpret_cast<const void*>(k), per_cu) * num_cus();
    if (grid > tiles) grid = tiles;
    if (EPI == EPI_ARGMAX && grid > kPartialStride) grid = kPartialStride;
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(64 * KS), 0, st, a);
    if (EPI == EPI_ARGMAX) launch_argmax_finalize(a.partial, grid, a.m_valid, a.idx, st);
}

template <int MT, int GW, int KS, int NMAT, int EPI, bool NORM, bool XREG>
void launch(const GemvParams& a, hipStream_t st) {
    // PF: the next tile's weights in flight while the current one is reduced
    // (when workgroups loop over several tiles); SBV: vector scale/bias loads
    // (whole rows of GW groups, aligned)
    const int tiles = (a.N + 15) / 16;
    const int G = a.K / 64;
    constexpr bool kCanPF = NMAT == 1 && (KS <= 4 || GW <= 4);   // registers for a second weight buffer
    const bool pf = kCanPF && tiles > num_cus();
    const bool sbv = G % GW == 0 && aligned(a.A.s, 16) && aligned(a.A.b, 16) &&
                     (NMAT == 1 || (aligned(a.B.s, 16) && aligned(a.B.b, 16)));
    if constexpr (kCanPF) {
        if (pf) {
            if (sbv) launch_one<MT, GW, KS, NMAT, EPI, NORM, XREG, true, true>(a, tiles, st);
            else launch_one<MT, GW, KS, NMAT, EPI, NORM, XREG, true, false>(a, tiles, st);
            return;
        }
    }
    if (sbv) launch_one<MT, GW, KS, NMAT, EPI, NORM, XREG, false, true>(a, tiles, st);
    else launch_one<MT, GW, KS, NMAT, EPI, NORM, XREG, false, false>(a, tiles, st);
}

// (MT, GW, XREG) fixed per shape class; KS = the smallest provided wave count
// covering all G groups, at most MAXKS (more waves per block would leave too
// few registers per lane and spill).
template <int MT, int GW, int MAXKS, int NMAT, int EPI, bool NORM, bool XREG>
int dispatch_ks(const GemvParams& a, hipStream_t st) {
    const int G = a.K / 64;
    const int need = (G + GW - 1) / GW;
    if (need <= 1) { launch<MT, GW, 1, NMAT, EPI, NORM, XREG>(a, st); return 0; }
    if (need <= 2) { launch<MT, GW, 2, NMAT, EPI, NORM, XREG>(a, st); return 0; }
    if (need <= 4) { launch<MT, GW, 4, NMAT, EPI, NORM, XREG>(a, st); return 0; }
    if constexpr (MAXKS >= 8) {
        if (need <= 8) { launch<MT, GW, 8, NMAT, EPI, NORM, XREG>(a, st); return 0; }
    }
    if constexpr (MAXKS >= 12) {
        if (need <= 12) { launch<MT, GW, 12, NMAT, EPI, NORM, XREG>(a, st); return 0; }
    }
    return -1;
}

template <int EPI, bool NORM>
int dispatch(const GemvParams& a, hipStream_t st) {
    constexpr int NMAT = EPI == EPI_SWIGLU ? 2 : 1;
    const int G = a.K / 64;
    if (NORM && a.K > 2048) return -1;                 // the LDS copy of the norm weights holds K <= 2048
    if (a.m_valid <= 16) {
        // Up to K = 2048: 4 groups per wave over up to 8 waves (activations
        // in registers, 32 VGPRs; about 115 VGPRs per lane, two 8-wave
        // workgroups per CU).  Beyond: 8 groups per wave (64 VGPRs) up to
        // K = 6144 for single-matrix stores and K = 4096 for the fused SwiGLU
        // and argmax epilogues.
        if (G <= 8 * 4) return dispatch_ks<1, 4, 8, NMAT, EPI, NORM, true>(a, st);
        constexpr int MAXKS = (NORM && NMAT == 2) ? 4 : (NMAT == 2 || EPI == EPI_ARGMAX) ? 8 : 12;
        if (G <= MAXKS * 8) return dispatch_ks<1, 8, MAXKS, NMAT, EPI, NORM, true>(a, st);
        return -1;
    }
    // two 16-row activation tiles: 4 groups per wave in registers up to
    // K = 2048; beyond, for the single-matrix stores, 8 groups per wave re-read
    // from L2 up to K = 6144.  Other shapes return -1 (the dot2 GEMV runs them).
    if (G <= 8 * 4) return dispatch_ks<2, 4, 8, NMAT, EPI, NORM, true>(a, st);
    if constexpr (!NORM && NMAT == 1 && EPI != EPI_ARGMAX) {
        if (G <= 12 * 8) return dispatch_ks<2, 8, 12, NMAT, EPI, false, false>(a, st);
    }
    return -1;
}

}  // namespace

namespace {

template <int MT, bool XREG, bool SBV>
void launch_split2(const GemvParams& a, int tiles, hipStream_t st) {
    static int per_cu = 0;
    auto* k = mf::q4_mfma_gemv_kernel<MT, 8, 6, 1, EPI_PARTIAL, false, XREG, false, SBV>;
    // two blocks (K parts) per tile; the grid stays within what the GPU holds at once
    int grid = resident_per_cu<6>(reinterpret_cast<const void*>(k), per_cu) * num_cus() / 2;
    if (grid < 1) grid = 1;
    if (grid > tiles) grid = tiles;
    hipLaunchKernelGGL(k, dim3((unsigned)grid, 2), dim3(64 * 6), 0, st, a);
}

}  // namespace

int launch_q4_mfma_gemv_split2(const GemvParams& a, float* part, hipStream_t st) {
    const int G = a.K / 64;
    // exactly the products the non-split dispatch runs on 12 waves of 8 groups
    if (a.m_valid < 1 || a.m_valid > kMfmaMaxM || a.K % 64 != 0 || G <= 64 || G > 96 || !part) return -1;
    GemvParams b = a;
    b.y = reinterpret_cast<uint16_t*>(part);
    const int tiles = (a.N + 15) / 16;
    const bool sbv = G % 8 == 0 && aligned(a.A.s, 16) && aligned(a.A.b, 16);
    if (a.m_valid <= 16) {
        if (sbv) launch_split2<1, true, true>(b, tiles, st);
        else launch_split2<1, true, false>(b, tiles, st);
    } else {
        if (sbv) launch_split2<2, false, true>(b, tiles, st);
        else launch_split2<2, false, false>(b, tiles, st);
    }
    return 0;
}

void launch_combine2_residual(const float* part, int M, int N, const uint16_t* res, uint16_t* y, hipStream_t st) {
    const int64_t n = (int64_t)M * N;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 2048) blocks = 2048;
    hipLaunchKernelGGL(mf::combine2_residual_kernel, dim3((unsigned)blocks), dim3(256), 0, st, part, n, res, y);
}

int launch_q4_mfma_gemv(const GemvParams& a, int epi, bool norm, hipStream_t st) {
    if (a.m_valid < 1 || a.m_valid > kMfmaMaxM) return -1;
    int rc = -1;
    switch (epi) {
        case EPI_STORE: rc = norm ? -1 : dispatch<EPI_STORE, false>(a, st); break;
        case EPI_STORE_F32: rc = norm ? -1 : dispatch<EPI_STORE_F32, false>(a, st); break;
        case EPI_RESIDUAL: rc = norm ? -1 : dispatch<EPI_RESIDUAL, false>(a, st); break;
        case EPI_SWIGLU: rc = norm ? dispatch<EPI_SWIGLU, true>(a, st) : dispatch<EPI_SWIGLU, false>(a, st); break;
        case EPI_ARGMAX:
            // K = 2048 (the model's lm_head): the weight-ring kernel, same arithmetic
            rc = launch_lm_ring(a, norm, st);
            if (rc != 0) rc = norm ? dispatch<EPI_ARGMAX, true>(a, st) : dispatch<EPI_ARGMAX, false>(a, st);
            break;
        default: rc = -1;
    }
    return rc;
}

}  // namespace mq4
