// Decode-shaped (small M) MLX-affine Q4 GEMV kernels for gfx950.
//
// Replaces mx::quantized_matmul(x, w, s, b, transpose=true, 64, 4) at the
// decode call sites: qmatmul (src/model/marlin.cpp:18-25) inside mlp_forward
// (src/model/marlin.cpp:31-35) and MarlinModel::lm_head
// (src/model/marlin.cpp:161-169), plus fusions of the ops around them: the
// (1 + w) rms_norm before the MLP and before the lm_head
// (src/model/marlin.cpp:12-16, 141, 145), swiglu (src/model/marlin.cpp:27-29),
// the residual add (src/model/marlin.cpp:142) and greedy argmax
// (src/sampling/sampler.cpp:15).
//
// Work decomposition (HBM-bound; every weight byte is read exactly once):
//  * A packed row of K/2 bytes is split into 16-byte slices (4 words = 32 K
//    elements = half a group).  Lane l of K-split wave kw owns slices
//    (kw*SPL + j)*64 + l, j < SPL, for every row it visits, so a wave's 16-byte
//    loads of one row are contiguous (1 KiB per load instruction).
//  * A lane's K range never changes, so its activations are loaded once and
//    kept in registers, pre-paired as bf16x2 to line up with the nibble pairs
//    (q_p, q_{p+4}) that one AND-OR extracts from a packed word.
//  * Nibbles become bf16 (128 + q) by OR-ing in the exponent bits of 128.0 and
//    v_dot2_f32_bf16 accumulates x*(128+q) in fp32.  Per half-group the lane
//    then adds s*D + (b - 128*s)*X, D the dot and X the precomputed sum of its
//    32 activations: sum_k x_k*(s*q_k + b) with the bias factored out of the
//    inner loop (about 11 VALU ops per packed word).
//  * The first batch of weight loads is issued before the activations are
//    read, so the two memory latencies overlap; with PF the next batch is in
//    flight while the current one is reduced (streaming kernels).
//  * RPI rows are processed per round; their RPI*M (x2 for gate/up) partial
//    sums are reduced across the wave by recursive halving, and across the KS
//    K-split waves of a wave group through LDS.  A block holds NG independent
//    wave groups.
#include <mutex>

#include "mq4_device.h"
#include "mq4_gemm.h"
#include "mq4_gemv.h"
#include "mq4_host.h"

namespace mq4 {

// Largest K the entry points accept: 1024 16-byte slices per row, two per
// lane of eight K-split waves (the M = 1 instance; 4-row chunks of x switch
// to single rows above K = 16384).  Larger K would need more slices per lane
// than the register file holds without spilling.
constexpr int kMaxK = 32768;

template <int SPL, int NMAT, int RPI>
struct WBatch {
    uint4 w[NMAT][RPI][SPL];
    uint32_t s[NMAT][RPI][SPL], b[NMAT][RPI][SPL];
};

// Loads of one row batch.  The addresses are clamped into the matrix (rows to
// N-1, slices to L-1) so that every load is unconditional: per-lane
// predicated loads split the load stream into exec-masked branches, which
// measured about 2.5 us slower per launch on a 14 MB gate/up pass.  The values
// of clamped lanes are never used: their activations are zero (invalid
// slices) or their rows are skipped by the epilogue (rows >= N).
template <int SPL, int NMAT, int RPI>
__device__ __forceinline__ void load_batch(WBatch<SPL, NMAT, RPI>& W, const QMat& A, const QMat& B, int r0,
                                           int N, int G, int64_t row_words, const int (&slice)[SPL]) {
#pragma unroll
    for (int t = 0; t < NMAT; ++t) {
        const QMat& Q = (t == 0) ? A : B;
#pragma unroll
        for (int r = 0; r < RPI; ++r) {
            const int row = (r0 + r) < N ? (r0 + r) : (N - 1);
#pragma unroll
            for (int j = 0; j < SPL; ++j) {
                W.w[t][r][j] = load_nt_u4(reinterpret_cast<const uint4*>(Q.wq + (int64_t)row * row_words) + slice[j]);
                W.s[t][r][j] = Q.s[(int64_t)row * G + (slice[j] >> 1)];
                W.b[t][r][j] = Q.b[(int64_t)row * G + (slice[j] >> 1)];
            }
        }
    }
}

template <int M, int SPL, int RPI, int KS, int NG, int EPI, bool PF, bool NORM>
__global__ __launch_bounds__(64 * KS * NG) void q4_gemv_kernel(GemvParams p) {
    constexpr int NMAT = (EPI == EPI_SWIGLU) ? 2 : 1;
    constexpr int V = NMAT * RPI * M;       // values reduced per row batch
    static_assert(V <= 64, "too many values per wave");
    constexpr int LOG2V = log2_const<V>();
    constexpr int SH = 6 - LOG2V;           // lane >> SH = value index after the wave reduce

    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    const int group = wid / KS;
    const int kw = wid % KS;
    const int N = p.N, K = p.K, m_valid = p.m_valid;
    const int L = K >> 5;
    const int G = K >> 6;
    const int64_t row_words = K >> 3;

    const int n_batches = (N + RPI - 1) / RPI;
    const int groups_total = gridDim.x * NG;
    const int gid = blockIdx.x * NG + group;
    const int rounds = (n_batches + groups_total - 1) / groups_total;   // block-uniform

    int slice[SPL];      // clamped into [0, L) so every load address is valid
    bool valid[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        const int sl = (kw * SPL + j) * 64 + lane;
        valid[j] = sl < L;
        slice[j] = valid[j] ? sl : (L - 1);
    }

    // ---- first weight batch in flight before the activations are read ----
    WBatch<SPL, NMAT, RPI> cur;
    load_batch(cur, p.A, p.B, gid * RPI, N, G, row_words, slice);

    // ---- activations of this lane's slices (optionally RMS-normalized);
    //      lanes of invalid slices or rows m >= m_valid hold zeros ----
    uint4 xv[M][SPL][4];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const int mm = m < m_valid ? m : (m_valid - 1);
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            const bool use = valid[j] && m < m_valid;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint4 v = reinterpret_cast<const uint4*>(p.x + (int64_t)mm * K)[slice[j] * 4 + w];
                xv[m][j][w] = use ? v : make_uint4(0u, 0u, 0u, 0u);
            }
        }
    }

    __shared__ float red[NG][(KS > 1) ? KS : 1][(V > M) ? V : M];
    if (NORM) {
        // sum of squares of each activation row over all K (this lane's part,
        // the wave, then the K-split waves of the group)
        float ss[M];
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < SPL; ++j)
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint4 a = xv[m][j][w];
                    const uint32_t e[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
                    for (int q = 0; q < 4; ++q) s = sumsq_word(s, e[q]);
                }
            ss[m] = wave_sum(s);
        }
        if (KS > 1) {
            if (lane == 0)
#pragma unroll
                for (int m = 0; m < M; ++m) red[group][kw][m] = ss[m];
            __syncthreads();
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float s = 0.0f;
#pragma unroll
                for (int k = 0; k < KS; ++k) s += red[group][k][m];
                ss[m] = s;
            }
            __syncthreads();
        }
        // x_k * r * (1 + w_k), one bf16 rounding (src/model/marlin.cpp:12-16)
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            uint4 wn[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) wn[w] = reinterpret_cast<const uint4*>(p.norm_w)[slice[j] * 4 + w];
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float r = rms_inv(ss[m], K, p.eps);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint4 e = xv[m][j][w];
                    xv[m][j][w] = make_uint4(norm_word(e.x, wn[w].x, r), norm_word(e.y, wn[w].y, r),
                                             norm_word(e.z, wn[w].z, r), norm_word(e.w, wn[w].w, r));
                }
            }
        }
    }

    uint32_t xp[M][SPL][16];
    float xs[M][SPL];
#pragma unroll
    for (int m = 0; m < M; ++m) {
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) sum = pair_chunk(xv[m][j][w], &xp[m][j][4 * w], sum);
            xs[m][j] = sum;
        }
    }

    uint64_t best = 0;   // EPI_ARGMAX: running max key of this lane's value slot

    for (int t = 0; t < rounds; ++t) {
        const int r0 = (t * groups_total + gid) * RPI;
        WBatch<SPL, NMAT, RPI> nxt;
        if (PF && t + 1 < rounds)
            load_batch(nxt, p.A, p.B, ((t + 1) * groups_total + gid) * RPI, N, G, row_words, slice);

        // ---- dot products: value index v = (r*M + m)*NMAT + mat ----
        float acc[V];
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = 0.0f;
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt) {
#pragma unroll
            for (int r = 0; r < RPI; ++r) {
#pragma unroll
                for (int j = 0; j < SPL; ++j) {
                    float d[M];
#pragma unroll
                    for (int m = 0; m < M; ++m) d[m] = 0.0f;
                    const uint32_t wd[4] = {cur.w[mt][r][j].x, cur.w[mt][r][j].y, cur.w[mt][r][j].z,
                                            cur.w[mt][r][j].w};
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        const uint32_t p0 = nib_pair_bf16<0>(wd[w]);
                        const uint32_t p1 = nib_pair_bf16<1>(wd[w]);
                        const uint32_t p2 = nib_pair_bf16<2>(wd[w]);
                        const uint32_t p3 = nib_pair_bf16<3>(wd[w]);
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            d[m] = dot2_bf16(xp[m][j][4 * w + 0], p0, d[m]);
                            d[m] = dot2_bf16(xp[m][j][4 * w + 1], p1, d[m]);
                            d[m] = dot2_bf16(xp[m][j][4 * w + 2], p2, d[m]);
                            d[m] = dot2_bf16(xp[m][j][4 * w + 3], p3, d[m]);
                        }
                    }
#pragma unroll
                    for (int m = 0; m < M; ++m)
                        acc[(r * M + m) * NMAT + mt] += affine_term(cur.s[mt][r][j], cur.b[mt][r][j], d[m], xs[m][j]);
                }
            }
        }

        // ---- reduce across the wave, then across the K-split waves ----
        float val = wave_multi_reduce<V>(acc, lane);
        int vidx = lane >> SH;                 // value index held by this lane
        bool holder = (lane & ((1 << SH) - 1)) == 0;
        bool active = true;
        if (KS > 1) {
            if (holder) red[group][kw][vidx] = val;
            __syncthreads();
            vidx = lane;
            holder = lane < V;
            active = kw == 0;
            float s = 0.0f;
            if (active && holder) {
#pragma unroll
                for (int k = 0; k < KS; ++k) s += red[group][k][lane];
            }
            val = s;
            __syncthreads();
        }

        // ---- epilogue ----
        if (active) {
            float other = 0.0f;
            if (EPI == EPI_SWIGLU) {
                // the up-projection partner of value index v is v ^ 1
                other = __shfl_xor(val, (KS > 1) ? 1 : (1 << SH));
            }
            const int mt = vidx % NMAT;
            const int m = (vidx / NMAT) % M;
            const int r = vidx / (NMAT * M);
            const int row = r0 + r;
            const bool live = holder && row < N && m < m_valid && (EPI != EPI_SWIGLU || mt == 0);
            if (EPI == EPI_STORE) {
                if (live) p.y[(int64_t)m * N + row] = (uint16_t)f32_to_bf16(val);
            } else if (EPI == EPI_STORE_F32) {
                if (live) reinterpret_cast<float*>(p.y)[(int64_t)m * N + row] = val;
            } else if (EPI == EPI_RESIDUAL) {
                if (live) {
                    const float rsd = bf16_to_f32(p.res[(int64_t)m * N + row]);
                    p.y[(int64_t)m * N + row] = (uint16_t)f32_to_bf16(rsd + round_bf16(val));
                }
            } else if (EPI == EPI_SWIGLU) {
                if (live) p.y[(int64_t)m * N + row] = (uint16_t)swiglu_bf16(val, other);
            } else {  // EPI_ARGMAX
                const uint32_t lb = f32_to_bf16(val);
                if (live) {
                    if (p.y) p.y[(int64_t)m * N + row] = (uint16_t)lb;
                    const uint64_t key = argmax_key(lb, (uint32_t)row);
                    best = key > best ? key : best;
                }
            }
        }

        if (t + 1 < rounds) {
            if (PF) cur = nxt;
            else load_batch(cur, p.A, p.B, ((t + 1) * groups_total + gid) * RPI, N, G, row_words, slice);
        }
    }

    if (EPI == EPI_ARGMAX) {
        // Lane -> m mapping: KS == 1: m = (lane >> SH) % M; KS > 1: m = lane % M
        // in the group's first wave.  Max-reduce over the lane bits that do not
        // encode m, then over the groups of the block through LDS.
        const int mshift = (KS > 1) ? 0 : SH;
        constexpr int MB = log2_const<M>();
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const bool is_m_bit = off >= (1 << mshift) && off < (1 << (mshift + MB));
            if (!is_m_bit) {
                const uint64_t o = shfl_xor_u64(best, off);
                best = o > best ? o : best;
            }
        }
        __shared__ uint64_t gbest[NG][M];
        const int m_of_lane = (lane >> mshift) & (M - 1);
        if (kw == 0 && (lane & ~((M - 1) << mshift)) == 0) gbest[group][m_of_lane] = best;
        __syncthreads();
        if (threadIdx.x < M && (int)threadIdx.x < m_valid) {
            uint64_t b = gbest[0][threadIdx.x];
#pragma unroll
            for (int g = 1; g < NG; ++g) b = gbest[g][threadIdx.x] > b ? gbest[g][threadIdx.x] : b;
            p.partial[(int64_t)threadIdx.x * kPartialStride + blockIdx.x] = b;
        }
    }
}

// idx[m] = index of the max key among partial[m, 0..count).
__global__ __launch_bounds__(256) void argmax_finalize_kernel(const uint64_t* __restrict__ partial,
                                                              int count, int stride,
                                                              uint32_t* __restrict__ idx) {
    const int m = blockIdx.x;
    uint64_t best = 0;
    for (int i = threadIdx.x; i < count; i += blockDim.x) {
        const uint64_t k = partial[(int64_t)m * stride + i];
        best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    __shared__ uint64_t wbest[4];
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = wbest[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) b = wbest[w] > b ? wbest[w] : b;
        idx[m] = argmax_key_index(b);
    }
}

// Per-block max key over a [M, N] bf16 logits matrix (grid.y = m).
__global__ __launch_bounds__(256) void argmax_partial_kernel(const uint16_t* __restrict__ logits,
                                                             int64_t N, uint64_t* __restrict__ partial,
                                                             int stride) {
    const int m = blockIdx.y;
    const uint16_t* row = logits + (int64_t)m * N;
    uint64_t best = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < N;
         i += (int64_t)gridDim.x * blockDim.x) {
        const uint64_t k = argmax_key(row[i], (uint32_t)i);
        best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    __shared__ uint64_t wbest[4];
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = wbest[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) b = wbest[w] > b ? wbest[w] : b;
        partial[(int64_t)m * stride + blockIdx.x] = b;
    }
}

__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t* __restrict__ g,
                                                     const uint16_t* __restrict__ u, int64_t n,
                                                     uint16_t* __restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = (uint16_t)swiglu_bf16(bf16_to_f32(g[i]), bf16_to_f32(u[i]));
}

// out[m, :] = bf16(x * rsqrt(mean(x^2) + eps) * (1 + w)) per row: the
// (1 + weight) RMSNorm of src/model/marlin.cpp:12-16, fp32 math, one rounding.
__global__ __launch_bounds__(256) void rms_norm_1pw_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ w, int K,
                                                           float eps, uint16_t* __restrict__ out) {
    const uint16_t* xr = x + (int64_t)blockIdx.x * K;
    uint16_t* orow = out + (int64_t)blockIdx.x * K;
    float ss = 0.0f;
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        const float v = bf16_to_f32(xr[k]);
        ss += v * v;
    }
    ss = wave_sum(ss);
    __shared__ float part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = part[0] + part[1] + part[2] + part[3];
    const float r = rms_inv(tot, K, eps);
    for (int k = threadIdx.x; k < K; k += blockDim.x)
        orow[k] = (uint16_t)f32_to_bf16(bf16_to_f32(xr[k]) * r * (1.0f + bf16_to_f32(w[k])));
}

// ------------------------------------------------------------ dispatch ---

constexpr int kRPI = 4;

void launch_argmax_finalize(const uint64_t* partial, int count, int M, uint32_t* idx, hipStream_t st) {
    hipLaunchKernelGGL(argmax_finalize_kernel, dim3((unsigned)M), dim3(256), 0, st, partial, count, kPartialStride,
                       idx);
}

static int g_cus = 0;
int num_cus() {
    if (g_cus == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            g_cus = n;
        else
            g_cus = 256;
    }
    return g_cus;
}

template <int M, int SPL, int KS, int EPI, bool NORM, int RPI>
static void launch_single(const GemvParams& a, hipStream_t st) {
    const int64_t batches = ((int64_t)a.N + RPI - 1) / RPI;
    hipLaunchKernelGGL((q4_gemv_kernel<M, SPL, RPI, KS, 1, EPI, false, NORM>), dim3((unsigned)batches),
                       dim3(64 * KS), 0, st, a);
}

template <int M, int SPL, int KS, int EPI, bool NORM, int RPI>
static void launch_stream(const GemvParams& a, hipStream_t st) {
    // Streaming: NG wave groups per block, a grid of a few blocks per CU and
    // the next batch in flight while the current one is reduced.
    constexpr int NG = (KS == 1) ? 4 : 1;
    const int64_t batches = ((int64_t)a.N + RPI - 1) / RPI;
    int64_t blocks = (batches + NG - 1) / NG;
    // 4 blocks per CU for the argmax path measured best on a 248320-row
    // lm_head (2: 61 us, 4: 58 us, 8-16: 60-67 us).
    const int64_t cap = EPI == EPI_ARGMAX ? (int64_t)num_cus() * 4 : (int64_t)num_cus() * 16 / (KS * NG);
    if (blocks > cap) blocks = cap;
    if (blocks > kPartialStride) blocks = kPartialStride;
    if (blocks < 1) blocks = 1;
    // Per-block partial keys; a small second kernel reduces them (a last-block
    // reduction needs a device-scope release fence per block, which measured
    // three times slower than the extra launch).
    hipLaunchKernelGGL((q4_gemv_kernel<M, SPL, RPI, KS, NG, EPI, true, NORM>), dim3((unsigned)blocks),
                       dim3(64 * KS * NG), 0, st, a);
    if (EPI == EPI_ARGMAX)
        hipLaunchKernelGGL(argmax_finalize_kernel, dim3((unsigned)a.m_valid), dim3(256), 0, st, a.partial,
                           (int)blocks, kPartialStride, a.idx);
}

template <int M, int SPL, int KS, int EPI, bool NORM>
static void launch_gemv(const GemvParams& a, hipStream_t st) {
    constexpr int RPI = (EPI == EPI_SWIGLU && M == 4) ? 2 : kRPI;
    const int64_t batches = ((int64_t)a.N + RPI - 1) / RPI;
    // RPI 4 measured best for both paths (1 and 2 rows per wave were slower
    // on the single-pass 6144x2048 gate/up; 8 rows slower when streaming).
    if (EPI == EPI_ARGMAX || batches > (int64_t)num_cus() * 16 / KS)
        launch_stream<M, SPL, KS, EPI, NORM, RPI>(a, st);
    else
        launch_single<M, SPL, KS, EPI, NORM, RPI>(a, st);
}

// Pick (SPL, KS) from the number of 16-byte slices per row L = K/32.
template <int M, int EPI, bool NORM>
static int dispatch_k(const GemvParams& a, hipStream_t st) {
    const int L = a.K / 32;
    if (L <= 64) { launch_gemv<M, 1, 1, EPI, NORM>(a, st); return 0; }
    if (L <= 128) { launch_gemv<M, 1, 2, EPI, NORM>(a, st); return 0; }
    if (L <= 192) { launch_gemv<M, 1, 3, EPI, NORM>(a, st); return 0; }
    if (L <= 256) { launch_gemv<M, 1, 4, EPI, NORM>(a, st); return 0; }
    if (L <= 512) { launch_gemv<M, 1, 8, EPI, NORM>(a, st); return 0; }
    if constexpr (M == 1) {
        if (L <= 1024) { launch_gemv<M, 2, 8, EPI, NORM>(a, st); return 0; }
    }
    return -1;
}

// The rows m0 .. m0+mc-1 of a call (x, y, residual, argmax partials, indices).
static GemvParams row_chunk(const GemvParams& base, int m0, int mc, int epi) {
    GemvParams a = base;
    a.x = base.x + (int64_t)m0 * base.K;
    a.m_valid = mc;
    if (base.y) a.y = base.y + (int64_t)m0 * base.N * (epi == EPI_STORE_F32 ? 2 : 1);
    if (base.res) a.res = base.res + (int64_t)m0 * base.N;
    if (base.partial) a.partial = base.partial + (int64_t)m0 * kPartialStride;
    if (base.idx) a.idx = base.idx + m0;
    return a;
}

template <int EPI, bool NORM>
static int run_gemv(const GemvParams& base, int M, hipStream_t st) {
    // Rows of x are processed in chunks of at most 4 (of 1 when K > 16384,
    // where four rows of activations would not fit the register file).
    const int chunk = (base.K / 32 > 512) ? 1 : 4;
    for (int m0 = 0; m0 < M; m0 += chunk) {
        const int mc = (M - m0) < chunk ? (M - m0) : chunk;
        const GemvParams a = row_chunk(base, m0, mc, EPI);
        int rc;
        if (mc == 1) rc = dispatch_k<1, EPI, NORM>(a, st);
        else if (mc == 2) rc = dispatch_k<2, EPI, NORM>(a, st);
        else rc = dispatch_k<4, EPI, NORM>(a, st);
        if (rc) return rc;
    }
    return 0;
}

// Small-M products: the MFMA GEMV (every weight byte read once per chunk of
// up to kMfmaMaxM rows) from kMfmaMinM rows on, the dot2 GEMV below that or
// where the MFMA kernel does not cover K.
template <int EPI, bool NORM>
static int run_small(const GemvParams& base, int M, hipStream_t st) {
    // the lm_head + argmax at K = 2048: the weight-ring kernels (1-2 rows
    // with the dot2 GEMV's arithmetic, 3-4 with the MFMA GEMV's, which
    // outruns the dot2 GEMV reading the 254 MB once per 4 rows at dot2 rate)
    if (EPI == EPI_ARGMAX && M < kMfmaMinM && launch_lm_ring(base, NORM, st) == 0) return 0;
    if (M < kMfmaMinM) return run_gemv<EPI, NORM>(base, M, st);
    for (int m0 = 0; m0 < M; m0 += kMfmaMaxM) {
        const int mc = (M - m0) < kMfmaMaxM ? (M - m0) : kMfmaMaxM;
        const GemvParams a = row_chunk(base, m0, mc, EPI);
        if (launch_q4_mfma_gemv(a, EPI, NORM, st) != 0)
            if (int rc = run_gemv<EPI, NORM>(a, mc, st)) return rc;
    }
    return 0;
}

static int check_qmm_args(const char* what, const uint16_t* x, int64_t M, int64_t K, const uint32_t* wq,
                          const uint16_t* s, const uint16_t* b, int64_t N) {
    if (int rc = check_k(what, K)) return rc;
    if (M <= 0 || N <= 0)
        return fail(MQ4_ERR_INVALID_ARG, "%s: M=%lld and N=%lld must be positive", what, (long long)M,
                    (long long)N);
    if (K > kMaxK)
        return fail(MQ4_ERR_UNSUPPORTED, "%s: K=%lld exceeds the supported maximum %d", what,
                    (long long)K, kMaxK);
    if (N > 0x7fffffffLL) return fail(MQ4_ERR_UNSUPPORTED, "%s: N too large", what);
    if (!x || !wq || !s || !b) return fail(MQ4_ERR_INVALID_ARG, "%s: null pointer", what);
    if (!aligned(x, 16) || !aligned(wq, 16) || !aligned(s, 2) || !aligned(b, 2))
        return fail(MQ4_ERR_ALIGNMENT, "%s: x and wq must be 16-byte aligned, scales/biases 2-byte",
                    what);
    return MQ4_OK;
}

static int check_norm(const char* what, const uint16_t* norm_w, float eps) {
    if (!norm_w) return fail(MQ4_ERR_INVALID_ARG, "%s: null norm weight", what);
    if (!aligned(norm_w, 16)) return fail(MQ4_ERR_ALIGNMENT, "%s: norm weight must be 16-byte aligned", what);
    if (!(eps >= 0.0f)) return fail(MQ4_ERR_INVALID_ARG, "%s: eps must be >= 0", what);
    return MQ4_OK;
}

// From kGemmMinM rows on, the entry points use the MFMA GEMM of mq4_gemm.hip
// (weights read once per 128-row tile instead of once per 4 rows).
static int run_gemm(const GemvParams& a, int64_t M, int epi, hipStream_t st, bool norm = false) {
    GemmArgs g{a.x, (int)M, a.N, a.K, a.A, a.B, a.y, a.res, a.norm_w, a.eps};
    return launch_q4_gemm(g, epi, norm, st);
}

static GemvParams params(const uint16_t* x, int64_t M, int64_t K, int64_t N, QMat A, QMat B, uint16_t* y) {
    GemvParams a{};
    a.x = x;
    a.m_valid = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.A = A;
    a.B = B;
    a.y = y;
    return a;
}

template <bool NORM>
static int gate_up_impl(const char* what, const uint16_t* x, int64_t M, int64_t K, const uint16_t* norm_w,
                        float eps, const uint32_t* gate_wq, const uint16_t* gate_scales,
                        const uint16_t* gate_biases, const uint32_t* up_wq, const uint16_t* up_scales,
                        const uint16_t* up_biases, int64_t N, uint16_t* h, void* stream) {
    if (int rc = check_qmm_args(what, x, M, K, gate_wq, gate_scales, gate_biases, N)) return rc;
    if (int rc = check_qmm_args(what, x, M, K, up_wq, up_scales, up_biases, N)) return rc;
    if (NORM)
        if (int rc = check_norm(what, norm_w, eps)) return rc;
    if (!h || !aligned(h, 2)) return fail(MQ4_ERR_INVALID_ARG, "%s: h must be a 2-byte aligned pointer", what);
    GemvParams a = params(x, M, K, N, {gate_wq, gate_scales, gate_biases}, {up_wq, up_scales, up_biases}, h);
    a.norm_w = norm_w;
    a.eps = eps;
    if (M >= kGemmMinM) {
        run_gemm(a, M, GEMM_SWIGLU, as_stream(stream), NORM);
        return launch_status(what);
    }
    if (run_small<EPI_SWIGLU, NORM>(a, (int)M, as_stream(stream)))
        return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported K", what);
    return launch_status(what);
}

static size_t lm_head_ws_bytes(int64_t M) {
    return M <= 0 ? 0 : (size_t)M * kPartialStride * sizeof(uint64_t);
}

template <bool NORM>
static int lm_head_impl(const char* what, const uint16_t* h, int64_t M, int64_t K, const uint16_t* norm_w,
                        float eps, const uint32_t* wq, const uint16_t* scales, const uint16_t* biases, int64_t N,
                        uint32_t* idx, uint16_t* logits, void* workspace, size_t workspace_bytes,
                        void* stream) {
    if (int rc = check_qmm_args(what, h, M, K, wq, scales, biases, N)) return rc;
    if (NORM)
        if (int rc = check_norm(what, norm_w, eps)) return rc;
    if (!idx || !aligned(idx, 4)) return fail(MQ4_ERR_INVALID_ARG, "%s: idx must be a 4-byte aligned pointer", what);
    if (logits && !aligned(logits, 2)) return fail(MQ4_ERR_ALIGNMENT, "%s: logits must be 2-byte aligned", what);
    if (!workspace || workspace_bytes < lm_head_ws_bytes(M) || !aligned(workspace, 8))
        return fail(MQ4_ERR_WORKSPACE, "%s: workspace needs %zu bytes, 8-byte aligned (got %zu)", what,
                    lm_head_ws_bytes(M), workspace_bytes);
    GemvParams a = params(h, M, K, N, {wq, scales, biases}, {nullptr, nullptr, nullptr}, logits);
    a.norm_w = norm_w;
    a.eps = eps;
    a.partial = reinterpret_cast<uint64_t*>(workspace);
    a.idx = idx;
    if (run_small<EPI_ARGMAX, NORM>(a, (int)M, as_stream(stream)))
        return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported K", what);
    return launch_status(what);
}

// ---- lm_head + argmax without a workspace argument ----
// The per-block partial keys of mq4_lm_head_argmax_noalloc live in this
// file-scope device array instead of a caller-provided workspace: one copy per
// GPU the library runs on, held until the process ends, shared by every call
// on that GPU (so calls that overlap in time on one GPU race).  The partial
// keys need no initialisation: every launch writes the slots it reads.
constexpr int kScratchMaxM = 32;
constexpr size_t kScratchWords = (size_t)kScratchMaxM * kPartialStride;       // 1 MiB
static __device__ __align__(256) uint64_t scratch[kScratchWords];

// In host code `scratch` names a host-side stand-in, not device memory: the
// device address of each GPU's copy comes from hipGetSymbolAddress, taken once
// per device with that device current, and only that address is handed to
// kernels.
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static uint64_t* g_scratch_dev[kMaxDevices] = {};

static int scratch_for_stream(const char* what, hipStream_t st, uint64_t** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(MQ4_ERR_HIP, "%s: hipGetDevice failed", what);
    if (st) {
        hipDevice_t sdev = 0;
        if (hipStreamGetDevice(st, &sdev) != hipSuccess)
            return fail(MQ4_ERR_HIP, "%s: hipStreamGetDevice failed", what);
        if ((int)sdev != dev)
            return fail(MQ4_ERR_INVALID_ARG, "%s: the stream belongs to device %d, the current device is %d", what,
                        (int)sdev, dev);
    }
    if (dev < 0 || dev >= kMaxDevices) return fail(MQ4_ERR_UNSUPPORTED, "%s: device %d out of range", what, dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(MQ4_ERR_HIP, "%s: hipGetSymbolAddress(scratch) failed: %s", what, hipGetErrorString(e));
        g_scratch_dev[dev] = reinterpret_cast<uint64_t*>(ptr);
    }
    *out = g_scratch_dev[dev];
    return MQ4_OK;
}

}  // namespace mq4

using namespace mq4;

extern "C" int mq4_lm_head_argmax_noalloc(const uint16_t* h, int64_t M, int64_t K, const uint32_t* wq,
                                          const uint16_t* scales, const uint16_t* biases, int64_t N,
                                          uint32_t* idx, uint16_t* logits, void* stream) {
    const char* what = "mq4_lm_head_argmax_noalloc";
    if (M > kScratchMaxM)
        return fail(MQ4_ERR_UNSUPPORTED, "%s: M=%lld exceeds the %d rows its static scratch holds", what,
                    (long long)M, kScratchMaxM);
    if (M <= 0) return fail(MQ4_ERR_INVALID_ARG, "%s: M=%lld must be positive", what, (long long)M);
    uint64_t* ws = nullptr;
    if (int rc = scratch_for_stream(what, as_stream(stream), &ws)) return rc;
    return lm_head_impl<false>(what, h, M, K, nullptr, 0.0f, wq, scales, biases, N, idx, logits, ws,
                               kScratchWords * sizeof(uint64_t), stream);
}

extern "C" int mq4_qmm(const uint16_t* x, int64_t M, int64_t K, const uint32_t* wq,
                       const uint16_t* scales, const uint16_t* biases, int64_t N, int transpose,
                       int group_size, int bits, uint16_t* y, void* stream) {
    const char* what = "mq4_qmm";
    if (int rc = check_format(what, group_size, bits)) return rc;
    if (transpose != 1)
        return fail(MQ4_ERR_UNSUPPORTED, "%s: only transpose=1 (x @ W^T) is implemented", what);
    if (int rc = check_qmm_args(what, x, M, K, wq, scales, biases, N)) return rc;
    if (!y || !aligned(y, 2)) return fail(MQ4_ERR_INVALID_ARG, "%s: y must be a 2-byte aligned pointer", what);
    GemvParams a = params(x, M, K, N, {wq, scales, biases}, {nullptr, nullptr, nullptr}, y);
    if (M >= kGemmMinM) {
        run_gemm(a, M, GEMM_STORE, as_stream(stream));
        return launch_status(what);
    }
    if (run_small<EPI_STORE, false>(a, (int)M, as_stream(stream)))
        return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported K", what);
    return launch_status(what);
}

extern "C" int mq4_qmm_f32(const uint16_t* x, int64_t M, int64_t K, const uint32_t* wq,
                           const uint16_t* scales, const uint16_t* biases, int64_t N, float* y,
                           void* stream) {
    const char* what = "mq4_qmm_f32";
    if (int rc = check_qmm_args(what, x, M, K, wq, scales, biases, N)) return rc;
    if (!y || !aligned(y, 4)) return fail(MQ4_ERR_INVALID_ARG, "%s: y must be a 4-byte aligned pointer", what);
    GemvParams a = params(x, M, K, N, {wq, scales, biases}, {nullptr, nullptr, nullptr},
                          reinterpret_cast<uint16_t*>(y));
    if (M >= kGemmMinM) {
        run_gemm(a, M, GEMM_STORE_F32, as_stream(stream));
        return launch_status(what);
    }
    if (run_small<EPI_STORE_F32, false>(a, (int)M, as_stream(stream)))
        return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported K", what);
    return launch_status(what);
}

extern "C" int mq4_qmm_residual(const uint16_t* x, int64_t M, int64_t K, const uint32_t* wq,
                                const uint16_t* scales, const uint16_t* biases, int64_t N,
                                const uint16_t* residual, uint16_t* y, void* stream) {
    const char* what = "mq4_qmm_residual";
    if (int rc = check_qmm_args(what, x, M, K, wq, scales, biases, N)) return rc;
    if (!y || !residual || !aligned(y, 2) || !aligned(residual, 2))
        return fail(MQ4_ERR_INVALID_ARG, "%s: y and residual must be 2-byte aligned pointers", what);
    GemvParams a = params(x, M, K, N, {wq, scales, biases}, {nullptr, nullptr, nullptr}, y);
    a.res = residual;
    if (M >= kGemmMinM) {
        run_gemm(a, M, GEMM_RESIDUAL, as_stream(stream));
        return launch_status(what);
    }
    if (run_small<EPI_RESIDUAL, false>(a, (int)M, as_stream(stream)))
        return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported K", what);
    return launch_status(what);
}

extern "C" int mq4_mlp_gate_up_silu(const uint16_t* x, int64_t M, int64_t K, const uint32_t* gate_wq,
                                    const uint16_t* gate_scales, const uint16_t* gate_biases,
                                    const uint32_t* up_wq, const uint16_t* up_scales,
                                    const uint16_t* up_biases, int64_t N, uint16_t* h, void* stream) {
    return gate_up_impl<false>("mq4_mlp_gate_up_silu", x, M, K, nullptr, 0.0f, gate_wq, gate_scales,
                               gate_biases, up_wq, up_scales, up_biases, N, h, stream);
}

extern "C" int mq4_rmsnorm_gate_up_silu(const uint16_t* x, int64_t M, int64_t K, const uint16_t* norm_weight,
                                        float eps, const uint32_t* gate_wq, const uint16_t* gate_scales,
                                        const uint16_t* gate_biases, const uint32_t* up_wq,
                                        const uint16_t* up_scales, const uint16_t* up_biases, int64_t N,
                                        uint16_t* h, void* stream) {
    return gate_up_impl<true>("mq4_rmsnorm_gate_up_silu", x, M, K, norm_weight, eps, gate_wq, gate_scales,
                              gate_biases, up_wq, up_scales, up_biases, N, h, stream);
}

namespace mq4 {

// ---- rms_norm + mlp_forward + residual in one call ----
// Workspace: h [M, N] bf16; on the GEMM path h is written in the GEMM's
// operand order by the SwiGLU epilogue, and the normalized x (by
// launch_pair_rows) too, both with their fp32 group sums, so neither GEMM
// forms them per wave.  On the MFMA GEMV path (kMfmaMinM <= M < kGemmMinM)
// part [2, M, K] fp32 holds the two K parts of the split down product.  On
// the fp16-weight path the down product in S > 1 K parts puts them in
// kpart [S, M, K] fp32, and silu holds the SwiGLU epilogue's table of the
// rounded SiLU (SILU_LUT_N bf16, written by the pre-pass).  Sections 256-byte
// aligned.
struct MlpWs {
    uint16_t* h = nullptr;
    uint16_t* xp = nullptr;
    float* xs = nullptr;
    uint16_t* hp = nullptr;
    float* hs = nullptr;
    float* part = nullptr;
    float* kpart = nullptr;
    uint16_t* silu = nullptr;
    size_t bytes = 0;
};

// Tiles and K parts of the fp16-weight down product ([M, N] . [K, N]^T,
// N / 64 groups) on the one-call path: 128 x 128 tiles (three blocks per CU)
// while there are at most two of them per CU, else 128 x 256; and the most
// of 1, 2 and 4 parts (whole 8-group scale slots per part) whose tiles times
// parts stay within one block per CU.  Measured on the 2048 x 6144 down
// product with its part combine, us for 1 / 2 / 4 parts, 128 x 256 tiles then
// 128 x 128:
//   M = 200:  84.4 / 48.6 / 31.0,    55.2 / 33.2 / 22.5
//   M = 1024: 91.7 / 54.8 / 45.6,    61.0 / 42.7 / 45.0
//   M = 2048: 99.1 / 71.2 / 79.1,    69.8 / 71.2 / 80.4
//   M = 3072: 108.0 / 105.0 / 113.4, 101.4 / 101.6 / 114.8
//   M = 4096: 119.5 / 126.2 / 146.4, 118.0 / 133.3 / 150.9
//   M = 8192: 212.5 / 250.5 / 315.0, 230.4 / 268.6 / 332.4
// Either tile width gives the same bits.  0 parts: N / 64 not a multiple of
// 8 (no fp16 down product).
static bool mlp_down_narrow(int64_t M, int64_t K) {
    return ((M + 127) / 128) * ((K + 127) / 128) <= 2 * (int64_t)num_cus();
}
static int mlp_down_parts(int64_t M, int64_t K, int64_t N) {
    const int64_t G = N / 64;
    if (N % 64 != 0 || G % 8 != 0) return 0;
    const int64_t BN = mlp_down_narrow(M, K) ? 128 : 256;
    const int64_t tiles = ((M + 127) / 128) * ((K + BN - 1) / BN);
    int S = 1;
    for (int s : {2, 4})
        if ((G / 8) % s == 0 && tiles * s <= (int64_t)num_cus()) S = s;
    return S;
}

static MlpWs mlp_ws_layout(void* base, int64_t M, int64_t K, int64_t N) {
    MlpWs w;
    char* b = reinterpret_cast<char*>(base);
    size_t off = 0;
    auto take = [&](size_t n) -> char* {
        char* q = b ? b + off : nullptr;
        off += (n + 255) & ~(size_t)255;
        return q;
    };
    // h (the other path's natural h, or the paired h)
    w.h = w.hp = reinterpret_cast<uint16_t*>(take((size_t)M * N * 2));
    if (M >= kGemmMinM) {
        w.xp = reinterpret_cast<uint16_t*>(take((size_t)M * K * 2));
        w.xs = reinterpret_cast<float*>(take((size_t)M * (K / 64) * 4));
        w.hs = reinterpret_cast<float*>(take((size_t)M * (N / 64) * 4));
        const int S = mlp_down_parts(M, K, N);
        if (S > 1) w.kpart = reinterpret_cast<float*>(take((size_t)S * M * K * 4));
        w.silu = reinterpret_cast<uint16_t*>(take((size_t)SILU_LUT_N * 2));
    } else if (M >= kMfmaMinM) {
        w.part = reinterpret_cast<float*>(take((size_t)2 * M * K * 4));
    }
    w.bytes = off;
    return w;
}

// The pre-paired GEMM path: K and N multiples of 512 (whole waves of chunks
// in launch_pair_rows, an even group count), scale/bias rows 4-byte aligned,
// byte offsets within 32 bits.
static bool mlp_paired_ok(int64_t M, int64_t K, int64_t N, const QMat& g, const QMat& u, const QMat& d) {
    auto a4 = [](const QMat& q) { return aligned(q.s, 4) && aligned(q.b, 4); };
    return M >= kGemmMinM && K % 512 == 0 && N % 512 == 0 && a4(g) && a4(u) && a4(d) &&
           M * K * 2 <= 0xFFFFFFFFLL && M * N * 2 <= 0xFFFFFFFFLL && N * K / 2 <= 0xFFFFFFFFLL;
}

}  // namespace mq4

// Enough for every call of at most M rows: the layout's size grows with the
// row count inside each of its three regimes (up to kMfmaMinM - 1 rows: h
// only; to kGemmMinM - 1: h and two fp32 K parts; from kGemmMinM: h, the
// paired operands and the down product's K parts), except where the K-part
// count drops, so the size is the largest over the regimes' top row counts
// and the row counts just below a drop (multiples of 128), up to M.
extern "C" size_t mq4_mlp_workspace_size(int64_t M, int64_t K, int64_t N) {
    if (M <= 0 || K <= 0 || N <= 0) return 0;
    size_t need = mlp_ws_layout(nullptr, M, K, N).bytes;
    auto at = [&](int64_t m) {
        if (m < 1 || m > M) return;
        const size_t b = mlp_ws_layout(nullptr, m, K, N).bytes;
        need = b > need ? b : need;
    };
    at(kMfmaMinM - 1);
    at(kGemmMinM - 1);
    for (int64_t m = 128; m < M; m += 128)
        if (mlp_down_parts(m, K, N) > mlp_down_parts(m + 1, K, N)) at(m);
    return need;
}

extern "C" int mq4_mlp_residual(const uint16_t* x, int64_t M, int64_t K, const uint16_t* norm_weight, float eps,
                                const uint32_t* gate_wq, const uint16_t* gate_scales, const uint16_t* gate_biases,
                                const uint32_t* up_wq, const uint16_t* up_scales, const uint16_t* up_biases,
                                const uint32_t* down_wq, const uint16_t* down_scales, const uint16_t* down_biases,
                                int64_t N, void* workspace, size_t workspace_bytes, uint16_t* y, void* stream) {
    const char* what = "mq4_mlp_residual";
    if (int rc = check_qmm_args(what, x, M, K, gate_wq, gate_scales, gate_biases, N)) return rc;
    if (int rc = check_qmm_args(what, x, M, K, up_wq, up_scales, up_biases, N)) return rc;
    if (int rc = check_norm(what, norm_weight, eps)) return rc;
    if (!y || !aligned(y, 2)) return fail(MQ4_ERR_INVALID_ARG, "%s: y must be a 2-byte aligned pointer", what);
    const size_t need = mlp_ws_layout(nullptr, M, K, N).bytes;
    if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
        return fail(MQ4_ERR_WORKSPACE, "%s: workspace needs %zu bytes, 256-byte aligned (got %zu)", what, need,
                    workspace_bytes);
    const MlpWs w = mlp_ws_layout(workspace, M, K, N);
    if (int rc = check_qmm_args(what, w.h, M, N, down_wq, down_scales, down_biases, K)) return rc;
    const QMat G{gate_wq, gate_scales, gate_biases}, U{up_wq, up_scales, up_biases},
        D{down_wq, down_scales, down_biases};
    hipStream_t st = as_stream(stream);
    if (mlp_paired_ok(M, K, N, G, U, D)) {
        // The fp16-weight GEMM (mq4_gemm16.hip) when every scale and bias row
        // is 16-byte aligned (else the exact-operand GEMM below): gate/up +
        // SwiGLU on an fp16 copy of the normalized x (its per-row
        // power-of-two scales in the xs area), and the down product on h
        // written as fp16 / 256 in the operand order (exact for |h| in
        // [2^-6, 1.6e7]), with the tiles and K parts of mlp_down_parts (2048
        // x 6144 down at M = 2048: 70 us, against 102 us on the
        // exact-operand GEMM with paired bf16 h).  With the down product's scale or bias rows
        // not 16-byte aligned, gate/up writes h paired in bf16 with its group
        // sums for the exact-operand GEMM's down product.
        auto a16 = [](const QMat& q) { return aligned(q.s, 16) && aligned(q.b, 16); };
        if (a16(G) && a16(U)) {
            // K parts need an 8-byte aligned y (one part stores any 2-byte
            // aligned y element by element)
            int parts = a16(D) ? mlp_down_parts(M, K, N) : 0;
            if (parts > 1 && !aligned(y, 8)) parts = 1;
            const bool down16 = parts > 0;
            if (launch_pair_rows16(x, (int)M, (int)K, norm_weight, eps, w.xp, w.xs, w.silu, st))
                return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported shape", what);
            Gemm16Args gu{w.xp, w.xs, (int)M, (int)N, (int)K, G, U, w.hp, nullptr, down16 ? nullptr : w.hs, 0.0f,
                          down16 ? 1.0f / 256.0f : 0.0f, 0, nullptr, 0, w.silu};
            if (launch_q4_gemm16(gu, GEMM_SWIGLU, st))
                return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported shape", what);
            if (down16) {
                Gemm16Args dn{w.hp, nullptr, (int)M, (int)K, (int)N, D, QMat{nullptr, nullptr, nullptr}, y, x,
                              nullptr, 256.0f, 0.0f, parts, w.kpart, mlp_down_narrow(M, K) ? 1 : 0};
                if (launch_q4_gemm16(dn, GEMM_RESIDUAL, st))
                    return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported shape", what);
                return launch_status(what);
            }
        } else {
            if (launch_pair_rows(x, (int)M, (int)K, norm_weight, eps, w.xp, w.xs, st))
                return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported shape", what);
            // gate/up + SwiGLU writes h already paired, with its group sums
            GemmArgs gu{w.xp, (int)M, (int)N, (int)K, G, U, w.hp, nullptr, nullptr, 0.0f, w.xs, w.hs};
            if (launch_q4_gemm(gu, GEMM_SWIGLU, false, st))
                return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported shape", what);
        }
        GemmArgs dn{w.hp, (int)M, (int)K, (int)N, D, QMat{nullptr, nullptr, nullptr}, y, x, nullptr, 0.0f, w.hs, nullptr};
        if (launch_q4_gemm(dn, GEMM_RESIDUAL, false, st)) return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported shape", what);
        return launch_status(what);
    }
    // otherwise the separate entries' kernels: norm + gate/up + SwiGLU into h,
    // then down + residual
    if (int rc = gate_up_impl<true>(what, x, M, K, norm_weight, eps, gate_wq, gate_scales, gate_biases, up_wq,
                                    up_scales, up_biases, N, w.h, stream))
        return rc;
    GemvParams a = params(w.h, M, N, K, D, {nullptr, nullptr, nullptr}, y);
    a.res = x;
    // from kMfmaMinM rows the down product runs as two K parts per tile (half
    // the activations per block, all CUs busy), bit-identical to the one-block
    // product of mq4_qmm_residual
    if (M >= kMfmaMinM && M < kGemmMinM && launch_q4_mfma_gemv_split2(a, w.part, st) == 0) {
        launch_combine2_residual(w.part, (int)M, (int)K, x, y, st);
        return launch_status(what);
    }
    if (M >= kGemmMinM) {
        run_gemm(a, M, GEMM_RESIDUAL, st);
        return launch_status(what);
    }
    if (run_small<EPI_RESIDUAL, false>(a, (int)M, st)) return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported K", what);
    return launch_status(what);
}

extern "C" size_t mq4_lm_head_argmax_workspace_size(int64_t M, int64_t N) {
    (void)N;
    return lm_head_ws_bytes(M);
}

extern "C" int mq4_lm_head_argmax(const uint16_t* h, int64_t M, int64_t K, const uint32_t* wq,
                                  const uint16_t* scales, const uint16_t* biases, int64_t N,
                                  uint32_t* idx, uint16_t* logits, void* workspace,
                                  size_t workspace_bytes, void* stream) {
    return lm_head_impl<false>("mq4_lm_head_argmax", h, M, K, nullptr, 0.0f, wq, scales, biases, N, idx, logits,
                               workspace, workspace_bytes, stream);
}

extern "C" int mq4_rmsnorm_lm_head_argmax(const uint16_t* h, int64_t M, int64_t K, const uint16_t* norm_weight,
                                          float eps, const uint32_t* wq, const uint16_t* scales,
                                          const uint16_t* biases, int64_t N, uint32_t* idx, uint16_t* logits,
                                          void* workspace, size_t workspace_bytes, void* stream) {
    return lm_head_impl<true>("mq4_rmsnorm_lm_head_argmax", h, M, K, norm_weight, eps, wq, scales, biases, N,
                              idx, logits, workspace, workspace_bytes, stream);
}

extern "C" size_t mq4_argmax_workspace_size(int64_t M, int64_t N) {
    (void)N;
    if (M <= 0) return 0;
    return (size_t)M * 1024 * sizeof(uint64_t);
}

extern "C" int mq4_argmax_bf16(const uint16_t* logits, int64_t M, int64_t N, uint32_t* idx,
                               void* workspace, size_t workspace_bytes, void* stream) {
    const char* what = "mq4_argmax_bf16";
    if (M <= 0 || N <= 0) return fail(MQ4_ERR_INVALID_ARG, "%s: M and N must be positive", what);
    if (N > 0x7fffffffLL || M > 65535) return fail(MQ4_ERR_UNSUPPORTED, "%s: M or N too large", what);
    if (!logits || !idx) return fail(MQ4_ERR_INVALID_ARG, "%s: null pointer", what);
    if (!workspace || workspace_bytes < mq4_argmax_workspace_size(M, N) || !aligned(workspace, 8))
        return fail(MQ4_ERR_WORKSPACE, "%s: workspace needs %zu bytes, 8-byte aligned", what,
                    mq4_argmax_workspace_size(M, N));
    int64_t blocks = (N + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    hipStream_t st = as_stream(stream);
    uint64_t* partial = reinterpret_cast<uint64_t*>(workspace);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3((unsigned)blocks, (unsigned)M), dim3(256), 0, st, logits,
                       N, partial, 1024);
    hipLaunchKernelGGL(argmax_finalize_kernel, dim3((unsigned)M), dim3(256), 0, st, partial, (int)blocks, 1024,
                       idx);
    return launch_status(what);
}

extern "C" int mq4_swiglu_bf16(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* out,
                               void* stream) {
    const char* what = "mq4_swiglu_bf16";
    if (n < 0) return fail(MQ4_ERR_INVALID_ARG, "%s: negative n", what);
    if (n == 0) return ok();
    if (!gate || !up || !out) return fail(MQ4_ERR_INVALID_ARG, "%s: null pointer", what);
    int64_t blocks = (n + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), gate, up, n,
                       out);
    return launch_status(what);
}

extern "C" int mq4_rms_norm(const uint16_t* x, int64_t M, int64_t K, const uint16_t* weight, float eps,
                            uint16_t* out, void* stream) {
    const char* what = "mq4_rms_norm";
    if (M <= 0 || K <= 0 || M > 0x7fffffffLL || K > 0x7fffffffLL)
        return fail(MQ4_ERR_INVALID_ARG, "%s: M and K must be positive", what);
    if (!x || !weight || !out) return fail(MQ4_ERR_INVALID_ARG, "%s: null pointer", what);
    hipLaunchKernelGGL(rms_norm_1pw_kernel, dim3((unsigned)M), dim3(256), 0, as_stream(stream), x, weight,
                       (int)K, eps, out);
    return launch_status(what);
}
