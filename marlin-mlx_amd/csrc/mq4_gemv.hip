// Decode-shaped (small M) MLX-affine Q4 GEMV kernels for gfx950.
//
// Replaces mx::quantized_matmul(x, w, s, b, transpose=true, 64, 4) at the
// decode call sites: qmatmul (src/model/marlin.cpp:18-25) inside mlp_forward
// (src/model/marlin.cpp:31-35) and MarlinModel::lm_head
// (src/model/marlin.cpp:161-169), plus the fusions of the ops around them:
// swiglu (src/model/marlin.cpp:27-29), the residual add
// (src/model/marlin.cpp:142) and greedy argmax (src/sampling/sampler.cpp:15).
//
// Work decomposition (HBM-bound; every weight byte is read exactly once):
//  * A packed row of K/2 bytes is split into 16-byte slices (4 words = 32 K
//    elements = half a group).  Lane l of K-split wave kw owns slices
//    (kw*SPL + j)*64 + l, j < SPL, for every row it visits, so a wave's 16-byte
//    loads of one row are contiguous (1 KiB per load instruction).
//  * Because a lane's K range never changes, its activations are loaded once
//    and kept in registers, pre-paired as bf16x2 to line up with the nibble
//    pairs (q_p, q_{p+4}) that one AND-OR extracts from a packed word.
//  * Nibbles become bf16 (128 + q) by OR-ing the exponent bits of 128.0, and
//    v_dot2_f32_bf16 accumulates x*(128+q) in fp32.  Per half-group the lane
//    then forms s*D + (b - 128*s)*X with D the dot and X the (precomputed)
//    sum of its 32 activations, i.e. sum_k x_k*(s*q_k + b) with the bias
//    factored out of the inner loop (≈11 VALU ops per packed word).
//  * RPI rows are processed per iteration; the RPI*M (x2 for gate/up) partial
//    sums are reduced across the wave by recursive halving, and across the KS
//    K-split waves of a block through LDS.
#include "mq4_device.h"
#include "mq4_host.h"

namespace mq4 {

enum Epilogue { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2, EPI_ARGMAX = 3, EPI_STORE_F32 = 4 };

struct QMat {
    const uint32_t* wq;
    const uint16_t* s;
    const uint16_t* b;
};

// bf16 SwiGLU in MLX's op order: every intermediate is a bf16 tensor.
__device__ __forceinline__ uint32_t swiglu_bf16(float g_acc, float u_acc) {
#pragma clang fp contract(off)
    const float g = round_bf16(g_acc);
    const float u = round_bf16(u_acc);
    const float sg = round_bf16(1.0f / (1.0f + expf(-g)));
    const float t = round_bf16(sg * g);
    return f32_to_bf16(t * u);
}

template <int M, int SPL, int RPI, int KS, int EPI>
__global__ __launch_bounds__(64 * KS) void q4_gemv_kernel(
    const uint16_t* __restrict__ x, int m_valid, QMat A, QMat B, int N, int K,
    uint16_t* __restrict__ y, const uint16_t* __restrict__ res, uint64_t* __restrict__ partial,
    int partial_stride) {
    constexpr int NMAT = (EPI == EPI_SWIGLU) ? 2 : 1;
    constexpr int V = NMAT * RPI * M;       // values reduced per row batch
    static_assert(V <= 64, "too many values per wave");
    constexpr int LOG2V = log2_const<V>();
    constexpr int SH = 6 - LOG2V;           // lane >> SH = value index after the wave reduce

    const int lane = threadIdx.x & 63;
    const int kw = threadIdx.x >> 6;
    const int L = K >> 5;
    const int G = K >> 6;
    const int64_t row_words = K >> 3;

    // ---- activations of this lane's slices, paired for the nibble layout ----
    uint32_t xp[M][SPL][16];
    float xs[M][SPL];
    int slice[SPL];
    bool valid[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        slice[j] = (kw * SPL + j) * 64 + lane;
        valid[j] = slice[j] < L;
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            float sum = 0.0f;
            if (valid[j] && m < m_valid) {
                const uint4* xv = reinterpret_cast<const uint4*>(x + (int64_t)m * K) + slice[j] * 4;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint4 a = xv[w];
                    xp[m][j][4 * w + 0] = (a.x & 0xffffu) | (a.z << 16);
                    xp[m][j][4 * w + 1] = (a.x >> 16) | (a.z & 0xffff0000u);
                    xp[m][j][4 * w + 2] = (a.y & 0xffffu) | (a.w << 16);
                    xp[m][j][4 * w + 3] = (a.y >> 16) | (a.w & 0xffff0000u);
                    sum += bf16_to_f32(a.x & 0xffffu) + bf16_to_f32(a.x >> 16) +
                           bf16_to_f32(a.y & 0xffffu) + bf16_to_f32(a.y >> 16) +
                           bf16_to_f32(a.z & 0xffffu) + bf16_to_f32(a.z >> 16) +
                           bf16_to_f32(a.w & 0xffffu) + bf16_to_f32(a.w >> 16);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) xp[m][j][i] = 0u;
            }
            xs[m][j] = sum;
        }
    }

    __shared__ float red[(KS > 1) ? KS : 1][V];
    uint64_t best = 0;   // EPI_ARGMAX: running max key of this lane's value slot

    for (int r0 = blockIdx.x * RPI; r0 < N; r0 += gridDim.x * RPI) {
        // ---- stream the packed slices of RPI rows (and both matrices) ----
        uint4 wv[NMAT][RPI][SPL];
        uint32_t sv[NMAT][RPI][SPL], bv[NMAT][RPI][SPL];
#pragma unroll
        for (int t = 0; t < NMAT; ++t) {
            const QMat& Q = (t == 0) ? A : B;
#pragma unroll
            for (int r = 0; r < RPI; ++r) {
                const int row = r0 + r;
#pragma unroll
                for (int j = 0; j < SPL; ++j) {
                    if (row < N && valid[j]) {
                        wv[t][r][j] = load_nt_u4(
                            reinterpret_cast<const uint4*>(Q.wq + (int64_t)row * row_words) + slice[j]);
                        sv[t][r][j] = Q.s[(int64_t)row * G + (slice[j] >> 1)];
                        bv[t][r][j] = Q.b[(int64_t)row * G + (slice[j] >> 1)];
                    } else {
                        wv[t][r][j] = make_uint4(0u, 0u, 0u, 0u);
                        sv[t][r][j] = 0u;
                        bv[t][r][j] = 0u;
                    }
                }
            }
        }

        // ---- dot products: value index v = (r*M + m)*NMAT + t ----
        float acc[V];
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = 0.0f;
#pragma unroll
        for (int t = 0; t < NMAT; ++t) {
#pragma unroll
            for (int r = 0; r < RPI; ++r) {
#pragma unroll
                for (int j = 0; j < SPL; ++j) {
                    float d[M];
#pragma unroll
                    for (int m = 0; m < M; ++m) d[m] = 0.0f;
                    const uint32_t wd[4] = {wv[t][r][j].x, wv[t][r][j].y, wv[t][r][j].z, wv[t][r][j].w};
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
                    const float s = bf16_to_f32(sv[t][r][j]);
                    const float c = bf16_to_f32(bv[t][r][j]) - 128.0f * s;
#pragma unroll
                    for (int m = 0; m < M; ++m)
                        acc[(r * M + m) * NMAT + t] += s * d[m] + c * xs[m][j];
                }
            }
        }

        // ---- reduce across the wave, then across the K-split waves ----
        float val = wave_multi_reduce<V>(acc, lane);
        int vidx = lane >> SH;                 // value index held by this lane
        bool holder = (lane & ((1 << SH) - 1)) == 0;
        if (KS > 1) {
            if (holder) red[kw][vidx] = val;
            __syncthreads();
            if (kw == 0) {
                vidx = lane;
                holder = lane < V;
                float s = 0.0f;
                if (holder) {
#pragma unroll
                    for (int k = 0; k < KS; ++k) s += red[k][lane];
                }
                val = s;
            }
            __syncthreads();
            if (kw != 0) continue;   // block-uniform loop: all waves still take every iteration
        }

        // ---- epilogue ----
        float other = 0.0f;
        if (EPI == EPI_SWIGLU) {
            // the up-projection partner of value index v is v ^ 1
            const int partner_off = (KS > 1) ? 1 : (1 << SH);
            other = __shfl_xor(val, partner_off);
        }
        const int t_mat = vidx % NMAT;
        const int m = (vidx / NMAT) % M;
        const int r = vidx / (NMAT * M);
        const int row = r0 + r;
        const bool live = holder && row < N && m < m_valid && (EPI != EPI_SWIGLU || t_mat == 0);
        if (EPI == EPI_STORE) {
            if (live) y[(int64_t)m * N + row] = (uint16_t)f32_to_bf16(val);
        } else if (EPI == EPI_STORE_F32) {
            if (live) reinterpret_cast<float*>(y)[(int64_t)m * N + row] = val;
        } else if (EPI == EPI_RESIDUAL) {
            if (live) {
                const float rsd = bf16_to_f32(res[(int64_t)m * N + row]);
                y[(int64_t)m * N + row] = (uint16_t)f32_to_bf16(rsd + round_bf16(val));
            }
        } else if (EPI == EPI_SWIGLU) {
            if (live) y[(int64_t)m * N + row] = (uint16_t)swiglu_bf16(val, other);
        } else {  // EPI_ARGMAX
            const uint32_t lb = f32_to_bf16(val);
            if (live) {
                if (y) y[(int64_t)m * N + row] = (uint16_t)lb;
                const uint64_t key = argmax_key(lb, (uint32_t)row);
                best = key > best ? key : best;
            }
        }
    }

    if (EPI == EPI_ARGMAX) {
        // Only wave 0 carries results when KS > 1.
        if (KS > 1 && kw != 0) return;
        // Lane -> m mapping: KS == 1: m = (lane >> SH) % M; KS > 1: m = lane % M.
        // Max-reduce over every lane bit that does not encode m.
        const int mshift = (KS > 1) ? 0 : SH;
        const int mbits = log2_const<M>();
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const bool is_m_bit = off >= (1 << mshift) && off < (1 << (mshift + mbits));
            if (!is_m_bit) {
                const uint64_t o = shfl_xor_u64(best, off);
                best = o > best ? o : best;
            }
        }
        const int m = (lane >> mshift) & (M - 1);
        if ((lane & ~((M - 1) << mshift)) == 0 && m < m_valid)
            partial[(int64_t)m * partial_stride + blockIdx.x] = best;
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

// ------------------------------------------------------------ dispatch ---

constexpr int kMaxGemvBlocks = 4096;     // also the argmax partial stride
constexpr int kRPI = 4;

struct GemvArgs {
    const uint16_t* x;
    int m_valid;
    QMat A, B;
    int N, K;
    uint16_t* y;
    const uint16_t* res;
    uint64_t* partial;
};

template <int M, int SPL, int KS, int EPI>
static void launch_gemv(const GemvArgs& a, hipStream_t st) {
    constexpr int RPI = (EPI == EPI_SWIGLU && M == 4) ? 2 : kRPI;
    int64_t batches = ((int64_t)a.N + RPI - 1) / RPI;
    // About 16 waves per CU at the cap; the argmax partial buffer has one
    // slot per block, so its grid is capped at the partial stride.
    int cap = (KS > 1) ? (16 * 256) / KS : kMaxGemvBlocks;
    if (EPI == EPI_ARGMAX) cap = kMaxGemvBlocks;
    int grid = (int)(batches < cap ? batches : cap);
    if (grid < 1) grid = 1;
    hipLaunchKernelGGL((q4_gemv_kernel<M, SPL, RPI, KS, EPI>), dim3(grid), dim3(64 * KS), 0, st, a.x,
                       a.m_valid, a.A, a.B, a.N, a.K, a.y, a.res, a.partial, kMaxGemvBlocks);
}

// Pick (SPL, KS) from the number of 16-byte slices per row L = K/32.
template <int M, int EPI>
static int dispatch_k(const GemvArgs& a, hipStream_t st) {
    const int L = a.K / 32;
    if (L <= 64) { launch_gemv<M, 1, 1, EPI>(a, st); return 0; }
    if (L <= 128) { launch_gemv<M, 1, 2, EPI>(a, st); return 0; }
    if (L <= 192) { launch_gemv<M, 1, 3, EPI>(a, st); return 0; }
    if (L <= 256) { launch_gemv<M, 1, 4, EPI>(a, st); return 0; }
    if (L <= 512) { launch_gemv<M, 1, 8, EPI>(a, st); return 0; }
    if constexpr (M == 1) {
        if (L <= 1024) { launch_gemv<M, 2, 8, EPI>(a, st); return 0; }
        if (L <= 2048) { launch_gemv<M, 4, 8, EPI>(a, st); return 0; }
    }
    return -1;
}

template <int EPI>
static int run_gemv(const GemvArgs& base, int M, hipStream_t st) {
    // Rows of x are processed in chunks of at most 4 (of 1 when K > 16384,
    // where four rows of activations would not fit the register file).
    const int chunk = (base.K / 32 > 512) ? 1 : 4;
    for (int m0 = 0; m0 < M; m0 += chunk) {
        GemvArgs a = base;
        const int mc = (M - m0) < chunk ? (M - m0) : chunk;
        a.x = base.x + (int64_t)m0 * base.K;
        a.m_valid = mc;
        if (base.y) a.y = base.y + (int64_t)m0 * base.N * (EPI == EPI_STORE_F32 ? 2 : 1);
        if (base.res) a.res = base.res + (int64_t)m0 * base.N;
        if (base.partial) a.partial = base.partial + (int64_t)m0 * kMaxGemvBlocks;
        int rc;
        if (mc == 1) rc = dispatch_k<1, EPI>(a, st);
        else if (mc == 2) rc = dispatch_k<2, EPI>(a, st);
        else rc = dispatch_k<4, EPI>(a, st);
        if (rc) return rc;
    }
    return 0;
}

static int check_qmm_args(const char* what, const uint16_t* x, int64_t M, int64_t K, const uint32_t* wq,
                          const uint16_t* s, const uint16_t* b, int64_t N) {
    if (int rc = check_k(what, K)) return rc;
    if (M <= 0 || N <= 0)
        return fail(MQ4_ERR_INVALID_ARG, "%s: M=%lld and N=%lld must be positive", what, (long long)M,
                    (long long)N);
    if (K > 65536)
        return fail(MQ4_ERR_UNSUPPORTED, "%s: K=%lld exceeds the supported maximum 65536", what,
                    (long long)K);
    if (N > 0x7fffffffLL) return fail(MQ4_ERR_UNSUPPORTED, "%s: N too large", what);
    if (!x || !wq || !s || !b) return fail(MQ4_ERR_INVALID_ARG, "%s: null pointer", what);
    if (!aligned(x, 16) || !aligned(wq, 16) || !aligned(s, 2) || !aligned(b, 2))
        return fail(MQ4_ERR_ALIGNMENT, "%s: x and wq must be 16-byte aligned, scales/biases 2-byte",
                    what);
    return MQ4_OK;
}

}  // namespace mq4

using namespace mq4;

extern "C" int mq4_qmm(const uint16_t* x, int64_t M, int64_t K, const uint32_t* wq,
                       const uint16_t* scales, const uint16_t* biases, int64_t N, int transpose,
                       int group_size, int bits, uint16_t* y, void* stream) {
    const char* what = "mq4_qmm";
    if (int rc = check_format(what, group_size, bits)) return rc;
    if (transpose != 1)
        return fail(MQ4_ERR_UNSUPPORTED, "%s: only transpose=1 (x @ W^T) is implemented", what);
    if (int rc = check_qmm_args(what, x, M, K, wq, scales, biases, N)) return rc;
    if (!y || !aligned(y, 2)) return fail(MQ4_ERR_INVALID_ARG, "%s: y must be a 2-byte aligned pointer", what);
    GemvArgs a{x, (int)M, {wq, scales, biases}, {nullptr, nullptr, nullptr}, (int)N, (int)K, y, nullptr,
               nullptr};
    if (run_gemv<EPI_STORE>(a, (int)M, as_stream(stream)))
        return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported K", what);
    return launch_status(what);
}

extern "C" int mq4_qmm_f32(const uint16_t* x, int64_t M, int64_t K, const uint32_t* wq,
                           const uint16_t* scales, const uint16_t* biases, int64_t N, float* y,
                           void* stream) {
    const char* what = "mq4_qmm_f32";
    if (int rc = check_qmm_args(what, x, M, K, wq, scales, biases, N)) return rc;
    if (!y || !aligned(y, 4)) return fail(MQ4_ERR_INVALID_ARG, "%s: y must be a 4-byte aligned pointer", what);
    GemvArgs a{x, (int)M, {wq, scales, biases}, {nullptr, nullptr, nullptr}, (int)N, (int)K,
               reinterpret_cast<uint16_t*>(y), nullptr, nullptr};
    if (run_gemv<EPI_STORE_F32>(a, (int)M, as_stream(stream)))
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
    GemvArgs a{x, (int)M, {wq, scales, biases}, {nullptr, nullptr, nullptr}, (int)N, (int)K, y, residual,
               nullptr};
    if (run_gemv<EPI_RESIDUAL>(a, (int)M, as_stream(stream)))
        return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported K", what);
    return launch_status(what);
}

extern "C" int mq4_mlp_gate_up_silu(const uint16_t* x, int64_t M, int64_t K, const uint32_t* gate_wq,
                                    const uint16_t* gate_scales, const uint16_t* gate_biases,
                                    const uint32_t* up_wq, const uint16_t* up_scales,
                                    const uint16_t* up_biases, int64_t N, uint16_t* h, void* stream) {
    const char* what = "mq4_mlp_gate_up_silu";
    if (int rc = check_qmm_args(what, x, M, K, gate_wq, gate_scales, gate_biases, N)) return rc;
    if (int rc = check_qmm_args(what, x, M, K, up_wq, up_scales, up_biases, N)) return rc;
    if (!h || !aligned(h, 2)) return fail(MQ4_ERR_INVALID_ARG, "%s: h must be a 2-byte aligned pointer", what);
    GemvArgs a{x, (int)M, {gate_wq, gate_scales, gate_biases}, {up_wq, up_scales, up_biases}, (int)N, (int)K,
               h, nullptr, nullptr};
    if (run_gemv<EPI_SWIGLU>(a, (int)M, as_stream(stream)))
        return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported K", what);
    return launch_status(what);
}

extern "C" size_t mq4_lm_head_argmax_workspace_size(int64_t M, int64_t N) {
    (void)N;
    if (M <= 0) return 0;
    return (size_t)M * kMaxGemvBlocks * sizeof(uint64_t);
}

extern "C" int mq4_lm_head_argmax(const uint16_t* h, int64_t M, int64_t K, const uint32_t* wq,
                                  const uint16_t* scales, const uint16_t* biases, int64_t N,
                                  uint32_t* idx, uint16_t* logits, void* workspace,
                                  size_t workspace_bytes, void* stream) {
    const char* what = "mq4_lm_head_argmax";
    if (int rc = check_qmm_args(what, h, M, K, wq, scales, biases, N)) return rc;
    if (!idx || !aligned(idx, 4)) return fail(MQ4_ERR_INVALID_ARG, "%s: idx must be a 4-byte aligned pointer", what);
    if (logits && !aligned(logits, 2)) return fail(MQ4_ERR_ALIGNMENT, "%s: logits must be 2-byte aligned", what);
    if (!workspace || workspace_bytes < mq4_lm_head_argmax_workspace_size(M, N) || !aligned(workspace, 8))
        return fail(MQ4_ERR_WORKSPACE, "%s: workspace needs %zu bytes, 8-byte aligned (got %zu)", what,
                    mq4_lm_head_argmax_workspace_size(M, N), workspace_bytes);
    uint64_t* partial = reinterpret_cast<uint64_t*>(workspace);
    GemvArgs a{h, (int)M, {wq, scales, biases}, {nullptr, nullptr, nullptr}, (int)N, (int)K, logits, nullptr,
               partial};
    hipStream_t st = as_stream(stream);
    if (run_gemv<EPI_ARGMAX>(a, (int)M, st)) return fail(MQ4_ERR_UNSUPPORTED, "%s: unsupported K", what);
    // Every block of the GEMV wrote its partial; blocks = min(row batches, cap).
    const int64_t batches = (N + kRPI - 1) / kRPI;
    const int count = (int)(batches < kMaxGemvBlocks ? batches : kMaxGemvBlocks);
    hipLaunchKernelGGL(argmax_finalize_kernel, dim3((unsigned)M), dim3(256), 0, st, partial, count,
                       kMaxGemvBlocks, idx);
    return launch_status(what);
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
    if (N > 0x7fffffffLL) return fail(MQ4_ERR_UNSUPPORTED, "%s: N too large", what);
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
