// MLX-affine Q4 (group 64) quantize/pack, dequantize and the synthetic
// normal generator, for gfx950.
//
// quantize follows mx::quantize(w, 64, 4) as called from quantize_weight
// (src/model/weights.cpp:45-56) and the lm_head load
// (src/model/weights.cpp:180-194); the arithmetic is MLX v0.25.2's CPU affine
// quantize (mlx/backend/cpu/quantized.cpp), restated here in float32 with
// correctly rounded division and round-half-even rint, so that packed words,
// scales and biases are bit-identical.
//
// Layout observation that shapes the kernel: with K % 64 == 0 the groups of a
// row-major [N, K] matrix are consecutive 64-element (128-byte) runs, and the
// packed words, scales and biases of group g sit at wq[8g..8g+7], scales[g],
// biases[g].  So the whole matrix is one flat stream of groups and the kernel
// never needs N or K: four lanes share a group, each reading 32 bytes
// (16 bf16) and writing two packed words per step, and a wave covers 16
// groups = 2 KiB of input per step with coalesced 16-byte loads.
#include "mq4_device.h"
#include "mq4_host.h"

namespace mq4 {

__device__ __forceinline__ float mlx_max(float a, float b) { return (a < b) ? b : a; }
__device__ __forceinline__ float mlx_min(float a, float b) { return (b < a) ? b : a; }

// The correctly rounded quotient d / scale without a division: inv =
// RN(1 / scale) is the correctly rounded reciprocal, q0 = RN(d * inv) is
// within 2 ulps of d / scale, and each correction q' = RN(q + r * inv) with
// the exact FMA residual r = d - q * scale (Markstein's iteration) leaves it
// within 1/2 ulp plus a small fraction after the first step and correctly
// rounded after the second (a quotient of two floats is never a rounding
// midpoint, so no tie can be decided the wrong way).  This holds without
// overflow or underflow; an infinite q0 means |d / scale| > 2^127, whose
// code is the clamp of q0 itself (GUARD), and an underflowing quotient codes
// to 0 either way (|scale| >= 5e-8: the 1e-7 floor, at most halved by the
// edge adjustment).  So rint of this quotient equals rint(d / scale) as MLX
// computes it, element by element.
template <bool GUARD>
__device__ __forceinline__ float quotient(float d, float scale, float inv) {
#pragma clang fp contract(off)
    const float q0 = d * inv;
    if (GUARD && !(fabsf(q0) <= 3.4028234663852886e38f)) return q0;   // +-inf, or NaN from a NaN d
    const float r0 = __builtin_fmaf(-q0, scale, d);
    const float q1 = __builtin_fmaf(r0, inv, q0);
    const float r1 = __builtin_fmaf(-q1, scale, d);
    return __builtin_fmaf(r1, inv, q1);
}

// x / 15 correctly rounded for finite x >= 0, without a division: one
// Markstein step q + RN(x - 15 q) * y from q = RN(x * y), y = RN(1 / 15).
// Checked against IEEE x / 15 for every non-negative finite float
// (subnormals and zero included), with no mismatch.
__device__ __forceinline__ float div15(float x) {
#pragma clang fp contract(off)
    const float y = 0x1.111112p-4f;
    const float q = x * y;
    return __builtin_fmaf(__builtin_fmaf(-q, 15.0f, x), y, q);
}

// The packed words of V consecutive weights f of a group.  The code of each
// weight, clamp(rint(x), 0, 15) of its quotient x = (f - bias) / scale with
// NaN -> 0 (fmaxf/fminf give the same code as MLX's max/min-then-NaN-check),
// lands in the low byte of t: the clamp comes first (to integer bounds, so
// the order does not matter), then rint by adding 1.5 * 2^23, whose float
// sum has unit spacing and rounds half to even, leaving the integer in the
// low mantissa bits (0x4B40000k).  Byte b of word i is then
// (code 8i+2b+1) << 4 | code 8i+2b, gathered by two byte permutes.
template <bool GUARD, int V>
__device__ __forceinline__ void pack_words(const float (&f)[V], float bias, float scale, float inv,
                                           uint32_t (&word)[V / 8]) {
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < V / 8; ++i) {
        uint32_t t[8];
#pragma unroll
        for (int p = 0; p < 8; ++p)
            t[p] = __builtin_bit_cast(
                uint32_t, fminf(fmaxf(quotient<GUARD>(f[8 * i + p] - bias, scale, inv), 0.0f), 15.0f) + 12582912.0f);
        uint32_t u[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) u[b] = (t[2 * b + 1] << 4) | t[2 * b];
        const uint32_t lo = __builtin_amdgcn_perm(u[1], u[0], 0x0c0c0400u);
        const uint32_t hi = __builtin_amdgcn_perm(u[3], u[2], 0x0c0c0400u);
        word[i] = lo | (hi << 16);
    }
}

// LPG lanes (consecutive, all active or all inactive) share a group of 64
// weights, V = 64 / LPG each (v: the lane's V / 8 consecutive 16-byte
// chunks) -> the lane's packed words, and the group's scale and bias (the
// same in every lane of the group).
template <int LPG>
__device__ __forceinline__ void pack_group(const uint4 (&v)[8 / LPG], uint32_t (&word)[8 / LPG],
                                           float& scale_out, float& bias_out) {
#pragma clang fp contract(off)
    constexpr int V = 64 / LPG;
    float f[V];
#pragma unroll
    for (int k = 0; k < V / 8; ++k) {
        f[8 * k + 0] = bf16_to_f32(v[k].x & 0xffffu); f[8 * k + 1] = bf16_to_f32(v[k].x >> 16);
        f[8 * k + 2] = bf16_to_f32(v[k].y & 0xffffu); f[8 * k + 3] = bf16_to_f32(v[k].y >> 16);
        f[8 * k + 4] = bf16_to_f32(v[k].z & 0xffffu); f[8 * k + 5] = bf16_to_f32(v[k].z >> 16);
        f[8 * k + 6] = bf16_to_f32(v[k].w & 0xffffu); f[8 * k + 7] = bf16_to_f32(v[k].w >> 16);
    }
    // Group extremes; NaN never wins (IEEE maxNum/minNum), matching MLX's
    // std::max/std::min scan from -inf/+inf.
    float mx = -__builtin_inff(), mn = __builtin_inff();
#pragma unroll
    for (int p = 0; p < V; ++p) { mx = fmaxf(mx, f[p]); mn = fminf(mn, f[p]); }
#pragma unroll
    for (int m = 1; m < LPG; m <<= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, m));
        mn = fminf(mn, __shfl_xor(mn, m));
    }
    const float n_bins = 15.0f;
    const float eps = 1e-7f;
    // With a finite range max - min every element lies within it, so
    // |d / scale| <= 15 (about 16 after roundings) and no quotient below can
    // overflow; the guards only matter for groups holding an infinity or
    // only NaNs.  The choice is wave-uniform (one branch per wave).
    const float range = mx - mn;
    const bool finite = __all(fabsf(range) <= 3.4028234663852886e38f);
    float scale;
    if (finite)
        scale = mlx_max(div15(range), eps);
    else
        scale = mlx_max(range / n_bins, eps);
    const bool side = fabsf(mn) > fabsf(mx);
    scale = side ? scale : -scale;
    const float edge = side ? mn : mx;
    const float q0 = __builtin_rintf(edge / scale);
    float bias = 0.0f;
    if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
    }
    const float inv = 1.0f / scale;
    if (finite)
        pack_words<false, V>(f, bias, scale, inv, word);
    else
        pack_words<true, V>(f, bias, scale, inv, word);
    scale_out = scale;
    bias_out = bias;
}

// Grid-stride pass over one flat stream of n_groups groups, LPG lanes per
// group and step, the next step's loads issued before this step's
// arithmetic.  Packed words go out as 16-byte stores when wq is 16-byte
// aligned, else as word stores.  Four lanes per group (16 weights, 66
// VGPRs, 7 waves per SIMD) measured fastest on MI355X; with two or one
// lane(s) per group the group's divisions are shared by fewer weights, but
// the 32 or 64 values held per lane cut the resident waves to 4 or 2 and
// the whole weight set took 1045 / 1548 us instead of 844 us.  Addresses
// are 32-bit byte offsets from the (scalar) base pointers, so a stream
// holds fewer than kQuantMaxGroups groups (the host splits longer ones).
constexpr int kQuantLanesPerGroup = 4;
constexpr int64_t kQuantMaxGroups = int64_t(1) << 25;       // 2^25 groups x 128 B = 4 GiB of input
__device__ __forceinline__ void quantize_stream(const uint4* __restrict__ w, uint32_t n_groups,
                                                uint32_t* __restrict__ wq, uint16_t* __restrict__ scales,
                                                uint16_t* __restrict__ biases) {
    constexpr int LPG = kQuantLanesPerGroup, NC = 8 / LPG;      // 16-byte chunks per lane
    const uint32_t stride = gridDim.x * blockDim.x / LPG;
    const bool wide = (reinterpret_cast<uintptr_t>(wq) & 15) == 0;
    const uint32_t part = threadIdx.x % LPG;
    const char* const wb = reinterpret_cast<const char*>(w);
    char* const qb = reinterpret_cast<char*>(wq);
    char* const sb = reinterpret_cast<char*>(scales);
    char* const bb = reinterpret_cast<char*>(biases);
    uint32_t g = (blockIdx.x * blockDim.x + threadIdx.x) / LPG;
    uint4 nxt[NC];
    if (g < n_groups) {
#pragma unroll
        for (int c = 0; c < NC; ++c) nxt[c] = load_nt_u4(reinterpret_cast<const uint4*>(wb + (g * 128u + part * (16u * NC) + c * 16u)));
    }
    for (; g < n_groups; g += stride) {
        uint4 cur[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) cur[c] = nxt[c];
        const uint32_t gn = g + stride;
        if (gn < n_groups) {
#pragma unroll
            for (int c = 0; c < NC; ++c)
                nxt[c] = load_nt_u4(reinterpret_cast<const uint4*>(wb + (gn * 128u + part * (16u * NC) + c * 16u)));
        }
        uint32_t word[NC];
        float scale, bias;
        pack_group<LPG>(cur, word, scale, bias);
        const uint32_t wo = g * 32u + part * (4u * NC);
        if (NC % 4 == 0 && wide) {
#pragma unroll
            for (int c = 0; c < NC; c += 4)
                *reinterpret_cast<uint4*>(qb + (wo + 4u * c)) = make_uint4(word[c], word[c + 1], word[c + 2], word[c + 3]);
        } else {
#pragma unroll
            for (int c = 0; c < NC; ++c) *reinterpret_cast<uint32_t*>(qb + (wo + 4u * c)) = word[c];
        }
        if (part == 0) {
            *reinterpret_cast<uint16_t*>(sb + g * 2u) = (uint16_t)f32_to_bf16(scale);
            *reinterpret_cast<uint16_t*>(bb + g * 2u) = (uint16_t)f32_to_bf16(bias);
        }
    }
}

__global__ __launch_bounds__(256) void quantize_g64_kernel(const uint4* __restrict__ w, uint32_t n_groups,
                                                           uint32_t* __restrict__ wq,
                                                           uint16_t* __restrict__ scales,
                                                           uint16_t* __restrict__ biases) {
    quantize_stream(w, n_groups, wq, scales, biases);
}

// Several matrices in one launch: the jobs' flat streams one after the other
// (every workgroup takes its share of job j, then moves on to job j + 1
// without waiting for the others), so the launch ramp and tail are paid once
// instead of per matrix.  The job table travels in the kernel arguments.
constexpr int kQuantBatch = 32;
struct QuantBatch {
    const uint4* w[kQuantBatch];
    uint32_t* wq[kQuantBatch];
    uint16_t* s[kQuantBatch];
    uint16_t* b[kQuantBatch];
    uint32_t n_groups[kQuantBatch];
    int n;
};

__global__ __launch_bounds__(256) void quantize_g64_batch_kernel(QuantBatch a) {
    for (int j = 0; j < a.n; ++j) quantize_stream(a.w[j], a.n_groups[j], a.wq[j], a.s[j], a.b[j]);
}

// One packed word per lane: 8 outputs = scale * q + bias (q * scale is exact
// for a bf16 scale and a 4-bit q; the add rounds once in float).
template <bool F32>
__global__ __launch_bounds__(256) void dequantize_g64_kernel(const uint32_t* __restrict__ wq,
                                                             const uint16_t* __restrict__ scales,
                                                             const uint16_t* __restrict__ biases,
                                                             int64_t n_words, void* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_words; i += stride) {
        const uint32_t word = wq[i];
        const float s = bf16_to_f32(scales[i >> 3]);
        const float b = bf16_to_f32(biases[i >> 3]);
        float o[8];
#pragma unroll
        for (int p = 0; p < 8; ++p) o[p] = __fmaf_rn(s, (float)((word >> (4 * p)) & 0xfu), b);
        if (F32) {
            float4* dst = reinterpret_cast<float4*>(out) + 2 * i;
            dst[0] = make_float4(o[0], o[1], o[2], o[3]);
            dst[1] = make_float4(o[4], o[5], o[6], o[7]);
        } else {
            uint4 r;
            r.x = f32_to_bf16(o[0]) | (f32_to_bf16(o[1]) << 16);
            r.y = f32_to_bf16(o[2]) | (f32_to_bf16(o[3]) << 16);
            r.z = f32_to_bf16(o[4]) | (f32_to_bf16(o[5]) << 16);
            r.w = f32_to_bf16(o[6]) | (f32_to_bf16(o[7]) << 16);
            reinterpret_cast<uint4*>(out)[i] = r;
        }
    }
}

// ------------------------------------------------------------ generator ---

__device__ __forceinline__ uint64_t sm64_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// double -> bf16 bits in one round-to-nearest-even step (normal range; the
// tiny or non-finite cases go through float).
__device__ __forceinline__ uint32_t f64_to_bf16(double d) {
    const uint64_t u = (uint64_t)__double_as_longlong(d);
    const uint64_t sign = u >> 63;
    const int e = (int)((u >> 52) & 0x7ff);
    const int eb = e - 1023 + 127;
    if (e == 0x7ff || eb <= 0) return f32_to_bf16((float)d);
    uint64_t v = ((uint64_t)eb << 52) | (u & ((1ull << 52) - 1));
    v += (1ull << 44) - 1 + ((v >> 45) & 1ull);
    v >>= 45;
    if (v >= 0xff80ull) v = 0x7f80ull;
    return (uint32_t)((sign << 15) | v);
}

// Element pair j of stream state s0: SplitMix64 outputs 2j and 2j+1 feed one
// Box-Muller draw (cos -> element 2j, sin -> element 2j+1).
__global__ __launch_bounds__(256) void fill_normal_bf16_kernel(uint16_t* __restrict__ out, int64_t n,
                                                               uint64_t s0, double mu, double sigma,
                                                               int64_t offset) {
#pragma clang fp contract(off)
    const uint64_t gamma = 0x9E3779B97F4A7C15ull;
    const double two_pi = 6.283185307179586476925286766559;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t first_pair = offset >> 1;
    const int64_t last_pair = (offset + n - 1) >> 1;
    for (int64_t j = first_pair + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j <= last_pair;
         j += stride) {
        const uint64_t a = sm64_mix(s0 + (uint64_t)(2 * j + 1) * gamma);
        const uint64_t b = sm64_mix(s0 + (uint64_t)(2 * j + 2) * gamma);
        const double u1 = (double)((a >> 11) + 1) * (1.0 / 9007199254740992.0);
        const double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
        const double r = sqrt(-2.0 * log(u1));
        const double t = two_pi * u2;
        const int64_t e0 = 2 * j - offset;
        if (e0 >= 0 && e0 < n) out[e0] = (uint16_t)f64_to_bf16(mu + sigma * (r * cos(t)));
        if (e0 + 1 >= 0 && e0 + 1 < n) out[e0 + 1] = (uint16_t)f64_to_bf16(mu + sigma * (r * sin(t)));
    }
}

static int grid_for(int64_t work_items, int block, int max_blocks) {
    int64_t g = (work_items + block - 1) / block;
    if (g > max_blocks) g = max_blocks;
    if (g < 1) g = 1;
    return (int)g;
}

}  // namespace mq4

using namespace mq4;

extern "C" int mq4_quantize(const uint16_t* w, int64_t N, int64_t K, int group_size, int bits,
                            uint32_t* wq, uint16_t* scales, uint16_t* biases, void* stream) {
    const char* what = "mq4_quantize";
    if (int rc = check_format(what, group_size, bits)) return rc;
    if (int rc = check_k(what, K)) return rc;
    if (N <= 0) return fail(MQ4_ERR_INVALID_ARG, "%s: N=%lld must be positive", what, (long long)N);
    if (!w || !wq || !scales || !biases) return fail(MQ4_ERR_INVALID_ARG, "%s: null pointer", what);
    if (!aligned(w, 16) || !aligned(wq, 4) || !aligned(scales, 2) || !aligned(biases, 2))
        return fail(MQ4_ERR_ALIGNMENT, "%s: w must be 16-byte aligned, wq 4-byte, scales/biases 2-byte",
                    what);
    const int64_t n_groups = N * (K / 64);
    const int block = 256;
    // pieces of at most kQuantMaxGroups groups (32-bit offsets in the kernel)
    for (int64_t g0 = 0; g0 < n_groups; g0 += kQuantMaxGroups) {
        const int64_t n = n_groups - g0 < kQuantMaxGroups ? n_groups - g0 : kQuantMaxGroups;
        const int grid = grid_for(n * kQuantLanesPerGroup, block, 256 * 32);
        hipLaunchKernelGGL(quantize_g64_kernel, dim3(grid), dim3(block), 0, as_stream(stream),
                           reinterpret_cast<const uint4*>(w) + 8 * g0, (uint32_t)n, wq + 8 * g0, scales + g0,
                           biases + g0);
        if (int rc = launch_status(what)) return rc;
    }
    return ok();
}

extern "C" int mq4_quantize_batch(const mq4_quantize_job* jobs, int64_t n_jobs, int group_size, int bits,
                                  void* stream) {
    const char* what = "mq4_quantize_batch";
    if (int rc = check_format(what, group_size, bits)) return rc;
    if (n_jobs < 0 || (n_jobs > 0 && !jobs))
        return fail(MQ4_ERR_INVALID_ARG, "%s: n_jobs=%lld with %s job table", what, (long long)n_jobs,
                    jobs ? "a" : "no");
    for (int64_t j = 0; j < n_jobs; ++j) {
        const mq4_quantize_job& q = jobs[j];
        if (q.K <= 0 || q.K % 64 != 0)
            return fail(MQ4_ERR_INVALID_ARG, "%s: job %lld: K=%lld must be a positive multiple of 64", what,
                        (long long)j, (long long)q.K);
        if (q.N <= 0) return fail(MQ4_ERR_INVALID_ARG, "%s: job %lld: N=%lld must be positive", what, (long long)j,
                                  (long long)q.N);
        if (!q.w || !q.wq || !q.scales || !q.biases)
            return fail(MQ4_ERR_INVALID_ARG, "%s: job %lld: null pointer", what, (long long)j);
        if (!aligned(q.w, 16) || !aligned(q.wq, 4) || !aligned(q.scales, 2) || !aligned(q.biases, 2))
            return fail(MQ4_ERR_ALIGNMENT,
                        "%s: job %lld: w must be 16-byte aligned, wq 4-byte, scales/biases 2-byte", what,
                        (long long)j);
    }
    // the jobs' streams in pieces of at most kQuantMaxGroups groups (32-bit
    // offsets in the kernel), kQuantBatch pieces per launch
    QuantBatch a{};
    auto flush = [&]() -> int {
        if (a.n == 0) return 0;
        // enough lanes to keep HBM busy, not more than the largest piece uses
        int64_t largest = 0;
        for (int i = 0; i < a.n; ++i) largest = a.n_groups[i] > largest ? a.n_groups[i] : largest;
        const int grid = grid_for(largest * kQuantLanesPerGroup, 256, 256 * 32);
        hipLaunchKernelGGL(quantize_g64_batch_kernel, dim3(grid), dim3(256), 0, as_stream(stream), a);
        a = QuantBatch{};
        return launch_status(what);
    };
    for (int64_t j = 0; j < n_jobs; ++j) {
        const mq4_quantize_job& q = jobs[j];
        const int64_t n_groups = q.N * (q.K / 64);
        for (int64_t g0 = 0; g0 < n_groups; g0 += kQuantMaxGroups) {
            const int i = a.n++;
            a.w[i] = reinterpret_cast<const uint4*>(q.w) + 8 * g0;
            a.wq[i] = q.wq + 8 * g0;
            a.s[i] = q.scales + g0;
            a.b[i] = q.biases + g0;
            a.n_groups[i] = (uint32_t)(n_groups - g0 < kQuantMaxGroups ? n_groups - g0 : kQuantMaxGroups);
            if (a.n == kQuantBatch)
                if (int rc = flush()) return rc;
        }
    }
    if (int rc = flush()) return rc;
    return ok();
}

extern "C" int mq4_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                              int64_t N, int64_t K, int group_size, int bits, void* out, int out_f32,
                              void* stream) {
    const char* what = "mq4_dequantize";
    if (int rc = check_format(what, group_size, bits)) return rc;
    if (int rc = check_k(what, K)) return rc;
    if (N <= 0) return fail(MQ4_ERR_INVALID_ARG, "%s: N=%lld must be positive", what, (long long)N);
    if (!wq || !scales || !biases || !out) return fail(MQ4_ERR_INVALID_ARG, "%s: null pointer", what);
    if (!aligned(wq, 4) || !aligned(scales, 2) || !aligned(biases, 2) || !aligned(out, 16))
        return fail(MQ4_ERR_ALIGNMENT, "%s: out must be 16-byte aligned, wq 4-byte", what);
    const int64_t n_words = N * (K / 8);
    const int block = 256;
    const int grid = grid_for(n_words, block, 256 * 32);
    if (out_f32)
        hipLaunchKernelGGL(dequantize_g64_kernel<true>, dim3(grid), dim3(block), 0, as_stream(stream),
                           wq, scales, biases, n_words, out);
    else
        hipLaunchKernelGGL(dequantize_g64_kernel<false>, dim3(grid), dim3(block), 0, as_stream(stream),
                           wq, scales, biases, n_words, out);
    return launch_status(what);
}

extern "C" int mq4_fill_normal_bf16(uint16_t* out, int64_t n, uint64_t seed, uint64_t stream_id,
                                    double mu, double sigma, int64_t offset, void* stream) {
    const char* what = "mq4_fill_normal_bf16";
    if (!out) return fail(MQ4_ERR_INVALID_ARG, "%s: null pointer", what);
    if (n < 0 || offset < 0) return fail(MQ4_ERR_INVALID_ARG, "%s: negative n or offset", what);
    if (n == 0) return ok();
    const int64_t pairs = ((offset + n - 1) >> 1) - (offset >> 1) + 1;
    const int block = 256;
    const int grid = grid_for(pairs, block, 256 * 64);
    hipLaunchKernelGGL(fill_normal_bf16_kernel, dim3(grid), dim3(block), 0, as_stream(stream), out, n,
                       seed ^ stream_id, mu, sigma, offset);
    return launch_status(what);
}
