/*
 * mq4_oracle.c -- CPU restatement of the MLX-affine Q4 path used by marlin-mlx.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP product path.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it, and only to check or to time a CPU baseline.  The product library
 * (libmq4.so) never links, loads or calls anything in this directory.
 *
 * What each function restates (reference paths are relative to the reference
 * repository root):
 *
 *   mq4o_quantize         mx::quantize(w, 64, 4) as called by quantize_weight
 *                         (src/model/weights.cpp:45-56) and by the lm_head load
 *                         (src/model/weights.cpp:180-194).  The arithmetic lives
 *                         in the un-vendored dependency ml-explore/mlx v0.25.2
 *                         (CMakeLists.txt:15-19), CPU backend
 *                         mlx/backend/cpu/quantized.cpp (quantize), restated from
 *                         its published source.
 *   mq4o_qmm_f64          mx::quantized_matmul(x, w, s, b, transpose=true, 64, 4)
 *                         (src/model/marlin.cpp:18-25, 161-169) evaluated exactly
 *                         in fp64 over the dequantized weights (the fp64 oracle).
 *   mq4o_qmm_f64_x32      the same fp64 product on float32 x (the C++ promotion
 *                         reading, in which float32 activations reach qmatmul and
 *                         MLX promotes the bf16 scales and biases to float32).
 *   mq4o_qmm_f32          same product, fp32 accumulation, OpenMP over rows
 *                         (CPU baseline "all cores" mode).
 *   mq4o_qmm_mlx_bf16     the literal scalar loop of MLX's CPU _qmm_t for T=bf16
 *                         (mlx/backend/cpu/quantized.cpp), every op rounded to
 *                         bf16, accumulator of type T (CPU baseline
 *                         "1 thread, MLX order" mode).
 *   mq4o_swiglu_bf16      (sigmoid(g) * g) * u with a bf16 result after each op
 *                         (src/model/marlin.cpp:27-29).
 *   mq4o_argmax_bf16      mx::argmax(last_logits, -1) on bf16 logits
 *                         (src/sampling/sampler.cpp:14-16): strict '>' scan, the
 *                         first index wins ties.
 *   mq4o_rmsnorm_1pw      x * rsqrt(mean(x^2) + eps) * (1 + w)
 *                         (src/model/marlin.cpp:12-16) with the sum of squares
 *                         in fp64, r = 1/sqrtf(mean + eps) and (x*r)*(1+w) in
 *                         fp32, one bf16 rounding: the formula the HIP kernels
 *                         implement (their sum of squares is fp32), and the
 *                         parity target for the fused norm entry points.
 *   mq4o_rmsnorm_mlx      the same rms_norm as the chain of MLX ops it is
 *                         written as (square, mean, + eps, rsqrt, *, 1 + w, *),
 *                         each op producing an array of its MLX result dtype:
 *                         square and mean of a bf16 array are bf16 (mean =
 *                         bf16(sum) * bf16(1/K)); the float scalars eps and
 *                         1.0f are float32 arrays in MLX's C++ API, so from
 *                         "+ eps" on the chain is float32 (flag
 *                         MQ4O_NORM_BF16_OPS instead keeps every op in bf16, the
 *                         reading in which scalars do not promote).  The sum
 *                         inside mean accumulates in fp32 (flag
 *                         MQ4O_NORM_BF16_SUM: a bf16 accumulator, rounded after
 *                         every add).  The float32 result is rounded once to
 *                         bf16, the activation type of this path.  Used to
 *                         bound how far the kernels' formula is from the
 *                         reference's op order (which MLX itself, absent here,
 *                         would fix).
 *   mq4o_add_bf16         hidden + mlp(...) (src/model/marlin.cpp:142) on two
 *                         bf16 arrays: bf16(a + b).
 *   mq4o_gen_normal_bf16  the synthetic-input generator (SplitMix64 counter
 *                         stream -> Box-Muller in fp64 -> mu + sigma*z -> bf16
 *                         round-to-nearest-even directly from fp64).
 *
 * Pinning (see tests/test_oracle_*.py): quantize is pinned by hand-derived
 * known-answer groups, invariants (bias is a group extreme or 0, q in [0,15],
 * the edge element reconstructs exactly) and a brute-force exact-rational
 * nearest-level check; qmm_f64 by exact Fraction arithmetic on tiny shapes and
 * numpy's float64 dot; argmax by numpy.argmax; bf16 rounding by torch's
 * float->bfloat16 cast; the generator by a committed SHA-256 fixture;
 * rmsnorm_1pw by exact known answers on tiny rows (each failing a misplaced
 * eps, a w in place of 1 + w or a mean over the wrong count) and by an
 * independent float64 formula on random rows; rmsnorm_mlx by torch's bf16 and
 * float32 CPU ops replaying the same chain; add_bf16 by torch's bf16 add and by
 * exact rationals.
 * Parity unpinned (needs a run of MLX itself, absent here): the tie-rounding
 * mode MLX uses inside quantize, MLX's bf16 accumulation order in _qmm_t, the
 * exact bf16 bit pattern of MLX's sigmoid, and which rms_norm chain (dtype
 * promotion of the scalars, accumulator of the sum) MLX evaluates; the tests
 * bound the distance between the kernels' formula and each reading instead.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <stddef.h>
#include <string.h>

#define MQ4O_GROUP 64
#define MQ4O_BITS 4

/* ---------------------------------------------------------------- bf16 --- */

static inline float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* float -> bf16, round to nearest even; NaN stays a quiet NaN. */
static inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

/* double -> bf16 with a single round-to-nearest-even step (no detour through
 * float, which could round twice).  Handles the normal bf16 range; values
 * below the smallest normal bf16 go through float (never produced by the
 * generator's distributions). */
static inline uint16_t f64_to_bf16(double d) {
    uint64_t u;
    memcpy(&u, &d, 8);
    uint64_t sign = u >> 63;
    int e = (int)((u >> 52) & 0x7ff);
    if (e == 0x7ff) return f32_to_bf16((float)d);
    int eb = e - 1023 + 127;
    if (eb <= 0) return f32_to_bf16((float)d);
    uint64_t mant = u & ((1ull << 52) - 1);
    uint64_t v = ((uint64_t)eb << 52) | mant;       /* rebias, keep 52-bit mantissa */
    uint64_t lsb = (v >> 45) & 1ull;
    v += (1ull << 44) - 1 + lsb;                    /* RNE at bit 45 */
    v >>= 45;                                       /* 8-bit exp | 7-bit mantissa */
    if (v >= 0xff80ull) v = 0x7f80ull;              /* overflow -> inf */
    return (uint16_t)((sign << 15) | v);
}

uint16_t mq4o_f32_to_bf16(float f) { return f32_to_bf16(f); }
float mq4o_bf16_to_f32(uint16_t h) { return bf16_to_f32(h); }
uint16_t mq4o_f64_to_bf16(double d) { return f64_to_bf16(d); }

void mq4o_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(in[i]);
}
void mq4o_f64_to_bf16_array(const double* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f64_to_bf16(in[i]);
}

/* ----------------------------------------------------------- generator --- */

/* SplitMix64 (Steele, Lea & Flood, OOPSLA 2014), used as a counter-based
 * stream: output i of a stream with state s0 is mix(s0 + (i+1)*gamma). */
static inline uint64_t sm64_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
#define SM64_GAMMA 0x9E3779B97F4A7C15ull

/* Element pair j of stream (seed ^ stream_id): u1 = ((a>>11)+1) * 2^-53 in
 * (0,1], u2 = (b>>11) * 2^-53 in [0,1) with a, b the stream outputs 2j and
 * 2j+1; r = sqrt(-2 ln u1), t = 2*pi*u2; element 2j = mu + sigma*r*cos t,
 * element 2j+1 = mu + sigma*r*sin t, each rounded once to bf16. */
void mq4o_gen_normal_bf16(uint64_t seed, uint64_t stream_id, double mu, double sigma,
                          int64_t offset, int64_t n, uint16_t* out) {
    const uint64_t s0 = seed ^ stream_id;
    const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        int64_t e = offset + i;
        int64_t j = e >> 1;
        uint64_t a = sm64_mix(s0 + (uint64_t)(2 * j + 1) * SM64_GAMMA);
        uint64_t b = sm64_mix(s0 + (uint64_t)(2 * j + 2) * SM64_GAMMA);
        double u1 = (double)((a >> 11) + 1) * (1.0 / 9007199254740992.0);
        double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1));
        double t = two_pi * u2;
        double z = (e & 1) ? r * sin(t) : r * cos(t);
        out[i] = f64_to_bf16(mu + sigma * z);
    }
}

/* ------------------------------------------------------------ quantize --- */

/* MLX affine quantize, one contiguous group of 64 at a time (the groups of a
 * row-major [N, K] array with K % 64 == 0 are simply consecutive 64-element
 * runs).  All arithmetic in float32:
 *   w_max, w_min over the group (max/min ignore NaN);
 *   scale = max((w_max - w_min) / 15, 1e-7);
 *   side  = |w_min| > |w_max|;  scale = side ? scale : -scale;
 *   edge  = side ? w_min : w_max;
 *   q0 = rint(edge / scale);  if q0 != 0 { scale = edge / q0; bias = edge }
 *   else bias = 0;
 *   q_i = clip(rint((w_i - bias) / scale), 0, 15)   (float32 scale)
 *   word j of the group = sum_p q_{8j+p} << 4p  (low nibble first);
 *   stored scale/bias are bf16(scale), bf16(bias) with round-to-nearest-even.
 * rint is round-half-to-even (the default FE_TONEAREST mode). */
static inline float fmax_mlx(float a, float b) { return (a < b) ? b : a; }
static inline float fmin_mlx(float a, float b) { return (b < a) ? b : a; }

void mq4o_quantize_groups(const uint16_t* w, int64_t n_groups, uint32_t* wq,
                          uint16_t* scales, uint16_t* biases) {
    const float n_bins = 15.0f;
    const float eps = 1e-7f;
#pragma omp parallel for schedule(static)
    for (int64_t g = 0; g < n_groups; ++g) {
        const uint16_t* wg = w + g * MQ4O_GROUP;
        float w_min = INFINITY, w_max = -INFINITY;
        for (int j = 0; j < MQ4O_GROUP; ++j) {
            float v = bf16_to_f32(wg[j]);
            w_max = fmax_mlx(w_max, v);
            w_min = fmin_mlx(w_min, v);
        }
        int side = fabsf(w_min) > fabsf(w_max);
        float range = w_max - w_min;
        float scale = fmax_mlx(range / n_bins, eps);
        scale = side ? scale : -scale;
        float edge = side ? w_min : w_max;
        float q0 = rintf(edge / scale);
        float bias = 0.0f;
        if (q0 != 0.0f) {
            scale = edge / q0;
            bias = edge;
        }
        for (int j = 0; j < MQ4O_GROUP / 8; ++j) {
            uint32_t word = 0;
            for (int p = 0; p < 8; ++p) {
                float d = bf16_to_f32(wg[8 * j + p]) - bias;
                float t = d / scale;
                float q = rintf(t);
                q = fmin_mlx(fmax_mlx(q, 0.0f), n_bins);
                uint32_t qi = (q == q) ? (uint32_t)q : 0u;   /* NaN -> 0 */
                word |= qi << (4 * p);
            }
            wq[g * 8 + j] = word;
        }
        scales[g] = f32_to_bf16(scale);
        biases[g] = f32_to_bf16(bias);
    }
}

int mq4o_quantize(const uint16_t* w, int64_t N, int64_t K, uint32_t* wq,
                  uint16_t* scales, uint16_t* biases) {
    if (K % MQ4O_GROUP != 0 || N < 0 || K <= 0) return -1;
    mq4o_quantize_groups(w, N * (K / MQ4O_GROUP), wq, scales, biases);
    return 0;
}

/* Dequantize to fp64: w = s*q + b with s, b the stored bf16 values (exact). */
void mq4o_dequantize_f64(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                         int64_t N, int64_t K, double* out) {
    const int64_t G = K / MQ4O_GROUP;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            uint32_t word = wq[n * (K / 8) + k / 8];
            uint32_t q = (word >> (4 * (k % 8))) & 0xfu;
            double s = bf16_to_f32(scales[n * G + k / MQ4O_GROUP]);
            double b = bf16_to_f32(biases[n * G + k / MQ4O_GROUP]);
            out[n * K + k] = s * (double)q + b;
        }
}

/* ------------------------------------------------------------------ qmm --- */

/* y[m, n] = sum_k x[m, k] * (s[n, k/64] * q[n, k] + b[n, k/64]) in fp64.
 * Every product and partial sum here is exact or rounded at 2^-53, so the
 * result is the true value to ~1e-16 relative; y_bf16 (optional) is its
 * single round-to-nearest-even to bf16. */
void mq4o_qmm_f64(const uint16_t* x, int64_t M, int64_t K, const uint32_t* wq,
                  const uint16_t* scales, const uint16_t* biases, int64_t N,
                  double* y, uint16_t* y_bf16) {
    const int64_t G = K / MQ4O_GROUP;
#pragma omp parallel
    {
        /* row n dequantized once (w = s*q + b, exact in fp64), then dotted with
         * every row of x in k order */
        double* w = (double*)malloc((size_t)K * sizeof(double));
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; ++n) {
            for (int64_t g = 0; g < G; ++g) {
                double s = bf16_to_f32(scales[n * G + g]);
                double b = bf16_to_f32(biases[n * G + g]);
                for (int j = 0; j < 8; ++j) {
                    uint32_t word = wq[n * (K / 8) + g * 8 + j];
                    for (int p = 0; p < 8; ++p) w[g * 64 + j * 8 + p] = s * (double)((word >> (4 * p)) & 0xfu) + b;
                }
            }
            for (int64_t m = 0; m < M; ++m) {
                const uint16_t* xr = x + m * K;
                double acc = 0.0;
                for (int64_t k = 0; k < K; ++k) acc += (double)bf16_to_f32(xr[k]) * w[k];
                if (y) y[m * N + n] = acc;
                if (y_bf16) y_bf16[m * N + n] = f64_to_bf16(acc);
            }
        }
        free(w);
    }
}

/* mx::quantized_matmul on float32 x (src/model/marlin.cpp:18-25 when the
 * activation reaching qmatmul is float32, as in the C++ promotion reading of
 * rms_norm: MLX then promotes the bf16 scales and biases to float32, exactly),
 * evaluated in fp64 over the dequantized weights like mq4o_qmm_f64: each
 * weight row is dequantized once and dotted with every row of x, products and
 * sums in fp64 (y[m, n] is the true value to ~1e-16 relative).  For x whose
 * values are bf16-representable it equals mq4o_qmm_f64 on the same values bit
 * for bit (same terms, same order). */
void mq4o_qmm_f64_x32(const float* x, int64_t M, int64_t K, const uint32_t* wq,
                      const uint16_t* scales, const uint16_t* biases, int64_t N, double* y) {
    const int64_t G = K / MQ4O_GROUP;
#pragma omp parallel
    {
        double* w = (double*)malloc((size_t)K * sizeof(double));
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; ++n) {
            for (int64_t g = 0; g < G; ++g) {
                double s = bf16_to_f32(scales[n * G + g]);
                double b = bf16_to_f32(biases[n * G + g]);
                for (int j = 0; j < 8; ++j) {
                    uint32_t word = wq[n * (K / 8) + g * 8 + j];
                    for (int p = 0; p < 8; ++p) w[g * 64 + j * 8 + p] = s * (double)((word >> (4 * p)) & 0xfu) + b;
                }
            }
            for (int64_t m = 0; m < M; ++m) {
                const float* xr = x + m * K;
                double acc = 0.0;
                for (int64_t k = 0; k < K; ++k) acc += (double)xr[k] * w[k];
                y[m * N + n] = acc;
            }
        }
        free(w);
    }
}

/* fp32 accumulation per row, dequantized weight s*q+b formed in fp32; OpenMP
 * over rows (CPU baseline, all cores). */
void mq4o_qmm_f32(const uint16_t* x, int64_t M, int64_t K, const uint32_t* wq,
                  const uint16_t* scales, const uint16_t* biases, int64_t N,
                  uint16_t* y_bf16) {
    const int64_t G = K / MQ4O_GROUP;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t m = 0; m < M; ++m) {
            const uint16_t* xr = x + m * K;
            float acc = 0.0f;
            for (int64_t g = 0; g < G; ++g) {
                float s = bf16_to_f32(scales[n * G + g]);
                float b = bf16_to_f32(biases[n * G + g]);
                const uint32_t* wr = wq + n * (K / 8) + g * 8;
                for (int j = 0; j < 8; ++j) {
                    uint32_t word = wr[j];
                    for (int p = 0; p < 8; ++p) {
                        float w = s * (float)((word >> (4 * p)) & 0xfu) + b;
                        acc += bf16_to_f32(xr[g * 64 + j * 8 + p]) * w;
                    }
                }
            }
            y_bf16[m * N + n] = f32_to_bf16(acc);
        }
    }
}

/* MLX CPU _qmm_t literal order for T = bf16: the accumulator and every
 * intermediate are bf16 (each binary op computes in float and rounds the
 * result back to bf16).  Single thread. */
static inline uint16_t bmul(uint16_t a, uint16_t b) { return f32_to_bf16(bf16_to_f32(a) * bf16_to_f32(b)); }
static inline uint16_t badd(uint16_t a, uint16_t b) { return f32_to_bf16(bf16_to_f32(a) + bf16_to_f32(b)); }

void mq4o_qmm_mlx_bf16(const uint16_t* x, int64_t M, int64_t K, const uint32_t* wq,
                       const uint16_t* scales, const uint16_t* biases, int64_t N,
                       uint16_t* y_bf16) {
    const int64_t G = K / MQ4O_GROUP;
    for (int64_t m = 0; m < M; ++m) {
        const uint32_t* w_local = wq;
        const uint16_t* s_local = scales;
        const uint16_t* b_local = biases;
        for (int64_t n = 0; n < N; ++n) {
            const uint16_t* x_local = x + m * K;
            uint16_t sum = 0;
            for (int64_t g = 0; g < G; ++g) {
                uint16_t scale = *s_local++;
                uint16_t bias = *b_local++;
                for (int j = 0; j < 8; ++j) {
                    uint32_t wi = *w_local++;
                    for (int p = 0; p < 8; ++p) {
                        uint16_t qv = f32_to_bf16((float)(wi & 0xfu));
                        uint16_t wv = badd(bmul(scale, qv), bias);
                        sum = badd(sum, bmul(*x_local++, wv));
                        wi >>= 4;
                    }
                }
            }
            y_bf16[m * N + n] = sum;
        }
    }
}

/* -------------------------------------------------------- swiglu/argmax --- */

/* (sigmoid(g) * g) * u, bf16 after each op; sigmoid computed in float as
 * 1 / (1 + exp(-g)) and rounded once. */
void mq4o_swiglu_bf16(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) {
        float gv = bf16_to_f32(g[i]);
        uint16_t sg = f32_to_bf16(1.0f / (1.0f + expf(-gv)));
        uint16_t t = f32_to_bf16(bf16_to_f32(sg) * gv);
        out[i] = f32_to_bf16(bf16_to_f32(t) * bf16_to_f32(u[i]));
    }
}

/* argmax over each row of bf16 logits [M, N]: strict '>' scan from index 0,
 * so the lowest index wins ties; NaN never compares greater. */
void mq4o_argmax_bf16(const uint16_t* logits, int64_t M, int64_t N, uint32_t* idx) {
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* r = logits + m * N;
        float best = bf16_to_f32(r[0]);
        uint32_t bi = 0;
        for (int64_t n = 1; n < N; ++n) {
            float v = bf16_to_f32(r[n]);
            if (v > best || (best != best && v == v)) { best = v; bi = (uint32_t)n; }
        }
        idx[m] = bi;
    }
}

/* x * rsqrt(mean(x^2) + eps) * (1 + w) per row, fp32 math, one bf16 rounding. */
void mq4o_rmsnorm_1pw(const uint16_t* x, const uint16_t* w, int64_t M, int64_t K, float eps,
                      uint16_t* out) {
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* xr = x + m * K;
        double ss = 0.0;
        for (int64_t k = 0; k < K; ++k) { float v = bf16_to_f32(xr[k]); ss += (double)v * v; }
        float r = 1.0f / sqrtf((float)(ss / (double)K) + eps);
        for (int64_t k = 0; k < K; ++k)
            out[m * K + k] = f32_to_bf16(bf16_to_f32(xr[k]) * r * (1.0f + bf16_to_f32(w[k])));
    }
}

/* rms_norm as the MLX op chain of src/model/marlin.cpp:12-16 (see the header
 * for the two readings selected by the flags). */
#define MQ4O_NORM_BF16_SUM 1
#define MQ4O_NORM_BF16_OPS 2
void mq4o_rmsnorm_mlx(const uint16_t* x, const uint16_t* w, int64_t M, int64_t K, float eps, int flags,
                      uint16_t* out) {
    const uint16_t inv_k = f32_to_bf16(1.0f / (float)K);        /* array(1.0 / n, bf16) */
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* xr = x + m * K;
        float sumf = 0.0f;
        uint16_t sumb = 0;
        for (int64_t k = 0; k < K; ++k) {
            float v = bf16_to_f32(xr[k]);
            uint16_t sq = f32_to_bf16(v * v);                    /* square: bf16 */
            if (flags & MQ4O_NORM_BF16_SUM) sumb = f32_to_bf16(bf16_to_f32(sumb) + bf16_to_f32(sq));
            else sumf += bf16_to_f32(sq);
        }
        uint16_t sum = (flags & MQ4O_NORM_BF16_SUM) ? sumb : f32_to_bf16(sumf);   /* sum: bf16 */
        uint16_t mean = f32_to_bf16(bf16_to_f32(sum) * bf16_to_f32(inv_k));       /* mean: bf16 */
        if (flags & MQ4O_NORM_BF16_OPS) {
            uint16_t v = f32_to_bf16(bf16_to_f32(mean) + bf16_to_f32(f32_to_bf16(eps)));
            uint16_t r = f32_to_bf16(1.0f / sqrtf(bf16_to_f32(v)));
            for (int64_t k = 0; k < K; ++k) {
                uint16_t t = f32_to_bf16(bf16_to_f32(xr[k]) * bf16_to_f32(r));
                uint16_t w1 = f32_to_bf16(1.0f + bf16_to_f32(w[k]));
                out[m * K + k] = f32_to_bf16(bf16_to_f32(t) * bf16_to_f32(w1));
            }
        } else {
            float v = bf16_to_f32(mean) + eps;                     /* float32 from here on */
            float r = 1.0f / sqrtf(v);
            for (int64_t k = 0; k < K; ++k) {
                float t = bf16_to_f32(xr[k]) * r;
                float w1 = 1.0f + bf16_to_f32(w[k]);
                out[m * K + k] = f32_to_bf16(t * w1);
            }
        }
    }
}

/* bf16 residual add: out = bf16(a + b). */
void mq4o_add_bf16(const uint16_t* a, const uint16_t* b, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(bf16_to_f32(a[i]) + bf16_to_f32(b[i]));
}

/* Threads an OpenMP region of this library uses (for reporting the CPU
 * baseline's core count). */
int mq4o_omp_threads(void) { return omp_get_max_threads(); }
