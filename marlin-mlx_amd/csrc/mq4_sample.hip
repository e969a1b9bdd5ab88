// Stochastic sample_token for gfx950: temperature, top-k, top-p and a
// categorical draw over bf16 logits, one workgroup per row.
//
// Restates src/sampling/sampler.cpp:18-39 (the branch taken when
// temperature > 0):
//   scaled = last_logits / temperature                       (float32)
//   top_k > 0:  scaled = where(scaled < min(topk(scaled, k)), -inf, scaled)
//   0 < top_p < 1:
//     probs = softmax(scaled); order = argsort(probs) (ascending)
//     mask  = cumsum(probs[order]) - probs[order] > top_p, scattered back
//     scaled = where(mask, -inf, scaled)
//   token = categorical(log(softmax(scaled)))
// The sort is ascending, so an element is masked when the probability mass
// of all smaller elements exceeds top_p: the mask removes the largest
// probabilities and keeps the low tail.  That is the reference's behaviour
// and it is kept as is.  With temperature <= 0 the row's greedy argmax is
// returned (sampler.cpp:14-16), lowest index among equal maxima.
//
// How each step is computed:
//  * Division by a positive temperature is monotone, so the order of
//    `scaled` is the order of the 16-bit order keys of the logits
//    (bf16_order_key; NaN is key 0 and never kept).  top-k: the k-th largest
//    key by a two-pass radix select (256-bin histograms of the high, then the
//    low key byte); keys below it are masked (ties at the k-th value are kept,
//    as `scaled < min_val` keeps them).
//  * top-p: e = exp(scaled - max) of every element top-k kept, in fixed point
//    (round(e * 2^40) in 64-bit integers, so every sum is exact and the same
//    in any summation order; N <= 2^23 keeps the total below 2^63).  The
//    largest key k* whose preceding mass E(< k*) is <= top_p * Z is found by
//    two radix passes over per-byte mass histograms; keys below k* are kept,
//    keys above are masked, and of the elements equal to k* (equal
//    probabilities) the first r in index order are kept, r the count with
//    E(< k*) + t * e(k*) <= top_p * Z for t = 0..r-1 (argsort taken as
//    stable, so equal probabilities keep index order).  The reference sums in
//    float32, so the two agree except where a cumulative sum lies within
//    float32 rounding of top_p.
//  * The categorical draw is Gumbel-max, the method mx::random::categorical
//    uses: argmax over kept i of scaled_i + g_i, g_i = -log(-log(u_i));
//    log(softmax(scaled)) and scaled differ by a per-row constant.  u_i comes
//    from this library's counter-based generator (SplitMix64 finaliser of
//    seed, row and i), not MLX's key stream, so draws match the reference in
//    distribution, not bit for bit; the draw is a pure function of (logits,
//    parameters, seed, row, i) and does not depend on the launch shape.
//
// Layout: wave w of the 16 owns the contiguous index range [w*S, (w+1)*S);
// within it the lanes read 64*VEC consecutive logits per step (VEC = 8: one
// 16-byte load per lane), so index order inside a wave is (step, lane,
// element) and the tie ranks of the top-p boundary come from a lane prefix
// sum plus per-wave offsets.  Every pass reads the row from L2 (a row of
// 151936 logits is 297 KiB, more than the LDS).
#include "mq4_device.h"
#include "mq4_host.h"

namespace mq4 {

namespace smp {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr double kFix = 1099511627776.0;   // 2^40: fixed-point scale of exp(scaled - max) in [0, 1]
// Upper bound of the Gumbel noise: u <= 1 - 2^-24 gives -log(-log(u)) < 16.7.
constexpr float kGumbelMax = 18.0f;

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Uniform on the 2^23 points (j + 1/2) * 2^-23 of (0, 1) for element i of
// row m: 23 random bits, so j + 1/2 is exact in float32 and u is never 0 or 1
// (the resolution of a float32 uniform in [0, 1), which MLX's gumbel uses).
__device__ __forceinline__ float uniform01(uint64_t seed, int64_t m, int64_t i) {
    const uint64_t state = mix64(seed ^ ((uint64_t)(m + 1) * 0xD1B54A32D192ED03ull));
    const uint64_t z = mix64(state + (uint64_t)(i + 1) * 0x9E3779B97F4A7C15ull);
    return ((float)(z >> 41) + 0.5f) * 1.1920928955078125e-7f;     // 2^-23
}

__device__ __forceinline__ float scaled_of(uint32_t h, float temperature) {
    return bf16_to_f32(h & 0xffffu) / temperature;
}

// bf16 bits of the value whose order key is `key` (the inverse of
// bf16_order_key for keys >= 1).
__device__ __forceinline__ uint32_t bf16_of_key(uint32_t key) {
    return (key & 0x8000u) ? (key & 0x7fffu) : (~key & 0xffffu);
}

// Fixed-point probability weight of scaled value s: round(exp(s - smax) * 2^40).
__device__ __forceinline__ uint64_t fixed_mass(float s, float smax) {
#pragma clang fp contract(off)
    return (uint64_t)((double)expf(s - smax) * kFix + 0.5);
}

// The Gumbel-perturbed value of kept element i (scaled value s) and its
// 64-bit draw key: the float's order key in the high word, ~i in the low word
// (the lowest index wins equal values).
__device__ __forceinline__ uint64_t draw_key(float s, uint64_t seed, int64_t m, int64_t i, float* val) {
#pragma clang fp contract(off)
    const float g = -logf(-logf(uniform01(seed, m, i)));
    const float v = s + g;
    const uint32_t fb = __float_as_uint(v);
    const uint32_t fk = (fb & 0x80000000u) ? ~fb : (fb | 0x80000000u);
    *val = v;
    return ((uint64_t)fk << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
}

// Eight keep flags (bit e of keepbits) as eight bytes at an 8-byte aligned kp.
__device__ __forceinline__ void store_keep8(uint8_t* kp, uint32_t keepbits) {
    uint2 w;
    w.x = ((keepbits >> 0) & 1u) | (((keepbits >> 1) & 1u) << 8) | (((keepbits >> 2) & 1u) << 16) |
          (((keepbits >> 3) & 1u) << 24);
    w.y = ((keepbits >> 4) & 1u) | (((keepbits >> 5) & 1u) << 8) | (((keepbits >> 6) & 1u) << 16) |
          (((keepbits >> 7) & 1u) << 24);
    *reinterpret_cast<uint2*>(kp) = w;
}

__device__ __forceinline__ uint64_t shfl_up_u64(uint64_t v, int d) {
    const uint32_t lo = __shfl_up((uint32_t)v, d);
    const uint32_t hi = __shfl_up((uint32_t)(v >> 32), d);
    return ((uint64_t)hi << 32) | lo;
}

// Block-wide sum / max of one value per thread over NW waves; tmp holds NW
// words of LDS.  Every thread gets the result; both contain barriers.
template <int NW>
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t* tmp) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += shfl_xor_u64(v, off);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) tmp[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t t = 0;
    for (int i = 0; i < NW; ++i) t += tmp[i];
    return t;
}

template <int NW>
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* tmp) {
    v = wave_max_u64(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) tmp[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t t = 0;
    for (int i = 0; i < NW; ++i) t = tmp[i] > t ? tmp[i] : t;
    return t;
}

// Wave 0: over 256 count bins, the largest b with count(bins >= b) >= need
// (need >= 1 and the total >= need); out[0] = b, out[1] = count(bins > b).
__device__ void select_top_bin(const uint32_t* hist, uint32_t need, uint32_t* out) {
    const int lane = threadIdx.x & 63;
    uint32_t h[4], t = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) { h[j] = hist[4 * lane + j]; t += h[j]; }
    // inclusive suffix sum over lanes (lane l: sum of lanes >= l)
    uint32_t suf = t;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = __shfl_down(suf, d);
        if (lane + d < 64) suf += o;
    }
    uint32_t above = suf - t;                // bins of lanes > l
    uint32_t cand = 0, cabove = 0;           // 1 + the largest bin of this lane meeting need
#pragma unroll
    for (int j = 3; j >= 0; --j) {
        if (!cand && above + h[j] >= need) { cand = 4 * lane + j + 1; cabove = above; }
        above += h[j];
    }
    const uint64_t best = wave_max_u64(((uint64_t)cand << 32) | cabove);
    if (lane == 0) { out[0] = (uint32_t)(best >> 32) - 1u; out[1] = (uint32_t)best; }
}

// Wave 0: over 256 mass bins with `base` mass before bin 0, the largest bin
// b with mass[b] != 0 and base + mass(bins < b) <= limit (bins ascending);
// out[0] = b (or ~0 if none), out[1] = base + mass(bins < b).
__device__ void select_mass_bin(const unsigned long long* mass, uint64_t base, uint64_t limit, uint64_t* out) {
    const int lane = threadIdx.x & 63;
    uint64_t h[4], t = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) { h[j] = mass[4 * lane + j]; t += h[j]; }
    uint64_t pre = t;                        // inclusive prefix over lanes
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint64_t o = shfl_up_u64(pre, d);
        if (lane >= d) pre += o;
    }
    uint64_t before = base + pre - t;
    uint64_t cand = 0, cbefore = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (h[j] != 0 && before <= limit) { cand = 4 * lane + j + 1; cbefore = before; }
        before += h[j];
    }
    // the candidate with the largest bin also has the largest `before`
    const uint64_t best = wave_max_u64(cand);
    const int src = best ? (int)((best - 1) >> 2) : 0;
    const uint64_t bb = ((uint64_t)__shfl((uint32_t)(cbefore >> 32), src) << 32) | __shfl((uint32_t)cbefore, src);
    if (lane == 0) { out[0] = best ? best - 1 : ~0ull; out[1] = bb; }
}

// Calls f(i0, v, ok) once per step for every lane of the calling wave
// (wave-uniform trip count): v[0..VEC) are logits i0..i0+VEC-1 when ok.
template <int VEC, class F>
__device__ __forceinline__ void for_each_step(const uint16_t* __restrict__ row, int64_t N, int64_t S, F&& f) {
    const int lane = threadIdx.x & 63;
    const int64_t beg = (int64_t)(threadIdx.x >> 6) * S;
    const int64_t end = beg + S < N ? beg + S : N;
    for (int64_t b = beg; b < end; b += 64 * VEC) {
        const int64_t i0 = b + (int64_t)lane * VEC;
        const bool ok = i0 < end;
        uint32_t v[VEC];
        if constexpr (VEC == 8) {
            uint4 q = make_uint4(0, 0, 0, 0);
            if (ok) q = *reinterpret_cast<const uint4*>(row + i0);
            v[0] = q.x & 0xffffu; v[1] = q.x >> 16; v[2] = q.y & 0xffffu; v[3] = q.y >> 16;
            v[4] = q.z & 0xffffu; v[5] = q.z >> 16; v[6] = q.w & 0xffffu; v[7] = q.w >> 16;
        } else {
            v[0] = ok ? (uint32_t)row[i0] : 0u;
        }
        f(i0, v, ok);
    }
}

template <int VEC>
__global__ __launch_bounds__(kThreads) void sample_kernel(const uint16_t* __restrict__ logits, int64_t N, int64_t S,
                                                          float temperature, int top_k, float top_p, uint64_t seed,
                                                          uint32_t* __restrict__ idx, uint8_t* __restrict__ keep_out) {
#pragma clang fp contract(off)
    const int64_t m = blockIdx.x;
    const uint16_t* row = logits + m * N;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ uint32_t hist[256];
    __shared__ unsigned long long mass[256];
    __shared__ uint32_t wcnt[kWaves][256];
    __shared__ uint64_t tmp[kWaves];
    __shared__ uint64_t sel[2];
    __shared__ uint32_t selk[2];
    __shared__ uint32_t woff[kWaves];

    if (!(temperature > 0.0f)) {                       // greedy
        uint64_t best = 0;
        for_each_step<VEC>(row, N, S, [&](int64_t i0, const uint32_t* v, bool ok) {
            if (!ok) return;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const uint64_t k = argmax_key(v[e], (uint32_t)(i0 + e));
                best = k > best ? k : best;
            }
        });
        best = block_max_u64<kWaves>(best, tmp);
        if (tid == 0) idx[m] = best ? argmax_key_index(best) : 0u;
        return;
    }

    // ---- pass 1: largest key, and the top-k high-byte histogram ----
    const bool use_k = top_k > 0 && (int64_t)top_k < N;
    if (use_k)
        for (int i = tid; i < 256; i += kThreads) hist[i] = 0;
    __syncthreads();
    uint64_t mk = 0;
    for_each_step<VEC>(row, N, S, [&](int64_t, const uint32_t* v, bool ok) {
        if (!ok) return;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const uint32_t k = bf16_order_key(v[e]);
            mk = k > mk ? k : mk;
            if (use_k) atomicAdd(&hist[k >> 8], 1u);
        }
    });
    const uint32_t kmax = (uint32_t)block_max_u64<kWaves>(mk, tmp);   // its barriers also complete hist

    // ---- top-k: keys below kmin are masked (kmin = 1 masks NaN only) ----
    uint32_t kmin = 1;
    if (use_k) {
        if (wave == 0) select_top_bin(hist, (uint32_t)top_k, selk);
        __syncthreads();
        const uint32_t hb = selk[0], above = selk[1];
        for (int i = tid; i < 256; i += kThreads) hist[i] = 0;
        __syncthreads();
        for_each_step<VEC>(row, N, S, [&](int64_t, const uint32_t* v, bool ok) {
            if (!ok) return;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const uint32_t k = bf16_order_key(v[e]);
                if ((k >> 8) == hb) atomicAdd(&hist[k & 0xffu], 1u);
            }
        });
        __syncthreads();
        if (wave == 0) select_top_bin(hist, (uint32_t)top_k - above, selk);
        __syncthreads();
        kmin = (hb << 8) | selk[0];
        if (kmin == 0) kmin = 1;
    }
    if (kmax < kmin) {                                 // nothing but NaN
        if (tid == 0) idx[m] = 0u;
        if (keep_out)
            for (int64_t i = tid; i < N; i += kThreads) keep_out[m * N + i] = 0;
        return;
    }
    const float smax = scaled_of(bf16_of_key(kmax), temperature);
    auto fixed_e = [&](float s) -> uint64_t { return fixed_mass(s, smax); };

    // ---- top-p: keys above kstar masked, the first tie_keep ties at kstar kept ----
    uint32_t kstar = 0xffffu;
    int64_t tie_keep = -1;                             // -1: every element equal to kstar is kept
    if (top_p > 0.0f && top_p < 1.0f) {
        for (int i = tid; i < 256; i += kThreads) mass[i] = 0;
        for (int i = tid; i < kWaves * 256; i += kThreads) (&wcnt[0][0])[i] = 0;
        __syncthreads();
        uint64_t z = 0;
        for_each_step<VEC>(row, N, S, [&](int64_t, const uint32_t* v, bool ok) {
            if (!ok) return;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const uint32_t k = bf16_order_key(v[e]);
                if (k < kmin) continue;
                const uint64_t f = fixed_e(scaled_of(v[e], temperature));
                z += f;
                if (f) atomicAdd(&mass[k >> 8], (unsigned long long)f);
            }
        });
        const uint64_t Z = block_sum_u64<kWaves>(z, tmp);      // its barriers also complete mass
        const uint64_t limit = (uint64_t)((double)top_p * (double)Z);
        if (wave == 0) select_mass_bin(mass, 0, limit, sel);
        __syncthreads();
        const uint32_t hb = (uint32_t)sel[0];
        const uint64_t before_hb = sel[1];
        __syncthreads();
        for (int i = tid; i < 256; i += kThreads) mass[i] = 0;
        __syncthreads();
        for_each_step<VEC>(row, N, S, [&](int64_t, const uint32_t* v, bool ok) {
            if (!ok) return;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const uint32_t k = bf16_order_key(v[e]);
                if (k < kmin || (k >> 8) != hb) continue;
                const uint64_t f = fixed_e(scaled_of(v[e], temperature));
                if (f) atomicAdd(&mass[k & 0xffu], (unsigned long long)f);
                atomicAdd(&wcnt[wave][k & 0xffu], 1u);
            }
        });
        __syncthreads();
        if (wave == 0) select_mass_bin(mass, before_hb, limit, sel);
        __syncthreads();
        const uint32_t lb = (uint32_t)sel[0];
        const uint64_t before_k = sel[1];
        kstar = (hb << 8) | lb;
        const uint64_t fe = fixed_e(scaled_of(bf16_of_key(kstar), temperature));
        tie_keep = (int64_t)((limit - before_k) / fe) + 1;
        if (tid == 0) {
            uint32_t acc = 0;
            for (int w = 0; w < kWaves; ++w) {
                woff[w] = acc;
                acc += wcnt[w][lb];
            }
        }
        __syncthreads();
    }

    // ---- Gumbel-max draw over the kept elements ----
    const bool track = tie_keep >= 0;
    uint32_t run = track ? woff[wave] : 0u;            // ties at kstar before this wave's current step
    uint64_t best = 0;
    float bv = -__builtin_inff();                      // best value of this thread so far
    for_each_step<VEC>(row, N, S, [&](int64_t i0, const uint32_t* v, bool ok) {
        uint32_t below = 0;                            // ties at kstar before this lane's first element
        if (track) {
            uint32_t c = 0;
            if (ok)
#pragma unroll
                for (int e = 0; e < VEC; ++e) c += bf16_order_key(v[e]) == kstar ? 1u : 0u;
            uint32_t inc = c;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t o = __shfl_up(inc, d);
                if (lane >= d) inc += o;
            }
            below = run + inc - c;
            run += __shfl(inc, 63);
        }
        uint32_t keepbits = 0;
        if (ok) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const uint32_t k = bf16_order_key(v[e]);
                bool keep = k >= kmin && k <= kstar;
                if (track && k == kstar) {
                    keep = keep && (int64_t)below < tie_keep;
                    ++below;
                }
                if (!keep) continue;
                keepbits |= 1u << e;
                const float s = scaled_of(v[e], temperature);
                // s + g <= fl(s + kGumbelMax) < bv: cannot reach a value already drawn
                if (s + kGumbelMax < bv) continue;
                float val;
                const uint64_t key = draw_key(s, seed, m, i0 + e, &val);
                if (key > best) best = key;
                bv = val > bv ? val : bv;
            }
        }
        // share the largest value drawn so far across the wave (a pruning bound only)
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            const float o = __shfl_xor(bv, d);
            bv = o > bv ? o : bv;
        }
        if (!ok) return;
        if (keep_out) {
            uint8_t* kp = keep_out + m * N + i0;
            if constexpr (VEC == 8) {
                store_keep8(kp, keepbits);
            } else {
                kp[0] = (uint8_t)(keepbits & 1u);
            }
        }
    });
    best = block_max_u64<kWaves>(best, tmp);
    if (tid == 0) idx[m] = best ? argmax_key_index(best) : 0u;
}

// ---------------------------------------------------------------------------
// Chunked path for a few long rows (decode batches): row m is cut into P
// chunks of C logits (C a multiple of kStep), one 256-thread workgroup each,
// and the selection runs as a chain of kernels on the stream, each reducing
// the previous stage's per-chunk partials from the workspace:
//   chunk_stats    chunk max key; top-k high-byte counts
//   chunk_topk     kmax and the top-k high byte; low-byte counts inside it
//   chunk_mass_hi  kmin; top-p mass per high byte of the keys >= kmin
//   chunk_mass_lo  the top-p high byte; mass and counts per low byte inside it
//   chunk_draw     k*, the ties kept, this chunk's earlier ties; Gumbel-max
//   chunk_final    the row's token from the chunks' best keys
// Only the stages the parameters need are launched.  The integer sums,
// thresholds and per-element draws are sample_kernel's, so the two paths give
// identical tokens and keep masks.
constexpr int kCT = 256;                    // threads per chunk workgroup
constexpr int kCW = kCT / 64;
constexpr int kStep = kCT * 8;              // logits per step: one 16-byte load per thread
constexpr int64_t kChunkMaxRows = 128;
constexpr int64_t kChunkMinN = 8192;

struct RowSel {                             // per-row results handed down the chain
    uint64_t limit, before_hb;
    uint32_t kmax, hb, above, kmin, hbp, pad;
};

struct ChunkArgs {
    const uint16_t* logits;
    int64_t N, C;
    int P;
    float temperature;
    int top_k;
    float top_p;
    uint64_t seed;
    int use_k, use_p;
    uint64_t* part_max;                     // [M][P]
    uint64_t* best;                         // [M][P]
    uint32_t* cnt_hi;                       // [M][P][256]
    uint32_t* cnt_lo;                       // [M][P][256]
    uint32_t* tcnt;                         // [M][P][256]
    unsigned long long* mass_hi;            // [M][P][256]
    unsigned long long* mass_lo;            // [M][P][256]
    RowSel* sel;                            // [M]
    uint32_t* idx;
    uint8_t* keep;
};

// f(i0, v, ok, step) for each step of chunk p (block-uniform trip count);
// thread t holds logits i0 = base + 8t .. +7 when ok.
template <class F>
__device__ __forceinline__ void for_chunk(const uint16_t* __restrict__ row, int64_t N, int64_t C, int p, F&& f) {
    const int64_t beg = (int64_t)p * C;
    const int64_t end = beg + C < N ? beg + C : N;
    int step = 0;
    for (int64_t b = beg; b < end; b += kStep, ++step) {
        const int64_t i0 = b + (int64_t)threadIdx.x * 8;
        const bool ok = i0 < end;
        uint4 q = make_uint4(0, 0, 0, 0);
        if (ok) q = *reinterpret_cast<const uint4*>(row + i0);
        const uint32_t v[8] = {q.x & 0xffffu, q.x >> 16, q.y & 0xffffu, q.y >> 16,
                               q.z & 0xffffu, q.z >> 16, q.w & 0xffffu, q.w >> 16};
        f(i0, v, ok, step);
    }
}

// Thread t (< 256) sums bin t over the P partial histograms part[P][256]
// into lds[t]; the caller synchronises before reading lds.  The sums are
// integers (counts, fixed-point masses), so the order does not matter: 64
// loads per batch are issued before any is added (clamped addresses, the
// ones past P added as 0), so P <= 128 chunks cost two round trips to L2.
template <class T>
__device__ __forceinline__ T reduce_bins(const T* __restrict__ part, int P, T* lds) {
    constexpr int kBatch = 64;
    T s = 0;
    const T* p = part + threadIdx.x;
    for (int q = 0; q < P; q += kBatch) {
        T v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) v[j] = p[(size_t)(q + j < P ? q + j : P - 1) * 256];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) s += q + j < P ? v[j] : (T)0;
    }
    lds[threadIdx.x] = s;
    return s;
}

// kmin of the top-k stage: the top_k - above largest keys inside high byte hb.
__device__ uint32_t resolve_kmin(const ChunkArgs& a, int64_t m, uint32_t* hist, uint32_t* selk) {
    const uint32_t hb = a.sel[m].hb, above = a.sel[m].above;
    reduce_bins(a.cnt_lo + (size_t)m * a.P * 256, a.P, hist);
    __syncthreads();
    if (threadIdx.x < 64) select_top_bin(hist, (uint32_t)a.top_k - above, selk);
    __syncthreads();
    const uint32_t kmin = (hb << 8) | selk[0];
    return kmin ? kmin : 1u;
}

__global__ __launch_bounds__(kCT) void chunk_stats_kernel(ChunkArgs a) {
    const int p = blockIdx.x;
    const int64_t m = blockIdx.y;
    const uint16_t* row = a.logits + m * a.N;
    __shared__ uint32_t hist[256];
    __shared__ uint64_t tmp[kCW];
    const bool use_k = a.use_k;
    hist[threadIdx.x] = 0;
    __syncthreads();
    uint64_t mk = 0;
    for_chunk(row, a.N, a.C, p, [&](int64_t, const uint32_t* v, bool ok, int) {
        if (!ok) return;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t k = bf16_order_key(v[e]);
            mk = k > mk ? k : mk;
            if (use_k) atomicAdd(&hist[k >> 8], 1u);
        }
    });
    mk = block_max_u64<kCW>(mk, tmp);               // its barriers also complete hist
    const size_t mp = (size_t)m * a.P + p;
    if (threadIdx.x == 0) a.part_max[mp] = mk;
    if (use_k) a.cnt_hi[mp * 256 + threadIdx.x] = hist[threadIdx.x];
}

__global__ __launch_bounds__(kCT) void chunk_topk_kernel(ChunkArgs a) {
    const int p = blockIdx.x;
    const int64_t m = blockIdx.y;
    const uint16_t* row = a.logits + m * a.N;
    __shared__ uint32_t hist[256];
    __shared__ uint32_t selk[2];
    __shared__ uint64_t tmp[kCW];
    uint64_t mk = 0;
    for (int q = threadIdx.x; q < a.P; q += kCT) {
        const uint64_t v = a.part_max[(size_t)m * a.P + q];
        mk = v > mk ? v : mk;
    }
    reduce_bins(a.cnt_hi + (size_t)m * a.P * 256, a.P, hist);
    const uint32_t kmax = (uint32_t)block_max_u64<kCW>(mk, tmp);   // its barriers also complete hist
    if (threadIdx.x < 64) select_top_bin(hist, (uint32_t)a.top_k, selk);
    __syncthreads();
    const uint32_t hb = selk[0], above = selk[1];
    hist[threadIdx.x] = 0;
    __syncthreads();
    for_chunk(row, a.N, a.C, p, [&](int64_t, const uint32_t* v, bool ok, int) {
        if (!ok) return;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t k = bf16_order_key(v[e]);
            if ((k >> 8) == hb) atomicAdd(&hist[k & 0xffu], 1u);
        }
    });
    __syncthreads();
    const size_t mp = (size_t)m * a.P + p;
    a.cnt_lo[mp * 256 + threadIdx.x] = hist[threadIdx.x];
    if (p == 0 && threadIdx.x == 0) {
        a.sel[m].kmax = kmax;
        a.sel[m].hb = hb;
        a.sel[m].above = above;
    }
}

__global__ __launch_bounds__(kCT) void chunk_mass_hi_kernel(ChunkArgs a) {
    const int p = blockIdx.x;
    const int64_t m = blockIdx.y;
    const uint16_t* row = a.logits + m * a.N;
    __shared__ uint32_t hist[256];
    __shared__ uint32_t selk[2];
    __shared__ unsigned long long mass[256];
    __shared__ uint64_t tmp[kCW];
    uint32_t kmax;
    if (a.use_k) {
        kmax = a.sel[m].kmax;
    } else {
        uint64_t mk = 0;
        for (int q = threadIdx.x; q < a.P; q += kCT) {
            const uint64_t v = a.part_max[(size_t)m * a.P + q];
            mk = v > mk ? v : mk;
        }
        kmax = (uint32_t)block_max_u64<kCW>(mk, tmp);
    }
    const uint32_t kmin = a.use_k ? resolve_kmin(a, m, hist, selk) : 1u;
    if (p == 0 && threadIdx.x == 0) {
        a.sel[m].kmin = kmin;
        a.sel[m].kmax = kmax;
    }
    mass[threadIdx.x] = 0;
    __syncthreads();
    if (kmax >= kmin) {
        const float T = a.temperature;
        const float smax = scaled_of(bf16_of_key(kmax), T);
        for_chunk(row, a.N, a.C, p, [&](int64_t, const uint32_t* v, bool ok, int) {
            if (!ok) return;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t k = bf16_order_key(v[e]);
                if (k < kmin) continue;
                const uint64_t f = fixed_mass(scaled_of(v[e], T), smax);
                if (f) atomicAdd(&mass[k >> 8], (unsigned long long)f);
            }
        });
    }
    __syncthreads();
    const size_t mp = (size_t)m * a.P + p;
    a.mass_hi[mp * 256 + threadIdx.x] = mass[threadIdx.x];
}

__global__ __launch_bounds__(kCT) void chunk_mass_lo_kernel(ChunkArgs a) {
    const int p = blockIdx.x;
    const int64_t m = blockIdx.y;
    const uint16_t* row = a.logits + m * a.N;
    __shared__ unsigned long long mass[256];
    __shared__ uint32_t tc[256];
    __shared__ uint64_t sel2[2];
    __shared__ uint64_t tmp[kCW];
    const uint32_t kmin = a.sel[m].kmin, kmax = a.sel[m].kmax;
    const uint64_t mine = reduce_bins(a.mass_hi + (size_t)m * a.P * 256, a.P, mass);
    const uint64_t Z = block_sum_u64<kCW>(mine, tmp);   // its barriers also complete mass
    const uint64_t limit = (uint64_t)((double)a.top_p * (double)Z);
    if (threadIdx.x < 64) select_mass_bin(mass, 0, limit, sel2);
    __syncthreads();
    const uint32_t hbp = (uint32_t)sel2[0];
    const uint64_t before_hb = sel2[1];
    __syncthreads();
    mass[threadIdx.x] = 0;
    tc[threadIdx.x] = 0;
    __syncthreads();
    if (kmax >= kmin) {
        const float T = a.temperature;
        const float smax = scaled_of(bf16_of_key(kmax), T);
        for_chunk(row, a.N, a.C, p, [&](int64_t, const uint32_t* v, bool ok, int) {
            if (!ok) return;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t k = bf16_order_key(v[e]);
                if (k < kmin || (k >> 8) != hbp) continue;
                const uint64_t f = fixed_mass(scaled_of(v[e], T), smax);
                if (f) atomicAdd(&mass[k & 0xffu], (unsigned long long)f);
                atomicAdd(&tc[k & 0xffu], 1u);
            }
        });
    }
    __syncthreads();
    const size_t mp = (size_t)m * a.P + p;
    a.mass_lo[mp * 256 + threadIdx.x] = mass[threadIdx.x];
    a.tcnt[mp * 256 + threadIdx.x] = tc[threadIdx.x];
    if (p == 0 && threadIdx.x == 0) {
        a.sel[m].limit = limit;
        a.sel[m].hbp = hbp;
        a.sel[m].before_hb = before_hb;
    }
}

__global__ __launch_bounds__(kCT) void chunk_draw_kernel(ChunkArgs a) {
#pragma clang fp contract(off)
    const int p = blockIdx.x;
    const int64_t m = blockIdx.y;
    const uint16_t* row = a.logits + m * a.N;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t mp = (size_t)m * a.P + p;
    __shared__ uint32_t hist[256];
    __shared__ uint32_t selk[2];
    __shared__ unsigned long long mass[256];
    __shared__ uint64_t sel2[2];
    __shared__ uint64_t tmp[kCW];
    __shared__ uint32_t wsum[2][kCW];
    const float T = a.temperature;

    if (!(T > 0.0f)) {                                 // greedy: argmax keys
        uint64_t best = 0;
        for_chunk(row, a.N, a.C, p, [&](int64_t i0, const uint32_t* v, bool ok, int) {
            if (!ok) return;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint64_t k = argmax_key(v[e], (uint32_t)(i0 + e));
                best = k > best ? k : best;
            }
        });
        best = block_max_u64<kCW>(best, tmp);
        if (tid == 0) a.best[mp] = best;
        return;
    }

    uint32_t kmin = 1, kmax = 0xffffu;
    if (a.use_p) {
        kmin = a.sel[m].kmin;
        kmax = a.sel[m].kmax;
    } else if (a.use_k) {
        kmax = a.sel[m].kmax;
        kmin = resolve_kmin(a, m, hist, selk);
    }
    if (kmax < kmin) {                                 // nothing but NaN
        if (tid == 0) a.best[mp] = 0;
        if (a.keep) {
            const int64_t beg = (int64_t)p * a.C, end = beg + a.C < a.N ? beg + a.C : a.N;
            for (int64_t i = beg + tid; i < end; i += kCT) a.keep[m * a.N + i] = 0;
        }
        return;
    }
    uint32_t kstar = 0xffffu;
    int64_t tie_keep = -1;
    uint32_t run = 0;                                  // ties at kstar before the current step
    if (a.use_p) {
        const uint64_t limit = a.sel[m].limit, before_hb = a.sel[m].before_hb;
        const uint32_t hbp = a.sel[m].hbp;
        reduce_bins(a.mass_lo + (size_t)m * a.P * 256, a.P, mass);
        __syncthreads();
        if (tid < 64) select_mass_bin(mass, before_hb, limit, sel2);
        __syncthreads();
        const uint32_t lb = (uint32_t)sel2[0];
        const uint64_t before_k = sel2[1];
        kstar = (hbp << 8) | lb;
        const float smax = scaled_of(bf16_of_key(kmax), T);
        const uint64_t fe = fixed_mass(scaled_of(bf16_of_key(kstar), T), smax);
        tie_keep = (int64_t)((limit - before_k) / fe) + 1;
        uint64_t c = 0;                                // ties at kstar in the chunks before p
        for (int q = tid; q < p; q += kCT) c += a.tcnt[((size_t)m * a.P + q) * 256 + lb];
        run = (uint32_t)block_sum_u64<kCW>(c, tmp);
    }

    const bool track = tie_keep >= 0;
    const uint64_t seed = a.seed;
    uint64_t best = 0;
    float bv = -__builtin_inff();
    for_chunk(row, a.N, a.C, p, [&](int64_t i0, const uint32_t* v, bool ok, int step) {
        uint32_t below = 0;                            // ties at kstar before this thread's first logit
        if (track) {
            uint32_t c = 0;
            if (ok)
#pragma unroll
                for (int e = 0; e < 8; ++e) c += bf16_order_key(v[e]) == kstar ? 1u : 0u;
            uint32_t inc = c;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t o = __shfl_up(inc, d);
                if (lane >= d) inc += o;
            }
            if (lane == 63) wsum[step & 1][wave] = inc;
            __syncthreads();
            uint32_t pre = 0, tot = 0;
#pragma unroll
            for (int w = 0; w < kCW; ++w) {
                const uint32_t x = wsum[step & 1][w];
                pre += w < wave ? x : 0u;
                tot += x;
            }
            below = run + pre + inc - c;
            run += tot;
        }
        uint32_t keepbits = 0;
        if (ok) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t k = bf16_order_key(v[e]);
                bool keep = k >= kmin && k <= kstar;
                if (track && k == kstar) {
                    keep = keep && (int64_t)below < tie_keep;
                    ++below;
                }
                if (!keep) continue;
                keepbits |= 1u << e;
                const float s = scaled_of(v[e], T);
                if (s + kGumbelMax < bv) continue;     // cannot reach a value already drawn
                float val;
                const uint64_t key = draw_key(s, seed, m, i0 + e, &val);
                if (key > best) best = key;
                bv = val > bv ? val : bv;
            }
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            const float o = __shfl_xor(bv, d);
            bv = o > bv ? o : bv;
        }
        if (ok && a.keep) store_keep8(a.keep + m * a.N + i0, keepbits);
    });
    best = block_max_u64<kCW>(best, tmp);
    if (tid == 0) a.best[mp] = best;
}

__global__ __launch_bounds__(64) void chunk_final_kernel(const uint64_t* __restrict__ best, int P,
                                                         uint32_t* __restrict__ idx) {
    const int64_t m = blockIdx.x;
    uint64_t b = 0;
    for (int q = threadIdx.x; q < P; q += 64) {
        const uint64_t v = best[(size_t)m * P + q];
        b = v > b ? v : b;
    }
    b = wave_max_u64(b);
    if (threadIdx.x == 0) idx[m] = b ? argmax_key_index(b) : 0u;
}

// Chunk shape of the chunked path: about 1024 workgroups (four per CU) over
// the M rows, at least one step of logits each.
inline void chunk_shape(int64_t M, int64_t N, int* P, int64_t* C) {
    const int64_t target = 1024 / M > 1 ? 1024 / M : 1;
    const int64_t steps = (N + kStep - 1) / kStep;
    *C = ((steps + target - 1) / target) * kStep;
    *P = (int)((N + *C - 1) / *C);
}

inline bool chunk_eligible(int64_t M, int64_t N) {
    return M <= kChunkMaxRows && N >= kChunkMinN && N % 8 == 0;
}

inline size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// Workspace carve-up of the chunked path; returns the bytes needed.
inline size_t chunk_layout(int64_t M, int P, char* base, ChunkArgs* a) {
    const size_t mp = (size_t)M * P, bins = mp * 256;
    size_t off = 0;
    auto take = [&](size_t bytes) -> char* {
        char* r = base ? base + off : nullptr;
        off += align256(bytes);
        return r;
    };
    char* part_max = take(mp * 8);
    char* best = take(mp * 8);
    char* cnt_hi = take(bins * 4);
    char* cnt_lo = take(bins * 4);
    char* tcnt = take(bins * 4);
    char* mass_hi = take(bins * 8);
    char* mass_lo = take(bins * 8);
    char* sel = take((size_t)M * sizeof(RowSel));
    if (a) {
        a->part_max = reinterpret_cast<uint64_t*>(part_max);
        a->best = reinterpret_cast<uint64_t*>(best);
        a->cnt_hi = reinterpret_cast<uint32_t*>(cnt_hi);
        a->cnt_lo = reinterpret_cast<uint32_t*>(cnt_lo);
        a->tcnt = reinterpret_cast<uint32_t*>(tcnt);
        a->mass_hi = reinterpret_cast<unsigned long long*>(mass_hi);
        a->mass_lo = reinterpret_cast<unsigned long long*>(mass_lo);
        a->sel = reinterpret_cast<RowSel*>(sel);
    }
    return off;
}

}  // namespace smp

}  // namespace mq4

using namespace mq4;

extern "C" size_t mq4_sample_workspace_size(int64_t M, int64_t N) {
    if (M <= 0 || N <= 0 || !smp::chunk_eligible(M, N)) return 0;
    int P;
    int64_t C;
    smp::chunk_shape(M, N, &P, &C);
    return smp::chunk_layout(M, P, nullptr, nullptr);
}

extern "C" int mq4_sample_bf16(const uint16_t* logits, int64_t M, int64_t N, float temperature, int top_k,
                               float top_p, uint64_t seed, uint32_t* idx, uint8_t* keep, void* workspace,
                               size_t workspace_bytes, void* stream) {
    const char* what = "mq4_sample_bf16";
    if (M <= 0 || N <= 0) return fail(MQ4_ERR_INVALID_ARG, "%s: M and N must be positive", what);
    if (M > 65535 || N > (1LL << 23))
        return fail(MQ4_ERR_UNSUPPORTED, "%s: at most 65535 rows of 2^23 logits (got %lld x %lld)", what,
                    (long long)M, (long long)N);
    if (!logits || !idx) return fail(MQ4_ERR_INVALID_ARG, "%s: null pointer", what);
    if (!aligned(logits, 2) || !aligned(idx, 4)) return fail(MQ4_ERR_ALIGNMENT, "%s: misaligned pointer", what);
    if (top_k < 0) return fail(MQ4_ERR_INVALID_ARG, "%s: top_k must be >= 0 (got %d)", what, top_k);
    if (temperature != temperature || top_p != top_p)
        return fail(MQ4_ERR_INVALID_ARG, "%s: temperature and top_p must not be NaN", what);
    const bool vec8 = N % 8 == 0 && aligned(logits, 16) && (!keep || aligned(keep, 8));
    const hipStream_t st = as_stream(stream);
    const size_t need = mq4_sample_workspace_size(M, N);
    if (workspace && need && vec8) {
        if (workspace_bytes < need || !aligned(workspace, 256))
            return fail(MQ4_ERR_WORKSPACE, "%s: workspace of %zu bytes (256-byte aligned) needed, got %zu", what,
                        need, workspace_bytes);
        smp::ChunkArgs a{};
        smp::chunk_shape(M, N, &a.P, &a.C);
        smp::chunk_layout(M, a.P, static_cast<char*>(workspace), &a);
        a.logits = logits;
        a.N = N;
        a.temperature = temperature;
        a.top_k = top_k;
        a.top_p = top_p;
        a.seed = seed;
        a.use_k = temperature > 0.0f && top_k > 0 && (int64_t)top_k < N;
        a.use_p = temperature > 0.0f && top_p > 0.0f && top_p < 1.0f;
        a.idx = idx;
        a.keep = keep;
        const dim3 grid((unsigned)a.P, (unsigned)M);
        if (a.use_k || a.use_p) hipLaunchKernelGGL(smp::chunk_stats_kernel, grid, dim3(smp::kCT), 0, st, a);
        if (a.use_k) hipLaunchKernelGGL(smp::chunk_topk_kernel, grid, dim3(smp::kCT), 0, st, a);
        if (a.use_p) {
            hipLaunchKernelGGL(smp::chunk_mass_hi_kernel, grid, dim3(smp::kCT), 0, st, a);
            hipLaunchKernelGGL(smp::chunk_mass_lo_kernel, grid, dim3(smp::kCT), 0, st, a);
        }
        hipLaunchKernelGGL(smp::chunk_draw_kernel, grid, dim3(smp::kCT), 0, st, a);
        hipLaunchKernelGGL(smp::chunk_final_kernel, dim3((unsigned)M), dim3(64), 0, st, a.best, a.P, idx);
        return launch_status(what);
    }
    if (vec8) {
        const int64_t S = ((N + smp::kWaves * 512 - 1) / (smp::kWaves * 512)) * 512;
        hipLaunchKernelGGL(smp::sample_kernel<8>, dim3((unsigned)M), dim3(smp::kThreads), 0, st, logits, N, S,
                           temperature, top_k, top_p, seed, idx, keep);
    } else {
        const int64_t S = (N + smp::kWaves - 1) / smp::kWaves;
        hipLaunchKernelGGL(smp::sample_kernel<1>, dim3((unsigned)M), dim3(smp::kThreads), 0, st, logits, N, S,
                           temperature, top_k, top_p, seed, idx, keep);
    }
    return launch_status(what);
}
