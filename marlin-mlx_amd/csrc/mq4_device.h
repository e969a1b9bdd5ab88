// Device-side helpers shared by the gfx950 kernels of libmq4.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mq4 {

constexpr int kWave = 64;     // CDNA wavefront width
constexpr int kGroup = 64;    // MLX affine group size along K
constexpr int kSlice = 32;    // K elements per 16-byte packed slice (4 words)

// One MLX-layout Q4 matrix: packed words [N, K/8], bf16 scales/biases [N, K/64].
struct QMat {
    const uint32_t* wq;
    const uint16_t* s;
    const uint16_t* b;
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming load (non-temporal hint: data read once).
__device__ __forceinline__ uint4 load_nt_u4(const void* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t h) {
    return __uint_as_float(h << 16);
}

// float -> bf16 bits, round to nearest even; NaN becomes the quiet NaN
// (bits >> 16) | 0x40.  gfx950's v_cvt_pk_bf16_f32 does exactly this (it is
// bit-identical to the integer formulation, add 0x7fff + lsb then shift, with
// that NaN rule, over all 2^32 inputs), one instruction for two values.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
    const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// Round to bf16 and back (the value a bf16 tensor would hold).
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// 2-way bf16 dot product with fp32 accumulate: a.lo*b.lo + a.hi*b.hi + c.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Nibbles p and p+4 of a packed word as the bf16 pair (128 + q_p, 128 + q_{p+4}):
// 0x4300 is bf16 128.0 and its 7 mantissa bits hold q exactly.
// One v_and_or_b32 per pair (plus a shift for P > 0): the compiler emits a
// separate AND and OR because gfx9 VOP3 encodings take no literal constant,
// so the mask is passed in an SGPR and the exponent bits in a VGPR.
template <int P>
__device__ __forceinline__ uint32_t nib_pair_bf16(uint32_t word) {
    const uint32_t s = P ? (word >> (4 * P)) : word;
    uint32_t m, c;
    asm("s_mov_b32 %0, 0x000f000f" : "=s"(m));
    asm("v_mov_b32 %0, 0x43004300" : "=v"(c));
    return (s & m) | c;
}

// ---- per-element arithmetic shared by every decode kernel ----
// The separate kernels (mq4_gemv.hip) and the persistent decode step
// (mq4_decode.hip) call these same functions in the same order, so the two
// paths produce bit-identical results.  FP contraction is off inside them and
// every fused multiply-add is written out, so the compiler cannot fuse
// differently in different kernels.

// Contribution of one 16-byte slice (32 K elements, half a group):
// sum_k x_k*(s*q_k + b) = s*D + (b - 128*s)*X with D = sum_k x_k*(128 + q_k)
// (the dot2 of the nibble pairs) and X = sum_k x_k.
__device__ __forceinline__ float affine_c(float s, uint32_t bbits) {
#pragma clang fp contract(off)
    return bf16_to_f32(bbits) - 128.0f * s;    // 128*s is exact
}
__device__ __forceinline__ float affine_term_f(float s, float c, float d, float xsum) {
#pragma clang fp contract(off)
    return __builtin_fmaf(s, d, c * xsum);
}
__device__ __forceinline__ float affine_term(uint32_t sbits, uint32_t bbits, float d, float xsum) {
    const float s = bf16_to_f32(sbits);
    return affine_term_f(s, affine_c(s, bbits), d, xsum);
}

// The four nibble pairs of one packed word (see nib_pair_bf16).
__device__ __forceinline__ void nib_pairs(uint32_t word, uint32_t* out4) {
    out4[0] = nib_pair_bf16<0>(word);
    out4[1] = nib_pair_bf16<1>(word);
    out4[2] = nib_pair_bf16<2>(word);
    out4[3] = nib_pair_bf16<3>(word);
}

// s + lo^2 + hi^2 of one word holding two bf16 values.
__device__ __forceinline__ float sumsq_word(float s, uint32_t v) {
#pragma clang fp contract(off)
    const float lo = bf16_to_f32(v & 0xffffu), hi = bf16_to_f32(v >> 16);
    return s + __builtin_fmaf(lo, lo, hi * hi);
}

// 1 / sqrt(mean(x^2) + eps) from the fp32 sum of squares of K values.
__device__ __forceinline__ float rms_inv(float ss, int K, float eps) {
#pragma clang fp contract(off)
    return 1.0f / sqrtf(ss / (float)K + eps);
}

// (1 + w) RMSNorm of one word of two bf16 values, one bf16 rounding each
// (src/model/marlin.cpp:12-16).
__device__ __forceinline__ uint32_t norm_word(uint32_t x, uint32_t w, float r) {
#pragma clang fp contract(off)
    return f32x2_to_bf16x2(bf16_to_f32(x & 0xffffu) * r * (1.0f + bf16_to_f32(w & 0xffffu)),
                           bf16_to_f32(x >> 16) * r * (1.0f + bf16_to_f32(w >> 16)));
}

// One 16-byte activation chunk (8 bf16 values in words a.x..a.w) -> the four
// dot2 pairs (v_p, v_{p+4}) matching nib_pair_bf16<0..3> of one packed word,
// and sum + (the 8 values, left to right).
__device__ __forceinline__ float pair_chunk(const uint4& a, uint32_t* out4, float sum) {
#pragma clang fp contract(off)
    out4[0] = (a.x & 0xffffu) | (a.z << 16);
    out4[1] = (a.x >> 16) | (a.z & 0xffff0000u);
    out4[2] = (a.y & 0xffffu) | (a.w << 16);
    out4[3] = (a.y >> 16) | (a.w & 0xffff0000u);
    return sum + (bf16_to_f32(a.x & 0xffffu) + bf16_to_f32(a.x >> 16) + bf16_to_f32(a.y & 0xffffu) +
                  bf16_to_f32(a.y >> 16) + bf16_to_f32(a.z & 0xffffu) + bf16_to_f32(a.z >> 16) +
                  bf16_to_f32(a.w & 0xffffu) + bf16_to_f32(a.w >> 16));
}

// bf16 SwiGLU in MLX's op order (src/model/marlin.cpp:27-29): every
// intermediate is a bf16 tensor.
__device__ __forceinline__ uint32_t swiglu_bf16(float g_acc, float u_acc) {
#pragma clang fp contract(off)
    const float g = round_bf16(g_acc);
    const float u = round_bf16(u_acc);
    const float sg = round_bf16(1.0f / (1.0f + expf(-g)));
    const float t = round_bf16(sg * g);
    return f32_to_bf16(t * u);
}

// swiglu_bf16 of N (gate, up) pairs through a table of the rounded SiLU
// t(g) = round_bf16(round_bf16(1 / (1 + expf(-g))) * g), the same bits.  The
// table holds t for the bf16 g with 2^-9 <= |g| < 128 (exponent fields
// 118-133; entry (sign << 11) | (exponent - 118) << 7 | mantissa, 4096 x 2
// bytes, silu_lut_entry).  Below 2^-9 the rounded sigmoid is 0.5 exactly, so
// t = g / 2: the exponent field less one for exponent fields 2-117, and
// +-0 for +-0.  The rest (|g| >= 128, inf, NaN, and |g| < 2^-125 where g / 2
// is subnormal) take the exact formula, in one branch for the batch.
constexpr int SILU_LUT_N = 4096;
constexpr uint32_t SILU_LUT_LO = 118u << 7;          // |g| bits of 2^-9
__device__ __forceinline__ uint32_t silu_lut_entry(uint32_t i) {
#pragma clang fp contract(off)
    const uint32_t bits = ((i >> 11) << 15) | (SILU_LUT_LO + (i & 2047u));
    const float g = bf16_to_f32(bits);
    return f32_to_bf16(round_bf16(1.0f / (1.0f + expf(-g))) * g);
}
template <int N>
__device__ __forceinline__ void swiglu_bf16_lut_batch(const float (&g_acc)[N], const float (&u_acc)[N],
                                                      uint32_t (&out)[N], const uint16_t* lut) {
#pragma clang fp contract(off)
    static_assert(N <= 32, "one mask word");
    uint32_t gb[N], tb[N];
    uint32_t need = 0;
#pragma unroll
    for (int e = 0; e < N; ++e) {
        gb[e] = f32_to_bf16(g_acc[e]);
        const uint32_t mag = gb[e] & 0x7fffu;
        const uint32_t k = mag - SILU_LUT_LO;                            // unsigned
        const uint32_t idx = (k < 2048u ? k : 0u) | ((gb[e] >> 4) & 0x800u);
        const uint32_t lt = lut[idx];
        const bool half = mag - 0x100u < SILU_LUT_LO - 0x100u;           // exponent fields 2-117
        tb[e] = k < 2048u ? lt : half ? gb[e] - 0x80u : gb[e];           // +-0 keeps its bits
        if (k >= 2048u && !half && mag != 0u) need |= 1u << e;
    }
    if (need) {
#pragma unroll
        for (int e = 0; e < N; ++e)
            if (need & (1u << e)) {
                const float g = bf16_to_f32(gb[e]);
                tb[e] = f32_to_bf16(round_bf16(1.0f / (1.0f + expf(-g))) * g);
            }
    }
#pragma unroll
    for (int e = 0; e < N; ++e) out[e] = f32_to_bf16(bf16_to_f32(tb[e]) * round_bf16(u_acc[e]));
}

// Monotone 16-bit key of a bf16 value for max-selection: larger value ->
// larger key; -0 maps like +0 and NaN maps to 0 (below every number).
__device__ __forceinline__ uint32_t bf16_order_key(uint32_t h) {
    h &= 0xffffu;
    if ((h & 0x7fffu) > 0x7f80u) return 0u;     // NaN
    if (h == 0x8000u) h = 0u;                   // -0 -> +0
    return (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
}

// 64-bit argmax key: value key in the high word, ~index in the low word so
// that among equal values the lowest index is the maximum.
__device__ __forceinline__ uint64_t argmax_key(uint32_t bf16_bits, uint32_t index) {
    return ((uint64_t)bf16_order_key(bf16_bits) << 32) | (uint64_t)(0xffffffffu - index);
}
__device__ __forceinline__ uint32_t argmax_key_index(uint64_t key) {
    return 0xffffffffu - (uint32_t)(key & 0xffffffffu);
}

// Workgroup barrier without a memory fence: waits for this wave's LDS
// operations only (lgkmcnt), not for outstanding global loads or LDS DMA.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Wait until at most N vector-memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// ---- cross-lane butterfly on the VALU (no LDS round trip) ----
// Level OFF pairs lane l with partner(l): OFF = 32 -> l^32 and 16 -> l^16
// (v_permlane32_swap / v_permlane16_swap, which move two registers at once),
// 8 -> l^8 (DPP row_ror:8 within a 16-lane row), 4 -> l^7 (DPP
// row_half_mirror), 2 -> l^2 and 1 -> l^1 (DPP quad_perm).  Each level flips
// bit log2(OFF) of the lane index, and the six partners span all 64 lanes, so
// six levels sum every lane exactly once.
template <int OFF>
__device__ __forceinline__ uint32_t dpp_partner(uint32_t v) {
    static_assert(OFF == 8 || OFF == 4 || OFF == 2 || OFF == 1, "DPP levels");
    constexpr int ctrl = OFF == 8 ? 0x128 : OFF == 4 ? 0x141 : OFF == 2 ? 0x4E : 0xB1;
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, ctrl, 0xF, 0xF, false);
}
__device__ __forceinline__ float dpp_partner_f(float v, int off) {
    switch (off) {
        case 8: return __uint_as_float(dpp_partner<8>(__float_as_uint(v)));
        case 4: return __uint_as_float(dpp_partner<4>(__float_as_uint(v)));
        case 2: return __uint_as_float(dpp_partner<2>(__float_as_uint(v)));
        default: return __uint_as_float(dpp_partner<1>(__float_as_uint(v)));
    }
}

// Value of v in lane `src` (wave-uniform result).  The readlane builtin is
// typed int, so the float travels as its bit pattern.
__device__ __forceinline__ float lane_value(float v, int src) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}

__device__ __forceinline__ uint32_t lane_bits(uint32_t v, int src) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, src);
}

// Value of lane K of this lane's quad (DPP quad_perm broadcast).
template <int K>
__device__ __forceinline__ float quad_lane(float v) {
    constexpr int ctrl = K | (K << 2) | (K << 4) | (K << 6);
    return __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(v), ctrl, 0xF, 0xF, false));
}

// (a', b') of v_permlane32_swap / v_permlane16_swap on (a, b): in the lower
// half of each pair of lane groups a' = a and b' = a of the partner lane; in
// the upper half a' = b of the partner lane and b' = b.  So a' + b' is the
// pair sum of a in the lower half and of b in the upper half.
template <int OFF>
__device__ __forceinline__ void swap_halves(float a, float b, float& a2, float& b2) {
    static_assert(OFF == 32 || OFF == 16, "swap levels");
    if constexpr (OFF == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
        a2 = __uint_as_float(r[0]);
        b2 = __uint_as_float(r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
        a2 = __uint_as_float(r[0]);
        b2 = __uint_as_float(r[1]);
    }
}

// Sum of v over the 64 lanes (every lane receives it).
__device__ __forceinline__ float wave_sum(float v) {
    float a, b;
    swap_halves<32>(v, v, a, b);
    v = a + b;
    swap_halves<16>(v, v, a, b);
    v = a + b;
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) v += dpp_partner_f(v, off);
    return v;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = shfl_xor_u64(v, m);
        v = o > v ? o : v;
    }
    return v;
}

// Reduce V per-lane values (V a power of two, 1..64) over the 64 lanes of a
// wave by recursive halving over the butterfly levels 32, 16, 8, 4, 2, 1: at
// each level the lanes of the lower half (bit log2(level) clear) keep the
// first half of their values and the upper lanes the second half, each adding
// the partner's copy.  Afterwards v[0] of lane l holds the wave-wide sum of
// value index (l >> (6 - log2 V)), identical in all lanes of that index.
template <int V>
__device__ __forceinline__ float wave_multi_reduce(float (&v)[V], int lane) {
    static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "V must be a power of two <= 64");
    int count = V;
#pragma unroll
    for (int lvl = 0; lvl < 2; ++lvl) {          // levels 32 and 16
        const int h = count > 1 ? count >> 1 : 0;
#pragma unroll
        for (int i = 0; i < (V > 1 ? V / 2 : 1); ++i) {
            if (count == 1 && i == 0) {
                float a, b;
                if (lvl == 0) swap_halves<32>(v[0], v[0], a, b);
                else swap_halves<16>(v[0], v[0], a, b);
                v[0] = a + b;
            } else if (i < h) {
                float a, b;
                if (lvl == 0) swap_halves<32>(v[i], v[i + h], a, b);
                else swap_halves<16>(v[i], v[i + h], a, b);
                v[i] = a + b;
            }
        }
        if (count > 1) count = h;
    }
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) {
        if (count > 1) {
            const bool upper = (lane & off) != 0;
            const int h = count >> 1;
#pragma unroll
            for (int i = 0; i < V / 2; ++i) {
                if (i < h) {
                    // both values read first: a select between two array
                    // elements would keep v[] in memory instead of registers
                    const float lo = v[i], hi = v[i + h];
                    const float send = upper ? lo : hi;
                    const float keep = upper ? hi : lo;
                    v[i] = keep + dpp_partner_f(send, off);
                }
            }
            count = h;
        } else {
            v[0] += dpp_partner_f(v[0], off);
        }
    }
    return v[0];
}

template <int V>
__device__ __forceinline__ constexpr int log2_const() {
    return V <= 1 ? 0 : 1 + log2_const<V / 2>();
}

}  // namespace mq4
