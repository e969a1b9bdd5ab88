// MFMA operand helpers shared by the MFMA GEMV (mq4_mfma.hip) and the
// batched one-launch MLP half (mq4_rows.hip): gfx950 v_mfma_f32_16x16x32_bf16
// on activations in the nibble-pair k order and the exact (128 + q) weights.
#pragma once

#include "mq4_device.h"

namespace mq4 {
namespace mf {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma16(const uint4& a, const uint4& b, const f32x4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

// 8 bf16 in natural k order -> nibble-pair order (k0, k4, k1, k5, k2, k6, k3, k7)
__device__ __forceinline__ uint4 pair_order(const uint4& a) {
    return make_uint4((a.x & 0xffffu) | (a.z << 16), (a.x >> 16) | (a.z & 0xffff0000u), (a.y & 0xffffu) | (a.w << 16),
                      (a.y >> 16) | (a.w & 0xffff0000u));
}

// The 8 (128 + q) bf16 of one packed word, pair P = (q_P, q_{P+4}).
__device__ __forceinline__ uint4 unpack_word(uint32_t w) {
    return make_uint4(nib_pair_bf16<0>(w), nib_pair_bf16<1>(w), nib_pair_bf16<2>(w), nib_pair_bf16<3>(w));
}

__device__ __forceinline__ void sumsq4(float& s, const uint4& v) {
    s = sumsq_word(s, v.x);
    s = sumsq_word(s, v.y);
    s = sumsq_word(s, v.z);
    s = sumsq_word(s, v.w);
}

}  // namespace mf
}  // namespace mq4
