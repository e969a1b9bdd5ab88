// Device-side checks of mq4_device.h helpers for the test suite (built into
// _build/libmq4_devcheck.so, never into libmq4.so): helpers whose whole input
// domain fits one launch are compared with their exact formulation on every
// input.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mq4_device.h"

namespace {

// One thread per bf16 bit pattern b of g.  status[b]: bit 0 = the fast
// sigmoid path decided (no exact fallback), bit 1 = sigmoid_bf16(g) differs
// from round_bf16(1 / (1 + expf(-g))), bit 2 = swiglu_bf16_fast(g, u)
// differs from swiglu_bf16(g, u) for one of the u below (bits compared; both
// NaN counts as equal), bit 3 = swiglu_bf16_batch<16> over g and 15 other
// bf16 patterns (b + 4099 k, u cycling through the same values) differs
// from swiglu_bf16 in any of the 16.
__global__ void sigmoid_check_kernel(uint32_t* status) {
#pragma clang fp contract(off)
    const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= 65536u) return;
    const float g = mq4::bf16_to_f32(b);
    float fast;
    const bool decided = mq4::sigmoid_bf16_fast(g, fast);
    const float exact = mq4::round_bf16(1.0f / (1.0f + expf(-g)));
    const float got = mq4::sigmoid_bf16(g);
    auto same = [](float x, float y) {
        return __builtin_bit_cast(uint32_t, x) == __builtin_bit_cast(uint32_t, y) || (x != x && y != y);
    };
    uint32_t st = decided ? 1u : 0u;
    if (!same(got, exact) || (decided && !same(fast, exact))) st |= 2u;
    const float us[4] = {1.0f, -3.5f, 0.01233f, 250.0f};
    for (int k = 0; k < 4; ++k) {
        const uint32_t a = mq4::swiglu_bf16_fast(g, us[k]), r = mq4::swiglu_bf16(g, us[k]);
        const bool nan_a = (a & 0x7fffu) > 0x7f80u, nan_r = (r & 0x7fffu) > 0x7f80u;
        if (a != r && !(nan_a && nan_r)) st |= 4u;
    }
    float ga[16], ua[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        ga[e] = mq4::bf16_to_f32((b + 4099u * (uint32_t)e) & 0xffffu);
        ua[e] = us[e & 3];
    }
    uint32_t hv[16];
    mq4::swiglu_bf16_batch<16>(ga, ua, hv);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const uint32_t r = mq4::swiglu_bf16(ga[e], ua[e]);
        const bool nan_a = (hv[e] & 0x7fffu) > 0x7f80u, nan_r = (r & 0x7fffu) > 0x7f80u;
        if (hv[e] != r && !(nan_a && nan_r)) st |= 8u;
    }
    status[b] = st;
}

}  // namespace

// status: 65536 words of device memory.  0, or -1 on a launch error.
extern "C" int mq4check_sigmoid(uint32_t* status, void* stream) {
    hipLaunchKernelGGL(sigmoid_check_kernel, dim3(256), dim3(256), 0, (hipStream_t)stream, status);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
