// Device-side checks of mq4_device.h helpers for the test suite (built into
// _build/libmq4_devcheck.so, never into libmq4.so): helpers whose whole input
// domain fits one launch are compared with their exact formulation on every
// input.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mq4_device.h"

namespace {

// One thread per bf16 bit pattern b of g; every block builds the SiLU table
// in its LDS with silu_lut_entry.  status[b]: bit 0 = swiglu_bf16_lut_batch<1>
// (g, u) differs from swiglu_bf16(g, u) for one of the u below, bit 1 =
// swiglu_bf16_lut_batch<16> over g and 15 other bf16 patterns (b + 4099 k, u
// cycling through the same values) differs from swiglu_bf16 in any of the
// 16 (bits compared; both NaN counts as equal); 0: no difference.
__global__ __launch_bounds__(256) void swiglu_lut_check_kernel(uint32_t* status) {
#pragma clang fp contract(off)
    __shared__ uint16_t lut[mq4::SILU_LUT_N];
    for (uint32_t i = threadIdx.x; i < (uint32_t)mq4::SILU_LUT_N; i += blockDim.x)
        lut[i] = (uint16_t)mq4::silu_lut_entry(i);
    __syncthreads();
    const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= 65536u) return;
    auto differ = [](uint32_t x, uint32_t y) {
        const bool nan_x = (x & 0x7fffu) > 0x7f80u, nan_y = (y & 0x7fffu) > 0x7f80u;
        return x != y && !(nan_x && nan_y);
    };
    const float us[4] = {1.0f, -3.5f, 0.01233f, 250.0f};
    uint32_t st = 0;
    for (int k = 0; k < 4; ++k) {
        const float g1[1] = {mq4::bf16_to_f32(b)}, u1[1] = {us[k]};
        uint32_t h1[1];
        mq4::swiglu_bf16_lut_batch<1>(g1, u1, h1, lut);
        if (differ(h1[0], mq4::swiglu_bf16(g1[0], us[k]))) st |= 1u;
    }
    float ga[16], ua[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        ga[e] = mq4::bf16_to_f32((b + 4099u * (uint32_t)e) & 0xffffu);
        ua[e] = us[e & 3];
    }
    uint32_t hv[16];
    mq4::swiglu_bf16_lut_batch<16>(ga, ua, hv, lut);
#pragma unroll
    for (int e = 0; e < 16; ++e)
        if (differ(hv[e], mq4::swiglu_bf16(ga[e], ua[e]))) st |= 2u;
    status[b] = st;
}

}  // namespace

// status: 65536 words of device memory.  0, or -1 on a launch error.
extern "C" int mq4check_swiglu_lut(uint32_t* status, void* stream) {
    hipLaunchKernelGGL(swiglu_lut_check_kernel, dim3(256), dim3(256), 0, (hipStream_t)stream, status);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
