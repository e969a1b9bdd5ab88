/* Exactness check of the quantize kernel's division by 15 (div15 in
 * marlin-mlx_amd/csrc/mq4_quantize.hip): one Markstein step
 * q + RN(x - 15 q) * y from q = RN(x * y), y = RN(1 / 15), against IEEE
 * x / 15, for the non-negative finite floats x whose bit pattern is a
 * multiple of the stride given as argv[1] (1 = all 2^31 of them), plus every
 * subnormal and every float in [2^-30, 2^-20] (around the 1e-7 scale
 * floor).  Prints the count of mismatches; exit status 1 if any. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static int bad(uint32_t bits) {
    const float y = 0x1.111112p-4f;
    const float x = f_of(bits);
    volatile float ref = x / 15.0f;
    const float q = x * y;
    const float q1 = fmaf(fmaf(-q, 15.0f, x), y, q);
    return u_of(q1) != u_of(ref);
}

int main(int argc, char** argv) {
    const int64_t stride = argc > 1 ? atoll(argv[1]) : 1;
    long mismatches = 0;
    for (int64_t b = 0; b <= 0x7F7FFFFFLL; b += stride) mismatches += bad((uint32_t)b);
    for (uint32_t b = 0; b < 0x00800000u; ++b) mismatches += bad(b);                       /* subnormals */
    for (uint32_t b = u_of(0x1p-30f); b <= u_of(0x1p-20f); ++b) mismatches += bad(b);      /* near 1e-7 */
    printf("div15 mismatches: %ld\n", mismatches);
    return mismatches ? 1 : 0;
}
