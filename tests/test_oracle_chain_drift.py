"""How far two correct implementations of the 24-layer MLP chain drift apart.

The decode step's hidden state after the per-layer residual adds
(src/model/marlin.cpp:141-142) is a bf16 stream: a 1-ulp difference in one
layer's output flips roundings in the next layers, so two implementations
that each meet the per-op bar (1e-2 of rms on every GEMV) disagree by a
growing amount.  This test measures that drift on the oracle itself, between
its fp64 GEMV (each output rounded once from fp64) and its fp32-accumulating
GEMV, on the benchmark's synthetic model (24 layers, 6144x2048 / 2048x6144,
the same seeded generator streams): it grows roughly linearly, about 1e-3 of
rms per layer, to ~1.9e-2 after 24 layers.  The GPU decode-step test's bar
against the oracle after 24 layers (5e-2) is set from this number.
"""
import numpy as np


def test_two_correct_chains_drift_apart(O):
    H, I = 2048, 6144
    layers = []
    for l in range(24):
        g = O.quantize(O.gen_normal_bf16(1000 + 3 * l, I * H, 0.0, 0.02).reshape(I, H))
        u = O.quantize(O.gen_normal_bf16(1001 + 3 * l, I * H, 0.0, 0.02).reshape(I, H))
        d = O.quantize(O.gen_normal_bf16(1002 + 3 * l, H * I, 0.0, 0.02).reshape(H, I))
        layers.append((g, u, d, O.gen_normal_bf16(2100 + l, H, 0.1, 0.02)))
    x0 = O.gen_normal_bf16(3000, H).reshape(1, H)

    def run(f64):
        x, out = x0, []
        for g, u, d, nw in layers:
            n = O.rmsnorm_1pw(x, nw, 1e-6)
            if f64:
                h = O.swiglu_bf16(O.qmm_f64(n, *g)[1], O.qmm_f64(n, *u)[1])
                y = O.qmm_f64(h, *d)[1]
            else:
                h = O.swiglu_bf16(O.qmm_f32(n, *g), O.qmm_f32(n, *u))
                y = O.qmm_f32(h, *d)
            x = O.add_bf16(x, y)
            out.append(O.bf16_to_f32(x).astype(np.float64))
        return out

    a, b = run(True), run(False)
    drift = [float(np.sqrt(np.mean((p - q) ** 2)) / np.sqrt(np.mean(p * p))) for p, q in zip(a, b)]
    print("drift per layer:", " ".join(f"{d:.1e}" for d in drift))
    assert drift[0] < 1e-3                 # one layer: ulp-level
    assert 1e-2 <= drift[-1] <= 3e-2       # 24 layers: the measured ~1.9e-2
    assert drift[-1] > drift[5] > drift[1]
