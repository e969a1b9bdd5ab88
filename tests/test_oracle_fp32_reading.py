"""The reference's activation dtype at the quantized-matmul seam.

In MLX's C++ API a float scalar is a float32 array, so rms_norm
(src/model/marlin.cpp:12-16) returns float32 ("variance + eps" and
"1.0f + weight" promote), and from there the reference's MLP half
(marlin.cpp:141-142: qmatmul on float32 x with the bf16 scales and biases
promoted, float32 SwiGLU and residual) and its lm_head + argmax
(marlin.cpp:161-169, sampler.cpp:15) run in float32.  The kernels follow the
benchmark configurations' bf16 activations instead (every op boundary
bf16, as the bf16 chain of the oracle).  This file pins the oracle's
float32-reading functions and measures how far the two readings are apart
on the benchmark's 24-layer synthetic model over 64 tokens: the hidden
state's drift and the greedy tokens.

Measured (printed by test_fp32_reading_against_bf16_chain_64_tokens): the
hidden states after 24 layers differ by 2.2e-2 of rms on average (at most
2.5e-2; the bf16 roundings of the residual stream and of every
intermediate, absent in the float32 reading; about what two bf16 chains
that differ only in accumulation drift apart), and 60 of the 64 tokens
agree; the 4 differing tokens are near-ties whose float32 logits lie 1e-3
to 2e-2 of rms(logits) below the float32 maximum, against a drift bound of
about 0.13.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

H, I, V, LAYERS, EPS = 2048, 6144, 248320, 24, 1e-6


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------- pinning ---

def test_qmm_f64_x32_pins(O):
    """Equal to the bf16-x fp64 oracle on bf16-representable x (same terms,
    same order); exact rationals on a tiny shape; numpy float64 on the
    dequantized weights for general float32 x."""
    N, K = 24, 128
    w = O.gen_normal_bf16(71, N * K, 0.0, 0.02).reshape(N, K)
    wq, s, b = O.quantize(w)
    xb = O.gen_normal_bf16(72, 3 * K).reshape(3, K)
    y32 = O.qmm_f64_x32(O.bf16_to_f32(xb), wq, s, b)
    y64, _ = O.qmm_f64(xb, wq, s, b)
    assert np.array_equal(y32, y64)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, K)).astype(np.float32) * np.float32(3.7)
    got = O.qmm_f64_x32(x, wq, s, b)
    deq = O.dequantize_f64(wq, s, b)
    ref = x.astype(np.float64) @ deq.T
    assert np.max(np.abs(got - ref)) <= 1e-12 * np.max(np.abs(ref))
    # exact: one row, the first 8 outputs
    for n in range(8):
        exact = sum(Fraction(float(x[0, k])) * Fraction(float(deq[n, k])) for k in range(K))
        assert abs(Fraction(got[0, n]) - exact) <= abs(exact) * Fraction(1, 2 ** 50) + Fraction(1, 2 ** 80)


def test_rmsnorm_f32_known_answers(O):
    """Hand-derived answers of the float32 reading.  [3, 4]: mean(x^2) = 12.5,
    r = 1/sqrt(12.5 + 1e-6), out = x * r * (1 + w).  The bf16 input's square
    is bf16 (1 + 2^-7 squares to 1 + 2^-6 + 2^-14, stored as 1 + 2^-6), the
    float32 input's is not: the two results differ exactly there."""
    x = torch.tensor([[3.0, 4.0]], dtype=torch.bfloat16)
    w = torch.tensor([0.0, 0.5], dtype=torch.bfloat16)
    got = O.rmsnorm_f32(bits(x), bits(w), EPS)
    r = np.float32(1.0) / np.sqrt(np.float32(12.5) + np.float32(EPS))
    assert got.dtype == np.float32
    assert np.array_equal(got, np.array([[np.float32(3.0) * r * np.float32(1.0),
                                          np.float32(4.0) * r * np.float32(1.5)]], np.float32))
    # one element: mean = x^2, so out = x / sqrt(x^2 + eps) ~ 1; bf16 square rounds
    v = 1.0 + 2.0 ** -7
    xb = torch.tensor([[v]], dtype=torch.bfloat16)
    got_b = O.rmsnorm_f32(bits(xb), bits(torch.zeros(1, dtype=torch.bfloat16)), 0.0)
    got_f = O.rmsnorm_f32(np.array([[v]], np.float32), bits(torch.zeros(1, dtype=torch.bfloat16)), 0.0)
    assert got_b[0, 0] == np.float32(v) / np.sqrt(np.float32(1.0 + 2.0 ** -6))
    assert got_f[0, 0] == np.float32(v) / np.sqrt(np.float32(v) * np.float32(v))
    assert got_b[0, 0] != got_f[0, 0]


def test_rmsnorm_f32_matches_torch_promotion(O):
    """The chain replayed with torch CPU ops and MLX C++'s promotion made
    explicit (eps and 1.0 as float32 tensors): bf16 square / sum / mean,
    float32 from "+ eps" on.  torch's float32 reductions may sum in another
    order, so the bar is a few float32 ulps."""
    g = torch.Generator().manual_seed(3)
    x = (torch.randn((4, H), generator=g) * 1.7).to(torch.bfloat16)
    w = (torch.randn(H, generator=g) * 0.02 + 0.1).to(torch.bfloat16)
    # 1-element tensors: torch treats 0-dim tensors as weak scalars that do not promote
    eps32, one32 = torch.tensor([EPS], dtype=torch.float32), torch.tensor([1.0], dtype=torch.float32)
    var = (x * x).sum(dim=-1, keepdim=True).to(torch.bfloat16) * torch.tensor([1.0 / H], dtype=torch.bfloat16)
    ref = (x * torch.rsqrt(var + eps32)) * (one32 + w)
    assert ref.dtype == torch.float32
    got = O.rmsnorm_f32(bits(x), bits(w), EPS)
    assert np.max(np.abs(got - ref.numpy()) / np.maximum(np.abs(ref.numpy()), 1e-30)) <= 4 * 2.0 ** -24
    # float32 input: torch's mean divides by K where the restatement multiplies
    # by float32(1/K), and its rsqrt and summation order differ, a few ulps
    # each; a formula mistake (no eps, w for 1 + w, a mean over another
    # count) is orders of magnitude larger
    xf = torch.randn((3, H), generator=g) * 2.1
    ref2 = (xf * torch.rsqrt((xf * xf).mean(dim=-1, keepdim=True) + eps32)) * (one32 + w)
    got2 = O.rmsnorm_f32(xf.numpy(), bits(w), EPS)
    assert np.max(np.abs(got2 - ref2.numpy()) / np.maximum(np.abs(ref2.numpy()), 1e-30)) <= 8 * 2.0 ** -24


def test_swiglu_f32(O):
    """Known answers (g = 0 gives 0; g = 0 or u = 0 gives 0) and torch's
    float32 chain: its sigmoid is a different float32 evaluation (a few ulps
    apart), which the two products carry into the result, so the bar is 6
    float32 ulps of the result; sigmoid(-g), a missing factor g or the
    order (g * u) * sigmoid are far outside it."""
    assert O.swiglu_f32(np.float32([0.0, 2.0]), np.float32([5.0, 0.0])).tolist() == [0.0, 0.0]
    g = torch.Generator().manual_seed(4)
    a, b = torch.randn(4096, generator=g) * 4, torch.randn(4096, generator=g)
    ref = (torch.sigmoid(a) * a) * b
    got = O.swiglu_f32(a.numpy(), b.numpy())
    assert np.all(np.abs(got - ref.numpy()) <= 6 * np.spacing(np.abs(ref.numpy()).astype(np.float32)) + 1e-38)


def test_decode_chain_f32_zero_mlp(O):
    """With all-zero MLP weights (every quantized group of zeros dequantizes to
    exactly 0) the MLP halves add 0: the hidden state is the input promoted
    to float32 (the residual add of a bf16 and a float32 array), so the
    final norm takes the float32 path: logits = lm_head(rmsnorm_f32(float32
    x)), which differs from the norm of the bf16 input."""
    K, N = 256, 64
    zero = O.quantize(np.zeros((K, K), np.uint16))
    assert not O.dequantize_f64(*zero).any()
    lm = O.quantize(O.gen_normal_bf16(73, N * K, 0.0, 0.02).reshape(N, K))
    nw = O.gen_normal_bf16(74, K, 0.1, 0.02)
    fn = O.gen_normal_bf16(75, K, 0.1, 0.02)
    x = O.gen_normal_bf16(76, 2 * K).reshape(2, K)
    h, logits, tok = O.decode_chain_f32(x, [(nw, zero, zero, zero)] * 2, fn, lm, EPS)
    assert h.dtype == np.float32 and np.array_equal(h, O.bf16_to_f32(x))
    want = O.qmm_f64_x32(O.rmsnorm_f32(O.bf16_to_f32(x), fn, EPS), *lm).astype(np.float32)
    assert np.array_equal(logits, want)
    assert not np.array_equal(logits, O.qmm_f64_x32(O.rmsnorm_f32(x, fn, EPS), *lm).astype(np.float32))
    assert np.array_equal(tok, np.argmax(want, axis=-1))


# --------------------------------------------------------- measurement ---

@pytest.fixture(scope="module")
def model(O):
    layers = []
    for l in range(LAYERS):
        g = O.quantize(O.gen_normal_bf16(1000 + 3 * l, I * H, 0.0, 0.02).reshape(I, H))
        u = O.quantize(O.gen_normal_bf16(1001 + 3 * l, I * H, 0.0, 0.02).reshape(I, H))
        d = O.quantize(O.gen_normal_bf16(1002 + 3 * l, H * I, 0.0, 0.02).reshape(H, I))
        layers.append((O.gen_normal_bf16(2100 + l, H, 0.1, 0.02), g, u, d))
    lm = O.quantize(O.gen_normal_bf16(2000, V * H, 0.0, 0.02).reshape(V, H))
    return layers, O.gen_normal_bf16(2001, H, 0.1, 0.02), lm


def test_fp32_reading_against_bf16_chain_64_tokens(O, model):
    """64 tokens (the decode rows of the benchmark's generator, streams
    3000..3063) through the 24-layer model in both readings.  Bars:
    * hidden-state drift between the readings after 24 layers <= 6e-2 of rms
      per row (two bf16 chains that differ only in accumulation drift 1.9e-2,
      tests/test_oracle_chain_drift.py; here every intermediate's bf16
      rounding differs);
    * a token of the bf16 chain may differ from the float32 reading's only
      on a near-tie: its float32 logit within 4.5 x rel x rms(logits) of the
      float32 maximum (rel the row's hidden drift; a drift of rel moves each
      logit by about rel x rms, two logits' difference by sqrt(2) times that,
      so 4.5 x rel is over 3 standard deviations) plus one bf16 ulp of the
      maximum (the bf16 chain's argmax runs over bf16 logits)."""
    layers, fnorm, lm = model
    M = 64
    x = np.stack([O.gen_normal_bf16(3000 + m, H) for m in range(M)])
    hb, lb64, tok_b = O.decode_chain_bf16(x, layers, fnorm, lm, EPS)
    hf, l32, tok_f = O.decode_chain_f32(x, layers, fnorm, lm, EPS)
    hbf = O.bf16_to_f32(hb).astype(np.float64)
    hff = hf.astype(np.float64)
    rel = np.sqrt(np.mean((hbf - hff) ** 2, axis=1) / np.mean(hff * hff, axis=1))
    l32 = l32.astype(np.float64)
    lrms = np.sqrt(np.mean(l32 * l32, axis=1))
    rows = np.arange(M)
    gap = l32.max(axis=1) - l32[rows, tok_b]
    ulp = np.exp2(np.floor(np.log2(np.abs(l32.max(axis=1)))) - 7)
    bar = 4.5 * rel * lrms + ulp
    agree = float(np.mean(tok_b == tok_f))
    diff = rows[tok_b != tok_f]
    print(f"hidden drift fp32 vs bf16 reading after {LAYERS} layers: mean {rel.mean():.2e}, max {rel.max():.2e}; "
          f"tokens agree {agree:.3f} ({int(np.sum(tok_b == tok_f))}/{M}); differing rows' gap / rms(logits): "
          + ", ".join(f"{gap[m] / lrms[m]:.2e} (bar {bar[m] / lrms[m]:.2e})" for m in diff))
    assert rel.max() <= 6e-2
    assert np.all(gap <= bar)
