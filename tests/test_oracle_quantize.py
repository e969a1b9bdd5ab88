"""Pins the oracle's MLX affine quantize (oracle/mq4_oracle.c, mq4o_quantize).

The reference calls mx::quantize(w, 64, 4) at src/model/weights.cpp:46 and
:183; the arithmetic is in the un-vendored MLX v0.25.2, so no reference test or
fixture exists.  The oracle is pinned here by

* hand-derived known answers (tests/golden/quantize_kat.json), each chosen so
  that a plausible mistake fails it:
    all_zero            eps = 1e-7 and the negative-scale default: scale is
                        bf16(-1e-7) = 0xb3d7, bias 0, all nibbles 0.
    max_edge            |max| >= |min| picks the max as edge/bias with a
                        negative scale: s = 1.5/(-15) = -0.1f, q(0) = 15.
    max_edge_f32_scale  nibbles use the float32 scale, not the stored bf16
                        one: (0.44921875-1.5)/-0.1f = 10.5078 -> 11, while
                        bf16(-0.1) = -0.10009766 would give 10.4976 -> 10.
    min_edge            |min| > |max| picks the min with a positive scale.
    constant            zero range: scale = -1e-7f, q0 = rint(0.25/-1e-7f) =
                        -2500000, scale = 0.25/q0 = -1e-7f, bias 0.25, q 0.
    half_even_ties      scale 0.125, bias -1.875: quotients 0.5, 1.5, 2.5,
                        3.5, 14.5 must round half-to-even to 0, 2, 2, 4, 14
                        (round-half-away would give 1, 2, 3, 4, 15).
    clip_high           s = 1/(-8), q(-0.9453125) = rint(15.5625) = 16 is
                        clipped to 15; q(0) = 8.
* invariants on N(0, 0.02) data: the bias is the larger-magnitude group
  extreme (max on ties) or 0, the edge element has nibble 0, the scale's sign
  follows the edge side, and every unclipped element lies within half a
  scale step (plus the bf16 rounding of the stored scale) of its level;
* the packing layout, re-derived by an independent numpy unpack.
"""
import json
import os

import numpy as np
import pytest

KAT = os.path.join(os.path.dirname(__file__), "golden", "quantize_kat.json")


def kat_cases():
    with open(KAT) as f:
        return json.load(f)["cases"]


def kat_group(O, case):
    v = np.full(64, case["fill"], np.float32)
    for k, val in case["set"].items():
        v[int(k)] = val
    b = O.f32_to_bf16(v)
    assert np.array_equal(O.bf16_to_f32(b), v), "KAT values must be exact bf16"
    return b


@pytest.mark.parametrize("case", kat_cases(), ids=lambda c: c["name"])
def test_quantize_known_answers(O, case):
    w = kat_group(O, case)[None, :]
    wq, s, b = O.quantize(w)
    assert [f"0x{x:08x}" for x in wq[0]] == case["words"]
    assert f"0x{s[0, 0]:04x}" == case["scale"]
    assert f"0x{b[0, 0]:04x}" == case["bias"]


def test_quantize_groups_are_independent_and_row_major(O):
    cases = kat_cases()
    rows = [np.concatenate([kat_group(O, c) for c in cases[:4]]),
            np.concatenate([kat_group(O, c) for c in cases[3:7]])]
    w = np.stack(rows)   # [2, 256]: groups are consecutive 64-runs of each row
    wq, s, b = O.quantize(w)
    assert wq.shape == (2, 32) and s.shape == (2, 4)
    for r, sel in ((0, cases[:4]), (1, cases[3:7])):
        for g, c in enumerate(sel):
            assert [f"0x{x:08x}" for x in wq[r, 8 * g:8 * g + 8]] == c["words"]
            assert f"0x{s[r, g]:04x}" == c["scale"]
            assert f"0x{b[r, g]:04x}" == c["bias"]


def test_quantize_rejects_bad_k(O):
    with pytest.raises(ValueError):
        O.quantize(np.zeros((2, 96), np.uint16))


def unpack(wq):
    """Independent unpack: nibble p of word j -> element 8j + p."""
    N, W = wq.shape
    shifts = np.arange(8, dtype=np.uint32) * 4
    return ((wq[:, :, None] >> shifts[None, None, :]) & 0xF).reshape(N, W * 8).astype(np.int64)


@pytest.fixture(scope="module")
def random_quant(O):
    N, K = 192, 2048
    w = O.gen_normal_bf16(1000, N * K, 0.0, 0.02).reshape(N, K)
    return w, O.quantize(w)


def test_quantize_invariants(O, random_quant):
    w, (wq, s, b) = random_quant
    N, K = w.shape
    wf = O.bf16_to_f32(w).astype(np.float64).reshape(N, K // 64, 64)
    q = unpack(wq).reshape(N, K // 64, 64)
    sf = O.bf16_to_f32(s).astype(np.float64)
    bf = O.bf16_to_f32(b).astype(np.float64)
    gmax, gmin = wf.max(-1), wf.min(-1)
    side_min = np.abs(gmin) > np.abs(gmax)
    edge = np.where(side_min, gmin, gmax)
    # bias is exactly the edge extreme (bf16-exact, so no rounding) or 0
    assert np.all((bf == edge) | (bf == 0.0))
    assert np.mean(bf == edge) > 0.999
    # the scale points from the edge into the group
    assert np.all(np.sign(sf) == np.where(side_min, 1.0, -1.0))
    # the edge element reconstructs exactly: its nibble is 0
    at_edge = wf == edge[..., None]
    assert np.all(q[at_edge & (bf[..., None] != 0)] == 0)
    # every element lies within half a step of its level; the stored scale is
    # the float32 scale rounded to bf16, so allow its relative error 2^-8
    deq = sf[..., None] * q + bf[..., None]
    step = np.abs(sf)[..., None]
    unclipped = (q > 0) & (q < 15)
    err = np.abs(wf - deq)
    assert np.all(err[unclipped] <= step.repeat(64, -1)[unclipped] * (0.5 + 15 * 2.0 ** -8) + 1e-12)
    # clipping is rare and only ever at the far end from the edge
    assert np.mean(q == 15) < 0.05


def test_quantize_matches_independent_level_search(O, random_quant):
    """Brute force: for each element, the chosen level minimises |w - b - s*q|
    over q in [0, 15] with s the stored (bf16) scale, except near ties: the
    float32 scale used for the nibbles differs from the stored one by at most
    2^-8 |s|, which moves level q by at most 15 * 2^-8 |s|, so the two nearest
    distances can swap only when they differ by less than 2 * 16 * 2^-8 |s|."""
    w, (wq, s, b) = random_quant
    N, K = w.shape
    wf = O.bf16_to_f32(w).astype(np.float64).reshape(N, K // 64, 64)
    q = unpack(wq).reshape(N, K // 64, 64)
    sf = O.bf16_to_f32(s).astype(np.float64)[..., None, None]
    bf = O.bf16_to_f32(b).astype(np.float64)[..., None, None]
    levels = np.arange(16, dtype=np.float64)
    dist = np.abs(wf[..., None] - (bf + sf * levels))       # [N, G, 64, 16]
    best = dist.argmin(-1)
    sorted_d = np.sort(dist, -1)
    ambiguous = (sorted_d[..., 1] - sorted_d[..., 0]) <= 32 * np.abs(sf[..., 0]) * 2.0 ** -8
    assert np.all((best == q) | ambiguous)
    assert np.mean(ambiguous) < 0.2   # window is 1/8 of a step: about 12% of elements


def test_dequantize_f64_is_exact_affine(O, random_quant):
    w, (wq, s, b) = random_quant
    d = O.dequantize_f64(wq, s, b)
    q = unpack(wq)
    sf = np.repeat(O.bf16_to_f32(s).astype(np.float64), 64, axis=1)
    bf = np.repeat(O.bf16_to_f32(b).astype(np.float64), 64, axis=1)
    assert np.array_equal(d, sf * q + bf)
