"""Pins oracle/sampler.py, the restatement of sample_token's masks
(src/sampling/sampler.cpp:18-36), independently of its own formulas:
hand-worked probabilities, a per-element loop over the definition with exact
Fraction sums, brute-force top-k, and invariants.  The reference's tests hold
no sampler cases, so these are the pins."""
from fractions import Fraction

import numpy as np
import pytest

from oracle import sampler as S


def bf16(vals):
    f = np.asarray(vals, np.float32)
    return (f.view(np.uint32) >> 16).astype(np.uint16)   # exact for the values used here


# ---- hand-worked cases -------------------------------------------------
# logits 0,1,2,3 at temperature 1: p = e^k / (1 + e + e^2 + e^3)
#   = 0.0321, 0.0871, 0.2369, 0.6439; mass before (ascending) = 0, 0.0321,
#   0.1192, 0.3561.  Masked where that mass exceeds top_p.
@pytest.mark.parametrize("top_p,keep", [
    (0.5, [1, 1, 1, 1]),
    (0.1, [1, 1, 0, 0]),
    (0.03, [1, 0, 0, 0]),
    (0.0321, [1, 1, 0, 0]),      # mass before logit 1 is 0.03206 <= 0.0321
])
def test_hand_worked_top_p(top_p, keep):
    got = S.keep_mask(bf16([0, 1, 2, 3]), 1.0, 0, top_p)
    assert got.astype(int).tolist() == [keep]


def test_hand_worked_temperature():
    # temperature 0.5: scaled 0,2,4,6; p = 0.00214, 0.01584, 0.1171, 0.8650;
    # mass before = 0, 0.00214, 0.01798, 0.1351
    assert S.keep_mask(bf16([0, 1, 2, 3]), 0.5, 0, 0.1).astype(int).tolist() == [[1, 1, 1, 0]]
    assert S.keep_mask(bf16([0, 1, 2, 3]), 0.5, 0, 0.01).astype(int).tolist() == [[1, 1, 0, 0]]


def test_hand_worked_scatter_order():
    # the same values permuted: logit 3 at index 0, 0 at 1, 2 at 2, 1 at 3.
    # Scattering back through sorted_idx instead of its inverse would give
    # [1, 0, 0, 1].
    assert S.keep_mask(bf16([3, 0, 2, 1]), 1.0, 0, 0.1).astype(int).tolist() == [[0, 1, 0, 1]]


@pytest.mark.parametrize("vals,k,keep", [
    ([5, 1, 5, 3, 2], 2, [1, 0, 1, 0, 0]),     # the 2nd largest is 5: both 5s kept
    ([5, 1, 5, 3, 2], 3, [1, 0, 1, 1, 0]),
    ([4, 4, 4, 1], 1, [1, 1, 1, 0]),           # ties at the k-th value are kept
    ([4, 4, 4, 1], 4, [1, 1, 1, 1]),           # k = N masks nothing
    ([-1, -3, -2], 1, [1, 0, 0]),
])
def test_hand_worked_top_k(vals, k, keep):
    assert S.keep_mask(bf16(vals), 1.0, k, 1.0).astype(int).tolist() == [keep]


def test_nan_is_masked():
    x = bf16([1, 2, 3])
    x[1] = 0x7FC0
    assert S.keep_mask(x, 1.0, 0, 1.0).astype(int).tolist() == [[1, 0, 1]]


# ---- the definition, element by element, with exact sums ---------------
def loop_keep(vals_f64, top_k, top_p):
    """Kept iff fewer than k elements are strictly larger (top-k) and the
    exact mass of the elements sorted before it -- smaller probability, or
    equal probability and lower index -- is at most top_p."""
    n = len(vals_f64)
    kept = [True] * n
    if 0 < top_k < n:
        for i in range(n):
            kept[i] = sum(1 for j in range(n) if vals_f64[j] > vals_f64[i]) < top_k
    if 0.0 < top_p < 1.0:
        s = np.array([v if kept[i] else -np.inf for i, v in enumerate(vals_f64)])
        p = np.exp(s - s.max())
        p = p / p.sum()
        P = [Fraction(float(x)) for x in p]
        lim = Fraction(float(np.float32(top_p)))
        for i in range(n):
            before = sum((P[j] for j in range(n) if P[j] < P[i] or (P[j] == P[i] and j < i)), Fraction(0))
            kept[i] = kept[i] and before <= lim
    return kept


@pytest.mark.parametrize("seed", range(40))
def test_matches_loop_definition(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(2, 14))
    # few distinct values so ties are common
    vals = rng.integers(-6, 7, size=n) * (0.5 if seed % 2 else 0.75)
    x = bf16(vals)
    t = float(rng.choice([0.5, 1.0, 1.7]))
    k = int(rng.integers(0, n + 1))
    p = float(rng.choice([0.05, 0.2, 0.45, 0.8, 0.97]))
    if S.topp_margin(x, t, k, p) < 1e-9:
        p += 1e-4
    got = S.keep_mask(x, t, k, p, dtype=np.float64)[0].tolist()
    want = loop_keep(S.bf16_to_f32(x).astype(np.float64) / np.float64(np.float32(t)), k, p)
    assert got == want, (vals.tolist(), t, k, p)


# ---- invariants --------------------------------------------------------
def test_invariants():
    rng = np.random.default_rng(7)
    x = bf16(rng.normal(0, 3, size=(4, 500)).astype(np.float32))
    assert S.keep_mask(x, 1.0, 0, 1.0).all()                  # top_p = 1: no mask
    assert S.keep_mask(x, 1.0, 500, 1.0).all()                # top_k = N: no mask
    assert S.keep_mask(x, 1.0, 0, 0.999999).all()             # mass before any element < 1 - p_max
    small = S.keep_mask(x, 1.0, 0, 1e-9)
    s = S.bf16_to_f32(x)
    for r in range(4):                                        # the smallest probability is always kept
        assert small[r, np.argmin(s[r])]
    # top-k alone keeps exactly the elements at or above the k-th largest
    km = S.keep_mask(x, 0.8, 25, 1.0)
    for r in range(4):
        thr = np.sort(s[r])[::-1][24]
        assert np.array_equal(km[r], s[r] >= thr)
    # the top-p mask is monotone in top_p
    a = S.keep_mask(x, 1.0, 0, 0.2)
    b = S.keep_mask(x, 1.0, 0, 0.6)
    assert (a <= b).all()
