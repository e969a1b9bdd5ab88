"""CPU restatement of sample_token's masks (src/sampling/sampler.cpp:9-39).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the GPU
sampler, never by the product path.

keep_mask follows sampler.cpp step by step, vectorised over rows, in the
reference's float32 arithmetic (or float64 on request):
  scaled = last_logits / temperature                         (sampler.cpp:18)
  top_k > 0: where(scaled < min(topk(scaled, k)), -inf, ...)  (:20-25)
  0 < top_p < 1: probs = softmax(scaled); sorted_idx = argsort(probs);
    cumulative = cumsum(probs[sorted_idx]);
    mask = cumulative - sorted_probs > top_p, scattered back through
    argsort(sorted_idx)                                       (:27-36)
argsort is taken as stable (equal probabilities in index order); MLX does
not document its argsort's order among equal keys, so that choice is an
assumption of this restatement.  NaN logits count as masked.  The draw
(:38-39) is random and has no restatement here: kept_probs gives the
distribution it samples, softmax(scaled) over the kept elements in float64.

Pinned by tests/test_oracle_sampler.py: hand-worked cases (the ascending
mask drops the largest probabilities), a loop over elements that applies
the definition "masked iff the probability mass sorted before it exceeds
top_p" with exact Fraction sums, brute-force top-k thresholds, and
invariants (top_p -> 1 keeps everything, the smallest probability is
always kept, top_k = N keeps everything).
"""
from __future__ import annotations

import numpy as np


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def scaled_logits(logits_bf16: np.ndarray, temperature: float, dtype=np.float32) -> np.ndarray:
    """sampler.cpp:18: float(logit) / temperature, row-wise."""
    x = bf16_to_f32(logits_bf16).astype(dtype)
    return x / dtype(temperature)


def topk_masked(scaled: np.ndarray, top_k: int) -> np.ndarray:
    """sampler.cpp:20-25: True where scaled < min(topk(scaled, k)).  top_k >= N
    masks nothing (mx::topk would refuse it)."""
    N = scaled.shape[-1]
    if top_k <= 0 or top_k >= N:
        return np.zeros(scaled.shape, bool)
    s = np.where(np.isnan(scaled), -np.inf, scaled)
    kth = -np.partition(-s, top_k - 1, axis=-1)[..., top_k - 1:top_k]
    return s < kth


def softmax(x: np.ndarray, dtype=np.float32) -> np.ndarray:
    x = x.astype(dtype)
    mx = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - mx)
    return e / np.sum(e, axis=-1, keepdims=True, dtype=dtype)


def topp_masked(scaled: np.ndarray, top_p: float, dtype=np.float32) -> np.ndarray:
    """sampler.cpp:27-36 on rows of scaled logits (-inf where already masked)."""
    if not (0.0 < top_p < 1.0):
        return np.zeros(scaled.shape, bool)
    probs = softmax(scaled, dtype)
    sorted_idx = np.argsort(probs, axis=-1, kind="stable")
    sorted_probs = np.take_along_axis(probs, sorted_idx, axis=-1)
    cumulative = np.cumsum(sorted_probs, axis=-1, dtype=dtype)
    mask = (cumulative - sorted_probs) > dtype(top_p)
    inverse = np.argsort(sorted_idx, axis=-1, kind="stable")
    return np.take_along_axis(mask, inverse, axis=-1)


def keep_mask(logits_bf16: np.ndarray, temperature: float, top_k: int = 0, top_p: float = 1.0,
              dtype=np.float32) -> np.ndarray:
    """Boolean [M, N]: the elements sampler.cpp leaves unmasked (temperature > 0)."""
    logits_bf16 = np.atleast_2d(np.asarray(logits_bf16, np.uint16))
    s = scaled_logits(logits_bf16, temperature, dtype)
    nan = np.isnan(s)
    s = np.where(nan, -np.inf, s)
    km = topk_masked(s, top_k)
    s = np.where(km, -np.inf, s)
    pm = topp_masked(s, top_p, dtype)
    return ~(nan | km | pm)


def topp_margin(logits_bf16: np.ndarray, temperature: float, top_k: int, top_p: float) -> float:
    """Smallest |mass before an element - top_p| over all elements, in float64,
    after top-k (inf when top-p is off).  Where it exceeds the float32
    rounding of a cumulative sum, every exact or float32 summation gives the
    same top-p mask."""
    if not (0.0 < top_p < 1.0):
        return float("inf")
    logits_bf16 = np.atleast_2d(np.asarray(logits_bf16, np.uint16))
    s = scaled_logits(logits_bf16, temperature, np.float64)
    s = np.where(np.isnan(s), -np.inf, s)
    s = np.where(topk_masked(s, top_k), -np.inf, s)
    p = np.sort(softmax(s, np.float64), axis=-1)
    before = np.cumsum(p, axis=-1) - p
    return float(np.min(np.abs(before - top_p)))


def kept_probs(logits_bf16: np.ndarray, temperature: float, keep: np.ndarray) -> np.ndarray:
    """sampler.cpp:38-39's distribution: softmax(scaled) over kept elements, float64."""
    s = scaled_logits(np.atleast_2d(logits_bf16), temperature, np.float64)
    s = np.where(np.atleast_2d(keep), s, -np.inf)
    return softmax(s, np.float64)
