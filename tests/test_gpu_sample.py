"""GPU sampler (mq4_sample_bf16) against the oracle of sample_token's masks
(src/sampling/sampler.cpp:9-39).

* keep masks: bit-exact against oracle/sampler.py wherever the top-p boundary
  is clear of summation rounding (topp_margin); heavy-tie inputs exercise the
  index-order ranks at the boundary, N % 8 != 0 the scalar-load variant.
* draws: the token equals the Gumbel-max over the oracle's kept set computed
  here with the library's documented generator (SplitMix64 finaliser of seed,
  row and index; u = (j + 1/2) 2^-23), except at near-ties of the perturbed
  values; and the empirical distribution over many rows passes a chi-square
  test against softmax over the kept set.  The reference draws with MLX's
  global key, so individual draws are parity unpinned against it; the
  distribution is the pin.
"""
import numpy as np
import pytest
import torch

from oracle import sampler as S

pytestmark = pytest.mark.gpu


def mix64(z):
    z = np.asarray(z, np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def uniform01(seed, m, n):
    with np.errstate(over="ignore"):
        state = mix64(np.uint64(seed) ^ (np.uint64(m + 1) * np.uint64(0xD1B54A32D192ED03)))
        i = np.arange(n, dtype=np.uint64)
        z = mix64(state + (i + np.uint64(1)) * np.uint64(0x9E3779B97F4A7C15))
    return (((z >> np.uint64(41)).astype(np.float32) + np.float32(0.5)) * np.float32(2.0 ** -23)).astype(np.float32)


def gumbel_tokens(bits, keep, temperature, seed):
    """Token per row and the gap between its perturbed value and the runner-up."""
    s = S.scaled_logits(bits, temperature, np.float32)
    toks, gaps = [], []
    for m in range(bits.shape[0]):
        u = uniform01(seed, m, bits.shape[1])
        g = -np.log(-np.log(u))
        v = np.where(keep[m], s[m] + g, -np.inf).astype(np.float32)
        order = np.argsort(-v, kind="stable")
        toks.append(int(order[0]))
        gaps.append(float(v[order[0]] - v[order[1]]) if len(v) > 1 else np.inf)
    return np.array(toks), np.array(gaps)


def gen_logits(rng, M, N, kind):
    if kind == "normal":
        f = rng.normal(0.0, 3.0, size=(M, N)).astype(np.float32)
    else:                                               # few distinct values: many exact ties
        f = (rng.integers(-8, 9, size=(M, N)) * 0.5).astype(np.float32)
    return (f.view(np.uint32) >> 16).astype(np.uint16)   # truncation to bf16 is fine for inputs


def to_dev(bits, dev):
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).to(dev)


def run(mq4, bits, dev, temperature, top_k, top_p, seed):
    print(f"sample M={bits.shape[0]} N={bits.shape[1]} t={temperature} k={top_k} p={top_p} seed={seed}", flush=True)
    tok, keep = mq4.sample_token(to_dev(bits, dev), temperature, top_k, top_p, seed=seed, return_keep=True)
    torch.cuda.synchronize()
    return tok.cpu().numpy(), (keep.cpu().numpy().astype(bool) if keep is not None else None)


CASES = [
    # (M, N, kind, temperature, top_k, top_p)
    (3, 4096, "normal", 1.0, 0, 1.0),
    (3, 4096, "normal", 0.7, 40, 1.0),
    (3, 4096, "normal", 1.0, 0, 0.3),
    (3, 4096, "normal", 1.3, 0, 0.9),
    (3, 4096, "normal", 0.7, 200, 0.2),
    (2, 4096, "ties", 1.0, 0, 0.35),
    (2, 4096, "ties", 1.0, 100, 0.6),
    (2, 4096, "ties", 0.5, 1, 1.0),
    (2, 999, "normal", 1.0, 17, 0.4),      # N % 8 != 0: scalar loads
    (2, 999, "ties", 1.0, 0, 0.25),
    (1, 151936, "normal", 0.8, 0, 0.5),    # full vocabulary
    (1, 151936, "normal", 0.8, 50, 0.9),
    (1, 151936, "ties", 1.0, 0, 0.7),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_keep_mask_and_draw(mq4, dev, case):
    M, N, kind, t, k, p = case
    rng = np.random.default_rng(CASES.index(case))
    bits = gen_logits(rng, M, N, kind)
    # keep the top-p boundary clear of rounding: nudge top_p if a mass lands on it
    for _ in range(20):
        if S.topp_margin(bits, t, k, p) > 1e-6:
            break
        p = float(np.float32(p + 1e-3))
    assert S.topp_margin(bits, t, k, p) > 1e-6
    seed = 1234567 + N
    tok, keep = run(mq4, bits, dev, t, k, p, seed)
    want = S.keep_mask(bits, t, k, p, dtype=np.float64)
    assert np.array_equal(keep, want), f"{(keep != want).sum()} mask differences"
    if S.topp_margin(bits, t, k, p) > 1e-3:           # the reference's float32 sums agree too
        assert np.array_equal(keep, S.keep_mask(bits, t, k, p, dtype=np.float32))
    assert keep[np.arange(M), tok].all(), "drew a masked token"
    ref_tok, gaps = gumbel_tokens(bits, want, t, seed)
    for m in range(M):
        assert tok[m] == ref_tok[m] or gaps[m] < 1e-5, (m, tok[m], ref_tok[m], gaps[m])


def test_greedy_is_argmax(mq4, O, dev):
    rng = np.random.default_rng(3)
    bits = gen_logits(rng, 4, 151936, "ties")
    tok, keep = run(mq4, bits, dev, 0.0, 50, 0.5, 9)
    assert keep is None
    assert np.array_equal(tok, O.argmax_bf16(bits).astype(np.int64))
    tok2, _ = run(mq4, bits, dev, -1.0, 0, 1.0, 9)
    assert np.array_equal(tok2, tok)


def test_seed_determinism(mq4, dev):
    rng = np.random.default_rng(5)
    bits = gen_logits(rng, 64, 2048, "normal")
    bits[:] = bits[0]                                   # the same row 64 times
    a, _ = run(mq4, bits, dev, 1.5, 0, 1.0, 77)
    b, _ = run(mq4, bits, dev, 1.5, 0, 1.0, 77)
    c, _ = run(mq4, bits, dev, 1.5, 0, 1.0, 78)
    assert np.array_equal(a, b)
    assert (a != c).sum() > 8
    assert len(set(a.tolist())) > 4                     # rows draw independently


@pytest.mark.parametrize("t,k,p", [(1.0, 0, 1.0), (0.8, 8, 1.0), (1.0, 0, 0.6), (0.9, 10, 0.7)])
def test_distribution_chi_square(mq4, dev, t, k, p):
    V, M = 16, 65535
    base = np.array([2.0, 1.5, 1.5, 1.0, 0.5, 0.25, 0.0, -0.5, -1.0, 3.0, 2.5, 0.75, -2.0, 1.25, 0.0, 1.75],
                    np.float32)
    bits = np.tile((base.view(np.uint32) >> 16).astype(np.uint16), (M, 1))
    tok, keep = run(mq4, bits, dev, t, k, p, 2024)
    want = S.keep_mask(bits[:1], t, k, p, dtype=np.float64)[0]
    assert S.topp_margin(bits[:1], t, k, p) > 1e-6
    assert np.array_equal(keep[0], want) and (keep == keep[0]).all()
    probs = S.kept_probs(bits[:1], t, want)[0]
    counts = np.bincount(tok, minlength=V)
    assert counts[~want].sum() == 0
    kept = np.flatnonzero(want)
    exp = probs[kept] * M
    chi2 = float((((counts[kept] - exp) ** 2) / exp).sum())
    dof = len(kept) - 1
    # mean dof, sd sqrt(2 dof): 6 sd is far outside sampling noise for a fixed seed
    assert chi2 < dof + 6.0 * np.sqrt(2.0 * dof) + 5.0, (chi2, dof, counts[kept].tolist(), exp.round(1).tolist())


def test_last_position_of_3d_logits(mq4, dev):
    rng = np.random.default_rng(11)
    bits = gen_logits(rng, 5, 3000, "normal").reshape(1, 5, 3000)
    print("sample 3-D logits [1, 5, 3000]", flush=True)
    tok = mq4.sample_token(to_dev(bits, dev), 1.0, 20, 1.0, seed=5)
    torch.cuda.synchronize()
    tok = tok.cpu().numpy()
    want = S.keep_mask(bits[0, -1:], 1.0, 20, 1.0)
    ref, _ = gumbel_tokens(bits[0, -1:], want, 1.0, 5)
    assert tok.shape == (1,) and tok[0] == ref[0]


def c_sample(mq4, x, t, k, p, seed, chunked):
    """mq4_sample_bf16 through the C ABI, with (chunked) or without a workspace."""
    import ctypes
    L = mq4.lib()
    M, V = x.shape
    idx = torch.empty(M, dtype=torch.int32, device=x.device)
    keep = torch.empty((M, V), dtype=torch.uint8, device=x.device)
    n = L.mq4_sample_workspace_size(M, V) if chunked else 0
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=x.device)
    rc = L.mq4_sample_bf16(x.data_ptr(), M, V, ctypes.c_float(t), k, ctypes.c_float(p), seed, idx.data_ptr(),
                           keep.data_ptr(), ws.data_ptr() if n else None, n, None)
    assert rc == 0, L.mq4_last_error().decode()
    torch.cuda.synchronize()
    return idx.cpu().numpy(), keep.cpu().numpy()


@pytest.mark.parametrize("M", [1, 4, 32])
def test_chunked_and_single_workgroup_paths_agree(mq4, dev, M):
    rng = np.random.default_rng(100 + M)
    V = 151936
    bits = gen_logits(rng, M, V, "normal")
    bits[-1] = gen_logits(rng, 1, V, "ties")[0]          # one row with heavy ties
    x = to_dev(bits, dev)
    assert mq4.lib().mq4_sample_workspace_size(M, V) > 0
    for (t, k, p) in [(0.0, 0, 1.0), (1.0, 0, 1.0), (0.7, 50, 1.0), (1.0, 0, 0.5), (0.8, 1000, 0.9),
                      (1.2, 7, 0.05)]:
        print(f"paths M={M} t={t} k={k} p={p}", flush=True)
        a_idx, a_keep = c_sample(mq4, x, t, k, p, 99, chunked=True)
        b_idx, b_keep = c_sample(mq4, x, t, k, p, 99, chunked=False)
        assert np.array_equal(a_idx, b_idx), (t, k, p, a_idx, b_idx)
        if t > 0:
            assert np.array_equal(a_keep, b_keep), (t, k, p)
            want = S.keep_mask(bits, t, k, p, dtype=np.float64)
            if S.topp_margin(bits, t, k, p) > 1e-6:
                assert np.array_equal(a_keep.astype(bool), want)
