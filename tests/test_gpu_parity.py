"""GPU parity of libmq4 (called through its C ABI via the package's ctypes
bindings) against the CPU oracle on identical seeded inputs.

Bars (stated per test):
* quantize / pack, scales, biases, argmax indices: bit-exact.
* GEMV outputs: max |got - ref| <= 1e-2 * rms(ref) against the unrounded
  fp64 oracle, measured on the kernel's unrounded fp32 result (mq4_qmm_f32);
  the bf16 result itself is element-wise at most 1 bf16 ulp from bf16(fp64)
  or, for outputs near zero where a bf16 ulp is far below fp32 accumulation
  noise, within 2^-12 * rms(ref).  (Measured against unrounded fp64, bf16
  output rounding alone costs up to half an ulp of the largest output, about
  1% of the RMS, so the 1e-2 bar is stated on the fp32 result.)
* SwiGLU outputs (bf16 op chain): element-wise, see check_swiglu.
"""
import numpy as np
import pytest
import torch

from conftest import to_dev_bf16, to_host_u16

pytestmark = pytest.mark.gpu

TOL = 1e-2   # max |err| relative to the reference output's RMS


def words(t):
    return t.cpu().numpy().view(np.uint32)


def gen_weight(mq4, O, stream_id, N, K, sigma=0.02, dev="cuda:0"):
    """Generate on the GPU (fast) and return (device tensor, host bits)."""
    w = mq4.fill_normal_bf16((N, K), stream_id, 0.0, sigma, device=dev)
    return w, to_host_u16(w)


def rel_err_f32(got_f32, ref64):
    r = np.asarray(ref64, np.float64)
    rms = float(np.sqrt(np.mean(r * r)))
    return float(np.max(np.abs(np.asarray(got_f32, np.float64) - r)) / rms)


def check_close(O, got_bits, ref64, what, got_f32=None):
    """bf16 output: <= 1 ulp of bf16(fp64) (or 2^-12 rms near zero); fp32
    output (when given): max|err| <= 1e-2 * rms against fp64."""
    ref64 = np.asarray(ref64, np.float64)
    ref_b = O.f64_to_bf16(ref64)
    ulp = O.bf16_ulp_diff(got_bits, ref_b)
    rms = float(np.sqrt(np.mean(ref64 * ref64)))
    abs_err = np.abs(O.bf16_to_f32(got_bits).astype(np.float64) - ref64)
    bad = (ulp > 1) & (abs_err > 2.0 ** -12 * rms)
    msg = (f"{what}: bf16 identical={np.mean(ulp == 0):.4f} max_ulp={int(ulp.max())} "
           f"bf16 max|err|/rms={O.rel_rms_err(got_bits, ref64):.2e}")
    if got_f32 is not None:
        e32 = rel_err_f32(got_f32, ref64)
        msg += f" fp32 max|err|/rms={e32:.2e}"
        assert e32 <= TOL, f"{what}: fp32 max|err|/rms = {e32:.3e}"
    print(msg)
    assert not bad.any(), f"{what}: {int(bad.sum())} outputs beyond 1 ulp and 2^-12 rms"
    assert np.mean(ulp == 0) >= 0.98


# ---------------------------------------------------------- generator ---

@pytest.mark.parametrize("sid,n,mu,sigma,off", [(1000, 65536, 0.0, 0.02, 0), (2000, 4097, 0.0, 0.02, 12345),
                                               (2001, 2048, 0.1, 0.02, 0), (3000, 2048, 0.0, 1.0, 0)])
def test_generator_gpu_matches_cpu(mq4, O, dev, sid, n, mu, sigma, off):
    g = to_host_u16(mq4.fill_normal_bf16((n,), sid, mu, sigma, device=dev, offset=off))
    assert np.array_equal(g, O.gen_normal_bf16(sid, n, mu, sigma, offset=off))


# ----------------------------------------------------------- quantize ---

def test_quantize_known_answers(mq4, O, dev):
    import json, os
    cases = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "quantize_kat.json")))["cases"]
    groups = []
    for c in cases:
        v = np.full(64, c["fill"], np.float32)
        for k, val in c["set"].items():
            v[int(k)] = val
        groups.append(O.f32_to_bf16(v))
    w = np.stack(groups)                 # one KAT group per row
    wq, s, b = mq4.quantize(to_dev_bf16(w, dev))
    torch.cuda.synchronize()
    for i, c in enumerate(cases):
        assert [f"0x{x:08x}" for x in words(wq)[i]] == c["words"], c["name"]
        assert f"0x{to_host_u16(s)[i, 0]:04x}" == c["scale"], c["name"]
        assert f"0x{to_host_u16(b)[i, 0]:04x}" == c["bias"], c["name"]


@pytest.mark.parametrize("N,K,sid", [(6144, 2048, 1000), (2048, 6144, 1002), (248320, 2048, 2000),
                                     (1, 64, 5), (3, 192, 6), (7, 4160, 7)])
def test_quantize_bit_exact(mq4, O, dev, N, K, sid):
    print(f"quantize N={N} K={K}", flush=True)
    w, wh = gen_weight(mq4, O, sid, N, K)
    wq, s, b = mq4.quantize(w)
    torch.cuda.synchronize()
    rq, rs, rb = O.quantize(wh)
    assert np.array_equal(words(wq), rq)
    assert np.array_equal(to_host_u16(s), rs)
    assert np.array_equal(to_host_u16(b), rb)


def test_quantize_planted_ties_and_special_groups(mq4, O, dev):
    """Random rows with exact-.5 tie groups, constant groups, all-zero groups and
    wide-range (clipping) groups planted at random positions."""
    N, K = 512, 2048
    wh = O.gen_normal_bf16(77, N * K, 0.0, 0.02).reshape(N, K).copy()
    ties = O.f32_to_bf16(np.array([-1.875, 0.0, -1.8125, -1.6875, -1.5625, -1.4375, -0.0625] + [-1.0] * 57,
                                  np.float32))
    rng = np.random.default_rng(5)
    for n, g in zip(rng.integers(0, N, 200), rng.integers(0, K // 64, 200)):
        kind = rng.integers(0, 4)
        blk = wh[n, 64 * g:64 * g + 64]
        if kind == 0:
            blk[:] = rng.permutation(ties)
        elif kind == 1:
            blk[:] = O.f32_to_bf16(np.full(64, rng.standard_normal() * 0.02, np.float32))
        elif kind == 2:
            blk[:] = 0
        else:
            blk[rng.integers(0, 64)] = O.f32_to_bf16(np.array([rng.standard_normal() * 2.0], np.float32))[0]
    wq, s, b = mq4.quantize(to_dev_bf16(wh, dev))
    torch.cuda.synchronize()
    rq, rs, rb = O.quantize(wh)
    assert np.array_equal(words(wq), rq)
    assert np.array_equal(to_host_u16(s), rs)
    assert np.array_equal(to_host_u16(b), rb)


def test_quantize_quotients_at_half_integers(mq4, O, dev):
    """Groups whose values sit on, or one bf16 ulp either side of, the
    half-integer quotients k + 1/2 of their own scale (where rounding the
    quotient decides the code), plus denormal-range groups (a reciprocal of
    the scale overflows) and groups near the bf16 maximum: the kernel's
    reciprocal-multiply path must give the codes of the exact division."""
    N, K = 384, 2048
    rng = np.random.default_rng(11)
    groups = []
    for gi in range(N * K // 64):
        kind = gi % 4
        if kind <= 1:
            lo = rng.standard_normal() * 0.02
            span = abs(rng.standard_normal()) * 0.05 + 1e-3
            k = rng.integers(0, 15, 64)
            v = (lo + (k + 0.5) * span / 15).astype(np.float32)
            v[0], v[1] = lo, lo + span                     # pin the extremes
            bits = O.f32_to_bf16(v).astype(np.int32)
            bits[2:] += rng.integers(-1, 2, 62) * (kind == 1)   # one ulp either side
            groups.append(bits.astype(np.uint16))
        elif kind == 2:
            groups.append(O.f32_to_bf16((rng.standard_normal(64) * 1e-39).astype(np.float32)))
        else:
            groups.append(O.f32_to_bf16((rng.standard_normal(64) * 1e37).astype(np.float32)))
    wh = np.stack(groups).reshape(N, K)
    print(f"quantize half-integer quotients N={N} K={K}", flush=True)
    wq, s, b = mq4.quantize(to_dev_bf16(wh, dev))
    torch.cuda.synchronize()
    rq, rs, rb = O.quantize(wh)
    assert np.array_equal(to_host_u16(s), rs)
    assert np.array_equal(to_host_u16(b), rb)
    assert np.array_equal(words(wq), rq)


def test_quantize_batch_matches_oracle(mq4, O, dev):
    """mq4_quantize_batch over 41 jobs of mixed shapes (two launches of at most
    32 jobs; K differs between jobs; ragged N): every job bit-identical to the
    oracle and to its own mq4_quantize call."""
    rng = np.random.default_rng(21)
    shapes = [(6144, 2048), (2048, 6144), (1, 64), (3, 192), (7, 4160)]
    shapes += [(int(rng.integers(1, 300)), 64 * int(rng.integers(1, 40))) for _ in range(36)]
    ws, whs = [], []
    for i, (N, K) in enumerate(shapes):
        w, wh = gen_weight(mq4, O, 3000 + i, N, K)
        ws.append(w)
        whs.append(wh)
    print(f"quantize_batch {len(shapes)} jobs", flush=True)
    outs = mq4.quantize_batch(ws)
    torch.cuda.synchronize()
    for i, ((wq, s, b), w, wh) in enumerate(zip(outs, ws, whs)):
        rq, rs, rb = O.quantize(wh)
        assert np.array_equal(words(wq), rq), i
        assert np.array_equal(to_host_u16(s), rs), i
        assert np.array_equal(to_host_u16(b), rb), i
        sq, ss, sb = mq4.quantize(w)
        assert torch.equal(sq, wq) and torch.equal(ss, s) and torch.equal(sb, b), i


def test_quantize_stream_past_2_25_groups(mq4, O, dev):
    """A matrix of 2^25 + 64 groups (4.3 GB of bf16): the kernels address one
    stream by 32-bit byte offsets and the host splits longer streams at 2^25
    groups.  The last rows, on both sides of the split, quantized within the
    whole matrix (single call, and batched beside a small job) are
    bit-identical to the same rows quantized alone and to the oracle."""
    K = 2048
    N = (1 << 25) // (K // 64) + 2                  # the split falls before row N - 2
    print(f"quantize {N}x{K} (2^25 + 64 groups)", flush=True)
    w = mq4.fill_normal_bf16((N, K), 3200, 0.0, 0.02, device=dev)
    rows = slice(N - 4, N)
    part = w[rows].contiguous()
    pq, ps, pb = mq4.quantize(part)
    wq, s, b = mq4.quantize(w)
    torch.cuda.synchronize()
    assert torch.equal(wq[rows], pq) and torch.equal(s[rows], ps) and torch.equal(b[rows], pb)
    del wq, s, b
    (bq0, bs0, bb0), (bq, bs, bb) = mq4.quantize_batch([part, w])
    torch.cuda.synchronize()
    assert torch.equal(bq[rows], pq) and torch.equal(bs[rows], ps) and torch.equal(bb[rows], pb)
    assert torch.equal(bq0, pq) and torch.equal(bs0, ps) and torch.equal(bb0, pb)
    rq, rs, rb = O.quantize(to_host_u16(part))
    assert np.array_equal(words(pq), rq)
    assert np.array_equal(to_host_u16(ps), rs) and np.array_equal(to_host_u16(pb), rb)
    del w, bq, bs, bb
    torch.cuda.empty_cache()


def test_quantize_non_finite_groups(mq4, O, dev):
    """Groups holding +-inf, NaN (some or all elements) or extremes whose range
    overflows float32 (+-3e38): the kernel's guarded quotient path (any group
    with a non-finite range in the wave) must give the oracle's codes, scales
    and biases, and the finite groups of the same waves theirs."""
    rng = np.random.default_rng(13)
    groups = []
    specials = [np.inf, -np.inf, np.nan]
    for gi in range(256):
        v = (rng.standard_normal(64) * 0.02).astype(np.float32)
        kind = gi % 8
        if kind == 0:
            v[rng.integers(0, 64)] = specials[gi // 8 % 3]
        elif kind == 1:
            v[rng.integers(0, 64, 5)] = np.nan
        elif kind == 2:
            v[:] = np.nan
        elif kind == 3:
            v[0], v[1] = 3.0e38, -3.0e38
        groups.append(O.f32_to_bf16(v))
    wh = np.stack(groups).reshape(64, 256)
    print("quantize non-finite groups", flush=True)
    wq, s, b = mq4.quantize(to_dev_bf16(wh, dev))
    torch.cuda.synchronize()
    rq, rs, rb = O.quantize(wh)
    assert np.array_equal(to_host_u16(s), rs)
    assert np.array_equal(to_host_u16(b), rb)
    assert np.array_equal(words(wq), rq)


def test_quantize_word_output_only_4_byte_aligned(mq4, O, dev):
    """wq needs only 4-byte alignment (the kernels store 4-byte words): a wq
    4 bytes past an 8-byte boundary gets the oracle's words, single and
    batched, and nothing is written outside it."""
    import ctypes
    N, K = 96, 640
    w, wh = gen_weight(mq4, O, 3100, N, K)
    rq, rs, rb = O.quantize(wh)
    L = mq4.lib()
    store = torch.zeros(N * K // 8 + 2, dtype=torch.int32, device=dev)
    wq = store[1:1 + N * K // 8]                     # 4 bytes past an 8-byte boundary
    assert wq.data_ptr() % 8 == 4
    s = torch.empty((N, K // 64), dtype=torch.bfloat16, device=dev)
    b = torch.empty_like(s)
    print("quantize into a 4-byte-aligned wq", flush=True)
    assert L.mq4_quantize(w.data_ptr(), N, K, 64, 4, wq.data_ptr(), s.data_ptr(), b.data_ptr(), None) == 0
    torch.cuda.synchronize()
    assert np.array_equal(wq.cpu().numpy().view(np.uint32).reshape(N, K // 8), rq)
    assert np.array_equal(to_host_u16(s), rs) and np.array_equal(to_host_u16(b), rb)
    store.zero_()
    jobs = (mq4._QuantJobC * 2)(mq4._QuantJobC(w.data_ptr(), N, K, wq.data_ptr(), s.data_ptr(), b.data_ptr()),
                                mq4._QuantJobC(w.data_ptr(), N, K, wq.data_ptr(), s.data_ptr(), b.data_ptr()))
    assert L.mq4_quantize_batch(ctypes.cast(jobs, ctypes.c_void_p), 1, 64, 4, None) == 0
    torch.cuda.synchronize()
    assert np.array_equal(wq.cpu().numpy().view(np.uint32).reshape(N, K // 8), rq)
    assert int(store[0].item()) == 0 and int(store[-1].item()) == 0      # nothing written outside wq


def test_dequantize_matches_affine_formula(mq4, O, dev):
    N, K = 96, 2048
    w, wh = gen_weight(mq4, O, 9, N, K)
    wq, s, b = mq4.quantize(w)
    d32 = mq4.dequantize(wq, s, b, dtype=torch.float32).cpu().numpy().astype(np.float64)
    d16 = to_host_u16(mq4.dequantize(wq, s, b))
    ref = O.dequantize_f64(*O.quantize(wh))
    assert np.array_equal(d32, ref)              # s*q + b is exact in float for these data
    assert np.array_equal(d16, O.f64_to_bf16(ref))


# --------------------------------------------------------------- GEMV ---

QMM_SHAPES = [
    (1, 6144, 2048), (1, 2048, 6144), (2, 6144, 2048), (3, 100, 2048), (4, 2048, 6144),
    (5, 64, 1024), (8, 33, 4096), (16, 512, 2048), (32, 256, 2048), (1, 7, 64), (1, 1, 64),
    (2, 130, 128), (1, 64, 16384), (1, 32, 20480), (2, 8, 20480), (3, 50, 8256),
]


@pytest.mark.parametrize("M,N,K", QMM_SHAPES)
def test_qmm_matches_fp64_oracle(mq4, O, dev, M, N, K):
    print(f"qmm M={M} N={N} K={K}", flush=True)
    w, wh = gen_weight(mq4, O, 1000 + N % 97, N, K)
    xh = O.gen_normal_bf16(3000 + M, M * K).reshape(M, K)
    qt = mq4.quantize_weight(w)
    xd = to_dev_bf16(xh, dev)
    y = mq4.qmatmul(xd, qt)
    y32 = mq4.quantized_matmul_f32(xd, qt.weight, qt.scales, qt.biases)
    torch.cuda.synchronize()
    ref, _ = O.qmm_f64(xh, *O.quantize(wh))
    check_close(O, to_host_u16(y), ref, f"qmm {M}x{N}x{K}", y32.cpu().numpy())
    # the bf16 output is the fp32 result rounded once
    assert np.array_equal(to_host_u16(y), O.f32_to_bf16(y32.cpu().numpy()))


def test_qmm_batched_leading_dims(mq4, O, dev):
    """x of shape [1, S, K] like the reference's [1, M, K] activations."""
    S, N, K = 6, 300, 2048
    w, wh = gen_weight(mq4, O, 1234, N, K)
    xh = O.gen_normal_bf16(4000, S * K).reshape(S, K)
    qt = mq4.quantize_weight(w)
    y = mq4.qmatmul(to_dev_bf16(xh, dev).view(1, S, K), qt)
    assert y.shape == (1, S, N)
    ref, _ = O.qmm_f64(xh, *O.quantize(wh))
    check_close(O, to_host_u16(y).reshape(S, N), ref, "qmm [1,S,K]")


def test_empty_batches(mq4, O, dev):
    """Zero activation rows give empty results of the right shapes (as
    mx::quantized_matmul, argmax and rms_norm do on empty inputs) without
    reaching the C ABI, which rejects M = 0."""
    N, K, I = 256, 512, 1024
    w, _ = gen_weight(mq4, O, 1234, N, K)
    g, _ = gen_weight(mq4, O, 1235, I, K)
    u, _ = gen_weight(mq4, O, 1236, I, K)
    d, _ = gen_weight(mq4, O, 1237, K, I)
    qw, qg, qu, qd = (mq4.quantize_weight(t) for t in (w, g, u, d))
    nw = torch.zeros(K, dtype=torch.bfloat16, device=dev)
    for lead in ((0,), (1, 0)):
        x = torch.empty((*lead, K), dtype=torch.bfloat16, device=dev)
        assert mq4.qmatmul(x, qw).shape == (*lead, N)
        assert mq4.quantized_matmul_f32(x, qw.weight, qw.scales, qw.biases).shape == (*lead, N)
        assert mq4.mlp_gate_up_silu(x, qg, qu).shape == (*lead, I)
        assert mq4.mlp_gate_up_silu(x, qg, qu, norm_weight=nw).shape == (*lead, I)
        h = torch.empty((*lead, I), dtype=torch.bfloat16, device=dev)
        assert mq4.qmatmul_residual(h, qd, x).shape == (*lead, K)
        assert mq4.mlp_residual(x, mq4.MLPWeights(qg, qu, qd), nw).shape == (*lead, K)
        assert mq4.rms_norm(x, nw).shape == (*lead, K)
        idx, logits = mq4.lm_head_argmax(x, qw, return_logits=True)
        assert idx.shape == lead and logits.shape == (*lead, N)
        assert mq4.argmax(torch.empty((*lead, N), dtype=torch.bfloat16, device=dev)).shape == lead
    torch.cuda.synchronize()


def check_swiglu(O, got, ref, what):
    """h is bf16(bf16(bf16(sigmoid(g))*g)*u) of bf16-rounded GEMV outputs g, u.
    A 1-ulp difference in the rounding of g or u (when the fp32 sum sits next
    to a bf16 rounding boundary) can flip bf16(sigmoid(g)) by a whole ulp and
    so move h by several ulps (g = 0.2598 vs 0.2578 gives h = -0.1123 vs
    -0.1099, 5 ulps).  h is therefore checked element-wise: at least 99%
    bit-identical, the rest within 8 bf16 ulps or 2^-8 * rms(h) absolute.
    The 1e-2 RMS bar applies to the GEMV outputs g, u and to the MLP output."""
    d = O.bf16_ulp_diff(got, ref)
    rf = O.bf16_to_f32(ref).astype(np.float64)
    rms = float(np.sqrt(np.mean(rf * rf)))
    abs_err = np.abs(O.bf16_to_f32(got).astype(np.float64) - rf)
    print(f"{what}: identical={np.mean(d == 0):.5f} max_ulp={int(d.max())} "
          f"max|err|/rms={O.rel_rms_err(got, rf):.2e}")
    assert np.mean(d == 0) >= 0.99
    assert np.all((d <= 8) | (abs_err <= 2.0 ** -8 * rms))


@pytest.mark.parametrize("M", [1, 2, 4, 5])
def test_mlp_gate_up_silu(mq4, O, dev, M):
    N, K = 6144, 2048
    wg, wgh = gen_weight(mq4, O, 1000, N, K)
    wu, wuh = gen_weight(mq4, O, 1001, N, K)
    xh = O.gen_normal_bf16(3000, M * K).reshape(M, K)
    qg, qu = mq4.quantize_weight(wg), mq4.quantize_weight(wu)
    h = mq4.mlp_gate_up_silu(to_dev_bf16(xh, dev), qg, qu)
    torch.cuda.synchronize()
    g64, gb = O.qmm_f64(xh, *O.quantize(wgh))
    u64, ub = O.qmm_f64(xh, *O.quantize(wuh))
    check_swiglu(O, to_host_u16(h), O.swiglu_bf16(gb, ub), f"gate_up_silu M={M}")
    # the unfused ops of this library: g and u meet the GEMV bar, and swiglu
    # applied to them matches the oracle's swiglu on the same bf16 inputs
    g = mq4.qmatmul(to_dev_bf16(xh, dev), qg)
    u = mq4.qmatmul(to_dev_bf16(xh, dev), qu)
    xd = to_dev_bf16(xh, dev)
    check_close(O, to_host_u16(g), g64, "gate",
                mq4.quantized_matmul_f32(xd, qg.weight, qg.scales, qg.biases).cpu().numpy())
    check_close(O, to_host_u16(u), u64, "up",
                mq4.quantized_matmul_f32(xd, qu.weight, qu.scales, qu.biases).cpu().numpy())
    h2 = mq4.swiglu(g, u)
    # the device expf and libm's may differ in the last float ulp, which can
    # flip a bf16 rounding of sigmoid for a few elements
    d2 = O.bf16_ulp_diff(to_host_u16(h2), O.swiglu_bf16(to_host_u16(g), to_host_u16(u)))
    assert d2.max() <= 2 and np.mean(d2 > 0) < 1e-3
    check_swiglu(O, to_host_u16(h), to_host_u16(h2), "fused vs unfused")


@pytest.mark.parametrize("M", [1, 3])
def test_qmm_residual_in_place(mq4, O, dev, M):
    N, K = 2048, 6144
    w, wh = gen_weight(mq4, O, 1002, N, K)
    hh = O.gen_normal_bf16(3100, M * K, 0.0, 0.3).reshape(M, K)
    rh = O.gen_normal_bf16(3200, M * N).reshape(M, N)
    qt = mq4.quantize_weight(w)
    r = to_dev_bf16(rh, dev)
    out = mq4.qmatmul_residual(to_dev_bf16(hh, dev), qt, r, out=r)   # in place
    torch.cuda.synchronize()
    assert out.data_ptr() == r.data_ptr()
    y64, yb = O.qmm_f64(hh, *O.quantize(wh))
    ref = O.add_bf16(rh, yb)
    got = to_host_u16(r)
    # absolute bar: a residual sum that cancels to near zero turns the
    # product's 1-2 ulp rounding difference into many ulps of the sum
    err = np.abs(O.bf16_to_f32(got).astype(np.float64) - O.bf16_to_f32(ref))
    rms = float(np.sqrt(np.mean(y64 * y64)))
    assert np.all(err <= 2.0 ** -7 * (np.abs(O.bf16_to_f32(yb)) + np.abs(O.bf16_to_f32(ref))) + 2.0 ** -12 * rms)
    assert O.rel_rms_err(got, O.bf16_to_f32(ref).astype(np.float64)) <= TOL


@pytest.mark.parametrize("M,K", [(1, 2048), (3, 2048), (1, 6144), (2, 128)])
def test_rmsnorm_gate_up_silu(mq4, O, dev, M, K):
    """rms_norm(x) (src/model/marlin.cpp:12-16, 141) fused in front of gate/up:
    h against the oracle's rms_norm -> bf16(fp64 g), bf16(fp64 u) -> swiglu."""
    N = 1536
    wg, wgh = gen_weight(mq4, O, 1010, N, K)
    wu, wuh = gen_weight(mq4, O, 1011, N, K)
    xh = O.gen_normal_bf16(3000, M * K, 0.0, 1.5).reshape(M, K)
    nwh = O.gen_normal_bf16(2100, K, 0.1, 0.02)
    qg, qu = mq4.quantize_weight(wg), mq4.quantize_weight(wu)
    h = mq4.mlp_gate_up_silu(to_dev_bf16(xh, dev), qg, qu, norm_weight=to_dev_bf16(nwh, dev), eps=1e-6)
    torch.cuda.synchronize()
    n = O.rmsnorm_1pw(xh, nwh, 1e-6)
    _, gb = O.qmm_f64(n, *O.quantize(wgh))
    _, ub = O.qmm_f64(n, *O.quantize(wuh))
    check_swiglu(O, to_host_u16(h), O.swiglu_bf16(gb, ub), f"norm+gate_up M={M} K={K}")
    # the fused norm equals the standalone rms_norm kernel followed by the unfused op
    n_dev = mq4.rms_norm(to_dev_bf16(xh, dev), to_dev_bf16(nwh, dev), 1e-6)
    dn = O.bf16_ulp_diff(to_host_u16(n_dev), n)
    assert dn.max() <= 1 and np.mean(dn > 0) < 1e-3
    h2 = mq4.mlp_gate_up_silu(n_dev, qg, qu)
    check_swiglu(O, to_host_u16(h), to_host_u16(h2), "fused norm vs rms_norm kernel")


@pytest.mark.parametrize("M", [1, 4])
def test_rmsnorm_lm_head_argmax(mq4, O, dev, lm_head, M):
    qt, (rq, rs, rb) = lm_head
    xh = O.gen_normal_bf16(3300, M * 2048, 0.0, 3.0).reshape(M, 2048)
    nwh = O.gen_normal_bf16(2001, 2048, 0.1, 0.02)
    idx, logits = mq4.lm_head_argmax(to_dev_bf16(xh, dev), qt, return_logits=True,
                                     norm_weight=to_dev_bf16(nwh, dev), eps=1e-6)
    torch.cuda.synchronize()
    hn = O.rmsnorm_1pw(xh, nwh, 1e-6)
    ref64, refb = O.qmm_f64(hn, rq, rs, rb)
    lg = to_host_u16(logits)
    ulp = O.bf16_ulp_diff(lg, refb)
    print(f"norm+lm_head M={M}: identical={np.mean(ulp == 0):.5f} max_ulp={int(ulp.max())}")
    assert np.mean(ulp == 0) >= 0.98
    assert np.array_equal(idx.cpu().numpy().astype(np.uint32), O.argmax_bf16(lg))


def test_lm_head_workspace_reuse(mq4, O, dev):
    """One workspace serves many calls (different shapes and M) in a row."""
    L = mq4.lib()
    import ctypes
    V, K = 50000, 2048
    w, wh = gen_weight(mq4, O, 2000, V, K)
    qt = mq4.quantize_weight(w)
    ws_bytes = L.mq4_lm_head_argmax_workspace_size(5, V)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    P = ctypes.c_void_p
    for M, Nuse in ((1, V), (5, V), (2, 777), (1, 64), (3, V)):
        hh = O.gen_normal_bf16(3400 + M, M * K).reshape(M, K)
        hd = to_dev_bf16(hh, dev)
        idx = torch.zeros(M, dtype=torch.int32, device=dev)
        logits = torch.empty((M, Nuse), dtype=torch.bfloat16, device=dev)
        rc = L.mq4_lm_head_argmax(P(hd.data_ptr()), M, K, P(qt.weight.data_ptr()), P(qt.scales.data_ptr()),
                                  P(qt.biases.data_ptr()), Nuse, P(idx.data_ptr()), P(logits.data_ptr()),
                                  P(ws.data_ptr()), ws_bytes, P(torch.cuda.current_stream().cuda_stream))
        assert rc == 0
        torch.cuda.synchronize()
        assert np.array_equal(idx.cpu().numpy().astype(np.uint32), O.argmax_bf16(to_host_u16(logits)))


def test_mlp_chain_two_layers(mq4, O, dev):
    """hidden = hidden + mlp(hidden) for two layers (src/model/marlin.cpp:142),
    M=1, each step pinned on the GPU's own input to that step:
      h_l = swiglu(gate x_l, up x_l)   element-wise bar (check_swiglu)
      y_l = down h_l                   GEMV bar: 1e-2 * rms(y_l) vs fp64
      x_{l+1} = bf16(x_l + y_l)        bit-exact (same fp32 sum as y_l)
    The end-to-end stream is then compared with the oracle's own chain.  The
    bf16 residual stream amplifies ulp-level differences: a 1-ulp change of y
    flips the rounding of x + y for some elements, whose 1-ulp change (0.4% of
    the value) in turn flips roundings of the next layer's g and u.  Two
    correct implementations therefore agree only statistically after a few
    layers; the end-to-end bar is rms(got - ref) <= 1e-2 * rms(ref)."""
    N, K = 6144, 2048
    layers_d, layers_h = [], []
    for l in range(2):
        ws = [gen_weight(mq4, O, mq4.stream_id_layer(l, p), *((N, K) if p < 2 else (K, N))) for p in range(3)]
        layers_d.append(mq4.MLPWeights(*[mq4.quantize_weight(w) for w, _ in ws]))
        layers_h.append([O.quantize(h) for _, h in ws])
    xh = O.gen_normal_bf16(3000, K).reshape(1, K)
    x = to_dev_bf16(xh, dev)
    for lw, (g, u, d) in zip(layers_d, layers_h):
        xin = to_host_u16(x)
        h = mq4.mlp_gate_up_silu(x, lw.gate_proj, lw.up_proj)
        y = mq4.qmatmul(h, lw.down_proj)
        xn = mq4.mlp_forward(x, lw, residual=x)
        torch.cuda.synchronize()
        _, gb = O.qmm_f64(xin, *g)
        _, ub = O.qmm_f64(xin, *u)
        check_swiglu(O, to_host_u16(h), O.swiglu_bf16(gb, ub), "chain h")
        y64, _ = O.qmm_f64(to_host_u16(h), *d)
        y32 = mq4.quantized_matmul_f32(h, lw.down_proj.weight, lw.down_proj.scales, lw.down_proj.biases)
        check_close(O, to_host_u16(y), y64, "chain down", y32.cpu().numpy())
        assert np.array_equal(to_host_u16(xn), O.add_bf16(xin, to_host_u16(y)))
        x = xn
    ref = xh
    for g, u, d in layers_h:
        _, _, _, yb = O.mlp_forward(ref, g, u, d)
        ref = O.add_bf16(ref, yb)
    got = to_host_u16(x)
    rf = O.bf16_to_f32(ref).astype(np.float64)
    rms = float(np.sqrt(np.mean(rf * rf)))
    dd = O.bf16_ulp_diff(got, ref)
    ae = np.abs(O.bf16_to_f32(got).astype(np.float64) - rf)
    rel_rms = float(np.sqrt(np.mean(ae * ae))) / rms
    print(f"chain end: identical={np.mean(dd == 0):.5f} max_ulp={int(dd.max())} "
          f"max|err|/rms={O.rel_rms_err(got, rf):.2e} rms(err)/rms={rel_rms:.2e}")
    assert rel_rms <= TOL


# ------------------------------------------------------ lm_head/argmax ---

@pytest.fixture(scope="module")
def lm_head(mq4, O, dev):
    V, K = 248320, 2048
    w, wh = gen_weight(mq4, O, mq4.STREAM_LM_HEAD, V, K)
    qt = mq4.quantize_weight(w)
    torch.cuda.synchronize()
    return qt, O.quantize(wh)


def normed_hidden(O, M, K=2048):
    x = O.gen_normal_bf16(3000, M * K).reshape(M, K)
    nw = O.gen_normal_bf16(2001, K, 0.1, 0.02)
    return O.rmsnorm_1pw(x, nw)


@pytest.mark.parametrize("M", [1, 4])
def test_lm_head_argmax_full_vocab(mq4, O, dev, lm_head, M):
    qt, (rq, rs, rb) = lm_head
    hh = normed_hidden(O, M)
    idx, logits = mq4.lm_head_argmax(to_dev_bf16(hh, dev), qt, return_logits=True)
    torch.cuda.synchronize()
    lg = to_host_u16(logits)
    ref64, refb = O.qmm_f64(hh, rq, rs, rb)
    check_close(O, lg, ref64, "lm_head logits")
    got = idx.cpu().numpy().astype(np.uint32)
    # argmax semantics are bit-exact on the kernel's own logits
    assert np.array_equal(got, O.argmax_bf16(lg))
    # and equal to the argmax of bf16(fp64) logits unless that row's top two
    # bf16 values are within one ulp (a near-tie the rounding may flip)
    ref_idx = O.argmax_bf16(refb)
    for m in range(M):
        if got[m] != ref_idx[m]:
            top = np.sort(O.bf16_to_f32(refb[m]))[-2:]
            assert O.bf16_ulp_diff(O.f32_to_bf16(top[:1]), O.f32_to_bf16(top[1:]))[0] <= 1
    # the fused path equals the unfused lm_head + argmax
    idx2 = mq4.argmax(logits)
    assert np.array_equal(idx2.cpu().numpy(), idx.cpu().numpy())


def test_lm_head_argmax_planted_tie(mq4, O, dev):
    """Duplicate the winning row at an earlier and at a later index: the
    lowest index must win (mx::argmax first-occurrence rule)."""
    V, K = 40000, 2048
    w, wh = gen_weight(mq4, O, 2000, V, K)
    hh = normed_hidden(O, 1)
    qt = mq4.quantize_weight(w)
    i0 = int(mq4.lm_head_argmax(to_dev_bf16(hh, dev), qt).cpu()[0])
    for dst in (17, V - 3):
        if dst == i0:
            continue
        wh2 = wh.copy()
        wh2[dst] = wh[i0]        # identical rows give bit-identical logits
        idx = mq4.lm_head_argmax(to_dev_bf16(hh, dev), mq4.quantize_weight(to_dev_bf16(wh2, dev)))
        assert int(idx.cpu()[0]) == min(dst, i0)


def test_argmax_special_values(mq4, O, dev):
    rng = np.random.default_rng(9)
    M, N = 5, 300000
    v = rng.standard_normal((M, N)).astype(np.float32)
    v[0, [5, 200000]] = 40.0
    v[1, :] = -3.0
    v[2, 123456] = 1e30
    bits = O.f32_to_bf16(v)
    bits[3, :] = 0x8000
    bits[3, 77] = 0x0000          # +0 vs -0: equal, so index 0 wins
    bits[4, 10] = 0x7fc0          # NaN never wins
    bits[4, 11] = O.f32_to_bf16(np.array([100.0], np.float32))[0]
    idx = mq4.argmax(to_dev_bf16(bits, dev))
    got = idx.cpu().numpy().astype(np.uint32)
    assert np.array_equal(got, O.argmax_bf16(bits))
    assert list(got) == [5, 0, 123456, 0, 11]


def test_sample_token_greedy_last_row(mq4, O, dev):
    S, V = 3, 1000
    bits = O.gen_normal_bf16(42, S * V).reshape(1, S, V)
    tok = mq4.sample_token(to_dev_bf16(bits, dev), temperature=0.0)
    assert int(tok.cpu().reshape(-1)[0]) == int(O.argmax_bf16(bits[0, -1])[0])
