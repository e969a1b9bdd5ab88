"""Batched decode (M concurrent token rows, bench config 5a) on the model's
shapes through the C ABI, against the oracle on the same seeded inputs:

* fused gate/up + SwiGLU (6144x2048), with and without the (1 + w) RMSNorm
  in front (src/model/marlin.cpp:27-33, 141): element-wise SwiGLU bar of
  check_swiglu against the oracle's bf16 op chain on bf16(fp64) g and u;
* down + residual (2048x6144, src/model/marlin.cpp:34, 142): the fp32 product
  within 1e-2 x rms of fp64 (the GEMV bar); the residual output equal to
  bf16(residual + the kernel's own bf16 product) bit for bit, and within
  2^-7 (|bf16(fp64)| + |ref|) + 2^-12 rms of ref = bf16(residual + bf16(fp64));
* lm_head + greedy argmax over the full 248,320-row vocab
  (src/model/marlin.cpp:161-169, src/sampling/sampler.cpp:14-16): logits
  >= 98% identical to bf16(fp64), indices bit-exact on the kernel's own
  logits and equal to the fp64 argmax unless the top two are within 1 ulp;
* edge shapes (test_batched_edge_shapes): odd M on either side of the
  16-row tile, ragged N, K of 1024 to 6144, every epilogue, and a store
  with more tiles than resident workgroups.
"""
import numpy as np
import pytest
import torch

from conftest import to_dev_bf16, to_host_u16
from test_gpu_parity import TOL, check_close, check_swiglu, rel_err_f32

pytestmark = pytest.mark.gpu

H, I, V = 2048, 6144, 248320
MS = [16, 32]


def q_host(qt):
    return qt.weight.cpu().numpy().view(np.uint32), to_host_u16(qt.scales), to_host_u16(qt.biases)


@pytest.fixture(scope="module")
def mlp(mq4, dev):
    ws = [mq4.quantize_weight(mq4.fill_normal_bf16((I, H) if p < 2 else (H, I), mq4.stream_id_layer(0, p),
                                                   0.0, 0.02, device=dev)) for p in range(3)]
    torch.cuda.synchronize()
    return ws, [q_host(w) for w in ws]


@pytest.mark.parametrize("M", MS)
@pytest.mark.parametrize("norm", [False, True])
def test_batched_gate_up_silu(mq4, O, dev, mlp, M, norm):
    print(f"batched gate/up M={M} norm={norm}", flush=True)
    (g, u, _), (gh, uh, _) = mlp
    xh = O.gen_normal_bf16(3000, M * H, 0.0, 1.5).reshape(M, H)
    nwh = O.gen_normal_bf16(2100, H, 0.1, 0.02)
    x = to_dev_bf16(xh, dev)
    h = mq4.mlp_gate_up_silu(x, g, u, norm_weight=to_dev_bf16(nwh, dev) if norm else None, eps=1e-6)
    torch.cuda.synchronize()
    n = O.rmsnorm_1pw(xh, nwh, 1e-6) if norm else xh
    _, gb = O.qmm_f64(n, *gh)
    _, ub = O.qmm_f64(n, *uh)
    check_swiglu(O, to_host_u16(h), O.swiglu_bf16(gb, ub), f"gate/up M={M} norm={norm}")


@pytest.mark.parametrize("M", MS)
def test_batched_down_residual(mq4, O, dev, mlp, M):
    print(f"batched down M={M}", flush=True)
    (_, _, d), (_, _, dh) = mlp
    hh = O.gen_normal_bf16(3100, M * I, 0.0, 0.3).reshape(M, I)
    rh = O.gen_normal_bf16(3200, M * H).reshape(M, H)
    hd = to_dev_bf16(hh, dev)
    y = mq4.qmatmul_residual(hd, d, to_dev_bf16(rh, dev))
    y32 = mq4.quantized_matmul_f32(hd, d.weight, d.scales, d.biases)
    yq = mq4.qmatmul(hd, d)
    torch.cuda.synchronize()
    y64, yb = O.qmm_f64(hh, *dh)
    check_close(O, to_host_u16(yq), y64, f"down M={M}", y32.cpu().numpy())
    # the residual epilogue adds the bf16-rounded product of the same kernel family
    want = O.add_bf16(rh, to_host_u16(yq))
    assert np.array_equal(to_host_u16(y), want)
    # against the oracle: the product's error (<= 2 ulps of bf16(fp64), see
    # check_close) plus the sum's own rounding, in absolute terms (a sum that
    # cancels to near zero makes an ulp count meaningless)
    ref = O.add_bf16(rh, yb)
    err = np.abs(O.bf16_to_f32(to_host_u16(y)).astype(np.float64) - O.bf16_to_f32(ref))
    rms = float(np.sqrt(np.mean(y64 * y64)))
    # |yq - yb| <= 2^-7 |yb| + fp32 noise; the two sums round apart by <= 1 ulp
    allow = 2.0 ** -7 * np.abs(O.bf16_to_f32(yb)) + 2.0 ** -7 * np.abs(O.bf16_to_f32(ref)) + 2.0 ** -12 * rms
    worst = np.unravel_index(np.argmax(err - allow), err.shape)
    assert np.all(err <= allow), (f"at {worst}: y={O.bf16_to_f32(to_host_u16(y))[worst]} ref={O.bf16_to_f32(ref)[worst]} "
                                  f"yq={O.bf16_to_f32(to_host_u16(yq))[worst]} yb={O.bf16_to_f32(yb)[worst]}")


@pytest.fixture(scope="module")
def lm(mq4, dev):
    qt = mq4.quantize_weight(mq4.fill_normal_bf16((V, H), mq4.STREAM_LM_HEAD, 0.0, 0.02, device=dev))
    torch.cuda.synchronize()
    return qt, q_host(qt)


@pytest.mark.parametrize("M", MS)
def test_batched_lm_head_argmax(mq4, O, dev, lm, M):
    print(f"batched lm_head M={M}", flush=True)
    qt, qh = lm
    xh = O.gen_normal_bf16(3300, M * H, 0.0, 3.0).reshape(M, H)
    nwh = O.gen_normal_bf16(2001, H, 0.1, 0.02)
    idx, logits = mq4.lm_head_argmax(to_dev_bf16(xh, dev), qt, return_logits=True,
                                     norm_weight=to_dev_bf16(nwh, dev), eps=1e-6)
    torch.cuda.synchronize()
    hn = O.rmsnorm_1pw(xh, nwh, 1e-6)
    ref64, refb = O.qmm_f64(hn, *qh)
    lg = to_host_u16(logits)
    ulp = O.bf16_ulp_diff(lg, refb)
    print(f"lm_head M={M}: identical={np.mean(ulp == 0):.5f} max_ulp={int(ulp.max())}")
    assert np.mean(ulp == 0) >= 0.98
    rms = float(np.sqrt(np.mean(ref64 * ref64)))
    assert np.max(np.abs(O.bf16_to_f32(lg).astype(np.float64) - ref64)) <= TOL * rms + np.abs(ref64).max() * 2.0 ** -8
    got = idx.cpu().numpy().astype(np.uint32)
    assert np.array_equal(got, O.argmax_bf16(lg))
    want = O.argmax_bf16(refb)
    for m in range(M):
        if got[m] != want[m]:
            top = np.sort(O.bf16_to_f32(refb[m]))[-2:]
            assert O.bf16_ulp_diff(O.f32_to_bf16(top[:1]), O.f32_to_bf16(top[1:]))[0] <= 1, f"row {m}"


@pytest.mark.parametrize("M", MS)
def test_batched_qmm_f32_bar(mq4, O, dev, mlp, M):
    """The unrounded fp32 product of gate (6144x2048) at batched M against fp64."""
    (g, _, _), (gh, _, _) = mlp
    xh = O.gen_normal_bf16(3400, M * H).reshape(M, H)
    y32 = mq4.quantized_matmul_f32(to_dev_bf16(xh, dev), g.weight, g.scales, g.biases)
    torch.cuda.synchronize()
    ref, _ = O.qmm_f64(xh, *gh)
    err = rel_err_f32(y32.cpu().numpy(), ref)
    print(f"gate fp32 M={M}: max|err|/rms = {err:.2e}")
    assert err <= 1e-4


# (M, N, K, what): odd M on either side of the 16-row tile, ragged N, K beyond
# the model's 2048 (other wave layouts, activations re-read per group at
# M > 16 and K > 2048), and a store with more 16-row tiles (750) than
# resident workgroups, so that workgroups loop over rounds with the next
# round's weights in flight.
EDGE = [(5, 200, 1024, "store"), (9, 1000, 2048, "f32"), (17, 520, 4096, "residual"),
        (31, 12000, 1024, "store"), (12, 6144, 1024, "swiglu"), (23, 1000, 2048, "argmax"),
        (7, 3000, 2048, "norm_swiglu"), (20, 256, 6144, "f32"), (29, 1000, 2048, "norm_swiglu")]


@pytest.mark.parametrize("case", EDGE, ids=lambda c: "-".join(map(str, c)))
def test_batched_edge_shapes(mq4, O, dev, case):
    M, N, K, what = case
    print(f"batched edge M={M} N={N} K={K} {what}", flush=True)
    sid = 5000 + EDGE.index(case)
    w = mq4.quantize_weight(mq4.fill_normal_bf16((N, K), sid, 0.0, 0.02, device=dev))
    wh = q_host(w)
    xh = O.gen_normal_bf16(sid + 100, M * K, 0.0, 1.0).reshape(M, K)
    x = to_dev_bf16(xh, dev)
    if what in ("store", "f32"):
        y = mq4.qmatmul(x, w)
        y32 = mq4.quantized_matmul_f32(x, w.weight, w.scales, w.biases)
        torch.cuda.synchronize()
        y64, _ = O.qmm_f64(xh, *wh)
        check_close(O, to_host_u16(y), y64, f"edge {case}", y32.cpu().numpy())
        assert rel_err_f32(y32.cpu().numpy(), y64) <= 1e-4
    elif what == "residual":
        rh = O.gen_normal_bf16(sid + 200, M * N).reshape(M, N)
        y = mq4.qmatmul_residual(x, w, to_dev_bf16(rh, dev))
        yq = mq4.qmatmul(x, w)
        torch.cuda.synchronize()
        assert np.array_equal(to_host_u16(y), O.add_bf16(rh, to_host_u16(yq)))
        y64, _ = O.qmm_f64(xh, *wh)
        check_close(O, to_host_u16(yq), y64, f"edge {case}")
    elif what in ("swiglu", "norm_swiglu"):
        u = mq4.quantize_weight(mq4.fill_normal_bf16((N, K), sid + 300, 0.0, 0.02, device=dev))
        uh = q_host(u)
        nwh = O.gen_normal_bf16(sid + 400, K, 0.1, 0.02)
        norm = what == "norm_swiglu"
        h = mq4.mlp_gate_up_silu(x, w, u, norm_weight=to_dev_bf16(nwh, dev) if norm else None, eps=1e-6)
        torch.cuda.synchronize()
        n = O.rmsnorm_1pw(xh, nwh, 1e-6) if norm else xh
        _, gb = O.qmm_f64(n, *wh)
        _, ub = O.qmm_f64(n, *uh)
        check_swiglu(O, to_host_u16(h), O.swiglu_bf16(gb, ub), f"edge {case}")
    else:
        idx, logits = mq4.lm_head_argmax(x, w, return_logits=True)
        torch.cuda.synchronize()
        lg = to_host_u16(logits)
        got = idx.cpu().numpy().astype(np.uint32)
        assert np.array_equal(got, O.argmax_bf16(lg))
        y64, yb = O.qmm_f64(xh, *wh)
        check_close(O, lg, y64, f"edge {case}")


@pytest.mark.parametrize("M,N", [(1, V), (2, V), (1, 17), (2, 4097), (1, 4097), (1, 26384), (2, 21383),
                                 (5, V), (16, V), (17, V), (32, V), (16, 1000), (20, 4097), (8, 17)])
def test_lm_head_ring_equals_mfma_gemv(mq4, O, dev, lm, M, N):
    """From 5 rows at K = 2048 the lm_head + argmax runs as the weight-ring
    kernel (mq4_lmring.hip): the MFMA GEMV's arithmetic (8 waves x 4 groups,
    wave partials in wave order), so its logits equal, bit for bit, the MFMA
    GEMV's plain product (qmatmul, the same K split and order); 1-2 rows run
    the dot2 GEMV, whose plain product is the same kernel with another
    epilogue.  The tokens are the argmax of those logits.  Ragged N: fewer
    tiles than workgroups (1000 and 17 rows) and a last tile of one row
    (4097); for 1-2 rows, whose rows past the full rounds of 4-row batches
    go out as short batches of up to ceil(rest / waves) rows, rests of one
    row per wave (248320), two (4097, 21383: the last wave's batch cut to
    one row) and three (26384)."""
    print(f"lm_head ring vs MFMA GEMV: M={M} N={N}", flush=True)
    qt = lm[0] if N == V else mq4.quantize_weight(
        mq4.fill_normal_bf16((N, H), 7100 + N, 0.0, 0.02, device=dev))
    x = mq4.fill_normal_bf16((M, H), 3400 + M, 0.0, 2.0, device=dev)
    idx, logits = mq4.lm_head_argmax(x, qt, return_logits=True)
    ref = mq4.qmatmul(x, qt)
    idx2 = mq4.lm_head_argmax(x, qt)                   # without the logits store
    torch.cuda.synchronize()
    lg = to_host_u16(logits)
    assert np.array_equal(lg, to_host_u16(ref)), "logits differ from the MFMA GEMV product"
    got = idx.cpu().numpy().astype(np.uint32)
    assert np.array_equal(got, O.argmax_bf16(lg))
    assert np.array_equal(idx2.cpu().numpy().astype(np.uint32), got)


@pytest.mark.parametrize("M", [3, 4])
def test_lm_head_ring_small_m_rows_independent(mq4, O, dev, lm, M):
    """From 3 rows the lm_head + argmax takes the weight-ring kernel, whose
    rows are independent (16-row MFMA tiles, rows past M repeat the last
    one): the logits of M rows equal the first M rows of a 5-row call bit for
    bit (5 rows: pinned to the MFMA GEMV above), and against the oracle they
    meet the lm_head bars."""
    print(f"lm_head ring rows: M={M}", flush=True)
    qt, qh = lm
    x5 = mq4.fill_normal_bf16((5, H), 3500, 0.0, 2.0, device=dev)
    nw = mq4.fill_normal_bf16((H,), 2002, 0.1, 0.02, device=dev)
    idx, lg = mq4.lm_head_argmax(x5[:M].contiguous(), qt, return_logits=True, norm_weight=nw, eps=1e-6)
    idx5, lg5 = mq4.lm_head_argmax(x5, qt, return_logits=True, norm_weight=nw, eps=1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(to_host_u16(lg), to_host_u16(lg5)[:M])
    assert np.array_equal(idx.cpu().numpy(), idx5.cpu().numpy()[:M])
    hn = O.rmsnorm_1pw(to_host_u16(x5[:M]), to_host_u16(nw), 1e-6)
    ref64, refb = O.qmm_f64(hn, *qh)
    ulp = O.bf16_ulp_diff(to_host_u16(lg), refb)
    assert np.mean(ulp == 0) >= 0.98
