"""Large-M Q4 GEMM (bf16 MFMA, weights dequantized into LDS) through the C ABI.

From M = 33 rows on, mq4_qmm / mq4_qmm_f32 / mq4_qmm_residual /
mq4_mlp_gate_up_silu run the MFMA GEMM (prefill: the prompt's S tokens through
qmatmul, src/model/marlin.cpp:18-25, and mlp_forward, :31-35).  Bars, against
the oracle's fp64 product of the same bf16 inputs and Q4 weights:
* fp32 output: max|err| <= 1e-2 x rms(ref), the bar against MLX, and the
  GEMM's own accuracy bar GEMM_TOL_F32 = 1e-4 x rms (measured ~1e-5), which
  a single-bf16 weight (~2^-9 relative, ~1e-2 of rms at the maximum over a
  prefill's outputs) would fail;
* bf16 output: the fp32 bar plus the output's own rounding, half a bf16 ulp
  of |ref|, and >= 98% bit-identical to bf16(ref);
* fused SwiGLU: the GEMV's element-wise bar (check_swiglu): >= 99%
  bit-identical to the oracle's bf16 op chain on the fp64 gate/up, the rest
  within 8 bf16 ulps or 2^-8 rms (one ulp flip of g can move h by ~5 ulps
  through bf16(sigmoid(g)));
* residual: bf16(res + bf16(acc)) equals the same formula on the GEMM's own
  fp32 product bit for bit.
At the prefill sizes (M = 1960 / 2048 / 8192) the oracle checks a spread of
rows; the others are covered by the row-independent kernel (every row runs
the same code on its own data) and by the small ragged shapes.
"""
import ctypes

import numpy as np
import pytest
import torch

from conftest import to_dev_bf16, to_host_u16
from test_gpu_parity import check_swiglu

pytestmark = pytest.mark.gpu

TOL = 1e-2
GEMM_TOL_F32 = 1e-4


def q_host(wq, s, b):
    return wq.cpu().numpy().view(np.uint32), to_host_u16(s), to_host_u16(b)


def make(mq4, O, N, K, sid, dev):
    w = mq4.fill_normal_bf16((N, K), sid, 0.0, 0.02, device=dev)
    wq, s, b = mq4.quantize(w)
    return (wq, s, b), q_host(wq, s, b)


def check_f32(got, ref64, what, tol=GEMM_TOL_F32):
    ref64 = np.asarray(ref64, np.float64)
    rms = float(np.sqrt(np.mean(ref64 * ref64)))
    err = float(np.max(np.abs(np.asarray(got, np.float64) - ref64))) / rms
    print(f"{what}: fp32 max|err|/rms = {err:.2e}")
    assert err <= min(tol, TOL), f"{what}: {err:.3e}"


def check_bf16(O, got_bits, ref64, what):
    ref64 = np.asarray(ref64, np.float64)
    rms = float(np.sqrt(np.mean(ref64 * ref64)))
    got = O.bf16_to_f32(got_bits).astype(np.float64)
    allow = TOL * rms + np.abs(ref64) * 2.0 ** -9
    bad = np.abs(got - ref64) > allow
    same = float(np.mean(got_bits == O.f64_to_bf16(ref64)))
    print(f"{what}: bf16 max|err|/rms = {float(np.max(np.abs(got - ref64))) / rms:.2e}, "
          f"identical to bf16(ref) {same:.4f}")
    assert not bad.any(), f"{what}: {int(bad.sum())} outputs beyond the bar"
    assert same >= 0.98


@pytest.mark.parametrize("M,N,K", [(33, 128, 64), (64, 256, 512), (130, 200, 2048), (257, 384, 1024),
                                   (96, 6144, 2048), (40, 2048, 6144)])
def test_gemm_qmm_small_against_fp64(mq4, O, dev, M, N, K):
    print(f"gemm M={M} N={N} K={K}", flush=True)
    (wq, s, b), qh = make(mq4, O, N, K, 1000 + N + K, dev)
    xh = O.gen_normal_bf16(4000, M * K).reshape(M, K)
    x = to_dev_bf16(xh, dev)
    y32 = mq4.quantized_matmul_f32(x, wq, s, b)
    y = mq4.quantized_matmul(x, wq, s, b)
    torch.cuda.synchronize()
    ref64, _ = O.qmm_f64(xh, *qh)
    check_f32(y32.cpu().numpy(), ref64, f"M={M} N={N} K={K}")
    check_bf16(O, to_host_u16(y), ref64, f"M={M} N={N} K={K}")


@pytest.mark.parametrize("M", [1960, 2048, 8192])
def test_gemm_prefill_shapes_sampled_rows(mq4, O, dev, M):
    """Prefill shapes: M tokens through gate (6144x2048) and down (2048x6144)."""
    print(f"prefill M={M}", flush=True)
    rows = np.unique(np.concatenate([np.arange(0, M, max(1, M // 13)), [M - 1, M - 2, 127, 128]]))
    for (N, K, sid) in [(6144, 2048, 1000), (2048, 6144, 1002)]:
        (wq, s, b), qh = make(mq4, O, N, K, sid, dev)
        x = mq4.fill_normal_bf16((M, K), mq4.STREAM_PREFILL, 0.0, 1.0, device=dev)
        y32 = mq4.quantized_matmul_f32(x, wq, s, b)
        torch.cuda.synchronize()
        xs = to_host_u16(x)[rows]
        ref64, _ = O.qmm_f64(xs, *qh)
        check_f32(y32.cpu().numpy()[rows], ref64, f"prefill M={M} N={N} K={K}")


def test_gemm_swiglu_and_residual(mq4, O, dev):
    M, N, K = 200, 6144, 2048
    (g, gh), (u, uh) = make(mq4, O, N, K, 1003, dev), make(mq4, O, N, K, 1004, dev)
    xh = O.gen_normal_bf16(4001, M * K).reshape(M, K)
    x = to_dev_bf16(xh, dev)
    G = mq4.QuantizedTensor(*g)
    U = mq4.QuantizedTensor(*u)
    h = mq4.mlp_gate_up_silu(x, G, U)
    torch.cuda.synchronize()
    _, gb = O.qmm_f64(xh, *gh)
    _, ub = O.qmm_f64(xh, *uh)
    check_swiglu(O, to_host_u16(h), O.swiglu_bf16(gb, ub), "GEMM SwiGLU")

    # residual epilogue: down projection of h, added to a residual stream
    (d, dh) = make(mq4, O, K, N, 1005, dev)
    D = mq4.QuantizedTensor(*d)
    res = mq4.fill_normal_bf16((M, K), 3001, 0.0, 1.0, device=dev)
    y = mq4.qmatmul_residual(h, D, res)
    y32 = mq4.quantized_matmul_f32(h, *d)
    torch.cuda.synchronize()
    want = O.add_bf16(to_host_u16(res), O.f32_to_bf16(y32.cpu().numpy()))
    assert np.array_equal(to_host_u16(y), want)
    ref64, _ = O.qmm_f64(to_host_u16(h), *dh)
    check_f32(y32.cpu().numpy(), ref64, "down")


def test_gemm_and_gemv_agree_at_the_switch(mq4, O, dev):
    """M = 32 runs the GEMV, M = 33 the GEMM: both rows-0..31 results are
    within the bar of the same fp64 reference."""
    N, K = 512, 2048
    (wq, s, b), qh = make(mq4, O, N, K, 11, dev)
    xh = O.gen_normal_bf16(4002, 33 * K).reshape(33, K)
    x = to_dev_bf16(xh, dev)
    a = mq4.quantized_matmul_f32(x[:32].contiguous(), wq, s, b)
    c = mq4.quantized_matmul_f32(x, wq, s, b)
    torch.cuda.synchronize()
    ref64, _ = O.qmm_f64(xh, *qh)
    check_f32(a.cpu().numpy(), ref64[:32], "GEMV M=32")
    check_f32(c.cpu().numpy(), ref64, "GEMM M=33")


def sampled_rows(M):
    return np.unique(np.concatenate([np.arange(0, M, max(1, M // 11)), [M - 1, M - 2, M - 40, 127, 128, 1919, 1920]]))


def test_gemm_epilogues_at_prefill_m(mq4, O, dev):
    """M = 1960 (the 10-frame video turn; its last 128-row tile is ragged):
    bf16 store, fused SwiGLU, fused (1 + w) RMSNorm + SwiGLU and residual
    epilogues on sampled rows."""
    M, N, K = 1960, 6144, 2048
    print(f"prefill epilogues M={M}", flush=True)
    rows = sampled_rows(M)
    (g, gh), (u, uh) = make(mq4, O, N, K, 1000, dev), make(mq4, O, N, K, 1001, dev)
    G, U = mq4.QuantizedTensor(*g), mq4.QuantizedTensor(*u)
    x = mq4.fill_normal_bf16((M, K), mq4.STREAM_PREFILL, 0.0, 1.0, device=dev)
    y = mq4.quantized_matmul(x, *g)
    y32 = mq4.quantized_matmul_f32(x, *g)
    h = mq4.mlp_gate_up_silu(x, G, U)
    nw = mq4.fill_normal_bf16((K,), mq4.stream_id_layer_norm(0), 0.1, 0.02, device=dev)
    hn = mq4.mlp_gate_up_silu(x, G, U, norm_weight=nw, eps=1e-6)
    torch.cuda.synchronize()
    xs = to_host_u16(x)[rows]
    ref64, _ = O.qmm_f64(xs, *gh)
    assert np.array_equal(to_host_u16(y), O.f32_to_bf16(y32.cpu().numpy()))
    check_f32(y32.cpu().numpy()[rows], ref64, "prefill gate fp32")
    check_bf16(O, to_host_u16(y)[rows], ref64, "prefill gate bf16")
    _, gb = O.qmm_f64(xs, *gh)
    _, ub = O.qmm_f64(xs, *uh)
    check_swiglu(O, to_host_u16(h)[rows], O.swiglu_bf16(gb, ub), "prefill SwiGLU")
    n = O.rmsnorm_1pw(xs, to_host_u16(nw), 1e-6)
    _, gbn = O.qmm_f64(n, *gh)
    _, ubn = O.qmm_f64(n, *uh)
    check_swiglu(O, to_host_u16(hn)[rows], O.swiglu_bf16(gbn, ubn), "prefill norm+SwiGLU")
    # the C entry point with the norm fused into the GEMM (what the Python
    # binding replaces by two launches at this size)
    import ctypes
    hc = torch.empty_like(hn)
    P = ctypes.c_void_p
    rc = mq4.lib().mq4_rmsnorm_gate_up_silu(P(x.data_ptr()), M, K, P(nw.data_ptr()), ctypes.c_float(1e-6),
                                            *[P(t.data_ptr()) for t in g], *[P(t.data_ptr()) for t in u], N,
                                            P(hc.data_ptr()), None)
    assert rc == 0
    torch.cuda.synchronize()
    check_swiglu(O, to_host_u16(hc)[rows], O.swiglu_bf16(gbn, ubn), "prefill norm+SwiGLU (fused C entry)")

    # down projection of h with the residual add (src/model/marlin.cpp:142)
    (d, dh) = make(mq4, O, K, N, 1002, dev)
    D = mq4.QuantizedTensor(*d)
    res = mq4.fill_normal_bf16((M, K), 3001, 0.0, 1.0, device=dev)
    yr = mq4.qmatmul_residual(h, D, res)
    yd32 = mq4.quantized_matmul_f32(h, *d)
    torch.cuda.synchronize()
    assert np.array_equal(to_host_u16(yr), O.add_bf16(to_host_u16(res), O.f32_to_bf16(yd32.cpu().numpy())))
    ref64d, _ = O.qmm_f64(to_host_u16(h)[rows], *dh)
    check_f32(yd32.cpu().numpy()[rows], ref64d, "prefill down fp32")


@pytest.mark.parametrize("M,K,N", [(1960, 2048, 6144), (200, 2048, 6144), (40, 512, 1024), (5, 2048, 6144),
                                   (16, 2048, 6144), (32, 2048, 6144), (24, 2048, 4608), (7, 1024, 5120),
                                   (23, 2048, 6144), (70, 640, 1280), (4096, 2048, 6144), (8192, 2048, 6144),
                                   (200, 2048, 1536), (130, 1024, 2048)])
def test_mlp_residual_one_call(mq4, O, dev, M, K, N):
    """mq4_mlp_residual: x + mlp_forward(rms_norm(x)) in one call
    (src/model/marlin.cpp:141-142).  From 33 rows on with K, N multiples of 512
    and 16-byte aligned scales and biases both products run on the
    fp16-weight GEMM on operands stored in the matrix cores' order; the down
    + residual product on 128 x 128 tiles while they number at most two per
    CU, in the most K parts that keep one block per CU ((1960, 2048, 6144) and
    (4096, ...): one part; (200, ...): four; (40, 512, 1024): two), and on
    128 x 256 tiles beyond ((8192, ...), the prefill bench's M = 8192
    figure), checked on sampled rows that include three of the last 128-row
    tile (M - 1, M - 2, M - 40); (200, 2048, 1536): 12 gate/up column blocks
    (not a multiple of 8, the plain block order) and a 24-group down product
    in one part; (130, 1024, 2048): four down parts of one 8-group scale slot
    each; (5, ...),
    (16, ...), (32, ...), (23, ...), (24, 2048, 4608) and (7, 1024, 5120)
    take the MFMA GEMV kernels, the down product as two K parts per tile and
    a combine (72 and 80 groups: the second part partly empty), and (70, 640,
    1280) the separate GEMM kernels.
    * Against the separate entries (mq4_rmsnorm_gate_up_silu +
      mq4_qmm_residual, each pinned to the oracle): rms of the difference of
      the MLP parts <= 1e-2 of rms; on the GEMV path bit for bit.  From 33
      rows with 16-byte aligned scales and biases the one call runs the
      fp16-weight GEMM (weights fp16(s q + b), about 2e-6 of the output rms
      from the exact product), whose gate/up flips the bf16 rounding of about
      1-2% of h: >= 95% of the outputs bit-identical (measured ~98%, rms of
      the difference ~8e-4).
    * Against the oracle's chain (rms_norm, gate/up, bf16 SwiGLU, fp64 down,
      bf16 residual add) on sampled rows: rms(err) <= 1e-2 x rms of the
      oracle's MLP output."""
    print(f"mlp_residual M={M} K={K} N={N}", flush=True)
    ws = [make(mq4, O, *((N, K) if p < 2 else (K, N)), 1100 + p, dev) for p in range(3)]
    w = mq4.MLPWeights(*[mq4.QuantizedTensor(*d) for d, _ in ws])
    x = mq4.fill_normal_bf16((M, K), mq4.STREAM_PREFILL, 0.0, 1.0, device=dev)
    nw = mq4.fill_normal_bf16((K,), mq4.stream_id_layer_norm(0), 0.1, 0.02, device=dev)
    y = mq4.mlp_residual(x, w, nw, 1e-6)
    h = mq4.mlp_gate_up_silu(x, w.gate_proj, w.up_proj, norm_weight=nw, eps=1e-6)
    ys = mq4.qmatmul_residual(h, w.down_proj, x)
    yi = x.clone()
    mq4.mlp_residual(yi, w, nw, 1e-6, out=yi)                      # in place
    torch.cuda.synchronize()
    got, sep, xh = to_host_u16(y), to_host_u16(ys), to_host_u16(x)
    assert np.array_equal(to_host_u16(yi), got)
    same = float(np.mean(got == sep))
    xf = O.bf16_to_f32(xh).astype(np.float64)
    dm = (O.bf16_to_f32(got) - O.bf16_to_f32(sep)).astype(np.float64)
    ms = O.bf16_to_f32(sep).astype(np.float64) - xf
    rel = float(np.sqrt(np.mean(dm * dm) / np.mean(ms * ms)))
    print(f"vs separate entries: identical {same:.5f}, rms(diff)/rms(mlp) {rel:.2e}")
    if M < 33:
        assert np.array_equal(got, sep)
    assert same >= 0.95 and rel <= TOL
    rows = sampled_rows(M) if M > 64 else np.arange(M)
    rows = rows[(rows >= 0) & (rows < M)]
    xs = xh[rows]
    n = O.rmsnorm_1pw(xs, to_host_u16(nw), 1e-6)
    (g, gh), (u, uh), (d, dh) = ws
    _, _, _, yb = O.mlp_forward(n, gh, uh, dh)
    ref = O.add_bf16(xs, yb)
    err = (O.bf16_to_f32(got[rows]) - O.bf16_to_f32(ref)).astype(np.float64)
    mo = O.bf16_to_f32(yb).astype(np.float64)
    rel_o = float(np.sqrt(np.mean(err * err) / np.mean(mo * mo)))
    print(f"vs oracle chain: rms(err)/rms(mlp) {rel_o:.2e}")
    assert rel_o <= TOL


@pytest.mark.gpu
@pytest.mark.parametrize("M,shift", [(200, "down"), (1960, "down"), (4096, "down"), (200, "gate")])
def test_mlp_residual_paired_down(mq4, O, dev, M, shift):
    """The one-call MLP with one matrix's scales and biases 4-byte but not
    16-byte aligned.  down: gate/up on the fp16-weight GEMM writes h paired
    in bf16 (pair order through the per-chunk column permutation) with its
    group sums from the LDS tile, and the down product runs on the
    exact-operand GEMM (M = 4096: its 64 x 64 wave tiles, 512 blocks of
    128 x 128; below: 64 x 32).  gate: both products on the exact-operand
    GEMM with paired operands.  Against the separate entries: >= 95% of the bits
    identical, rms of the difference <= 1e-2 of the MLP output's rms; against
    the oracle chain on sampled rows: rms(err) <= 1e-2 of that rms."""
    import torch
    K, N = 2048, 6144
    print(f"mlp_residual shifted {shift} scales M={M}", flush=True)
    ws = [make(mq4, O, *((N, K) if p < 2 else (K, N)), 1400 + p, dev) for p in range(3)]
    (gd, _), (ud, _), (dd, _) = ws
    keep = []

    def shifted(t):                                       # the same values 4 bytes past a 16-byte boundary
        buf = torch.empty(t.numel() + 2, dtype=t.dtype, device=dev)
        v = buf[2:].view(t.shape)
        v.copy_(t)
        keep.append(buf)
        return v

    sel = dd if shift == "down" else gd
    ss, sb = shifted(sel[1]), shifted(sel[2])
    assert ss.data_ptr() % 16 != 0 and ss.data_ptr() % 4 == 0 and sb.data_ptr() % 16 != 0
    q = mq4.QuantizedTensor(sel[0], ss, sb)
    w = (mq4.MLPWeights(mq4.QuantizedTensor(*gd), mq4.QuantizedTensor(*ud), q) if shift == "down" else
         mq4.MLPWeights(q, mq4.QuantizedTensor(*ud), mq4.QuantizedTensor(*dd)))
    x = mq4.fill_normal_bf16((M, K), mq4.STREAM_PREFILL + 3, 0.0, 1.0, device=dev)
    nw = mq4.fill_normal_bf16((K,), mq4.stream_id_layer_norm(3), 0.1, 0.02, device=dev)
    y = mq4.mlp_residual(x, w, nw, 1e-6)
    h = mq4.mlp_gate_up_silu(x, w.gate_proj, w.up_proj, norm_weight=nw, eps=1e-6)
    ys = mq4.qmatmul_residual(h, w.down_proj, x)
    torch.cuda.synchronize()
    got, sep, xh = to_host_u16(y), to_host_u16(ys), to_host_u16(x)
    same = float(np.mean(got == sep))
    xf = O.bf16_to_f32(xh).astype(np.float64)
    dm = (O.bf16_to_f32(got) - O.bf16_to_f32(sep)).astype(np.float64)
    ms = O.bf16_to_f32(sep).astype(np.float64) - xf
    rel = float(np.sqrt(np.mean(dm * dm) / np.mean(ms * ms)))
    print(f"vs separate entries: identical {same:.5f}, rms(diff)/rms(mlp) {rel:.2e}")
    assert same >= 0.95 and rel <= TOL
    rows = sampled_rows(M)
    rows = rows[(rows >= 0) & (rows < M)]
    xs = xh[rows]
    n = O.rmsnorm_1pw(xs, to_host_u16(nw), 1e-6)
    (_, gh), (_, uh), (_, dh) = ws
    _, _, _, yb = O.mlp_forward(n, gh, uh, dh)
    ref = O.add_bf16(xs, yb)
    err = (O.bf16_to_f32(got[rows]) - O.bf16_to_f32(ref)).astype(np.float64)
    mo = O.bf16_to_f32(yb).astype(np.float64)
    rel_o = float(np.sqrt(np.mean(err * err) / np.mean(mo * mo)))
    print(f"vs oracle chain: rms(err)/rms(mlp) {rel_o:.2e}")
    assert rel_o <= TOL


@pytest.mark.gpu
def test_mlp_residual_down_tile_widths_agree(mq4, O, dev):
    """The one-call MLP's down product (2048 x 6144) runs on 128 x 128 tiles
    while they number at most two per CU (2048 and 3000 rows: 256 and 384
    tiles on 256 CUs) and on 128 x 256 tiles beyond (8192 rows), in one K
    part each.  Every row's result depends only on that row (its norm, its
    fp16 copy, its products in the same K order), so the 2048- and 3000-row
    calls equal the first rows of the 8192-row call bit for bit (3000: a
    ragged last tile of 56 rows)."""
    import torch
    K, N = 2048, 6144
    print("mlp_residual tile widths M=8192 / 3000 / 2048", flush=True)
    ws = [make(mq4, O, *((N, K) if p < 2 else (K, N)), 1500 + p, dev) for p in range(3)]
    w = mq4.MLPWeights(*[mq4.QuantizedTensor(*d) for d, _ in ws])
    x = mq4.fill_normal_bf16((8192, K), mq4.STREAM_PREFILL + 4, 0.0, 1.0, device=dev)
    nw = mq4.fill_normal_bf16((K,), mq4.stream_id_layer_norm(4), 0.1, 0.02, device=dev)
    full = mq4.mlp_residual(x, w, nw, 1e-6).view(torch.int16)
    for M in (3000, 2048):
        part = mq4.mlp_residual(x[:M], w, nw, 1e-6).view(torch.int16)
        torch.cuda.synchronize()
        same = float((part == full[:M]).float().mean())
        print(f"M={M}: identical to the 8192-row call {same:.6f}")
        assert torch.equal(part, full[:M])


@pytest.mark.gpu
def test_mlp_residual_unaligned_output(mq4, O, dev):
    """The one-call MLP at 200 rows (fp16-weight GEMM; four K parts of the
    down product for an 8-byte aligned y) into a y that is only 2-byte
    aligned, which the entry accepts: the down product then runs as one part
    and stores element by element.  Same result up to the parts' fp32
    summation order: >= 99% of the bits identical, rms of the difference
    <= 1e-3 of the MLP output's rms."""
    import torch
    M, K, N = 200, 2048, 6144
    print(f"mlp_residual unaligned y M={M}", flush=True)
    ws = [make(mq4, O, *((N, K) if p < 2 else (K, N)), 1300 + p, dev) for p in range(3)]
    w = mq4.MLPWeights(*[mq4.QuantizedTensor(*d) for d, _ in ws])
    x = mq4.fill_normal_bf16((M, K), mq4.STREAM_PREFILL + 2, 0.0, 1.0, device=dev)
    nw = mq4.fill_normal_bf16((K,), mq4.stream_id_layer_norm(2), 0.1, 0.02, device=dev)
    ref = mq4.mlp_residual(x, w, nw, 1e-6)
    buf = torch.zeros(M * K + 1, dtype=torch.bfloat16, device=dev)
    yo = buf[1:].view(M, K)                                # 2-byte aligned, not 8
    assert yo.data_ptr() % 8 != 0
    mq4.mlp_residual(x, w, nw, 1e-6, out=yo)
    torch.cuda.synchronize()
    got, want, xh = to_host_u16(yo), to_host_u16(ref), to_host_u16(x)
    same = float(np.mean(got == want))
    xf = O.bf16_to_f32(xh).astype(np.float64)
    d = (O.bf16_to_f32(got) - O.bf16_to_f32(want)).astype(np.float64)
    ms = O.bf16_to_f32(want).astype(np.float64) - xf
    rel = float(np.sqrt(np.mean(d * d) / np.mean(ms * ms)))
    print(f"identical {same:.5f}, rms(diff)/rms(mlp) {rel:.2e}")
    assert same >= 0.99 and rel <= 1e-3


@pytest.mark.parametrize("M", [16, 32, 200])
def test_mlp_residual_split_graph_replay(mq4, O, dev, M):
    """The one-call MLP with its down product in K parts plus a combine,
    captured in a HIP graph: at batched-decode sizes (16, 32: two parts per
    16-row tile, bit for bit the separate entries) and at 200 rows (the
    fp16-weight GEMM, four parts of 24 groups).  Every replay, with eager work
    and synchronizations between replays and the workspace overwritten with
    0xFF bytes before each, reproduces the eager call bit for bit, as the
    benches replay it."""
    K, N = 2048, 6144
    print(f"mlp_residual graph M={M}", flush=True)
    ws_ = [make(mq4, O, *((N, K) if p < 2 else (K, N)), 1200 + p, dev) for p in range(3)]
    w = mq4.MLPWeights(*[mq4.QuantizedTensor(*d) for d, _ in ws_])
    x = mq4.fill_normal_bf16((M, K), mq4.STREAM_PREFILL + 1, 0.0, 1.0, device=dev)
    nw = mq4.fill_normal_bf16((K,), mq4.stream_id_layer_norm(1), 0.1, 0.02, device=dev)
    L = mq4.lib()
    P = ctypes.c_void_p
    nb = L.mq4_mlp_workspace_size(M, K, N)
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)
    y = torch.empty_like(x)
    qa = lambda q: (P(q.weight.data_ptr()), P(q.scales.data_ptr()), P(q.biases.data_ptr()))

    def call(st):
        mq4._check(L.mq4_mlp_residual(P(x.data_ptr()), M, K, P(nw.data_ptr()), 1e-6, *qa(w.gate_proj),
                                      *qa(w.up_proj), *qa(w.down_proj), N, P(ws.data_ptr()), nb, P(y.data_ptr()),
                                      st))

    call(P(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    want = to_host_u16(y).copy()
    ref = to_host_u16(mq4.qmatmul_residual(mq4.mlp_gate_up_silu(x, w.gate_proj, w.up_proj, norm_weight=nw),
                                           w.down_proj, x))
    if M < 33:
        assert np.array_equal(want, ref)                   # same bits as the separate entries
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call(P(s.cuda_stream))
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(P(torch.cuda.current_stream().cuda_stream))
    for r in range(3):
        y.fill_(0)
        ws.fill_(0xFF)                                     # nothing of a call's workspace outlives it
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(to_host_u16(y), want), f"replay {r}"
        mq4.qmatmul(x, w.gate_proj)                        # eager work between replays
        torch.cuda.synchronize()
