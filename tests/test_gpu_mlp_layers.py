"""The batched one-launch MLP half (mq4_mlp_layers / BatchedMlpLayers).

Per layer and for M token rows (1 <= M <= 32) the kernel evaluates

    x = x + down(swiglu(gate n, up n)),   n = rms_norm(x, norm_l)

(src/model/marlin.cpp:141-142, rms_norm :12-16, mlp_forward :31-35) for M
concurrent decode streams (src/core/engine.cpp:79-94).  Its per-element
arithmetic is that of the other decode kernels (exact bf16 x (128 + q)
products, fp32 sums, the (1 + w) norm, bf16 SwiGLU and residual); only the
grouping of the fp32 sums differs, so results are pinned against the oracle
(fp64 products rounded once to bf16) with the bars of the separate entry
points, and against those entry points (mlp_residual) to fp32-rounding
agreement.  Invariances that need no tolerance: a row's result does not
depend on the other rows or on M, the per-layer calls equal the stacked
call, and graph replays equal the eager call bit for bit.
"""
import numpy as np
import pytest
import torch

from conftest import to_host_u16
from test_gpu_decode_step import EPS, H, build_model, token_row

pytestmark = pytest.mark.gpu


def q_host(w):
    return w.weight.cpu().numpy().view(np.uint32), to_host_u16(w.scales), to_host_u16(w.biases)


def rows_x(mq4, dev, M, first=0):
    return torch.stack([token_row(first + m, dev, mq4) for m in range(M)])


def oracle_layer(O, xh, ly):
    """One MLP half on the CPU: (hidden bf16 bits, y fp64, y bf16 bits)."""
    n = O.rmsnorm_1pw(xh, to_host_u16(ly.post_attn_norm), EPS)
    _, _, h, _ = O.mlp_forward(n, q_host(ly.mlp.gate_proj), q_host(ly.mlp.up_proj), q_host(ly.mlp.down_proj))
    y64, yb = O.qmm_f64(h, *q_host(ly.mlp.down_proj))
    return O.add_bf16(xh, yb), y64, yb


def check_residual(O, got, ref, y64, yb, what):
    """x + y element-wise against the oracle.  A 1-ulp rounding difference of
    gate or up can move an h element by up to 8 bf16 ulps (the SwiGLU bar of
    the separate kernels) in about 1% of the 6144 elements; through the down
    product that is about 3e-3 x rms(y) at most.  Bar: |err| <= 2^-7
    (|y| + |x + y|) + 2^-7 rms(y) per element (an index or layout mistake
    gives errors of order rms(y)), and rms(err) <= 1e-2 rms(x + y) per row."""
    g = O.bf16_to_f32(got).astype(np.float64)
    r = O.bf16_to_f32(ref).astype(np.float64)
    err = np.abs(g - r)
    yrms = float(np.sqrt(np.mean(y64 * y64)))
    bar = 2.0 ** -7 * (np.abs(O.bf16_to_f32(yb)) + np.abs(r)) + 2.0 ** -7 * yrms
    rel = np.sqrt(np.mean((g - r) ** 2, axis=-1) / np.mean(r * r, axis=-1))
    same = float(np.mean(got == ref))
    print(f"{what}: bit-identical {same:.4f}, worst element {np.max(err / bar):.3f} of its bar, "
          f"rms(err)/rms max {rel.max():.2e}", flush=True)
    assert np.all(err <= bar)
    assert rel.max() <= 1e-2


@pytest.fixture(scope="module")
def one_layer(mq4, dev):
    layers, _, _ = build_model(mq4, 1, 16, dev)
    return layers


@pytest.mark.parametrize("M", [1, 3, 16, 17, 32])
def test_one_layer_against_oracle(mq4, O, dev, one_layer, M):
    print(f"mlp_layers one layer vs oracle: M={M}", flush=True)
    ly = one_layer[0]
    B = mq4.BatchedMlpLayers(one_layer, max_rows=32, eps=EPS)
    x = rows_x(mq4, dev, M)
    got = B(x)
    sep = mq4.mlp_residual(x, ly.mlp, ly.post_attn_norm, EPS)
    torch.cuda.synchronize()
    ref, y64, yb = oracle_layer(O, to_host_u16(x), ly)
    check_residual(O, to_host_u16(got), ref, y64, yb, f"M={M} vs oracle")
    # the separate entry points' result meets the same bar against this one
    check_residual(O, to_host_u16(got), to_host_u16(sep), y64, yb, f"M={M} vs mlp_residual")


def test_rows_do_not_depend_on_M(mq4, dev, one_layer):
    """Every row's arithmetic is the same whatever the other rows hold and
    however many there are (one or two 16-row MFMA tiles)."""
    print("mlp_layers row independence: M=1..32", flush=True)
    B = mq4.BatchedMlpLayers(one_layer, max_rows=32, eps=EPS)
    x32 = rows_x(mq4, dev, 32)
    full = to_host_u16(B(x32))
    for M in (1, 2, 5, 15, 16, 17, 31):
        part = to_host_u16(B(x32[:M].contiguous()))
        assert np.array_equal(part, full[:M]), f"M={M}"
    # the same row placed at another position of another batch
    x = rows_x(mq4, dev, 20, first=40)
    x[13] = x32[7]
    got = to_host_u16(B(x))
    assert np.array_equal(got[13], full[7])


@pytest.fixture(scope="module")
def stack24(mq4, dev):
    print("mlp_layers: building 24 layers", flush=True)
    layers, _, _ = build_model(mq4, 24, 16, dev)
    torch.cuda.synchronize()
    return layers


@pytest.mark.parametrize("M", [4, 16, 32])
def test_24_layer_stack_against_oracle_chain(mq4, O, dev, stack24, M):
    """The benchmark's 24 layers against the oracle's chain: per row rms(err)
    <= 5e-2 rms after 24 layers (the bar of the batched chain test: two
    correct chains drift about 1e-3 of rms per layer through the bf16
    residual stream), and against the chain of mlp_residual calls, which
    drifts from this one by fp32 grouping only."""
    print(f"mlp_layers 24-layer stack vs oracle chain: M={M}", flush=True)
    B = mq4.BatchedMlpLayers(stack24, max_rows=32, eps=EPS)
    x0 = rows_x(mq4, dev, M)
    got = B(x0)
    xs = x0
    for ly in stack24:
        xs = mq4.mlp_residual(xs, ly.mlp, ly.post_attn_norm, EPS)
    # the per-layer entry, chained by the caller, equals the stacked call
    xl = x0
    for i in range(len(stack24)):
        xl = B.layer(i, xl)
    torch.cuda.synchronize()
    g = to_host_u16(got)
    assert np.array_equal(to_host_u16(xl), g), "per-layer calls differ from the stacked call"
    ref = to_host_u16(x0)
    for ly in stack24:
        ref, _, _ = oracle_layer(O, ref, ly)

    def rel(a, b):
        af, bf = O.bf16_to_f32(a).astype(np.float64), O.bf16_to_f32(b).astype(np.float64)
        return np.sqrt(np.mean((af - bf) ** 2, axis=1) / np.mean(bf * bf, axis=1))

    r_or, r_sep = rel(g, ref), rel(g, to_host_u16(xs))
    r_sep_or = rel(to_host_u16(xs), ref)
    print(f"M={M}: rms(err)/rms vs oracle chain max {r_or.max():.2e} (mlp_residual chain vs oracle "
          f"{r_sep_or.max():.2e}); vs mlp_residual chain max {r_sep.max():.2e}", flush=True)
    assert r_or.max() <= 5e-2
    assert r_sep.max() <= 5e-2


def test_epoch_counts_launches_and_graph_replay(mq4, dev, stack24):
    """The epoch word moves on once per launch (one launch per layer) and the
    arrival count by 256 per launch; a captured graph of a 3-layer stack
    replays bit-identically to the eager call, with eager launches on the
    same workspace between the replays."""
    print("mlp_layers epoch and graph replay: M=16, 3 layers", flush=True)
    B = mq4.BatchedMlpLayers(stack24[:3], max_rows=16, eps=EPS)
    x = rows_x(mq4, dev, 16)
    want = to_host_u16(B(x))
    torch.cuda.synchronize()
    ctrl = B.workspace[:128].view(torch.int32)
    assert int(ctrl[0].item()) == 3 and int(ctrl[16].item()) == 3 * 256
    out = torch.empty_like(x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        B(x, out)                                   # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        B(x, out)
    for r in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(to_host_u16(out), want), f"replay {r}"
        assert np.array_equal(to_host_u16(B(x)), want), f"eager call after replay {r}"
        torch.cuda.synchronize()
    # eager 1 + warm-up 1 + 3 replays + 3 eager calls, 3 launches each
    assert int(ctrl[0].item()) == 8 * 3 and int(ctrl[16].item()) == 8 * 3 * 256


def test_sticky_error(mq4, dev, one_layer):
    """A workspace whose error word is set makes every call write NaN rows,
    until the workspace is zero-filled."""
    B = mq4.BatchedMlpLayers(one_layer, max_rows=8, eps=EPS)
    x = rows_x(mq4, dev, 8)
    want = to_host_u16(B(x))
    B.workspace[128:132].view(torch.int32).fill_(1)        # error word (uint32 index 32)
    got = to_host_u16(B(x))
    assert np.all(got == 0x7FC0)
    B.reset()
    assert np.array_equal(to_host_u16(B(x)), want)


def test_rejects(mq4, dev, one_layer):
    B = mq4.BatchedMlpLayers(one_layer, max_rows=8, eps=EPS)
    x = rows_x(mq4, dev, 9)
    with pytest.raises(ValueError):
        B(x)                                        # more rows than the workspace was sized for
    x = rows_x(mq4, dev, 4)
    with pytest.raises(ValueError):
        B(x, x_out=torch.empty((4, H + 1), dtype=torch.bfloat16, device=dev))
    with pytest.raises(mq4.MQ4Error) as e:
        B(x, x_out=x)                               # in place: workgroups read x while others write
    assert e.value.code == -1
    with pytest.raises(NotImplementedError):
        mq4.BatchedMlpLayers(one_layer, max_rows=33)
