"""The header-only C++ host API (marlin-mlx_amd/csrc/mq4.hpp), driven by the
prebuilt tests/cpp/mq4_cpp_demo.cpp, gives bit-identical results to the same
decode-shaped computation issued through the Python binding, and the result
meets the oracle's bar."""
import os
import subprocess

import numpy as np
import pytest
import torch

from conftest import ROOT, to_host_u16

pytestmark = pytest.mark.gpu
DEMO = os.path.join(ROOT, "marlin-mlx_amd", "_build", "mq4_cpp_demo")


def test_cpp_demo_matches_python_binding(mq4, O, dev):
    assert os.path.exists(DEMO), "build the library first (it builds the C++ demo too)"
    out = subprocess.run([DEMO], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    lines = out.stdout.splitlines()
    tok = int(lines[0].split()[1])
    hid = np.array([int(v) for v in lines[1].split()[1:]], np.uint16)

    H, I, V = 512, 1024, 4096
    layers, norms = [], []
    for l in range(2):
        w = [mq4.fill_normal_bf16(shp, mq4.stream_id_layer(l, p), 0.0, 0.02, device=dev)
             for p, shp in enumerate(((I, H), (I, H), (H, I)))]
        layers.append(mq4.MLPWeights(*[mq4.quantize_weight(t) for t in w]))
        norms.append(mq4.fill_normal_bf16((H,), mq4.stream_id_layer_norm(l), 0.1, 0.02, device=dev))
    lm = mq4.quantize_weight(mq4.fill_normal_bf16((V, H), mq4.STREAM_LM_HEAD, 0.0, 0.02, device=dev))
    fn = mq4.fill_normal_bf16((H,), mq4.STREAM_NORM_WEIGHT, 0.1, 0.02, device=dev)
    x = mq4.fill_normal_bf16((1, H), mq4.stream_id_decode_row(0), 0.0, 1.0, device=dev)
    for lw, nw in zip(layers, norms):
        x = mq4.mlp_forward(x, lw, residual=x, norm_weight=nw)
    idx, logits = mq4.lm_head_argmax(x, lm, return_logits=True, norm_weight=fn)
    torch.cuda.synchronize()
    assert np.array_equal(to_host_u16(x).reshape(-1), hid)
    assert int(idx.cpu()[0]) == tok
    assert tok == int(O.argmax_bf16(to_host_u16(logits))[0])
    # mq4::Sampler: the first call draws with seed 5 + 0 calls, the second is greedy
    words = lines[2].split()
    assert words[0] == "sampled" and words[2] == "greedy"
    assert int(words[3]) == tok
    want = mq4.sample_token(logits, temperature=0.8, top_k=50, seed=5)
    assert int(words[1]) == int(want.cpu()[0])
    # mq4::MlpResidual (one mq4_mlp_residual call per layer) gave the same hidden state
    assert lines[3] == "mlp_residual_same 1"
    assert lines[4] == "empty_ok 1"
    # mq4::MlpResidual sized for 40 rows runs 24, 32 and 40 rows (a workspace
    # size that never shrinks as the row count grows), and bit for bit the
    # separate entries' result below 33 rows
    assert lines[5] == "mlp_residual_rows_ok 1"
    # tensors of another format are refused by the fused mirrors
    assert lines[6] == "format_rejected 1"
    # mq4::BatchedMlpLayers: a two-layer call equals two chained one-layer calls
    assert lines[7] == "batched_layers_ok 1"
