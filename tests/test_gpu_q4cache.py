"""The on-disk Q4 cache on the device: quantized weights saved and loaded
back are bit-identical and give bit-identical products; quantize_or_load
quantizes once and loads on the second call; the C++ demo's lm_head, saved
and reloaded through mq4_cache.hpp, still gives the Python binding's token."""
import os
import subprocess

import numpy as np
import pytest
import torch

from conftest import ROOT, to_host_u16

pytestmark = pytest.mark.gpu
DEMO = os.path.join(ROOT, "marlin-mlx_amd", "_build", "mq4_cpp_demo")


def test_save_load_bit_identical(mq4, dev, tmp_path):
    path = str(tmp_path / "m.safetensors")
    ws = {f"model.language_model.layers.0.mlp.{n}": mq4.fill_normal_bf16(shp, 1000 + i, 0.0, 0.02, device=dev)
          for i, (n, shp) in enumerate((("gate_proj", (6144, 2048)), ("up_proj", (6144, 2048)),
                                        ("down_proj", (2048, 6144))))}
    qs = {n: mq4.quantize_weight(w) for n, w in ws.items()}
    mq4.save_q4_cache(path, qs)
    back = mq4.load_q4_cache(path, device=dev)
    x = mq4.fill_normal_bf16((3, 2048), 3000, 0.0, 1.0, device=dev)
    for n, q in qs.items():
        b = back[n]
        assert torch.equal(b.weight, q.weight)
        assert torch.equal(b.scales.view(torch.int16), q.scales.view(torch.int16))
        assert torch.equal(b.biases.view(torch.int16), q.biases.view(torch.int16))
    g0 = mq4.qmatmul(x, qs["model.language_model.layers.0.mlp.gate_proj"])
    g1 = mq4.qmatmul(x, back["model.language_model.layers.0.mlp.gate_proj"])
    torch.cuda.synchronize()
    assert torch.equal(g0.view(torch.int16), g1.view(torch.int16))


def test_quantize_or_load_uses_the_cache(mq4, dev, tmp_path, monkeypatch):
    path = str(tmp_path / "c.safetensors")
    ws = {"lm_head": mq4.fill_normal_bf16((4096, 2048), 2000, 0.0, 0.02, device=dev)}
    first = mq4.quantize_or_load(path, ws, device=dev)
    assert os.path.exists(path)
    calls = []
    monkeypatch.setattr(mq4, "quantize_weights", lambda *a, **k: calls.append(1) or (_ for _ in ()).throw(
        AssertionError("quantize_weights called although the cache exists")))
    second = mq4.quantize_or_load(path, ws, device=dev)
    assert not calls
    assert torch.equal(first["lm_head"].weight, second["lm_head"].weight)


def test_quantize_or_load_ignores_a_stale_cache(mq4, dev, tmp_path):
    """A cache written from other weights under the same names (another
    checkpoint), or with other shapes, is not used: the weights passed in are
    quantized again and the cache is rewritten for them."""
    path = str(tmp_path / "s.safetensors")
    a = {"lm_head": mq4.fill_normal_bf16((4096, 2048), 2000, 0.0, 0.02, device=dev)}
    b = {"lm_head": mq4.fill_normal_bf16((4096, 2048), 2002, 0.0, 0.02, device=dev)}
    c = {"lm_head": mq4.fill_normal_bf16((2048, 2048), 2000, 0.0, 0.02, device=dev)}
    qa = mq4.quantize_or_load(path, a, device=dev)["lm_head"]
    for ws in (b, c, a):
        got = mq4.quantize_or_load(path, ws, device=dev)["lm_head"]
        want = mq4.quantize_weight(ws["lm_head"])
        torch.cuda.synchronize()
        assert torch.equal(got.weight, want.weight)
        assert torch.equal(got.scales.view(torch.int16), want.scales.view(torch.int16))
    assert not torch.equal(qa.weight[:2048], mq4.quantize_weight(b["lm_head"]).weight[:2048])


def test_cpp_cache_round_trip_keeps_the_token(mq4, dev, tmp_path):
    assert os.path.exists(DEMO)
    plain = subprocess.run([DEMO], capture_output=True, text=True, timeout=60)
    cached = subprocess.run([DEMO, str(tmp_path / "lm.safetensors")], capture_output=True, text=True, timeout=60)
    assert plain.returncode == 0 and cached.returncode == 0, cached.stderr
    assert plain.stdout == cached.stdout
    # the file the C++ side wrote loads through the Python module
    q = mq4.load_q4_cache(str(tmp_path / "lm.safetensors"), device=dev)["lm_head"]
    assert q.out_features == 4096 and q.in_features == 512
