"""On-disk Q4 cache (safetensors, MLX naming), checked on the CPU: the Python
module (marlin-mlx_amd/q4cache.py) and the C++ header
(marlin-mlx_amd/csrc/mq4_cache.hpp, driven by tests/cpp/mq4_cache_tool.cpp)
each read what the other and the safetensors library write, byte for byte,
and reject malformed files."""
import os
import struct
import subprocess

import numpy as np
import pytest
import torch

from conftest import ROOT

TOOL = os.path.join(ROOT, "marlin-mlx_amd", "_build", "mq4_cache_tool")


def fnv1a(b: bytes) -> str:
    h = 1469598103934665603
    for c in b:
        h ^= c
        h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return f"{h:016x}"


def cpp_dump(path):
    out = subprocess.run([TOOL, "dump", path], capture_output=True, text=True, timeout=30)
    assert out.returncode == 0, out.stderr
    meta, ts = {}, {}
    for line in out.stdout.splitlines():
        f = line.split()
        if f[0] == "meta":
            meta[f[1]] = f[2]
        else:
            ts[f[0]] = (f[1], tuple(int(v) for v in f[2:-1]), f[-1])
    return meta, ts


def random_q4(mq4, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    wq = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K // 8), generator=g, dtype=torch.int64).to(torch.int32)
    s = (torch.randn((N, K // 64), generator=g) * 0.01).to(torch.bfloat16)
    b = (torch.randn((N, K // 64), generator=g) * 0.05).to(torch.bfloat16)
    return mq4.QuantizedTensor(wq, s, b)


def test_python_writer_read_by_safetensors_and_cpp(mq4, tmp_path):
    from safetensors import safe_open
    path = str(tmp_path / "q4.safetensors")
    qs = {"model.layers.0.mlp.gate_proj": random_q4(mq4, 64, 2048, 1), "lm_head": random_q4(mq4, 33, 128, 2)}
    mq4.save_q4_cache(path, qs)
    with safe_open(path, "pt") as f:
        assert f.metadata()["quantization.group_size"] == "64" and f.metadata()["quantization.bits"] == "4"
        for name, q in qs.items():
            w = f.get_tensor(name + ".weight")
            assert w.dtype == torch.uint32 and tuple(w.shape) == tuple(q.weight.shape)
            assert torch.equal(w.view(torch.int32), q.weight)
            assert torch.equal(f.get_tensor(name + ".scales").view(torch.int16), q.scales.view(torch.int16))
            assert torch.equal(f.get_tensor(name + ".biases").view(torch.int16), q.biases.view(torch.int16))
    meta, ts = cpp_dump(path)
    assert meta["format"] == "mlx"
    for name, q in qs.items():
        for suf, t, dt in ((".weight", q.weight, "U32"), (".scales", q.scales, "BF16"), (".biases", q.biases, "BF16")):
            assert ts[name + suf] == (dt, tuple(t.shape), fnv1a(t.contiguous().view(torch.uint8).numpy().tobytes()))
    back = mq4.load_q4_cache(path, device="cpu")
    for name, q in qs.items():
        assert torch.equal(back[name].weight, q.weight)
        assert torch.equal(back[name].scales.view(torch.int16), q.scales.view(torch.int16))
        assert torch.equal(back[name].biases.view(torch.int16), q.biases.view(torch.int16))
        assert back[name].in_features == q.in_features and back[name].group_size == 64


def test_cpp_writer_read_by_python_and_safetensors(mq4, tmp_path):
    from safetensors import safe_open
    path = str(tmp_path / "cpp.safetensors")
    out = subprocess.run([TOOL, "write", path], capture_output=True, text=True, timeout=30)
    assert out.returncode == 0, out.stderr
    want = {"weight": bytes((i * 37 + 11) & 0xFF for i in range(3 * 16 * 4)),
            "scales": bytes((i * 13 + 60) & 0xFF for i in range(12)),
            "biases": bytes((i * 7 + 190) & 0xFF for i in range(12))}
    with safe_open(path, "pt") as f:
        for k, raw in want.items():
            assert f.get_tensor("layer.0.mlp.gate_proj." + k).contiguous().view(torch.uint8).numpy().tobytes() == raw
    q = mq4.load_q4_cache(path, device="cpu")["layer.0.mlp.gate_proj"]
    assert q.weight.contiguous().view(torch.uint8).numpy().tobytes() == want["weight"]
    assert q.scales.contiguous().view(torch.uint8).numpy().tobytes() == want["scales"]
    assert q.out_features == 3 and q.in_features == 128


def test_safetensors_library_file_loads(mq4, tmp_path):
    """A file in MLX's convention written by another producer (here the
    safetensors library itself) loads through both readers."""
    from safetensors.torch import save_file
    path = str(tmp_path / "lib.safetensors")
    q = random_q4(mq4, 16, 256, 3)
    save_file({"x.weight": q.weight.view(torch.uint32), "x.scales": q.scales, "x.biases": q.biases}, path,
              metadata={"quantization.group_size": "64", "quantization.bits": "4"})
    back = mq4.load_q4_cache(path, device="cpu")["x"]
    assert torch.equal(back.weight, q.weight)
    meta, ts = cpp_dump(path)
    assert ts["x.weight"] == ("U32", (16, 32), fnv1a(q.weight.contiguous().view(torch.uint8).numpy().tobytes()))


def test_malformed_files_are_rejected(mq4, tmp_path):
    good = str(tmp_path / "g.safetensors")
    mq4.save_q4_cache(good, {"a": random_q4(mq4, 4, 128, 4)})
    raw = open(good, "rb").read()
    (n,) = struct.unpack("<Q", raw[:8])
    cases = {
        "truncated": raw[:-16],
        "bad_len": struct.pack("<Q", len(raw) * 2) + raw[8:],
        "not_json": raw[:8] + b"{" * n + raw[8 + n:],
    }
    for name, data in cases.items():
        p = str(tmp_path / f"{name}.safetensors")
        open(p, "wb").write(data)
        with pytest.raises(ValueError):
            mq4.load_q4_cache(p, device="cpu")
        r = subprocess.run([TOOL, "dump", p], capture_output=True, text=True, timeout=30)
        assert r.returncode != 0, name
    # scales of the wrong width for the weight's K
    from safetensors.torch import save_file
    q = random_q4(mq4, 4, 128, 5)
    p = str(tmp_path / "shape.safetensors")
    save_file({"a.weight": q.weight.view(torch.uint32), "a.scales": q.scales[:, :1].contiguous(),
               "a.biases": q.biases[:, :1].contiguous()}, p)
    with pytest.raises(ValueError, match="do not match"):
        mq4.load_q4_cache(p, device="cpu")


@pytest.mark.parametrize("meta", [{"quantization.group_size": "128", "quantization.bits": "4"},
                                  {"quantization.group_size": "64", "quantization.bits": "2"}])
def test_other_formats_are_refused_by_both_loaders(mq4, tmp_path, meta):
    """MLX writes other group sizes and bit widths too.  Both loaders refuse
    them: the fused entry points take no format argument and would read a
    group-128 file's scales as K/64 groups, past their end."""
    from safetensors.torch import save_file
    K = 256
    bits = int(meta["quantization.bits"])
    gs = int(meta["quantization.group_size"])
    g = torch.Generator().manual_seed(9)
    wq = torch.randint(0, 2 ** 31 - 1, (8, K * bits // 32), generator=g, dtype=torch.int64).to(torch.int32)
    s = torch.zeros((8, K // gs), dtype=torch.bfloat16)
    p = str(tmp_path / "other.safetensors")
    save_file({"a.weight": wq.view(torch.uint32), "a.scales": s, "a.biases": s.clone()}, p, metadata=meta)
    with pytest.raises(NotImplementedError, match="group_size=64, bits=4"):
        mq4.load_q4_cache(p, device="cpu")
    r = subprocess.run([TOOL, "check", p], capture_output=True, text=True, timeout=30)
    assert r.returncode == 3 and "group_size=64, bits=4" in r.stderr, r.stderr
    good = str(tmp_path / "good.safetensors")
    mq4.save_q4_cache(good, {"a": random_q4(mq4, 4, 128, 6)})
    assert subprocess.run([TOOL, "check", good], capture_output=True, timeout=30).returncode == 0


def test_crafted_headers_are_rejected_by_cpp_reader(tmp_path):
    """A shape whose element count overflows 64 bits (it would wrap around to
    match the data offsets) and a header nested past any safetensors layout
    (recursion depth) are refused by the C++ reader."""
    def write(name, header: bytes, data: bytes = b"\0" * 16):
        header += b" " * (-len(header) % 8)
        p = str(tmp_path / name)
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", len(header)) + header + data)
        return p
    # 2^32 * 2^32 * 4 wraps to 0 in 64-bit arithmetic: the same as offsets [0, 0]
    wrap = write("wrap.safetensors", b'{"a.weight":{"dtype":"U32","shape":[4294967296,4294967296],'
                                     b'"data_offsets":[0,0]}}')
    r = subprocess.run([TOOL, "dump", wrap], capture_output=True, text=True, timeout=30)
    assert r.returncode != 0 and "shape" in r.stderr
    deep = write("deep.safetensors", b'{"__metadata__":' + b"[" * 100000 + b"]" * 100000 + b"}")
    r = subprocess.run([TOOL, "dump", deep], capture_output=True, text=True, timeout=30)
    assert r.returncode == 1 and "JSON" in r.stderr


def test_source_fingerprint(mq4):
    """The fingerprint quantize_or_load compares: equal for equal weights,
    different when any element or the shape differs."""
    from importlib import import_module
    qc = import_module(mq4.__name__ + ".q4cache")
    g = torch.Generator().manual_seed(3)
    w = torch.randn((64, 128), generator=g).to(torch.bfloat16)
    a = qc.source_fingerprint(w)
    assert a == qc.source_fingerprint(w.clone())
    w2 = w.clone()
    w2[63, 127] = w2[63, 127] + 1
    assert qc.source_fingerprint(w2) != a
    assert qc.source_fingerprint(w.reshape(128, 64)) != a
    assert a.startswith("64x128:")
