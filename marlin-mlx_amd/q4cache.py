"""On-disk cache of MLX-affine Q4 weights in the safetensors format.

The reference quantizes every MLP and lm_head weight at load time
(quantize_weight, src/model/weights.cpp:45-56, and the lm_head,
src/model/weights.cpp:180-194), about 2 s per start (RESEARCH.md, "No weight
cache").  This module stores the quantized tensors once and loads them back:
one safetensors file, three tensors per quantized matrix in MLX's naming
convention -- "<name>.weight" U32 [N, K/8] (eight nibbles per word, low nibble
first), "<name>.scales" and "<name>.biases" BF16 [N, K/64] -- so a file
written by MLX for the same group size and bit width loads unchanged.  The
group size and bit width are recorded in the file's metadata.

safetensors layout (public format): an 8-byte little-endian header length,
a JSON header mapping each tensor name to {"dtype", "shape", "data_offsets"}
(offsets relative to the data section) plus "__metadata__" (string values),
padded with spaces to a multiple of 8 bytes, then the raw little-endian
tensor bytes.  Only local paths are read or written.
"""
from __future__ import annotations

import json
import os
import struct

import torch

_DT = {"U32": (torch.int32, 4), "BF16": (torch.bfloat16, 2)}


def _tensor_bytes(t: torch.Tensor) -> bytes:
    return t.detach().contiguous().cpu().view(torch.uint8).numpy().tobytes()


def write_safetensors(path: str, tensors: list[tuple[str, str, list[int], bytes]],
                      metadata: dict[str, str] | None = None) -> None:
    """Write (name, dtype, shape, raw bytes) entries to a safetensors file."""
    header: dict = {}
    if metadata:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    offset = 0
    for name, dtype, shape, raw in tensors:
        if dtype not in _DT:
            raise ValueError(f"write_safetensors: unsupported dtype {dtype}")
        n = 1
        for d in shape:
            n *= int(d)
        if n * _DT[dtype][1] != len(raw):
            raise ValueError(f"write_safetensors: {name}: {len(raw)} bytes for shape {shape} of {dtype}")
        header[name] = {"dtype": dtype, "shape": [int(d) for d in shape], "data_offsets": [offset, offset + len(raw)]}
        offset += len(raw)
    hb = json.dumps(header, separators=(",", ":")).encode("utf-8")
    hb += b" " * (-len(hb) % 8)
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for _, _, _, raw in tensors:
            f.write(raw)
    os.replace(tmp, path)


def read_safetensors(path: str):
    """(header dict, data bytes) of a safetensors file; validates the offsets."""
    with open(path, "rb") as f:
        raw = f.read()
    if len(raw) < 8:
        raise ValueError(f"{path}: not a safetensors file")
    (n,) = struct.unpack("<Q", raw[:8])
    if 8 + n > len(raw):
        raise ValueError(f"{path}: header length {n} exceeds the file")
    header = json.loads(raw[8:8 + n].decode("utf-8"))
    data = memoryview(raw)[8 + n:]
    for name, e in header.items():
        if name == "__metadata__":
            continue
        b, t = e["data_offsets"]
        if not (0 <= b <= t <= len(data)):
            raise ValueError(f"{path}: {name}: data offsets {b}..{t} outside the data section")
    return header, data


def source_fingerprint(w: torch.Tensor) -> str:
    """Shape and an exact integer checksum of a bf16 weight, computed where
    the tensor lives: sum over i of bits_i * (i mod 65521 + 1) mod 2^64,
    with bits_i the 16-bit pattern of element i.  It tells a cache written
    for these source weights from one written for another checkpoint."""
    flat = w.detach().contiguous().view(-1).view(torch.int16)
    acc = 0
    step = 1 << 24
    for o in range(0, flat.numel(), step):
        v = flat[o:o + step].to(torch.int64) & 0xFFFF
        k = torch.arange(o, o + v.numel(), device=v.device, dtype=torch.int64) % 65521 + 1
        acc = (acc + int((v * k).sum().item())) & 0xFFFFFFFFFFFFFFFF
    return "x".join(str(int(d)) for d in w.shape) + f":{acc:016x}"


def save_q4_cache(path: str, tensors: dict, group_size: int = 64, bits: int = 4,
                  sources: dict | None = None) -> None:
    """Write {name: QuantizedTensor} as name.weight / .scales / .biases; with
    sources ({name: fingerprint string}) each matrix's source fingerprint is
    recorded in the metadata as "source.<name>"."""
    entries = []
    for name, q in tensors.items():
        if not q.quantized or q.group_size != group_size or q.bits != bits:
            raise ValueError(f"save_q4_cache: {name} is not a group-{group_size}, {bits}-bit quantized tensor")
        entries.append((name + ".weight", "U32", list(q.weight.shape), _tensor_bytes(q.weight)))
        entries.append((name + ".scales", "BF16", list(q.scales.shape), _tensor_bytes(q.scales)))
        entries.append((name + ".biases", "BF16", list(q.biases.shape), _tensor_bytes(q.biases)))
    meta = {"format": "mlx", "quantization.group_size": str(group_size), "quantization.bits": str(bits)}
    for name, fp in (sources or {}).items():
        meta["source." + name] = fp
    write_safetensors(path, entries, meta)


def load_q4_cache(path: str, device="cuda", group_size: int | None = None, bits: int | None = None) -> dict:
    """Read every name.weight / .scales / .biases triple of a safetensors file
    into {name: QuantizedTensor} on `device`, checking dtypes and shapes (the
    group size and bit width come from the metadata unless given)."""
    from . import QuantizedTensor
    header, data = read_safetensors(path)
    meta = header.get("__metadata__", {}) or {}
    gs = group_size if group_size is not None else int(meta.get("quantization.group_size", 64))
    bt = bits if bits is not None else int(meta.get("quantization.bits", 4))
    if gs != 64 or bt != 4:
        # MLX also writes other group sizes and bit widths; this library's
        # kernels read only the group-64, 4-bit layout
        raise NotImplementedError(f"load_q4_cache: {path} holds group_size={gs}, bits={bt}; "
                                  f"only group_size=64, bits=4 is implemented")
    names = sorted(k[:-len(".weight")] for k in header if k.endswith(".weight")
                   and k[:-len(".weight")] + ".scales" in header)

    def tensor(key, dtype):
        e = header[key]
        if e["dtype"] != dtype:
            raise ValueError(f"load_q4_cache: {key} is {e['dtype']}, expected {dtype}")
        b, t = e["data_offsets"]
        tdt, _ = _DT[dtype]
        buf = torch.frombuffer(bytearray(data[b:t]), dtype=torch.uint8)
        return buf.view(tdt).reshape(e["shape"]).to(device)

    out = {}
    for name in names:
        wq = tensor(name + ".weight", "U32")
        s = tensor(name + ".scales", "BF16")
        b = tensor(name + ".biases", "BF16")
        if wq.dim() != 2 or s.shape != b.shape or s.dim() != 2 or s.shape[0] != wq.shape[0]:
            raise ValueError(f"load_q4_cache: {name}: inconsistent shapes {tuple(wq.shape)} / {tuple(s.shape)}")
        K = wq.shape[1] * 32 // bt
        if K % gs != 0 or s.shape[1] != K // gs:
            raise ValueError(f"load_q4_cache: {name}: scales {tuple(s.shape)} do not match K={K}, group {gs}")
        out[name] = QuantizedTensor(wq, s, b, gs, bt, True)
    return out


def quantize_or_load(path: str, weights: dict, device="cuda") -> dict:
    """The load-time step of the reference (quantize each bf16 weight) with a
    cache: if `path` exists, holds every name with the weight's shape and was
    written from these very weights (the source fingerprints recorded at
    save time match), load it; otherwise quantize the given bf16 [N, K]
    tensors (one batched quantize) and write the cache.  A cache left by
    another checkpoint or model is therefore never used silently."""
    from . import quantize_weights
    names = list(weights)
    fps = {n: source_fingerprint(weights[n]) for n in names}
    if os.path.exists(path):
        header, _ = read_safetensors(path)
        meta = header.get("__metadata__", {}) or {}
        if all(meta.get("source." + n) == fps[n] for n in names):
            cached = load_q4_cache(path, device)
            if all(n in cached and (cached[n].out_features, cached[n].in_features) == tuple(weights[n].shape)
                   for n in names):
                return {n: cached[n] for n in names}
    out = dict(zip(names, quantize_weights([weights[n] for n in names])))
    save_q4_cache(path, out, sources=fps)
    return out
