"""marlin-mlx_amd: MI355X-native MLX-affine Q4 matrix products for marlin-mlx.

Python mirror of the reference's interface for the quantized path, over the
C ABI of libmq4.so (include/mq4.h).  torch provides device memory and the
current HIP stream only; every byte of arithmetic runs in the gfx950 kernels of
libmq4.so.  If that library is missing the import fails (there is no fallback).

Reference seams mirrored (paths relative to the marlin-mlx repository):
  QuantizedTensor        src/core/types.h:75-82
  quantize_weight        src/model/weights.cpp:45-56 (and :180-194 for lm_head)
  qmatmul                src/model/marlin.cpp:18-25
  swiglu                 src/model/marlin.cpp:27-29
  mlp_forward            src/model/marlin.cpp:31-35
  lm_head                src/model/marlin.cpp:161-169
  sample_token           src/sampling/sampler.cpp:9-39
and the MLX ops they call: quantize, dequantize, quantized_matmul, argmax.

Tensor conventions: bf16 tensors are torch.bfloat16; packed weights are
torch.int32 holding the uint32 words of MLX's layout; indices are torch.int32.
"""
from __future__ import annotations

import ctypes
import itertools
import os
from dataclasses import dataclass

import torch

__all__ = [
    "MQ4Error", "library_path", "lib", "QuantizedTensor", "MLPWeights",
    "quantize", "dequantize", "quantized_matmul", "quantized_matmul_f32", "argmax", "swiglu",
    "quantize_weight", "quantize_batch", "quantize_weights", "qmatmul", "mlp_gate_up_silu", "qmatmul_residual", "mlp_forward",
    "mlp_residual",
    "lm_head", "lm_head_argmax", "lm_head_last_row", "sample_token", "rms_norm", "fill_normal_bf16",
    "DecoderLayer", "DecodeStep", "BatchedMlpLayers", "save_q4_cache", "load_q4_cache", "quantize_or_load",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmq4.so")
_lib = None

GROUP_SIZE = 64
BITS = 4

# Stream ids of the synthetic-input generator (SplitMix64 seed ^ stream id).
SEED = 0x4D41524C  # "MARL"
GEMM_MIN_M = 33     # rows from which the C entry points take the MFMA GEMM (mq4_gemm.h kGemmMinM)


def stream_id_layer(layer: int, proj: int) -> int:
    """gate=0, up=1, down=2 of layer `layer`."""
    return 1000 + 3 * layer + proj


STREAM_LM_HEAD = 2000
STREAM_NORM_WEIGHT = 2001          # final norm (src/model/marlin.cpp:145)


def stream_id_layer_norm(layer: int) -> int:
    """post-attention norm of layer `layer` (src/model/marlin.cpp:141)."""
    return 2100 + layer



def stream_id_decode_row(m: int) -> int:
    return 3000 + m


STREAM_PREFILL = 4000


class MQ4Error(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"libmq4 error {code}: {message}")
        self.code = code


def library_path() -> str:
    return _LIB_PATH


def lib():
    """The loaded libmq4.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(
            f"{_LIB_PATH} is missing: build it with `python marlin-mlx_amd/build.py` "
            "(there is no non-HIP fallback)")
    L = ctypes.CDLL(_LIB_PATH)
    P, I64, I, SZ, U64, D = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t,
                             ctypes.c_uint64, ctypes.c_double)
    sig = {
        "mq4_last_error": ([], ctypes.c_char_p),
        "mq4_version": ([], I),
        "mq4_quantize": ([P, I64, I64, I, I, P, P, P, P], I),
        "mq4_quantize_batch": ([P, I64, I, I, P], I),
        "mq4_dequantize": ([P, P, P, I64, I64, I, I, P, I, P], I),
        "mq4_qmm": ([P, I64, I64, P, P, P, I64, I, I, I, P, P], I),
        "mq4_qmm_residual": ([P, I64, I64, P, P, P, I64, P, P, P], I),
        "mq4_qmm_f32": ([P, I64, I64, P, P, P, I64, P, P], I),
        "mq4_mlp_gate_up_silu": ([P, I64, I64, P, P, P, P, P, P, I64, P, P], I),
        "mq4_rmsnorm_gate_up_silu": ([P, I64, I64, P, ctypes.c_float, P, P, P, P, P, P, I64, P, P], I),
        "mq4_mlp_workspace_size": ([I64, I64, I64], ctypes.c_size_t),
        "mq4_mlp_residual": ([P, I64, I64, P, ctypes.c_float] + [P] * 9 + [I64, P, ctypes.c_size_t, P, P], I),
        "mq4_rmsnorm_lm_head_argmax": ([P, I64, I64, P, ctypes.c_float, P, P, P, I64, P, P, P, SZ, P], I),
        "mq4_swiglu_bf16": ([P, P, I64, P, P], I),
        "mq4_lm_head_argmax_workspace_size": ([I64, I64], SZ),
        "mq4_lm_head_argmax": ([P, I64, I64, P, P, P, I64, P, P, P, SZ, P], I),
        "mq4_lm_head_argmax_noalloc": ([P, I64, I64, P, P, P, I64, P, P, P], I),
        "mq4_argmax_workspace_size": ([I64, I64], SZ),
        "mq4_argmax_bf16": ([P, I64, I64, P, P, SZ, P], I),
        "mq4_sample_workspace_size": ([I64, I64], SZ),
        "mq4_sample_bf16": ([P, I64, I64, ctypes.c_float, I, ctypes.c_float, U64, P, P, P, SZ, P], I),
        "mq4_fill_normal_bf16": ([P, I64, U64, U64, D, D, I64, P], I),
        "mq4_rms_norm": ([P, I64, I64, P, ctypes.c_float, P, P], I),
        "mq4_decode_workspace_size": ([I64, I64, I64], SZ),
        "mq4_decode_step": ([P, I64, I64, I64, P, P, ctypes.c_float, P, P, P, I64, P, P, P, SZ, P], I),
        "mq4_mlp_layers_workspace_size": ([I64, I64, I64], SZ),
        "mq4_mlp_layers": ([P, I64, I64, I64, I64, P, ctypes.c_float, P, P, SZ, P], I),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != 0:
        raise MQ4Error(rc, lib().mq4_last_error().decode())


def _stream(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: torch.Tensor | None):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _need(t: torch.Tensor, dtype, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    return t.contiguous()


def _check_weight(fn: str, wq: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, K: int,
                  group_size: int = GROUP_SIZE, bits: int = BITS) -> int:
    """Shapes and dtypes of one MLX-layout quantized matrix against an input
    of K features (what mx::quantized_matmul validates): wq int32 [N, K*bits/32],
    scales and biases bf16 [N, K/group_size].  Returns N.  Checked before any
    pointer reaches the C ABI, which only sees raw addresses."""
    for t, name in ((wq, "weight"), (scales, "scales"), (biases, "biases")):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{fn}: {name} must be a torch.Tensor")
    if wq.dtype != torch.int32:
        raise TypeError(f"{fn}: packed weight must be int32 (uint32 words), got {wq.dtype}")
    if scales.dtype != torch.bfloat16 or biases.dtype != torch.bfloat16:
        raise TypeError(f"{fn}: scales and biases must be bfloat16")
    if wq.dim() != 2:
        raise ValueError(f"{fn}: packed weight must be 2-D [N, K/8], got shape {tuple(wq.shape)}")
    if group_size != GROUP_SIZE or bits != BITS:
        # the kernels are built for MLX's group-64, 4-bit layout only; another
        # format's scales/biases/words would be read past their ends
        raise NotImplementedError(f"{fn}: only group_size={GROUP_SIZE}, bits={BITS} is implemented "
                                  f"(got group_size={group_size}, bits={bits})")
    if K % group_size != 0 or (K * bits) % 32 != 0:
        raise ValueError(f"{fn}: K={K} is not a multiple of group_size={group_size}")
    N = wq.shape[0]
    if wq.shape[1] != K * bits // 32:
        raise ValueError(f"{fn}: input has K={K} features but the weight holds "
                         f"{wq.shape[1] * 32 // bits} (shape {tuple(wq.shape)})")
    want = (N, K // group_size)
    if tuple(scales.shape) != want or tuple(biases.shape) != want:
        raise ValueError(f"{fn}: scales/biases must be {want}, got {tuple(scales.shape)} and "
                         f"{tuple(biases.shape)}")
    return N


def _check_vector(fn: str, t: torch.Tensor, n: int, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{fn}: {name} must be a torch.Tensor")
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{fn}: {name} must be bfloat16")
    if t.numel() != n:
        raise ValueError(f"{fn}: {name} must hold {n} values, got {t.numel()}")


def _in_features(fn: str, x: torch.Tensor) -> int:
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{fn}: input must be a torch.Tensor")
    if x.dim() == 0 or x.shape[-1] == 0:
        raise ValueError(f"{fn}: input must have a non-empty last dimension")
    return x.shape[-1]


# ----------------------------------------------------------------- ops ---

def quantize(w: torch.Tensor, group_size: int = 64, bits: int = 4):
    """mx::quantize(w, group_size, bits) for bf16 w [..., K]: returns
    (wq int32 [..., K/8], scales bf16 [..., K/64], biases bf16 [..., K/64])."""
    w = _need(w, torch.bfloat16, "w")
    K = w.shape[-1]
    N = w.numel() // K if K else 0
    lead = w.shape[:-1]
    wq = torch.empty((*lead, K // 8), dtype=torch.int32, device=w.device)
    s = torch.empty((*lead, K // max(group_size, 1)), dtype=torch.bfloat16, device=w.device)
    b = torch.empty_like(s)
    _check(lib().mq4_quantize(_ptr(w), N, K, group_size, bits, _ptr(wq), _ptr(s), _ptr(b),
                              _stream(w.device)))
    return wq, s, b


class _QuantJobC(ctypes.Structure):
    """mq4_quantize_job (include/mq4.h)."""
    _fields_ = [("w", ctypes.c_void_p), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
                ("wq", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("biases", ctypes.c_void_p)]


def quantize_batch(ws, group_size: int = 64, bits: int = 4):
    """mx::quantize over a whole weight set in one batched call: the loader's
    loop of quantize_weight calls (src/model/weights.cpp:97-104, 147-160) plus
    the lm_head's (:180-194).  ws: bf16 tensors [..., K] on one device (K may
    differ between them).  Returns a list of (wq, scales, biases), bit for bit
    what quantize() returns for each."""
    fn = "quantize_batch"
    ws = list(ws)
    if not ws:
        return []
    dev = ws[0].device
    jobs = (_QuantJobC * len(ws))()
    outs = []
    for i, w in enumerate(ws):
        w = _need(w, torch.bfloat16, f"ws[{i}]")
        if w.device != dev:
            raise ValueError(f"{fn}: every weight must be on {dev} (ws[{i}] is on {w.device})")
        K = w.shape[-1]
        lead = w.shape[:-1]
        wq = torch.empty((*lead, K // 8), dtype=torch.int32, device=dev)
        s = torch.empty((*lead, K // max(group_size, 1)), dtype=torch.bfloat16, device=dev)
        b = torch.empty_like(s)
        jobs[i] = _QuantJobC(_ptr(w), w.numel() // K if K else 0, K, _ptr(wq), _ptr(s), _ptr(b))
        outs.append((w, wq, s, b))
    _check(lib().mq4_quantize_batch(ctypes.cast(jobs, ctypes.c_void_p), len(ws), group_size, bits, _stream(dev)))
    return [(wq, s, b) for (_, wq, s, b) in outs]


def quantize_weights(ws, bits: int = 4, group_size: int = 64) -> list:
    """quantize_weight (src/model/weights.cpp:45-56) for a list of bf16 [N, K]
    weights in one batched call; returns QuantizedTensors."""
    return [QuantizedTensor(wq, s, b, group_size, bits, True) for wq, s, b in quantize_batch(ws, group_size, bits)]


def dequantize(wq: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               group_size: int = 64, bits: int = 4, dtype=torch.bfloat16) -> torch.Tensor:
    wq = _need(wq, torch.int32, "wq")
    scales = _need(scales, torch.bfloat16, "scales")
    biases = _need(biases, torch.bfloat16, "biases")
    K = wq.shape[-1] * 8
    N = wq.numel() * 8 // K
    if dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("dequantize: dtype must be bfloat16 or float32")
    out = torch.empty((*wq.shape[:-1], K), dtype=dtype, device=wq.device)
    _check(lib().mq4_dequantize(_ptr(wq), _ptr(scales), _ptr(biases), N, K, group_size, bits,
                                _ptr(out), int(dtype == torch.float32), _stream(wq.device)))
    return out


def _mk(x: torch.Tensor, N: int):
    K = x.shape[-1]
    M = x.numel() // K
    y = torch.empty((*x.shape[:-1], N), dtype=torch.bfloat16, device=x.device)
    return M, K, y


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                     transpose: bool = True, group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """mx::quantized_matmul(x, w, scales, biases, transpose, group_size, bits):
    x bf16 [..., K] @ dequant(w [N, K/8])^T -> bf16 [..., N]."""
    N = _check_weight("quantized_matmul", w, scales, biases, _in_features("quantized_matmul", x),
                      group_size, bits)
    x = _need(x, torch.bfloat16, "x")
    w = _need(w, torch.int32, "w")
    scales = _need(scales, torch.bfloat16, "scales")
    biases = _need(biases, torch.bfloat16, "biases")
    M, K, y = _mk(x, N)
    if M == 0:                      # no rows: an empty result, as mx::quantized_matmul gives
        return y
    _check(lib().mq4_qmm(_ptr(x), M, K, _ptr(w), _ptr(scales), _ptr(biases), N, int(transpose),
                         group_size, bits, _ptr(y), _stream(x.device)))
    return y


def quantized_matmul_f32(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                         biases: torch.Tensor) -> torch.Tensor:
    """quantized_matmul with the fp32 accumulator returned unrounded (float32)."""
    N = _check_weight("quantized_matmul_f32", w, scales, biases, _in_features("quantized_matmul_f32", x))
    x = _need(x, torch.bfloat16, "x")
    w = _need(w, torch.int32, "w")
    scales = _need(scales, torch.bfloat16, "scales")
    biases = _need(biases, torch.bfloat16, "biases")
    K = x.shape[-1]
    M = x.numel() // K
    y = torch.empty((*x.shape[:-1], N), dtype=torch.float32, device=x.device)
    if M == 0:
        return y
    _check(lib().mq4_qmm_f32(_ptr(x), M, K, _ptr(w), _ptr(scales), _ptr(biases), N, _ptr(y),
                             _stream(x.device)))
    return y


def argmax(logits: torch.Tensor, axis: int = -1) -> torch.Tensor:
    """mx::argmax(logits, -1) over bf16 logits: lowest index wins ties."""
    if axis not in (-1, logits.dim() - 1):
        raise NotImplementedError("argmax: only the last axis is supported")
    logits = _need(logits, torch.bfloat16, "logits")
    N = logits.shape[-1]
    M = logits.numel() // N
    idx = torch.empty(logits.shape[:-1], dtype=torch.int32, device=logits.device)
    if M == 0:
        return idx
    L = lib()
    ws_bytes = L.mq4_argmax_workspace_size(M, N)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=logits.device)
    _check(L.mq4_argmax_bf16(_ptr(logits), M, N, _ptr(idx), _ptr(ws), ws_bytes,
                             _stream(logits.device)))
    return idx


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """(sigmoid(gate) * gate) * up with a bf16 result after each op
    (src/model/marlin.cpp:27-29)."""
    gate = _need(gate, torch.bfloat16, "gate")
    up = _need(up, torch.bfloat16, "up")
    if gate.shape != up.shape:
        raise ValueError("swiglu: gate and up shapes differ")
    out = torch.empty_like(gate)
    _check(lib().mq4_swiglu_bf16(_ptr(gate), _ptr(up), gate.numel(), _ptr(out),
                                 _stream(gate.device)))
    return out


# ------------------------------------------------- reference interface ---

@dataclass
class QuantizedTensor:
    """src/core/types.h:75-82: weight (packed uint32 words as int32), scales,
    biases (bf16), group_size=64, bits=4, quantized."""
    weight: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor
    group_size: int = 64
    bits: int = 4
    quantized: bool = True

    @property
    def out_features(self) -> int:
        return self.weight.shape[0]

    @property
    def in_features(self) -> int:
        return self.weight.shape[-1] * 32 // self.bits if self.quantized else self.weight.shape[-1]


@dataclass
class MLPWeights:
    """src/model/marlin.h:17-21."""
    gate_proj: QuantizedTensor
    up_proj: QuantizedTensor
    down_proj: QuantizedTensor


def quantize_weight(w: torch.Tensor, bits: int = 4, group_size: int = 64) -> QuantizedTensor:
    """src/model/weights.cpp:45-56: quantize a bf16 [N, K] weight."""
    wq, s, b = quantize(w, group_size, bits)
    return QuantizedTensor(wq, s, b, group_size, bits, True)


def _require_quantized(w: QuantizedTensor, fn: str) -> None:
    if not w.quantized:
        raise NotImplementedError(
            f"{fn}: unquantized (bf16 dense) weights are outside this library's path")


def qmatmul(x: torch.Tensor, w: QuantizedTensor) -> torch.Tensor:
    """src/model/marlin.cpp:18-25 (quantized branch)."""
    _require_quantized(w, "qmatmul")
    return quantized_matmul(x, w.weight, w.scales, w.biases, True, w.group_size, w.bits)


def mlp_gate_up_silu(x: torch.Tensor, gate: QuantizedTensor, up: QuantizedTensor,
                     norm_weight: torch.Tensor | None = None, eps: float = 1e-6) -> torch.Tensor:
    """swiglu(qmatmul(x, gate), qmatmul(x, up)) in one pass over both weights;
    with norm_weight, x is first rms_norm'ed with the (1 + w) multiplier
    (src/model/marlin.cpp:141): inside the same kernel for decode-sized M,
    and as the separate norm kernel into a temporary followed by the GEMM from
    33 rows on (the prefill GEMM with the norm fused re-reads each row block
    for its norm statistics; the two launches are faster and give the same
    normalized operand)."""
    fn = "mlp_gate_up_silu"
    _require_quantized(gate, fn)
    _require_quantized(up, fn)
    Kx = _in_features(fn, x)
    N = _check_weight(fn, gate.weight, gate.scales, gate.biases, Kx, gate.group_size, gate.bits)
    if _check_weight(fn, up.weight, up.scales, up.biases, Kx, up.group_size, up.bits) != N:
        raise ValueError(f"{fn}: gate and up must have the same shape")
    if norm_weight is not None:
        _check_vector(fn, norm_weight, Kx, "norm_weight")
    x = _need(x, torch.bfloat16, "x")
    M, K, h = _mk(x, N)
    if M == 0:
        return h
    g = (_ptr(gate.weight), _ptr(gate.scales), _ptr(gate.biases))
    u = (_ptr(up.weight), _ptr(up.scales), _ptr(up.biases))
    if norm_weight is None:
        _check(lib().mq4_mlp_gate_up_silu(_ptr(x), M, K, *g, *u, N, _ptr(h), _stream(x.device)))
    elif M >= GEMM_MIN_M:
        n = rms_norm(x, norm_weight, eps)
        _check(lib().mq4_mlp_gate_up_silu(_ptr(n), M, K, *g, *u, N, _ptr(h), _stream(x.device)))
    else:
        norm_weight = _need(norm_weight, torch.bfloat16, "norm_weight")
        _check(lib().mq4_rmsnorm_gate_up_silu(_ptr(x), M, K, _ptr(norm_weight), eps, *g, *u, N, _ptr(h),
                                              _stream(x.device)))
    return h


def qmatmul_residual(x: torch.Tensor, w: QuantizedTensor, residual: torch.Tensor,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """residual + qmatmul(x, w) with bf16 rounding of both (src/model/marlin.cpp:142);
    out may be residual itself (in-place)."""
    fn = "qmatmul_residual"
    _require_quantized(w, fn)
    N = _check_weight(fn, w.weight, w.scales, w.biases, _in_features(fn, x), w.group_size, w.bits)
    K = x.shape[-1]
    M = x.numel() // K
    if not isinstance(residual, torch.Tensor) or residual.numel() != M * N:
        raise ValueError(f"{fn}: residual must hold M*N = {M * N} values")
    if out is not None and (not isinstance(out, torch.Tensor) or out.dtype != torch.bfloat16
                            or out.numel() != M * N or not out.is_contiguous()):
        raise ValueError(f"{fn}: out must be a contiguous bf16 tensor of M*N = {M * N} values")
    x = _need(x, torch.bfloat16, "x")
    residual = _need(residual, torch.bfloat16, "residual")
    y = out if out is not None else torch.empty_like(residual)
    if M == 0:
        return y
    _check(lib().mq4_qmm_residual(_ptr(x), M, K, _ptr(w.weight), _ptr(w.scales), _ptr(w.biases), N,
                                  _ptr(residual), _ptr(y), _stream(x.device)))
    return y


def mlp_forward(x: torch.Tensor, w: MLPWeights, residual: torch.Tensor | None = None,
                norm_weight: torch.Tensor | None = None, eps: float = 1e-6) -> torch.Tensor:
    """src/model/marlin.cpp:31-35 (down(swiglu(gate x, up x))); with `residual`
    also the add of src/model/marlin.cpp:142, with `norm_weight` the rms_norm
    of src/model/marlin.cpp:141 in front.  With both and residual is x (the
    block's hidden state, :141-142), one mq4_mlp_residual call."""
    if residual is not None and norm_weight is not None and residual is x:
        return mlp_residual(x, w, norm_weight, eps)
    h = mlp_gate_up_silu(x, w.gate_proj, w.up_proj, norm_weight, eps)
    if residual is None:
        return qmatmul(h, w.down_proj)
    return qmatmul_residual(h, w.down_proj, residual)


def mlp_residual(x: torch.Tensor, w: MLPWeights, norm_weight: torch.Tensor, eps: float = 1e-6,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """x + mlp_forward(rms_norm(x, norm_weight)) (src/model/marlin.cpp:141-142,
    31-35) in one mq4_mlp_residual call; out may be x (in place)."""
    fn = "mlp_residual"
    for q in (w.gate_proj, w.up_proj, w.down_proj):
        _require_quantized(q, fn)
    Kx = _in_features(fn, x)
    N = _check_weight(fn, w.gate_proj.weight, w.gate_proj.scales, w.gate_proj.biases, Kx, w.gate_proj.group_size,
                      w.gate_proj.bits)
    if _check_weight(fn, w.up_proj.weight, w.up_proj.scales, w.up_proj.biases, Kx, w.up_proj.group_size,
                     w.up_proj.bits) != N:
        raise ValueError(f"{fn}: gate and up have different output sizes")
    if _check_weight(fn, w.down_proj.weight, w.down_proj.scales, w.down_proj.biases, N, w.down_proj.group_size,
                     w.down_proj.bits) != Kx:
        raise ValueError(f"{fn}: down_proj must map {N} back to {Kx} features")
    _check_vector(fn, norm_weight, Kx, "norm_weight")
    norm_weight = _need(norm_weight, torch.bfloat16, "norm_weight")
    x = _need(x, torch.bfloat16, "x")
    K = x.shape[-1]
    M = x.numel() // K
    y = torch.empty_like(x) if out is None else _need(out, torch.bfloat16, "out")
    if y.shape != x.shape:
        raise ValueError(f"{fn}: out has shape {tuple(y.shape)}, x {tuple(x.shape)}")
    if M == 0:
        return y
    L = lib()
    ws_bytes = L.mq4_mlp_workspace_size(M, K, N)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    qa = lambda q: (_ptr(q.weight), _ptr(q.scales), _ptr(q.biases))
    _check(L.mq4_mlp_residual(_ptr(x), M, K, _ptr(norm_weight), eps, *qa(w.gate_proj), *qa(w.up_proj),
                              *qa(w.down_proj), N, _ptr(ws), ws_bytes, _ptr(y), _stream(x.device)))
    return y


def lm_head(hidden: torch.Tensor, w: QuantizedTensor) -> torch.Tensor:
    """src/model/marlin.cpp:161-169 (quantized branch): bf16 logits."""
    return qmatmul(hidden, w)


def lm_head_argmax(hidden: torch.Tensor, w: QuantizedTensor, return_logits: bool = False,
                   norm_weight: torch.Tensor | None = None, eps: float = 1e-6):
    """Greedy next token of every row of `hidden`: argmax of the bf16 logits,
    fused with the lm_head product (marlin.cpp:161-169 + sampler.cpp:14-16);
    with norm_weight also the final rms_norm (marlin.cpp:145) in front."""
    fn = "lm_head_argmax"
    _require_quantized(w, fn)
    Kx = _in_features(fn, hidden)
    N = _check_weight(fn, w.weight, w.scales, w.biases, Kx, w.group_size, w.bits)
    if norm_weight is not None:
        _check_vector(fn, norm_weight, Kx, "norm_weight")
    hidden = _need(hidden, torch.bfloat16, "hidden")
    K = hidden.shape[-1]
    M = hidden.numel() // K
    idx = torch.empty(hidden.shape[:-1], dtype=torch.int32, device=hidden.device)
    logits = (torch.empty((*hidden.shape[:-1], N), dtype=torch.bfloat16, device=hidden.device)
              if return_logits else None)
    if M == 0:
        return (idx, logits) if return_logits else idx
    L = lib()
    ws_bytes = L.mq4_lm_head_argmax_workspace_size(M, N)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=hidden.device)
    wargs = (_ptr(w.weight), _ptr(w.scales), _ptr(w.biases), N, _ptr(idx), _ptr(logits), _ptr(ws), ws_bytes,
             _stream(hidden.device))
    if norm_weight is None:
        _check(L.mq4_lm_head_argmax(_ptr(hidden), M, K, *wargs))
    else:
        norm_weight = _need(norm_weight, torch.bfloat16, "norm_weight")
        _check(L.mq4_rmsnorm_lm_head_argmax(_ptr(hidden), M, K, _ptr(norm_weight), eps, *wargs))
    return (idx, logits) if return_logits else idx


def lm_head_last_row(hidden: torch.Tensor, w: QuantizedTensor, norm_weight: torch.Tensor | None = None,
                     eps: float = 1e-6, return_logits: bool = False):
    """Greedy next token after a prompt: the reference runs the lm_head over
    all S rows of the prefill hidden state (src/core/engine.cpp:64) and
    sample_token then keeps the last row (src/sampling/sampler.cpp:10-12);
    here only that row goes through the (fused norm +) lm_head + argmax.
    hidden: [S, K] or [1, S, K]; returns the int32 token [1] (and the last
    row's bf16 logits [1, N] with return_logits)."""
    fn = "lm_head_last_row"
    if not isinstance(hidden, torch.Tensor) or hidden.dim() not in (2, 3) or (hidden.dim() == 3 and hidden.shape[0] != 1):
        raise ValueError(f"{fn}: hidden must be [S, K] or [1, S, K]")
    last = hidden.reshape(-1, hidden.shape[-1])[-1:]
    return lm_head_argmax(last.contiguous(), w, return_logits=return_logits, norm_weight=norm_weight, eps=eps)


_sample_calls = itertools.count()
_proc_seed: list[int] = []


def _process_seed() -> int:
    """A 64-bit seed drawn once per process from the OS: like MLX's global
    random key, which is seeded from the clock, every process draws a
    different sequence."""
    if not _proc_seed:
        _proc_seed.append(int.from_bytes(os.urandom(8), "little"))
    return _proc_seed[0]


def sample_token(logits: torch.Tensor, temperature: float = 0.0, top_k: int = 0, top_p: float = 1.0,
                 seed: int | None = None, return_keep: bool = False):
    """sample_token (src/sampling/sampler.cpp:9-39) on the GPU, one kernel.

    logits: bf16 [1, S, V] (the last position is sampled, as the reference
    slices it) or [M, V] (every row is sampled).  temperature <= 0 is the
    greedy argmax; otherwise scaled = logits / temperature, top_k > 0 masks
    everything below the k-th largest value, 0 < top_p < 1 applies the
    reference's ascending-order mass mask (an element is masked when the
    probability mass of the smaller elements before it exceeds top_p), and
    the token is drawn from softmax(scaled) over the unmasked elements.
    seed: the draw is a pure function of (logits, parameters, seed, row);
    None takes a per-process random base (drawn once from the OS) plus a
    per-process call counter, so successive calls and separate processes
    draw independently, as the reference's clock-seeded global random key
    does.
    Returns int64 [M] (and the uint8 [M, V] keep mask with return_keep,
    None for the greedy case)."""
    fn = "sample_token"
    if not isinstance(logits, torch.Tensor) or logits.dim() not in (2, 3):
        raise ValueError(f"{fn}: logits must be [1, S, V] or [M, V]")
    if logits.dim() == 3:
        if logits.shape[0] != 1:
            raise ValueError(f"{fn}: [B, S, V] logits need B == 1 (got {tuple(logits.shape)})")
        logits = logits[0, -1:, :]
    if int(top_k) < 0:
        raise ValueError(f"{fn}: top_k must be >= 0")
    rows = _need(logits, torch.bfloat16, "logits").contiguous()
    M, V = rows.shape
    if seed is None:
        seed = (_process_seed() + next(_sample_calls)) & 0xFFFFFFFFFFFFFFFF
    idx = torch.empty(M, dtype=torch.int32, device=rows.device)
    keep = None
    if return_keep and temperature > 0.0:
        keep = torch.empty((M, V), dtype=torch.uint8, device=rows.device)
    L = lib()
    ws_bytes = L.mq4_sample_workspace_size(M, V)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=rows.device) if ws_bytes else None
    _check(L.mq4_sample_bf16(_ptr(rows), M, V, float(temperature), int(top_k), float(top_p),
                             int(seed) & 0xFFFFFFFFFFFFFFFF, _ptr(idx), _ptr(keep), _ptr(ws), ws_bytes,
                             _stream(rows.device)))
    out = idx.to(torch.int64)
    return (out, keep) if return_keep else out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """src/model/marlin.cpp:12-16: x * rsqrt(mean(x^2) + eps) * (1 + weight)."""
    _check_vector("rms_norm", weight, _in_features("rms_norm", x), "weight")
    x = _need(x, torch.bfloat16, "x")
    weight = _need(weight, torch.bfloat16, "weight")
    K = x.shape[-1]
    out = torch.empty_like(x)
    if out.numel() == 0:
        return out
    _check(lib().mq4_rms_norm(_ptr(x), x.numel() // K, K, _ptr(weight), eps, _ptr(out),
                              _stream(x.device)))
    return out


def fill_normal_bf16(shape, stream_id: int, mu: float = 0.0, sigma: float = 1.0,
                     device="cuda", seed: int = SEED, offset: int = 0) -> torch.Tensor:
    """Synthetic bf16 N(mu, sigma) tensor from the counter-based generator."""
    out = torch.empty(shape, dtype=torch.bfloat16, device=device)
    _check(lib().mq4_fill_normal_bf16(_ptr(out), out.numel(), seed, stream_id, mu, sigma, offset,
                                      _stream(out.device)))
    return out


# ------------------------------------------------------ whole decode step ---

class _MlpLayerC(ctypes.Structure):
    """struct mq4_mlp_layer of include/mq4.h."""
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "norm_weight", "gate_wq", "gate_scales", "gate_biases", "up_wq", "up_scales", "up_biases",
        "down_wq", "down_scales", "down_biases")]


@dataclass
class DecoderLayer:
    """The MLP half of one decoder layer (src/model/marlin.h:17-21 and the
    post-attention norm used at src/model/marlin.cpp:141)."""
    post_attn_norm: torch.Tensor
    mlp: MLPWeights


def _layer_array(fn: str, layers: list[DecoderLayer], H: int, I: int):
    """The struct mq4_mlp_layer array of `layers`.  Every pointer handed to a
    kernel is checked first: shapes and dtypes of all layers, then device and
    contiguity."""
    for i, ly in enumerate(layers):
        m = ly.mlp
        for w, k, n, name in ((m.gate_proj, H, I, "gate_proj"), (m.up_proj, H, I, "up_proj"),
                              (m.down_proj, I, H, "down_proj")):
            _require_quantized(w, fn)
            if _check_weight(f"{fn} layer {i} {name}", w.weight, w.scales, w.biases, k,
                             w.group_size, w.bits) != n:
                raise ValueError(f"{fn}: layer {i} {name} must have {n} rows")
        _check_vector(f"{fn} layer {i}", ly.post_attn_norm, H, "post_attn_norm")
    arr = (_MlpLayerC * max(1, len(layers)))()
    for i, ly in enumerate(layers):
        m = ly.mlp
        tensors = [(ly.post_attn_norm, "post_attn_norm")]
        for w, name in ((m.gate_proj, "gate_proj"), (m.up_proj, "up_proj"), (m.down_proj, "down_proj")):
            tensors += [(w.weight, f"{name}.weight"), (w.scales, f"{name}.scales"), (w.biases, f"{name}.biases")]
        for t, tn in tensors:
            if not t.is_cuda or not t.is_contiguous():
                raise ValueError(f"{fn}: layer {i} {tn} must be a contiguous device tensor")
        arr[i] = _MlpLayerC(*[t.data_ptr() for t, _ in tensors])
    return arr


class DecodeStep:
    """One greedy decode step for one token in a single launch:

        for layer in layers:  x = x + mlp_forward(rms_norm(x, layer.post_attn_norm))
        token = argmax(lm_head(rms_norm(x, final_norm)))

    (the MLP half of src/model/marlin.cpp:110-145, then :145, :161-169 and
    src/sampling/sampler.cpp:14-16).  Same arithmetic as the separate
    rmsnorm+gate/up, residual-down and rmsnorm+lm_head+argmax entry points, so
    the token and hidden state are identical to chaining those.  Holds its
    workspace (zero-filled once here); calls are stream-ordered and must not
    overlap other device work.  Built for hidden 2048 / intermediate 6144."""

    def __init__(self, layers: list[DecoderLayer], final_norm: torch.Tensor, lm: QuantizedTensor,
                 eps: float = 1e-6):
        fn = "DecodeStep"
        _require_quantized(lm, fn)
        self.layers = list(layers)
        self.hidden = lm.in_features
        _check_weight(fn, lm.weight, lm.scales, lm.biases, self.hidden, lm.group_size, lm.bits)
        _check_vector(fn, final_norm, self.hidden, "final_norm")
        self.lm = lm
        self.eps = float(eps)
        self.intermediate = self.layers[0].mlp.gate_proj.out_features if self.layers else 6144
        self._arr = _layer_array(fn, self.layers, self.hidden, self.intermediate)
        self.final_norm = _need(final_norm, torch.bfloat16, "final_norm")
        for t, tn in ((lm.weight, "weight"), (lm.scales, "scales"), (lm.biases, "biases")):
            if not t.is_cuda or not t.is_contiguous():
                raise ValueError(f"{fn}: lm_head {tn} must be a contiguous device tensor")
        L = lib()
        self.ws_bytes = L.mq4_decode_workspace_size(self.hidden, self.intermediate, lm.out_features)
        self.workspace = torch.zeros(self.ws_bytes, dtype=torch.uint8, device=self.final_norm.device)

    def reset(self) -> None:
        """Zero the workspace (clears the sticky error state)."""
        self.workspace.zero_()

    def __call__(self, x: torch.Tensor, x_out: torch.Tensor | None = None,
                 idx: torch.Tensor | None = None) -> torch.Tensor:
        """x: bf16 [hidden] (or [1, hidden]); returns the int32 token tensor [1]
        (0xFFFFFFFF as int32 -1 after an internal timeout).  x_out, if given,
        receives the hidden state after the last layer."""
        x = _need(x, torch.bfloat16, "x")
        if x.numel() != self.hidden:
            raise ValueError(f"DecodeStep: x must hold {self.hidden} values (one token)")
        if idx is None:
            idx = torch.empty((1,), dtype=torch.int32, device=x.device)
        if x_out is not None and (x_out.dtype != torch.bfloat16 or x_out.numel() != self.hidden
                                  or not x_out.is_contiguous()):
            raise ValueError("DecodeStep: x_out must be a contiguous bf16 tensor of hidden values")
        lm = self.lm
        _check(lib().mq4_decode_step(_ptr(x), self.hidden, self.intermediate, len(self.layers),
                                     ctypes.cast(self._arr, ctypes.c_void_p), _ptr(self.final_norm), self.eps,
                                     _ptr(lm.weight), _ptr(lm.scales), _ptr(lm.biases), lm.out_features,
                                     _ptr(idx), _ptr(x_out), _ptr(self.workspace), self.ws_bytes,
                                     _stream(x.device)))
        return idx

    def mlp_layer(self, i: int, x: torch.Tensor, x_out: torch.Tensor) -> torch.Tensor:
        """x_out = x + mlp_forward(rms_norm(x, layers[i].post_attn_norm)) for one
        token in one launch: the MLP half that the reference's layer loop runs
        between its attention / SSM halves (src/model/marlin.cpp:141-142), so a
        caller that interleaves other work per layer keeps the one-launch
        exchange structure (mq4_decode_step with one layer and vocab 0, on
        this object's workspace).  Bit-identical to the i-th layer of the
        whole step and to the separate entry points.  x_out may not alias x."""
        fn = "DecodeStep.mlp_layer"
        if not 0 <= i < len(self.layers):
            raise IndexError(f"{fn}: layer {i} of {len(self.layers)}")
        x = _need(x, torch.bfloat16, "x")
        if x.numel() != self.hidden:
            raise ValueError(f"{fn}: x must hold {self.hidden} values (one token)")
        if (not isinstance(x_out, torch.Tensor) or x_out.dtype != torch.bfloat16 or x_out.numel() != self.hidden
                or not x_out.is_contiguous()):
            raise ValueError(f"{fn}: x_out must be a contiguous bf16 tensor of hidden values")
        if x_out.data_ptr() == x.data_ptr():
            raise ValueError(f"{fn}: x_out must not alias x (workgroups read x while others write x_out)")
        layer_ptr = ctypes.c_void_p(ctypes.addressof(self._arr) + i * ctypes.sizeof(_MlpLayerC))
        _check(lib().mq4_decode_step(_ptr(x), self.hidden, self.intermediate, 1, layer_ptr, None, self.eps,
                                     None, None, None, 0, None, _ptr(x_out), _ptr(self.workspace), self.ws_bytes,
                                     _stream(x.device)))
        return x_out


class BatchedMlpLayers:
    """The MLP halves of a stack of decoder layers for M token rows
    (1 <= M <= max_rows <= 32), one launch per layer:

        for layer in layers:  x = x + mlp_forward(rms_norm(x, layer.post_attn_norm))

    i.e. src/model/marlin.cpp:141-142 for M concurrent decode streams
    (src/core/engine.cpp:79-94), through mq4_mlp_layers.  Same per-element
    arithmetic as mlp_residual (bf16 x (128 + q) products, fp32 sums, bf16
    SwiGLU and residual) with the sums grouped differently, so results agree
    with it to fp32 rounding, not bit for bit.  Holds its workspace
    (zero-filled once here); calls are stream-ordered and must not overlap
    other device work.  Built for hidden 2048 / intermediate 6144."""

    def __init__(self, layers: list[DecoderLayer], max_rows: int = 32, eps: float = 1e-6):
        fn = "BatchedMlpLayers"
        if not layers:
            raise ValueError(f"{fn}: needs at least one layer")
        self.layers = list(layers)
        self.hidden = self.layers[0].mlp.gate_proj.in_features
        self.intermediate = self.layers[0].mlp.gate_proj.out_features
        self.eps = float(eps)
        self._arr = _layer_array(fn, self.layers, self.hidden, self.intermediate)
        L = lib()
        self.max_rows = int(max_rows)
        self.ws_bytes = L.mq4_mlp_layers_workspace_size(self.max_rows, self.hidden, self.intermediate)
        if self.ws_bytes == 0:
            raise NotImplementedError(
                f"{fn}: built for hidden 2048, intermediate 6144 and 1..32 rows "
                f"(got {self.hidden}, {self.intermediate}, max_rows {max_rows})")
        dev = self.layers[0].post_attn_norm.device
        self.workspace = torch.zeros(self.ws_bytes, dtype=torch.uint8, device=dev)

    def reset(self) -> None:
        """Zero the workspace (clears the sticky error state)."""
        self.workspace.zero_()

    def _run(self, fn: str, x: torch.Tensor, x_out, first: int, count: int) -> torch.Tensor:
        x = _need(x, torch.bfloat16, "x")
        if x.dim() != 2 or x.shape[1] != self.hidden or not 1 <= x.shape[0] <= self.max_rows:
            raise ValueError(f"{fn}: x must be [M, {self.hidden}] with 1 <= M <= {self.max_rows}")
        if x_out is None:
            x_out = torch.empty_like(x)
        elif (not isinstance(x_out, torch.Tensor) or x_out.dtype != torch.bfloat16 or x_out.shape != x.shape
              or not x_out.is_contiguous()):
            raise ValueError(f"{fn}: x_out must be a contiguous bf16 tensor shaped like x")
        layer_ptr = ctypes.c_void_p(ctypes.addressof(self._arr) + first * ctypes.sizeof(_MlpLayerC))
        _check(lib().mq4_mlp_layers(_ptr(x), x.shape[0], self.hidden, self.intermediate, count, layer_ptr,
                                    self.eps, _ptr(x_out), _ptr(self.workspace), self.ws_bytes,
                                    _stream(x.device)))
        return x_out

    def __call__(self, x: torch.Tensor, x_out: torch.Tensor | None = None) -> torch.Tensor:
        """x: bf16 [M, hidden]; returns the hidden states after every layer
        (x_out, if given, receives them and must not overlap x)."""
        return self._run("BatchedMlpLayers", x, x_out, 0, len(self.layers))

    def layer(self, i: int, x: torch.Tensor, x_out: torch.Tensor | None = None) -> torch.Tensor:
        """x + mlp_forward(rms_norm(x, layers[i].post_attn_norm)) for the M rows
        of x in one launch: the MLP half the reference's layer loop runs
        between its attention / SSM halves, for callers that interleave other
        work per layer.  x_out must not overlap x."""
        if not 0 <= i < len(self.layers):
            raise IndexError(f"BatchedMlpLayers.layer: layer {i} of {len(self.layers)}")
        return self._run("BatchedMlpLayers.layer", x, x_out, i, 1)


# on-disk Q4 weight cache (safetensors, MLX naming): see q4cache.py
from .q4cache import load_q4_cache, quantize_or_load, save_q4_cache  # noqa: E402
