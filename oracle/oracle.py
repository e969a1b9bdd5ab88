"""ctypes + numpy front end of the CPU oracle (libmq4_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker (or the timed CPU
baseline), never as the product.  The product path (libmq4.so) does not load
anything from this directory.

Every function mirrors one in mq4_oracle.c; that file's header names the
reference file:line each follows.  Arrays of bf16 values are numpy uint16
holding the raw bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmq4_oracle.so")
_lib = None

GROUP = 64
BITS = 4
SEED = 0x4D41524C  # "MARL"


def build() -> None:
    """Compile libmq4_oracle.so with the Makefile beside this file."""
    subprocess.check_call(["make", "-s", "-C", _HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        L.mq4o_gen_normal_bf16.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double,
                                           ctypes.c_double, I64, I64, P]
        L.mq4o_quantize.argtypes = [P, I64, I64, P, P, P]
        L.mq4o_quantize.restype = ctypes.c_int
        L.mq4o_dequantize_f64.argtypes = [P, P, P, I64, I64, P]
        L.mq4o_qmm_f64.argtypes = [P, I64, I64, P, P, P, I64, P, P]
        L.mq4o_qmm_f32.argtypes = [P, I64, I64, P, P, P, I64, P]
        L.mq4o_qmm_f64_x32.argtypes = [P, I64, I64, P, P, P, I64, P]
        L.mq4o_qmm_mlx_bf16.argtypes = [P, I64, I64, P, P, P, I64, P]
        L.mq4o_swiglu_bf16.argtypes = [P, P, I64, P]
        L.mq4o_argmax_bf16.argtypes = [P, I64, I64, P]
        L.mq4o_rmsnorm_1pw.argtypes = [P, P, I64, I64, ctypes.c_float, P]
        L.mq4o_rmsnorm_mlx.argtypes = [P, P, I64, I64, ctypes.c_float, ctypes.c_int, P]
        L.mq4o_add_bf16.argtypes = [P, P, I64, P]
        L.mq4o_f32_to_bf16_array.argtypes = [P, P, I64]
        L.mq4o_f64_to_bf16_array.argtypes = [P, P, I64]
        L.mq4o_omp_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------ bf16 ---
def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().mq4o_f32_to_bf16_array(_p(f), _p(out), f.size)
    return out


def f64_to_bf16(d: np.ndarray) -> np.ndarray:
    d = np.ascontiguousarray(d, dtype=np.float64)
    out = np.empty(d.shape, np.uint16)
    lib().mq4o_f64_to_bf16_array(_p(d), _p(out), d.size)
    return out


# ------------------------------------------------------------- generator ---
def gen_normal_bf16(stream_id: int, n: int, mu: float = 0.0, sigma: float = 1.0,
                    seed: int = SEED, offset: int = 0) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().mq4o_gen_normal_bf16(seed, stream_id, mu, sigma, offset, n, _p(out))
    return out


# -------------------------------------------------------------- quantize ---
def quantize(w: np.ndarray):
    """w: uint16 bf16 bits [N, K] -> (wq uint32 [N, K/8], scales, biases uint16 [N, K/64])."""
    w = np.ascontiguousarray(w, dtype=np.uint16)
    N, K = w.shape
    wq = np.empty((N, K // 8), np.uint32)
    s = np.empty((N, K // GROUP), np.uint16)
    b = np.empty((N, K // GROUP), np.uint16)
    rc = lib().mq4o_quantize(_p(w), N, K, _p(wq), _p(s), _p(b))
    if rc != 0:
        raise ValueError(f"oracle quantize: K={K} must be a positive multiple of {GROUP}")
    return wq, s, b


def dequantize_f64(wq, s, b) -> np.ndarray:
    N = wq.shape[0]
    K = wq.shape[1] * 8
    out = np.empty((N, K), np.float64)
    lib().mq4o_dequantize_f64(_p(np.ascontiguousarray(wq)), _p(np.ascontiguousarray(s)),
                              _p(np.ascontiguousarray(b)), N, K, _p(out))
    return out


# ------------------------------------------------------------------- qmm ---
def _qmm_args(x, wq, s, b):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    if x.ndim == 1:
        x = x[None, :]
    M, K = x.shape
    N = wq.shape[0]
    assert wq.shape == (N, K // 8) and s.shape == (N, K // GROUP) and b.shape == s.shape
    return x, M, K, N, np.ascontiguousarray(wq), np.ascontiguousarray(s), np.ascontiguousarray(b)


def qmm_f64(x, wq, s, b):
    """fp64 oracle: returns (y_f64 [M, N], y_bf16 [M, N] = RNE(y_f64))."""
    x, M, K, N, wq, s, b = _qmm_args(x, wq, s, b)
    y = np.empty((M, N), np.float64)
    yb = np.empty((M, N), np.uint16)
    lib().mq4o_qmm_f64(_p(x), M, K, _p(wq), _p(s), _p(b), N, _p(y), _p(yb))
    return y, yb


def qmm_f32(x, wq, s, b):
    x, M, K, N, wq, s, b = _qmm_args(x, wq, s, b)
    yb = np.empty((M, N), np.uint16)
    lib().mq4o_qmm_f32(_p(x), M, K, _p(wq), _p(s), _p(b), N, _p(yb))
    return yb


def qmm_mlx_bf16(x, wq, s, b):
    x, M, K, N, wq, s, b = _qmm_args(x, wq, s, b)
    yb = np.empty((M, N), np.uint16)
    lib().mq4o_qmm_mlx_bf16(_p(x), M, K, _p(wq), _p(s), _p(b), N, _p(yb))
    return yb


# ---------------------------------------------------- swiglu/argmax/norm ---
def swiglu_bf16(g, u):
    g = np.ascontiguousarray(g, dtype=np.uint16)
    u = np.ascontiguousarray(u, dtype=np.uint16)
    out = np.empty(g.shape, np.uint16)
    lib().mq4o_swiglu_bf16(_p(g), _p(u), g.size, _p(out))
    return out


def argmax_bf16(logits):
    logits = np.ascontiguousarray(logits, dtype=np.uint16)
    if logits.ndim == 1:
        logits = logits[None, :]
    M, N = logits.shape
    idx = np.empty(M, np.uint32)
    lib().mq4o_argmax_bf16(_p(logits), M, N, _p(idx))
    return idx


def rmsnorm_1pw(x, w, eps: float = 1e-6):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    if x.ndim == 1:
        x = x[None, :]
    M, K = x.shape
    w = np.ascontiguousarray(w, dtype=np.uint16)
    out = np.empty((M, K), np.uint16)
    lib().mq4o_rmsnorm_1pw(_p(x), _p(w), M, K, eps, _p(out))
    return out


NORM_BF16_SUM = 1   # mean's sum accumulates in bf16 (rounded after every add)
NORM_BF16_OPS = 2   # every op of the chain returns bf16 (scalars do not promote)


def rmsnorm_mlx(x, w, eps: float = 1e-6, flags: int = 0):
    """rms_norm (src/model/marlin.cpp:12-16) evaluated as its chain of MLX ops;
    flags 0 = MLX C++ promotion (bf16 square/mean, float32 from + eps on,
    fp32 sum), see mq4_oracle.c for the flag meanings."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    if x.ndim == 1:
        x = x[None, :]
    M, K = x.shape
    w = np.ascontiguousarray(w, dtype=np.uint16)
    out = np.empty((M, K), np.uint16)
    lib().mq4o_rmsnorm_mlx(_p(x), _p(w), M, K, eps, flags, _p(out))
    return out


def add_bf16(a, b):
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(a.shape, np.uint16)
    lib().mq4o_add_bf16(_p(a), _p(b), a.size, _p(out))
    return out


def mlp_forward(x, gate, up, down):
    """down(swiglu(gate x, up x)) with each qmm rounded once from fp64 to bf16
    (src/model/marlin.cpp:31-35); gate/up/down are (wq, s, b) triples."""
    _, g = qmm_f64(x, *gate)
    _, u = qmm_f64(x, *up)
    h = swiglu_bf16(g, u)
    _, y = qmm_f64(h, *down)
    return g, u, h, y


# ------------------------------------- the C++ promotion reading (fp32) ---
# In MLX's C++ API a float scalar operand is a float32 array, and a bf16 array
# combined with a float32 one gives float32.  rms_norm (src/model/marlin.cpp:
# 12-16) adds eps and 1.0f, so it returns float32; qmatmul (marlin.cpp:18-25)
# then multiplies float32 activations (MLX promotes the bf16 scales and biases
# to float32, exactly); swiglu (marlin.cpp:27-29), the residual add (:142) and
# the lm_head logits (:161-169) are float32, and sample_token's argmax
# (src/sampling/sampler.cpp:15) runs over float32 logits.  After the first
# residual add the hidden state itself is float32.  These functions evaluate
# that reading; the kernels (and the chain above) follow the bf16 activations
# of the benchmark configurations instead.


def qmm_f64_x32(x32, wq, s, b) -> np.ndarray:
    """mx::quantized_matmul on float32 x in fp64 (mq4o_qmm_f64_x32): [M, N] fp64."""
    x32 = np.ascontiguousarray(x32, dtype=np.float32)
    if x32.ndim == 1:
        x32 = x32[None, :]
    M, K = x32.shape
    N = wq.shape[0]
    assert wq.shape == (N, K // 8) and s.shape == (N, K // GROUP) and b.shape == s.shape
    y = np.empty((M, N), np.float64)
    lib().mq4o_qmm_f64_x32(_p(x32), M, K, _p(np.ascontiguousarray(wq)), _p(np.ascontiguousarray(s)),
                           _p(np.ascontiguousarray(b)), N, _p(y))
    return y


def rmsnorm_f32(x, w, eps: float = 1e-6) -> np.ndarray:
    """rms_norm (src/model/marlin.cpp:12-16) in the C++ promotion reading:
    square and mean keep the input's dtype (bf16 bits as uint16, the first
    layer's input, or float32), "+ eps" promotes to float32, rsqrt, the
    product with x and with (1.0f + w) are float32.  Returns float32."""
    one = np.float32(1.0)
    if x.dtype == np.uint16:
        xf = bf16_to_f32(x)
        sq = bf16_to_f32(f32_to_bf16(xf * xf))                        # square: bf16
        sm = bf16_to_f32(f32_to_bf16(sq.sum(axis=-1, dtype=np.float32)))   # sum: bf16
        inv = bf16_to_f32(f32_to_bf16(np.float32(1.0 / x.shape[-1])))
        mean = bf16_to_f32(f32_to_bf16(sm * inv))                     # mean: bf16
    else:
        xf = np.asarray(x, np.float32)
        mean = (xf * xf).sum(axis=-1, dtype=np.float32) * np.float32(1.0 / x.shape[-1])
    r = one / np.sqrt(mean.astype(np.float32) + np.float32(eps))
    return (xf * r[..., None]) * (one + bf16_to_f32(w))


def swiglu_f32(g, u) -> np.ndarray:
    """(sigmoid(g) * g) * u (src/model/marlin.cpp:27-29) on float32 arrays,
    every op rounded to float32."""
    g = np.asarray(g, np.float32)
    sg = np.float32(1.0) / (np.float32(1.0) + np.exp(-g))
    return (sg * g) * np.asarray(u, np.float32)


def decode_chain_f32(x, layers, final_norm, lm, eps: float = 1e-6):
    """The decode step's MLP halves and lm_head in the C++ promotion reading:
    x bf16 bits [M, K]; layers a list of (norm_w, gate, up, down) with Q4
    (wq, s, b) triples.  Returns (hidden float32 [M, K], logits float32
    [M, N], tokens = first index of the float32 maximum)."""
    h = np.asarray(x, np.uint16)
    for nw, g, u, d in layers:
        n = rmsnorm_f32(h, nw, eps)
        gg = qmm_f64_x32(n, *g).astype(np.float32)
        uu = qmm_f64_x32(n, *u).astype(np.float32)
        y = qmm_f64_x32(swiglu_f32(gg, uu), *d).astype(np.float32)
        hf = bf16_to_f32(h) if h.dtype == np.uint16 else h
        h = hf + y
    logits = qmm_f64_x32(rmsnorm_f32(h, final_norm, eps), *lm).astype(np.float32)
    return h, logits, np.argmax(logits, axis=-1)


def decode_chain_bf16(x, layers, final_norm, lm, eps: float = 1e-6):
    """The same step with bf16 activations at every op boundary, as the
    kernels compute it: rmsnorm_1pw, each qmm rounded once from fp64 to bf16,
    the bf16 SwiGLU chain and residual add, argmax over bf16 logits.  Returns
    (hidden bf16 bits, logits fp64 [M, N], tokens)."""
    h = np.asarray(x, np.uint16)
    for nw, g, u, d in layers:
        _, _, _, y = mlp_forward(rmsnorm_1pw(h, nw, eps), g, u, d)
        h = add_bf16(h, y)
    l64, lb = qmm_f64(rmsnorm_1pw(h, final_norm, eps), *lm)
    return h, l64, argmax_bf16(lb)


def omp_threads() -> int:
    return int(lib().mq4o_omp_threads())


# ---------------------------------------------------- tolerance helpers ---
def rel_rms_err(got_bf16, ref_f64) -> float:
    """max |got - ref| / rms(ref) with got as bf16 bits, ref as fp64 values."""
    g = bf16_to_f32(np.asarray(got_bf16)).astype(np.float64)
    r = np.asarray(ref_f64, dtype=np.float64)
    rms = float(np.sqrt(np.mean(r * r)))
    return float(np.max(np.abs(g - r)) / rms) if rms > 0 else float(np.max(np.abs(g - r)))


def bf16_ulp_diff(a_bf16, b_bf16) -> np.ndarray:
    """Distance in bf16 ulps between two bf16 bit arrays (monotone integer map)."""
    def key(h):
        h = np.asarray(h, dtype=np.uint16).astype(np.int32)
        return np.where(h & 0x8000, 0x8000 - (h & 0x7FFF), 0x8000 + h)
    return np.abs(key(a_bf16) - key(b_bf16))
