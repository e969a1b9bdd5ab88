"""C-ABI surface of libmq4.so, checked without a GPU: the library loads, it
exports every function include/mq4.h declares, and argument validation
rejects bad calls with the documented status codes before any HIP call."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mq4.h")

OK, INVALID, UNSUPPORTED, ALIGN, HIPERR, WORKSPACE = 0, -1, -2, -3, -4, -5


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mq4_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for must in ("mq4_quantize", "mq4_qmm", "mq4_mlp_gate_up_silu", "mq4_lm_head_argmax",
                 "mq4_argmax_bf16", "mq4_qmm_residual", "mq4_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol(mq4):
    L = mq4.lib()
    for name in declared_functions():
        assert hasattr(L, name), f"libmq4.so does not export {name}"
    assert L.mq4_version() >= 100


def fake(addr):
    """A non-null 'device pointer' with the given alignment; never dereferenced
    because every call below fails validation first."""
    return ctypes.c_void_p(addr)


A16 = 0x100000
S = ctypes.c_void_p(0)


def last_error(mq4):
    return mq4.lib().mq4_last_error().decode()


def test_quantize_validation(mq4):
    L = mq4.lib()
    assert L.mq4_quantize(fake(A16), 4, 128, 32, 4, fake(A16), fake(A16), fake(A16), S) == UNSUPPORTED
    assert "group_size" in last_error(mq4)
    assert L.mq4_quantize(fake(A16), 4, 128, 64, 8, fake(A16), fake(A16), fake(A16), S) == UNSUPPORTED
    assert L.mq4_quantize(fake(A16), 4, 96, 64, 4, fake(A16), fake(A16), fake(A16), S) == INVALID
    assert L.mq4_quantize(fake(A16), 0, 128, 64, 4, fake(A16), fake(A16), fake(A16), S) == INVALID
    assert L.mq4_quantize(None, 4, 128, 64, 4, fake(A16), fake(A16), fake(A16), S) == INVALID
    assert L.mq4_quantize(fake(A16 + 8), 4, 128, 64, 4, fake(A16), fake(A16), fake(A16), S) == ALIGN
    assert L.mq4_quantize(fake(A16), 4, 128, 64, 4, fake(A16 + 2), fake(A16), fake(A16), S) == ALIGN


def test_quantize_batch_validation(mq4):
    """Every job is checked before anything is enqueued; the message names the
    failing job.  (n_jobs = 0 is a no-op that enqueues nothing.)"""
    L = mq4.lib()
    good = mq4._QuantJobC(A16, 4, 128, A16, A16, A16)
    table = (mq4._QuantJobC * 3)(good, mq4._QuantJobC(A16, 4, 96, A16, A16, A16), good)
    jobs = ctypes.cast(table, ctypes.c_void_p)
    assert L.mq4_quantize_batch(jobs, 3, 64, 4, S) == INVALID
    assert "job 1" in last_error(mq4) and "K=96" in last_error(mq4)
    table[1] = mq4._QuantJobC(A16, 0, 128, A16, A16, A16)
    assert L.mq4_quantize_batch(jobs, 3, 64, 4, S) == INVALID and "job 1" in last_error(mq4)
    table[1] = mq4._QuantJobC(A16 + 8, 4, 128, A16, A16, A16)
    assert L.mq4_quantize_batch(jobs, 3, 64, 4, S) == ALIGN
    table[1] = mq4._QuantJobC(A16, 4, 128, None, A16, A16)
    assert L.mq4_quantize_batch(jobs, 3, 64, 4, S) == INVALID
    table[1] = good
    assert L.mq4_quantize_batch(jobs, 3, 32, 4, S) == UNSUPPORTED
    assert L.mq4_quantize_batch(jobs, -1, 64, 4, S) == INVALID
    assert L.mq4_quantize_batch(None, 2, 64, 4, S) == INVALID
    assert L.mq4_quantize_batch(None, 0, 64, 4, S) == OK


def test_qmm_validation(mq4):
    L = mq4.lib()
    args = lambda **kw: [kw.get("x", fake(A16)), kw.get("M", 1), kw.get("K", 2048), kw.get("wq", fake(A16)),
                         fake(A16), fake(A16), kw.get("N", 64), kw.get("tr", 1), kw.get("g", 64),
                         kw.get("bits", 4), kw.get("y", fake(A16)), S]
    assert L.mq4_qmm(*args(tr=0)) == UNSUPPORTED
    assert "transpose" in last_error(mq4)
    assert L.mq4_qmm(*args(g=128)) == UNSUPPORTED
    assert L.mq4_qmm(*args(K=100)) == INVALID
    assert L.mq4_qmm(*args(K=32768 + 64)) == UNSUPPORTED
    assert L.mq4_qmm(*args(M=0)) == INVALID
    assert L.mq4_qmm(*args(N=0)) == INVALID
    assert L.mq4_qmm(*args(x=fake(A16 + 2))) == ALIGN
    assert L.mq4_qmm(*args(wq=fake(A16 + 4))) == ALIGN
    assert L.mq4_qmm(*args(y=None)) == INVALID


def test_lm_head_workspace_validation(mq4):
    L = mq4.lib()
    need = L.mq4_lm_head_argmax_workspace_size(1, 248320)
    assert need > 0 and L.mq4_lm_head_argmax_workspace_size(4, 248320) == 4 * need
    rc = L.mq4_lm_head_argmax(fake(A16), 1, 2048, fake(A16), fake(A16), fake(A16), 248320,
                              fake(A16), None, fake(A16), need - 8, S)
    assert rc == WORKSPACE
    rc = L.mq4_lm_head_argmax(fake(A16), 1, 2048, fake(A16), fake(A16), fake(A16), 248320,
                              fake(A16), None, None, need, S)
    assert rc == WORKSPACE
    rc = L.mq4_argmax_bf16(fake(A16), 1, 10, fake(A16), fake(A16), 0, S)
    assert rc == WORKSPACE


def test_error_message_is_per_call(mq4):
    L = mq4.lib()
    L.mq4_quantize(fake(A16), 4, 128, 32, 4, fake(A16), fake(A16), fake(A16), S)
    assert last_error(mq4) != ""
    # a successful zero-length call clears it
    assert L.mq4_swiglu_bf16(fake(A16), fake(A16), 0, fake(A16), S) == OK
    assert last_error(mq4) == ""


def test_python_api_rejects_host_tensors(mq4):
    import torch
    with pytest.raises(ValueError):
        mq4.quantize(torch.zeros(4, 64, dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        mq4.quantize(torch.zeros(4, 64, dtype=torch.float32))
    with pytest.raises(ValueError):
        mq4.sample_token(torch.zeros(1, 1, 8, dtype=torch.bfloat16), temperature=0.7)
    with pytest.raises(ValueError):
        mq4.sample_token(torch.zeros(2, 1, 8, dtype=torch.bfloat16), temperature=0.7)
    with pytest.raises(ValueError):
        mq4.sample_token(torch.zeros(1, 8, dtype=torch.bfloat16), temperature=0.7, top_k=-1)


def test_sample_validation(mq4):
    L = mq4.lib()
    f = ctypes.c_float
    args = lambda M, N, t, k, p, lg=fake(A16), ix=fake(A16): (lg, M, N, f(t), k, f(p), 7, ix, None, None, 0, S)
    assert L.mq4_sample_bf16(*args(0, 8, 1.0, 0, 1.0)) == INVALID
    assert L.mq4_sample_bf16(*args(1, 0, 1.0, 0, 1.0)) == INVALID
    assert L.mq4_sample_bf16(*args(65536, 8, 1.0, 0, 1.0)) == UNSUPPORTED
    assert L.mq4_sample_bf16(*args(1, (1 << 23) + 1, 1.0, 0, 1.0)) == UNSUPPORTED
    assert L.mq4_sample_bf16(*args(1, 8, 1.0, -1, 1.0)) == INVALID
    assert "top_k" in last_error(mq4)
    assert L.mq4_sample_bf16(*args(1, 8, float("nan"), 0, 1.0)) == INVALID
    assert L.mq4_sample_bf16(*args(1, 8, 1.0, 0, float("nan"))) == INVALID
    assert L.mq4_sample_bf16(*args(1, 8, 1.0, 0, 1.0, lg=None)) == INVALID
    assert L.mq4_sample_bf16(*args(1, 8, 1.0, 0, 1.0, lg=fake(A16 + 1))) == ALIGN
    assert L.mq4_sample_bf16(*args(1, 8, 1.0, 0, 1.0, ix=fake(A16 + 2))) == ALIGN
    # the chunked path needs its whole workspace, 256-byte aligned
    need = L.mq4_sample_workspace_size(1, 151936)
    assert need > 0 and L.mq4_sample_workspace_size(1, 1000) == 0 and L.mq4_sample_workspace_size(129, 151936) == 0
    ws_args = (fake(A16), 1, 151936, f(1.0), 0, f(1.0), 7, fake(A16), None)
    assert L.mq4_sample_bf16(*ws_args, fake(A16), need - 1, S) == WORKSPACE
    assert L.mq4_sample_bf16(*ws_args, fake(A16 + 8), need, S) == WORKSPACE


class _Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "norm_weight", "gate_wq", "gate_scales", "gate_biases", "up_wq", "up_scales", "up_biases",
        "down_wq", "down_scales", "down_biases")]


def test_decode_step_validation(mq4):
    """Every rejection of mq4_decode_step happens before its first HIP call."""
    L = mq4.lib()
    need = L.mq4_decode_workspace_size(2048, 6144, 248320)
    assert need > 0 and need % 256 == 0
    good = _Layer(*([A16] * 10))
    arr = (_Layer * 2)(good, good)

    def call(**kw):
        return L.mq4_decode_step(
            kw.get("x", fake(A16)), kw.get("hidden", 2048), kw.get("inter", 6144), kw.get("n", 2),
            kw.get("layers", ctypes.cast(arr, ctypes.c_void_p)), kw.get("fn", fake(A16)), 1e-6,
            kw.get("wq", fake(A16)), fake(A16), fake(A16), kw.get("vocab", 248320), kw.get("idx", fake(A16)),
            kw.get("xo", None), kw.get("ws", fake(0x200000)), kw.get("wsb", need), S)

    assert call(hidden=4096) == UNSUPPORTED
    assert "hidden" in last_error(mq4)
    assert call(inter=8192) == UNSUPPORTED
    assert call(n=33) == UNSUPPORTED
    assert call(n=-1) == UNSUPPORTED
    assert call(vocab=-1) == INVALID
    assert call(vocab=0, n=0) == INVALID                # no layers and no lm_head: nothing to do
    assert "nothing to do" in last_error(mq4)
    # vocab 0 runs the layers only: the final norm, lm_head and idx may be NULL,
    # so the call passes every host check and reaches the device (absent here)
    assert call(vocab=0, idx=None, fn=None, wq=None) == HIPERR
    assert call(vocab=(1 << 30) + 1) == INVALID
    assert call(x=None) == INVALID
    assert call(idx=None) == INVALID
    assert call(layers=None) == INVALID
    assert call(x=fake(A16 + 2)) == ALIGN
    assert call(wq=fake(A16 + 4)) == ALIGN
    assert call(xo=fake(A16 + 2)) == ALIGN
    assert call(ws=None) == WORKSPACE
    assert call(wsb=need - 1) == WORKSPACE
    assert call(ws=fake(0x200000 + 128)) == WORKSPACE
    bad = (_Layer * 2)(good, _Layer(*([A16] * 9 + [0])))
    assert call(layers=ctypes.cast(bad, ctypes.c_void_p)) == INVALID
    assert "layer 1" in last_error(mq4)
    mis = (_Layer * 2)(good, _Layer(*([A16, A16 + 8] + [A16] * 8)))
    assert call(layers=ctypes.cast(mis, ctypes.c_void_p)) == ALIGN


def test_noalloc_lm_head_host_validation(mq4):
    """Rejected on the host, before any HIP call: more rows than the static
    scratch holds, and non-positive M."""
    L = mq4.lib()
    f = L.mq4_lm_head_argmax_noalloc
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64] + [ctypes.c_void_p] * 3 + \
        [ctypes.c_int64] + [ctypes.c_void_p] * 3
    assert f(fake(A16), 33, 2048, fake(A16), fake(A16), fake(A16), 1000, fake(A16), None, S) == UNSUPPORTED
    assert "32" in last_error(mq4)
    assert f(fake(A16), 0, 2048, fake(A16), fake(A16), fake(A16), 1000, fake(A16), None, S) == INVALID


def test_mlp_residual_workspace_and_validation(mq4):
    """mq4_mlp_workspace_size: h [M, N] bf16, plus for 5-32 rows the two fp32
    K parts of the down product [2, M, K], and from 33 rows on the paired x
    [M, K], the group sums of x and h and the fp16-weight down product's
    fp32 K parts [S, M, K] (S of 1, 2, 4 with tiles x S <= 256 CUs, the
    tiles 128 x 128 while ceil(M / 128) ceil(K / 128) <= 512, else 128 x
    256; no section for S = 1) and the SwiGLU epilogue's SiLU table (4096
    bf16), each section 256-byte aligned; the
    entry rejects a missing, small or misaligned workspace (and bad shapes)
    before enqueueing anything."""
    L = mq4.lib()
    up = lambda v: (v + 255) // 256 * 256
    assert L.mq4_mlp_workspace_size(0, 2048, 6144) == 0
    assert L.mq4_mlp_workspace_size(4, 2048, 6144) == up(4 * 6144 * 2)
    assert L.mq4_mlp_workspace_size(16, 2048, 6144) == up(16 * 6144 * 2) + up(2 * 16 * 2048 * 4)
    assert L.mq4_mlp_workspace_size(32, 2048, 6144) == up(32 * 6144 * 2) + up(2 * 32 * 2048 * 4)
    M, K, N = 2048, 2048, 6144
    # from 33 rows: h, the paired (or fp16) operand, its group sums (or row
    # scales), h's group sums, the K parts (M = 2048: 16 x 16 tiles of
    # 128 x 128, one part, no section) and the SiLU table
    lut = 4096 * 2
    assert L.mq4_mlp_workspace_size(M, K, N) == (up(M * N * 2) + up(M * K * 2) + up(M * K // 64 * 4) +
                                                 up(M * N // 64 * 4) + lut)
    # 1000 rows: 8 x 16 tiles, two parts
    M1 = 1000
    assert L.mq4_mlp_workspace_size(M1, K, N) >= (up(M1 * N * 2) + up(M1 * K * 2) + up(M1 * K // 64 * 4) +
                                                  up(M1 * N // 64 * 4) + up(2 * M1 * K * 4) + lut)
    # 8192 rows (64 x 8 tiles of 128 x 256): one part, no section
    M8 = 8192
    assert L.mq4_mlp_workspace_size(M8, K, N) == (up(M8 * N * 2) + up(M8 * K * 2) + up(M8 * K // 64 * 4) +
                                                  up(M8 * N // 64 * 4) + lut)
    # the size for M rows covers every smaller row count, also where the
    # K-part count drops (512 rows: four parts, 513: two)
    big = L.mq4_mlp_workspace_size(3000, K, N)
    assert all(L.mq4_mlp_workspace_size(m, K, N) <= big for m in (33, 512, 513, 1024, 1025, 2048, 2049, 3000))
    assert L.mq4_mlp_workspace_size(600, K, N) >= up(4 * 512 * K * 4)
    # the size for M rows covers every call of at most M rows (the paired
    # GEMM regime from 33 rows needs less per row than the two fp32 K parts of
    # 5-32 rows, so the size is the largest over the regimes up to M)
    for K, N in ((2048, 6144), (512, 1024), (6144, 2048)):
        sizes = [L.mq4_mlp_workspace_size(m, K, N) for m in range(1, 80)]
        assert all(b >= a for a, b in zip(sizes, sizes[1:])), (K, N)
    assert L.mq4_mlp_workspace_size(40, 2048, 6144) >= up(32 * 6144 * 2) + up(2 * 32 * 2048 * 4)
    # the call itself needs only its own row count's layout (40 rows: the
    # paired GEMM operands), less than the size that covers every M <= 40
    need = up(40 * 6144 * 2) + up(40 * 2048 * 2) + up(40 * 2048 // 64 * 4) + up(40 * 6144 // 64 * 4) + lut
    assert need < L.mq4_mlp_workspace_size(40, 2048, 6144)
    w = [fake(A16)] * 9
    call = lambda ws, nb, **kw: L.mq4_mlp_residual(kw.get("x", fake(A16)), kw.get("M", 40), kw.get("K", 2048),
                                                   fake(A16), ctypes.c_float(1e-6), *w, kw.get("N", 6144), ws, nb,
                                                   kw.get("y", fake(A16)), S)
    assert call(None, need) == WORKSPACE
    assert call(fake(A16), need - 1) == WORKSPACE
    assert "workspace" in last_error(mq4)
    assert call(fake(A16 + 16), need) == WORKSPACE
    assert call(fake(A16), need, K=100) == INVALID
    assert call(fake(A16), need, M=0) == INVALID
    assert call(fake(A16), need, y=None) == INVALID
    assert call(fake(A16), need, x=fake(A16 + 2)) == ALIGN


def test_mlp_layers_validation(mq4):
    """mq4_mlp_layers (the batched one-launch MLP half): the workspace size
    (control words, the h and part-sum exchange words sized for 32 rows, two
    ping-pong hidden states of M rows) and every rejection before the first
    HIP call."""
    L = mq4.lib()
    up = lambda v: (v + 255) // 256 * 256
    ws_size = L.mq4_mlp_layers_workspace_size
    for bad in ((0, 2048, 6144), (33, 2048, 6144), (4, 4096, 6144), (4, 2048, 8192)):
        assert ws_size(*bad) == 0
    exch = 256 + up(8 * 32 * 384 * 8) + up(8 * 32 * 64 * 32 * 8)
    for M in (1, 16, 32):
        assert ws_size(M, 2048, 6144) == exch + 2 * up(M * 2048 * 2)
    sizes = [ws_size(m, 2048, 6144) for m in range(1, 33)]
    assert all(b >= a for a, b in zip(sizes, sizes[1:]))
    need = ws_size(16, 2048, 6144)
    good = _Layer(*([A16] * 10))
    arr = (_Layer * 2)(good, good)
    WS = 0x4000000

    def call(**kw):
        return L.mq4_mlp_layers(
            kw.get("x", fake(A16)), kw.get("M", 16), kw.get("hidden", 2048), kw.get("inter", 6144),
            kw.get("n", 2), kw.get("layers", ctypes.cast(arr, ctypes.c_void_p)), 1e-6,
            kw.get("xo", fake(0x200000)), kw.get("ws", fake(WS)), kw.get("wsb", need), S)

    assert call(hidden=4096) == UNSUPPORTED
    assert "hidden" in last_error(mq4)
    assert call(inter=8192) == UNSUPPORTED
    assert call(M=0) == UNSUPPORTED
    assert call(M=33) == UNSUPPORTED
    assert call(n=0) == INVALID
    assert call(x=None) == INVALID
    assert call(xo=None) == INVALID
    assert call(layers=None) == INVALID
    assert call(x=fake(A16 + 2)) == ALIGN
    assert call(xo=fake(0x200000 + 8)) == ALIGN
    assert call(xo=fake(A16 + 16 * 2048)) == INVALID           # overlaps the last row of x
    assert "overlap" in last_error(mq4)
    assert call(xo=fake(A16 + 16 * 2048 * 2)) == HIPERR         # adjacent: passes the host checks
    assert call(ws=None) == WORKSPACE
    assert call(wsb=need - 1) == WORKSPACE
    assert call(M=32) == WORKSPACE                              # a 16-row workspace is too small for 32
    assert call(ws=fake(WS + 128)) == WORKSPACE
    assert call(xo=fake(WS + need - 16)) == INVALID             # inside the workspace
    bad = (_Layer * 2)(good, _Layer(*([A16] * 9 + [0])))
    assert call(layers=ctypes.cast(bad, ctypes.c_void_p)) == INVALID
    assert "layer 1" in last_error(mq4)
    mis = (_Layer * 2)(good, _Layer(*([A16, A16 + 8] + [A16] * 8)))
    assert call(layers=ctypes.cast(mis, ctypes.c_void_p)) == ALIGN
    mis = (_Layer * 2)(_Layer(*([A16] * 8 + [A16 + 8, A16])), good)   # down scales: 16-byte loads
    assert call(layers=ctypes.cast(mis, ctypes.c_void_p)) == ALIGN
    # every host check passed: the call reaches the device query (absent here)
    assert call() == HIPERR
    assert call(M=8) == HIPERR                                  # a larger workspace serves fewer rows
