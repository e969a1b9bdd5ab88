"""Exhaustive device checks of mq4_device.h helpers (tests/hip/mq4_device_check.hip,
built by build() into marlin-mlx_amd/_build/libmq4_devcheck.so).

swiglu_bf16_lut_batch (the fp16-weight GEMM's SwiGLU epilogue) replaces the
rounded SiLU of swiglu_bf16, round_bf16(round_bf16(1 / (1 + expf(-g))) * g)
(the bf16 SwiGLU of src/model/marlin.cpp:27-29), by a 4096-entry table for
2^-9 <= |g| < 128 (built by silu_lut_entry from that formula), g / 2 below
(where the rounded sigmoid is 0.5) and the formula itself beyond.  Its input
g is a bf16 value, so all 65536 inputs are checked against swiglu_bf16, bit
for bit: one value at a time for four values of u, and in 16-value batches
(the form the epilogue calls, with one branch for the values the table does
not cover) that cover every input 16 times."""
import ctypes
import os

import numpy as np
import pytest

from conftest import ROOT

LIB = os.path.join(ROOT, "marlin-mlx_amd", "_build", "libmq4_devcheck.so")


@pytest.mark.gpu
def test_swiglu_lut_all_inputs(mq4, dev):
    import torch
    print("swiglu_bf16_lut_batch: all 65536 bf16 gate values", flush=True)
    assert os.path.exists(LIB), "build() makes the device check library"
    L = ctypes.CDLL(LIB)
    L.mq4check_swiglu_lut.restype = ctypes.c_int
    st = torch.full((65536,), 0x7fffffff, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    assert L.mq4check_swiglu_lut(ctypes.c_void_p(st.data_ptr()), ctypes.c_void_p(stream)) == 0
    torch.cuda.synchronize()
    s = st.cpu().numpy().astype(np.uint32)
    assert (s <= 3).all(), "every input was checked"
    bad = np.nonzero(s)[0]
    print(f"mismatches: single {int((s & 1).sum())}, batched {int((s & 2).sum() // 2)}", flush=True)
    assert bad.size == 0, [hex(int(x)) for x in bad[:16]]
