"""Exhaustive device checks of mq4_device.h helpers (tests/hip/mq4_device_check.hip,
built by build() into marlin-mlx_amd/_build/libmq4_devcheck.so).

sigmoid_bf16 (used by the fp16-weight GEMM's SwiGLU epilogue) replaces
round_bf16(1 / (1 + expf(-g))) (the bf16 SwiGLU of src/model/marlin.cpp:27-29,
as swiglu_bf16 computes it) by v_exp_f32 / v_rcp_f32 with an exact fallback
near bf16 rounding midpoints.  Its input is a bf16 value, so all 65536 inputs
are checked: bit for bit against the exact formula, swiglu_bf16_fast
against swiglu_bf16 for four values of u, and swiglu_bf16_batch<16> (the
form the fp16-weight GEMM's epilogue calls, with the exact formula for the
undecided values in one branch) against swiglu_bf16 on 16-value batches
that cover every input 16 times."""
import ctypes
import os

import numpy as np
import pytest

from conftest import ROOT

LIB = os.path.join(ROOT, "marlin-mlx_amd", "_build", "libmq4_devcheck.so")


@pytest.mark.gpu
def test_sigmoid_bf16_all_inputs(mq4, dev):
    import torch
    print("sigmoid_bf16: all 65536 bf16 inputs", flush=True)
    assert os.path.exists(LIB), "build() makes the device check library"
    L = ctypes.CDLL(LIB)
    L.mq4check_sigmoid.restype = ctypes.c_int
    st = torch.full((65536,), 0x7fffffff, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    assert L.mq4check_sigmoid(ctypes.c_void_p(st.data_ptr()), ctypes.c_void_p(stream)) == 0
    torch.cuda.synchronize()
    s = st.cpu().numpy().astype(np.uint32)
    assert (s <= 15).all(), "every input was checked"
    bad = np.nonzero(s & 14)[0]
    b = np.arange(65536, dtype=np.uint32)
    g = (b << 16).view(np.float32)
    finite_small = np.isfinite(g) & (np.abs(g) < 64.0)
    decided = int((s & 1).sum())
    print(f"fast path decided {decided} of {int(finite_small.sum())} finite |g| < 64; "
          f"mismatches {bad.size}", flush=True)
    assert bad.size == 0, [hex(int(x)) for x in bad[:16]]
    assert not (s[~finite_small] & 1).any(), "|g| >= 64 and non-finite g take the exact formula"
    # the fast path decides nearly every input it covers (the exact formula
    # only within SIG_MARGIN fp32 ulps of a bf16 rounding midpoint)
    assert decided >= 0.97 * int(finite_small.sum())
