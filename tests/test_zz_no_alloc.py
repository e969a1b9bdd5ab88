"""mq4_lm_head_argmax_noalloc (the entry point that allocates nothing) against
mq4_lm_head_argmax with a caller workspace, through the C ABI: two calls in a
row on the same GPU, the second with a smaller input (fewer rows, a shorter
vocab), must give bit-identical indices and logits; M above the static
scratch's 32 rows is rejected on the host."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import to_host_u16

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p


def ptr(t):
    return P(t.data_ptr()) if t is not None else P(0)


def test_noalloc_lm_head_matches_workspace_variant(mq4, dev):
    L = mq4.lib()
    V, K = 50000, 2048
    w = mq4.quantize_weight(mq4.fill_normal_bf16((V, K), mq4.STREAM_LM_HEAD, 0.0, 0.02, device=dev))
    st = P(torch.cuda.current_stream().cuda_stream)
    for M, N in ((5, V), (2, 777), (32, V), (1, 64)):
        print(f"noalloc lm_head M={M} N={N}", flush=True)
        h = mq4.fill_normal_bf16((M, K), 3500 + M, 0.0, 1.0, device=dev)
        ws_bytes = L.mq4_lm_head_argmax_workspace_size(M, N)
        ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
        idx_a = torch.full((M,), -5, dtype=torch.int32, device=dev)
        idx_b = torch.full((M,), -7, dtype=torch.int32, device=dev)
        lg_a = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        lg_b = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        wp = (ptr(w.weight), ptr(w.scales), ptr(w.biases))
        assert L.mq4_lm_head_argmax(ptr(h), M, K, *wp, N, ptr(idx_a), ptr(lg_a), ptr(ws), ws_bytes, st) == 0
        assert L.mq4_lm_head_argmax_noalloc(ptr(h), M, K, *wp, N, ptr(idx_b), ptr(lg_b), st) == 0
        torch.cuda.synchronize()
        assert np.array_equal(idx_a.cpu().numpy(), idx_b.cpu().numpy()), f"M={M} N={N}"
        assert np.array_equal(to_host_u16(lg_a), to_host_u16(lg_b)), f"M={M} N={N}"
        assert int(idx_b.min()) >= 0 and int(idx_b.max()) < N
        # logits are optional (NULL) on the no-allocation path too
        idx_c = torch.full((M,), -9, dtype=torch.int32, device=dev)
        assert L.mq4_lm_head_argmax_noalloc(ptr(h), M, K, *wp, N, ptr(idx_c), None, st) == 0
        torch.cuda.synchronize()
        assert np.array_equal(idx_a.cpu().numpy(), idx_c.cpu().numpy())


def test_noalloc_rejects_too_many_rows(mq4, dev):
    L = mq4.lib()
    K, N = 2048, 128
    w = mq4.quantize_weight(mq4.fill_normal_bf16((N, K), 5, 0.0, 0.02, device=dev))
    h = torch.zeros((33, K), dtype=torch.bfloat16, device=dev)
    idx = torch.zeros((33,), dtype=torch.int32, device=dev)
    rc = L.mq4_lm_head_argmax_noalloc(ptr(h), 33, K, ptr(w.weight), ptr(w.scales), ptr(w.biases), N,
                                      ptr(idx), None, P(torch.cuda.current_stream().cuda_stream))
    assert rc == -2
    assert "32" in L.mq4_last_error().decode()
