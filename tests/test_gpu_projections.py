"""Q4 for the model's other projections (the SSM and attention layers): the same entry
points at the SSM and attention shapes -- in_proj_qkv 6144x2048
(src/model/gated_deltanet.cpp:108), in_proj_z / out_proj 2048x2048
(:109), q_proj 4096x2048, k_proj / v_proj 512x2048, o_proj 2048x2048
(src/model/attention.cpp:82-89) -- at decode (M = 1 dot2 GEMV), batched
(M = 16 MFMA GEMV) and prefill (M = 300 MFMA GEMM) sizes, against the fp64
oracle with the GEMV/GEMM bars of test_gpu_parity / test_gpu_gemm; plus the
last-row-only prefill lm_head (src/core/engine.cpp:64 with
src/sampling/sampler.cpp:10-12) against the full lm_head's last row."""
import numpy as np
import pytest
import torch

from conftest import to_dev_bf16, to_host_u16
from test_gpu_parity import check_close, rel_err_f32

pytestmark = pytest.mark.gpu

SHAPES = [(6144, 2048), (2048, 2048), (4096, 2048), (512, 2048)]


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("M", [1, 16, 300])
def test_projection_shapes(mq4, O, dev, N, K, M):
    print(f"projection N={N} K={K} M={M}", flush=True)
    w = mq4.fill_normal_bf16((N, K), 1500 + N, 0.0, 0.02, device=dev)
    qt = mq4.quantize_weight(w)
    xh = O.gen_normal_bf16(3600 + M, M * K).reshape(M, K)
    xd = to_dev_bf16(xh, dev)
    y = mq4.qmatmul(xd, qt)
    y32 = mq4.quantized_matmul_f32(xd, qt.weight, qt.scales, qt.biases)
    torch.cuda.synchronize()
    qh = (qt.weight.cpu().numpy().view(np.uint32), to_host_u16(qt.scales), to_host_u16(qt.biases))
    ref, _ = O.qmm_f64(xh, *qh)
    err = rel_err_f32(y32.cpu().numpy(), ref)
    assert err <= 1e-4, f"fp32 max|err|/rms = {err:.2e}"
    check_close(O, to_host_u16(y), ref, f"proj {N}x{K} M={M}", y32.cpu().numpy())
    assert np.array_equal(to_host_u16(y), O.f32_to_bf16(y32.cpu().numpy()))


def test_lm_head_last_row_only(mq4, O, dev):
    """Only the last prompt row goes through the lm_head (M = 1, dot2 GEMV);
    the full S-row lm_head runs the MFMA path, so the two agree within the
    GEMV bars of the fp64 oracle, not bit for bit."""
    V, K, S = 32768, 2048, 37
    lm = mq4.quantize_weight(mq4.fill_normal_bf16((V, K), mq4.STREAM_LM_HEAD, 0.0, 0.02, device=dev))
    hidden = mq4.fill_normal_bf16((1, S, K), 3700, 0.0, 1.0, device=dev)
    nw = mq4.fill_normal_bf16((K,), mq4.STREAM_NORM_WEIGHT, 0.1, 0.02, device=dev)
    tok, lg = mq4.lm_head_last_row(hidden, lm, norm_weight=nw, return_logits=True)
    idx_all, lg_all = mq4.lm_head_argmax(hidden.reshape(S, K), lm, return_logits=True, norm_weight=nw)
    torch.cuda.synchronize()
    qh = (lm.weight.cpu().numpy().view(np.uint32), to_host_u16(lm.scales), to_host_u16(lm.biases))
    hn = O.rmsnorm_1pw(to_host_u16(hidden).reshape(S, K)[-1:], to_host_u16(nw), 1e-6)
    ref64, refb = O.qmm_f64(hn, *qh)
    check_close(O, to_host_u16(lg).reshape(1, V), ref64, "last-row lm_head")
    check_close(O, to_host_u16(lg_all[-1:]), ref64, "full lm_head, last row")
    t = int(tok.reshape(-1)[0])
    assert t == int(O.argmax_bf16(to_host_u16(lg).reshape(1, V))[0])
    # the full path's token for the last row: equal unless the top two fp64
    # logits are within one bf16 ulp
    if t != int(idx_all[-1]):
        top = np.sort(O.bf16_to_f32(refb[0]))[-2:]
        assert O.bf16_ulp_diff(O.f32_to_bf16(top[:1]), O.f32_to_bf16(top[1:]))[0] <= 1
    # sample_token on the full logits keeps the last row (greedy)
    st = mq4.sample_token(lg_all.reshape(1, S, V), temperature=0.0)
    assert int(st.reshape(-1)[0]) == int(idx_all[-1])
