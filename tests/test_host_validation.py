"""Host-side validation of the Python mirror, checked on the CPU: every shape,
dtype and size mismatch that would let a kernel read past a buffer is
rejected with ValueError/TypeError before any pointer reaches the C ABI (as
mx::quantized_matmul rejects such shapes).  CPU tensors are used, so a check
that ran after the device check would show up here as the wrong message."""
import pytest
import torch


def qt(mq4, N, K, gs=64, extra_cols=0, s_cols=None):
    wq = torch.zeros((N, K // 8 + extra_cols), dtype=torch.int32)
    sc = K // gs if s_cols is None else s_cols
    s = torch.zeros((N, sc), dtype=torch.bfloat16)
    return mq4.QuantizedTensor(wq, s, s.clone())


def x_of(M, K):
    return torch.zeros((M, K), dtype=torch.bfloat16)


def test_quantized_matmul_rejects_k_mismatch(mq4):
    w = qt(mq4, 16, 2048)
    with pytest.raises(ValueError, match="K=1024"):
        mq4.quantized_matmul(x_of(1, 1024), w.weight, w.scales, w.biases)
    with pytest.raises(ValueError, match="K=1024"):
        mq4.qmatmul(x_of(1, 1024), w)
    with pytest.raises(ValueError, match="K=1024"):
        mq4.quantized_matmul_f32(x_of(2, 1024), w.weight, w.scales, w.biases)


def test_quantized_matmul_rejects_scale_shape(mq4):
    w = qt(mq4, 16, 2048, s_cols=16)
    with pytest.raises(ValueError, match="scales/biases"):
        mq4.qmatmul(x_of(1, 2048), w)
    good = qt(mq4, 16, 2048)
    with pytest.raises(ValueError, match="scales/biases"):
        mq4.quantized_matmul(x_of(1, 2048), good.weight, good.scales[:8], good.biases)


def test_quantized_matmul_rejects_dtypes(mq4):
    w = qt(mq4, 16, 2048)
    with pytest.raises(TypeError):
        mq4.quantized_matmul(x_of(1, 2048), w.weight.float(), w.scales, w.biases)
    with pytest.raises(TypeError):
        mq4.quantized_matmul(x_of(1, 2048), w.weight, w.scales.float(), w.biases)
    with pytest.raises(ValueError, match="2-D"):
        mq4.quantized_matmul(x_of(1, 2048), w.weight.reshape(-1), w.scales, w.biases)


def test_gate_up_checks_both_weights_and_norm(mq4):
    g, u = qt(mq4, 64, 2048), qt(mq4, 64, 2048)
    with pytest.raises(ValueError, match="same shape"):
        mq4.mlp_gate_up_silu(x_of(1, 2048), g, qt(mq4, 32, 2048))
    with pytest.raises(ValueError, match="K=1024"):
        mq4.mlp_gate_up_silu(x_of(1, 1024), g, u)
    with pytest.raises(ValueError, match="norm_weight must hold 2048"):
        mq4.mlp_gate_up_silu(x_of(1, 2048), g, u, norm_weight=torch.zeros(1024, dtype=torch.bfloat16))


def test_residual_and_out_sizes(mq4):
    d = qt(mq4, 2048, 6144)
    with pytest.raises(ValueError, match="K=2048"):
        mq4.qmatmul_residual(x_of(1, 2048), d, x_of(1, 2048))
    with pytest.raises(ValueError, match="residual"):
        mq4.qmatmul_residual(x_of(1, 6144), d, x_of(1, 1024))
    with pytest.raises(ValueError, match="out must be"):
        mq4.qmatmul_residual(x_of(1, 6144), d, x_of(1, 2048), out=x_of(1, 1024))


def test_lm_head_checks(mq4):
    w = qt(mq4, 1000, 2048)
    with pytest.raises(ValueError, match="K=1024"):
        mq4.lm_head_argmax(x_of(1, 1024), w)
    with pytest.raises(ValueError, match="norm_weight"):
        mq4.lm_head_argmax(x_of(1, 2048), w, norm_weight=torch.zeros(64, dtype=torch.bfloat16))


def test_rms_norm_weight_size(mq4):
    with pytest.raises(ValueError, match="weight must hold 2048"):
        mq4.rms_norm(x_of(2, 2048), torch.zeros(2047, dtype=torch.bfloat16))


def test_decode_step_checks_every_layer(mq4):
    H, I = 2048, 6144
    lm = qt(mq4, 4096, H)
    fn = torch.zeros(H, dtype=torch.bfloat16)
    good = mq4.MLPWeights(qt(mq4, I, H), qt(mq4, I, H), qt(mq4, H, I))
    bad_down = mq4.MLPWeights(qt(mq4, I, H), qt(mq4, I, H), qt(mq4, H, H))
    with pytest.raises(ValueError, match="layer 1 down_proj"):
        mq4.DecodeStep([mq4.DecoderLayer(fn, good), mq4.DecoderLayer(fn, bad_down)], fn, lm)
    bad_rows = mq4.MLPWeights(qt(mq4, I, H), qt(mq4, I - 64, H), qt(mq4, H, I))
    with pytest.raises(ValueError, match="layer 0 up_proj must have 6144 rows"):
        mq4.DecodeStep([mq4.DecoderLayer(fn, bad_rows)], fn, lm)
    with pytest.raises(ValueError, match="post_attn_norm"):
        mq4.DecodeStep([mq4.DecoderLayer(torch.zeros(H - 1, dtype=torch.bfloat16), good)], fn, lm)
    # all shapes right: the remaining complaint is that the tensors are host memory
    with pytest.raises(ValueError, match="device"):
        mq4.DecodeStep([mq4.DecoderLayer(fn, good)], fn, lm)


def test_fused_paths_reject_other_formats(mq4):
    """The kernels read the group-64, 4-bit layout only.  A tensor that
    claims another format (as a cache file MLX wrote with group 128 or 2 bits
    would give) is refused before its buffers reach an entry point; with
    group 128 the scales/biases of a matching shape would otherwise be read
    as if they held K/64 groups."""
    g = qt(mq4, 64, 2048)
    odd = mq4.QuantizedTensor(torch.zeros((64, 2048 // 8), dtype=torch.int32),
                              torch.zeros((64, 2048 // 128), dtype=torch.bfloat16),
                              torch.zeros((64, 2048 // 128), dtype=torch.bfloat16), 128, 4, True)
    two_bit = mq4.QuantizedTensor(torch.zeros((64, 2048 * 2 // 32), dtype=torch.int32),
                                  torch.zeros((64, 32), dtype=torch.bfloat16),
                                  torch.zeros((64, 32), dtype=torch.bfloat16), 64, 2, True)
    for bad in (odd, two_bit):
        with pytest.raises(NotImplementedError, match="group_size=64, bits=4"):
            mq4.mlp_gate_up_silu(x_of(1, 2048), g, bad)
        with pytest.raises(NotImplementedError, match="group_size=64, bits=4"):
            mq4.lm_head_argmax(x_of(1, 2048), bad)
        with pytest.raises(NotImplementedError, match="group_size=64, bits=4"):
            mq4.qmatmul(x_of(1, 2048), bad)
        with pytest.raises(NotImplementedError, match="group_size=64, bits=4"):
            mq4.mlp_residual(x_of(1, 2048), mq4.MLPWeights(g, g, bad), torch.zeros(2048, dtype=torch.bfloat16))
