"""The INT8 API contract that can be checked without a device -- the
reference's tests/test_int8_api.py:21-156 and tests/test_int8_autograd.py:20-61,
with the device wording of this build ("GPU" where the reference says "XPU")."""

import pytest
import torch

from xpu_kernels import int8


def _w(n=32, k=512):
    return torch.zeros((n, k), dtype=torch.int8)


def _x(m=4, k=512):
    return torch.zeros((m, k), dtype=torch.bfloat16)


def _scale(n=32):
    return torch.full((n,), 0.01, dtype=torch.float32)


def _device_only(reason):
    return reason is None or "libxpuint8" in reason or "GPU" in reason


def test_valid_call_passes_the_argument_checks():
    assert _device_only(int8.unsupported_reason(_x(), _w(), _scale()))


def test_activation_dtype_is_reported():
    assert "float16" in int8.unsupported_reason(_x().to(torch.float16), _w(), _scale())


def test_weight_must_be_int8_2d():
    assert "int8" in int8.unsupported_reason(_x(), _w().float(), _scale())
    assert "int8" in int8.unsupported_reason(_x(), _w()[0], _scale())


def test_column_count_must_match_the_weight():
    reason = int8.unsupported_reason(_x(k=512), _w(k=1024), _scale())
    assert "512" in reason and "1024" in reason


def test_pair_activation_wants_two_halves():
    reason = int8.unsupported_reason(_x(k=512), _w(k=512), _scale(), act="situ")
    assert "1024" in reason
    assert int8.unsupported_reason(_x(k=1024), _w(k=512), _scale(), act="situ") is not None
    assert "situ" in int8.unsupported_reason(_x(), _w(), _scale(), act="silu")


def test_the_activation_set():
    assert set(int8.ACTIVATIONS) >= {"gelu_tanh", "swiglu", "situ", "geglu_erf", "gelu_erf"}
    assert "situ" in int8.PAIRED_ACTIVATIONS and "geglu_erf" in int8.PAIRED_ACTIVATIONS
    assert "gelu_erf" not in int8.PAIRED_ACTIVATIONS


def test_the_new_activations_in_the_argument_checks():
    assert "1024" in int8.unsupported_reason(_x(k=512), _w(k=512), _scale(), act="geglu_erf")
    assert _device_only(int8.unsupported_reason(_x(k=512), _w(k=512), _scale(), act="gelu_erf"))


def test_ffn_rejects_an_unknown_activation_before_anything_else():
    with pytest.raises(TypeError) as exc:
        int8.ffn(_x(), _w(), _scale(), _w(), _scale(), act="silu")
    assert "silu" in str(exc.value)
    with pytest.raises(TypeError) as exc:
        int8.ffn(_x(), _w(), _scale(), _w(), _scale(), act="swiglu")
    assert "swiglu" in str(exc.value)


def test_group_size_multiple():
    assert "256" in int8.unsupported_reason(_x(k=384), _w(k=384), _scale())


def test_output_width_multiple_of_16():
    reason = int8.unsupported_reason(_x(), _w(n=24), _scale(24))
    assert "24" in reason and "16" in reason


def test_scale_shapes():
    assert "floating point" in int8.unsupported_reason(_x(), _w(), torch.zeros(32, dtype=torch.int32))
    assert "dims" in int8.unsupported_reason(_x(), _w(), torch.zeros((2, 2, 8)))
    assert "values" in int8.unsupported_reason(_x(), _w(), torch.zeros(7))
    assert "tensor or a python float" in int8.unsupported_reason(_x(), _w(), "0.01")
    for scale in (torch.zeros(1), torch.zeros(32), torch.zeros(32, 1), 0.01):
        assert _device_only(int8.unsupported_reason(_x(), _w(), scale))


def test_cpu_tensors_are_refused_with_a_reason():
    reason = int8.unsupported_reason(_x(), _w(), _scale())
    if int8.available():
        assert "GPU" in reason and "cpu" in reason


def test_linear_raises_the_same_message():
    reason = int8.unsupported_reason(_x(), _w(k=384), _scale())
    with pytest.raises(TypeError) as exc:
        int8.linear(_x(), _w(k=384), _scale())
    assert str(exc.value) == reason


def test_prepare_weight_checks_the_group_size():
    for fn in (int8.prepare_weight, int8.prepare_weight_fused):
        with pytest.raises(ValueError) as exc:
            fn(torch.zeros((32, 384), dtype=torch.bfloat16))
        assert "384" in str(exc.value) and "256" in str(exc.value)


def test_the_trainable_linear_checks_its_arguments():
    w = torch.zeros((32, 512), dtype=torch.bfloat16)
    with pytest.raises(ValueError) as exc:
        int8.TrainableInt8Linear(w, backward="exact")
    assert "exact" in str(exc.value)
    with pytest.raises(TypeError) as exc:
        int8.TrainableInt8Linear(torch.zeros((32, 512), dtype=torch.float16))
    assert "bfloat16" in str(exc.value)


def test_expand_scale():
    flat = _scale(32)
    assert int8.expand_scale(flat, 32, flat.device) is flat
    one = torch.tensor(0.25)
    got = int8.expand_scale(one, 5, one.device)
    assert got.shape == (5,) and got.dtype == torch.float32
    assert torch.equal(got, torch.full((5,), 0.25))
    col = torch.arange(4, dtype=torch.float32).reshape(4, 1)
    assert torch.equal(int8.expand_scale(col, 4, col.device), col.reshape(-1))
    assert int8.expand_scale(0.5, 3, torch.device("cpu")).shape == (3,)
    with pytest.raises(TypeError):
        int8.expand_scale(0.5, 3)
    with pytest.raises(TypeError):
        int8.expand_scale("0.5", 3, torch.device("cpu"))


# ---- tests/test_int8_autograd.py:20-61
def test_an_unknown_backward_mode_is_refused():
    with pytest.raises(ValueError) as exc:
        int8.int8_linear(torch.zeros(2, 4, dtype=torch.bfloat16), torch.zeros(4, 4, dtype=torch.int8),
                         torch.ones(4, dtype=torch.float32), mode="nope")
    assert "nope" in str(exc.value)


def test_an_unknown_mode_is_refused_by_the_module():
    with pytest.raises(ValueError):
        int8.Int8Linear(torch.zeros(4, 4, dtype=torch.int8), torch.ones(4, dtype=torch.float32),
                        backward="nope")


def test_linear_dw_contracts_over_the_batch():
    dy = torch.randn(8, 16, dtype=torch.bfloat16)
    x = torch.randn(8, 32, dtype=torch.bfloat16)
    dw = int8.linear_dw(dy, x)
    assert dw.shape == (16, 32)
    assert torch.equal(dw, dy.transpose(0, 1) @ x)


def test_linear_dw_rejects_mismatched_batches():
    with pytest.raises(ValueError) as exc:
        int8.linear_dw(torch.randn(8, 16, dtype=torch.bfloat16), torch.randn(4, 32, dtype=torch.bfloat16))
    assert "rows" in str(exc.value)


def test_linear_dw_flattens_leading_dims():
    dy = torch.randn(2, 3, 8, 16, dtype=torch.bfloat16)
    x = torch.randn(2, 3, 8, 32, dtype=torch.bfloat16)
    dw = int8.linear_dw(dy, x)
    assert dw.shape == (16, 32)
    assert torch.equal(dw, dy.reshape(-1, 16).transpose(0, 1) @ x.reshape(-1, 32))


def test_kernels_refuse_cpu_tensors_loudly():
    """No silent CPU fallback: a kernel call on a CPU tensor raises."""
    with pytest.raises((TypeError, RuntimeError)):
        int8.quantize(_x())
    with pytest.raises((TypeError, RuntimeError)):
        int8.rotate(_x())
