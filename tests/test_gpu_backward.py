"""The dense-mode backward on the GPU: linear_dx (the bf16 MFMA NN GEMM,
reference python/xpu_kernels/int8/ops.py:194-204), int8_linear(mode="dense")
(ops.py:241-317) and TrainableInt8Linear (ops.py:730-828), forward and
backward, for bf16 and fp32 models.

Bars.  The forward is bit-exact against the oracle (it is the INT8 linear).
Gradients computed by a bf16 kernel are checked element by element against
float64: within one bf16 rounding of the exact value plus the fp32
accumulation error, 2^-8 |ref| + 2^-14 sum |a||b|.  Gradients computed by
torch in fp32 (the fp32 model's products, as the reference computes them) are
checked with the fp32 form of the same bound, 2^-20 |ref| + 2^-18 sum |a||b|.
"""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import activation, bits, mismatch, npy, weight
from xpu_kernels import int8

pytestmark = pytest.mark.gpu


def _within(got, ref, mag, rel, acc):
    got = np.asarray(got, np.float64)
    bound = rel * np.abs(ref) + acc * mag
    err = np.abs(got - ref)
    ok = np.all(err <= bound)
    return ok, float(np.max(err / np.maximum(bound, 1e-300)))


def _bf16_bound(got_bf16_bits, ref, mag):
    return _within(O.bf16_to_f32(got_bf16_bits), ref, mag, 2.0 ** -8, 2.0 ** -14)


# (2100, 2048, 1200) and (4000, 2080, 1280) take the split-K kernel with
# ragged rows and columns and, for the second, an odd number of 32-row
# contraction steps (the teams' halves differ by one); small batches whose
# contraction is split across blocks (129 x 640 and 1024 x 1280: 4 slices,
# 200 x 1280 and the ragged 777 x 1040: 2)
@pytest.mark.parametrize("m,n,k", [(4096, 5120, 1280), (77, 48, 144), (1, 16, 16), (300, 1040, 272),
                                   (129, 4096, 640), (2100, 2048, 1200), (4000, 2080, 1280),
                                   (1024, 5120, 1280), (200, 2048, 1280), (777, 3072, 1040)])
def test_linear_dx_dense(dev, m, n, k):
    g = torch.Generator().manual_seed(m + n + k)
    dy = (torch.randn(m, n, generator=g) * 1e-3).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    dx = int8.linear_dx(dy.to(dev), w.to(dev))
    assert dx.dtype == torch.bfloat16 and tuple(dx.shape) == (m, k)
    ref = O.linear_dx(bits(dy), bits(w))
    mag = np.abs(O.bf16_to_f32(bits(dy)).astype(np.float64)) @ \
        np.abs(O.bf16_to_f32(bits(w)).astype(np.float64))
    ok, worst = _bf16_bound(bits(dx), ref, mag)
    assert ok, worst


def test_linear_dx_dense_batched_input(dev):
    """A [B, S, N] gradient keeps its batch dims, as dy @ w does."""
    g = torch.Generator().manual_seed(3)
    dy = (torch.randn(2, 40, 64, generator=g) * 1e-2).to(torch.bfloat16).to(dev)
    w = (torch.randn(64, 256, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    dx = int8.linear_dx(dy, w)
    assert tuple(dx.shape) == (2, 40, 256)
    flat = int8.linear_dx(dy.reshape(80, 64), w)
    assert torch.equal(dx.reshape(80, 256), flat)


def test_int8_linear_dense_backward(dev):
    """int8_linear(mode="dense"): dx = linear_dx(bf16(dy), dequant_weight(w8, ws)),
    the dequantized weight bit-exact against the oracle and the product within
    the bf16 bound of float64; dbias = dy.sum(0) (the column-sum kernel)."""
    m, n, k = 256, 512, 1280
    x = activation(m, k, seed=21).to(dev).requires_grad_(True)
    w8, ws = int8.prepare_weight(weight(n, k, seed=22).to(dev))
    bias = torch.zeros(n, device=dev, dtype=torch.bfloat16, requires_grad=True)
    dy = (torch.randn(m, n, generator=torch.Generator().manual_seed(23)) * 1e-2).to(torch.bfloat16)
    y = int8.int8_linear(x, w8, ws, bias, mode="dense")
    want_y = O.linear(bits(x.detach()), npy(w8), npy(ws), np.zeros(n, np.float32))
    assert np.array_equal(bits(y.detach()), want_y), mismatch(bits(y.detach()), want_y)
    y.backward(dy.to(dev))
    wd = O.dequant_weight(npy(w8), npy(ws))
    ref = O.linear_dx(bits(dy), wd)
    mag = np.abs(O.bf16_to_f32(bits(dy)).astype(np.float64)) @ \
        np.abs(O.bf16_to_f32(wd).astype(np.float64))
    ok, worst = _bf16_bound(bits(x.grad), ref, mag)
    assert ok, worst
    assert x.grad.dtype == torch.bfloat16
    # dbias: the HIP column sum, bit for bit the oracle's fixed order
    assert np.array_equal(bits(bias.grad), O.column_sum(bits(dy)))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("mode", ["ste", "dense"])
def test_trainable_int8_linear(dev, dtype, mode):
    """Forward: the INT8 linear of prepare_weight_fused(weight), bit for bit.
    Backward: dx = dy @ W (ste: the parameter; dense: the dequantized weight),
    dW = dy^T x, db = dy.sum(0), each in the parameter's dtype."""
    m, n, k = 192, 256, 512
    g = torch.Generator().manual_seed(31)
    w0 = (torch.randn(n, k, generator=g) * 0.02).to(dtype)
    b0 = (torch.randn(n, generator=g) * 0.01).to(dtype)
    mod = int8.TrainableInt8Linear(w0.to(dev), b0.to(dev), backward=mode)
    x = (torch.randn(m, k, generator=g)).to(dtype).to(dev).requires_grad_(True)
    dy = (torch.randn(m, n, generator=g) * 1e-2).to(dtype)
    y = mod(x)
    assert y.dtype == dtype
    # forward against the oracle: the activation and weight enter as bf16
    wq, wsc = O.prepare_weight_fused(bits(w0.to(torch.bfloat16)))
    want_y = O.linear(bits(x.detach().to(torch.bfloat16)), wq, wsc, O.bf16_to_f32(bits(b0.to(torch.bfloat16)))
                      if dtype == torch.bfloat16 else b0.numpy())
    assert np.array_equal(bits(y.detach().to(torch.bfloat16)), want_y)
    y.backward(dy.to(dev))

    f64 = lambda t: t.detach().cpu().double().numpy()
    dyd, xd = f64(dy), f64(x)
    wd = f64(w0) if mode == "ste" else O.bf16_to_f32(O.dequant_weight(wq, wsc)).astype(np.float64)
    bf16_dx = dtype == torch.bfloat16 or mode == "dense"      # dense: bf16 weight, dy cast to it
    dyx = O.bf16_to_f32(bits(dy.to(torch.bfloat16))).astype(np.float64) if bf16_dx else dyd
    ref_dx = dyx @ wd
    mag_dx = np.abs(dyx) @ np.abs(wd)
    if bf16_dx:
        ok, worst = _bf16_bound(bits(x.grad.to(torch.bfloat16)), ref_dx, mag_dx)
    else:
        ok, worst = _within(f64(x.grad), ref_dx, mag_dx, 2.0 ** -20, 2.0 ** -18)
    assert ok, ("dx", worst)
    assert mod.weight.grad.dtype == dtype
    ref_dw = dyd.T @ xd
    mag_dw = np.abs(dyd).T @ np.abs(xd)
    if dtype == torch.bfloat16:
        ok, worst = _bf16_bound(bits(mod.weight.grad), ref_dw, mag_dw)
    else:
        ok, worst = _within(f64(mod.weight.grad), ref_dw, mag_dw, 2.0 ** -20, 2.0 ** -18)
    assert ok, ("dw", worst)
    ref_db = dyd.sum(0)
    mag_db = np.abs(dyd).sum(0)
    rel = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -20
    ok, worst = _within(f64(mod.bias.grad), ref_db, mag_db, rel, 2.0 ** -14)
    assert ok, ("db", worst)
