"""Two accumulator-consumer and weight-format features of the reference's
linear, on the GPU:

* linear(residual=, residual_scale=) (python/xpu_kernels/int8/ops.py:639-644):
  with a bf16 activation and a bf16 per-column (or single) scale the update
  ``residual + residual_scale * out`` runs in the GEMM's store; it must equal
  the reference chain -- the dequant result rounded to bf16, then
  torch.addcmul on bf16 tensors -- bit for bit, through every GEMM kernel
  (persistent, two-block, small, split-K, skinny).  Other forms run the
  reference's torch chain and keep its dtype promotion.
* Weight formats: per-channel scales stored as [N, 1] (the checkpoint shape,
  reference tests/test_int8_api.py:148-150), per-tensor scales, and an
  Int8Linear state_dict saved and loaded again (torch.save / torch.load with
  weights_only=True) give the same outputs bit for bit.
"""

import io

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import activation, bits, from_bits, mismatch, npy, weight
from xpu_kernels import int8

pytestmark = pytest.mark.gpu


def _residual_reference(d_bits, res_bits, scale_bits):
    """torch.addcmul(res, d, scale) on bf16 CPU tensors -- the reference's op."""
    t = lambda b: torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)
    out = torch.addcmul(t(res_bits), t(d_bits), t(scale_bits))
    return out.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("m,n,k", [(4096, 10240, 1280), (300, 1040, 1280), (33, 48, 256),
                                   (4096, 1280, 5120), (1000, 5120, 1280)])
def test_linear_residual_fused_exact(dev, m, n, k):
    x = activation(m, k, seed=m + 1)
    w8, ws = int8.prepare_weight(weight(n, k, seed=n).to(dev))
    bias = weight(1, n, seed=3, std=0.01)[0]
    g = torch.Generator().manual_seed(m + n)
    res = torch.randn(m, n, generator=g).to(torch.bfloat16)
    rscale = (torch.rand(n, generator=g) * 2 - 0.5).to(torch.bfloat16)
    got = int8.linear(x.to(dev), w8, ws, bias.to(dev), residual=res.to(dev),
                      residual_scale=rscale.to(dev))
    assert got.dtype == torch.bfloat16 and tuple(got.shape) == (m, n)
    d = O.linear(bits(x), npy(w8), npy(ws), O.bf16_to_f32(bits(bias)))
    want = _residual_reference(d, bits(res), bits(rscale))
    assert np.array_equal(bits(got), want), mismatch(bits(got), want)
    # the closed form of the same update: one fp32 add of an exact product
    f = lambda b: O.bf16_to_f32(b)
    closed = O.f32_to_bf16(f(bits(res)) + f(d) * f(bits(rscale))[None, :])
    assert np.array_equal(closed, want)


def test_linear_residual_scale_forms(dev):
    """A single-value scale and a [1, 1, N] scale take the fused path; a 3-D
    activation keeps its shape; an fp32 scale follows torch's promotion to an
    fp32 result, as the reference's addcmul does."""
    m, n, k = 2 * 64, 256, 512
    x = activation(m, k, seed=5).reshape(2, 64, k)
    w8, ws = int8.prepare_weight(weight(n, k, seed=6).to(dev))
    res = torch.randn(2, 64, n, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    d = O.linear(bits(x.reshape(m, k)), npy(w8), npy(ws))
    for scale in (torch.tensor([0.75], dtype=torch.bfloat16),
                  (torch.rand(1, 1, n, generator=torch.Generator().manual_seed(8))).to(torch.bfloat16)):
        got = int8.linear(x.to(dev), w8, ws, residual=res.to(dev), residual_scale=scale.to(dev))
        assert tuple(got.shape) == (2, 64, n) and got.dtype == torch.bfloat16
        sc = np.broadcast_to(bits(scale.reshape(-1)), (n,)).copy()
        want = _residual_reference(d, bits(res.reshape(m, n)), sc)
        assert np.array_equal(bits(got.reshape(m, n)), want), mismatch(bits(got.reshape(m, n)), want)
    s32 = torch.rand(n, generator=torch.Generator().manual_seed(9))
    got = int8.linear(x.to(dev), w8, ws, residual=res.to(dev), residual_scale=s32.to(dev))
    assert got.dtype == torch.float32
    want = torch.addcmul(torch.from_numpy(bits(res.reshape(m, n)).view(np.int16)).view(torch.bfloat16),
                         torch.from_numpy(d.view(np.int16)).view(torch.bfloat16), s32)
    assert torch.allclose(got.reshape(m, n).cpu(), want, rtol=1e-6, atol=1e-6)


def test_per_channel_scale_as_column(dev):
    """[N, 1] scales (how checkpoints store them) and a per-tensor scale: the
    same kernels, the same bits as the flat [N] scale."""
    m, n, k = 96, 512, 1280
    x = activation(m, k, seed=11).to(dev)
    w8, ws = int8.prepare_weight(weight(n, k, seed=12).to(dev))
    flat = int8.linear(x, w8, ws)
    col = int8.linear(x, w8, ws.reshape(n, 1))
    assert torch.equal(flat, col)
    mod = int8.Int8Linear(w8, ws.reshape(n, 1))
    assert torch.equal(mod(x), flat)
    want = O.linear(bits(x), npy(w8), npy(ws))
    assert np.array_equal(bits(flat), want)
    # per-tensor: a one-element tensor and a python float
    one = int8.linear(x, w8, torch.tensor([0.004], device=dev))
    want1 = O.linear(bits(x), npy(w8), np.full(n, 0.004, np.float32))
    assert np.array_equal(bits(one), want1)
    assert torch.equal(int8.linear(x, w8, 0.004), one)


@pytest.mark.parametrize("scale_shape", ["flat", "column"])
def test_int8_linear_state_dict_round_trip(dev, scale_shape):
    n, k = 640, 1280
    w = weight(n, k, seed=13).to(dev)
    bias = weight(1, n, seed=14, std=0.01)[0].to(dev)
    lin = torch.nn.Linear(k, n, bias=True, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(w)
        lin.bias.copy_(bias)
    mod = int8.Int8Linear.from_linear(lin)
    if scale_shape == "column":
        mod.w_scale = mod.w_scale.reshape(n, 1)
    buf = io.BytesIO()
    torch.save(mod.state_dict(), buf)
    buf.seek(0)
    sd = torch.load(buf, weights_only=True, map_location=dev)
    assert set(sd) == {"w8", "w_scale", "bias"} and sd["w8"].dtype == torch.int8
    fresh = int8.Int8Linear(torch.empty_like(sd["w8"]), torch.empty_like(sd["w_scale"]),
                            torch.empty(n, device=dev))
    fresh.load_state_dict(sd)
    x = activation(200, k, seed=15).to(dev)
    assert torch.equal(fresh(x), mod(x))
    q, s = O.prepare_weight(bits(w))
    assert np.array_equal(npy(fresh.w8), q)
    assert np.array_equal(npy(fresh.w_scale).reshape(-1), s)
