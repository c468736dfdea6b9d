"""The bias gradient dy.sum(dim=0) (reference python/xpu_kernels/int8/ops.py:276)
as the HIP column-sum pass, on the GPU: bit for bit the oracle's fixed order
(oracle.column_sum, itself pinned to the float64 sums), at config 5's
gradient shape and at ragged ones, and through the int8_linear backward."""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import activation, bits, mismatch, weight
from xpu_kernels import int8
from xpu_kernels.int8 import _lib as L

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,n", [(4096, 5120), (1, 16), (31, 48), (33, 2064), (1000, 4112),
                                 (4097, 272)])
def test_column_sum_exact(dev, m, n):
    g = torch.Generator().manual_seed(m + n)
    dy = (torch.randn(m, n, generator=g) * 1e-3).to(torch.bfloat16)
    dy[:, :3] *= 300                                           # large columns
    got = int8.column_sum(dy.to(dev))
    want = O.column_sum(bits(dy))
    assert np.array_equal(bits(got), want), mismatch(bits(got), want)
    # within one bf16 ulp of torch's own reduction
    ref = dy.to(dev).sum(0).float().cpu()
    assert torch.all((got.float().cpu() - ref).abs() <= ref.abs() * 2.0 ** -7 + 1e-30)


def test_column_sum_more_chunks_than_grid_rows(dev):
    """More 32-row chunks than a launch's 65535 block rows: the partial-sum
    kernel takes chunks c, c + 65535, ... per block row."""
    m, n = 65535 * 32 + 100, 16
    g = torch.Generator().manual_seed(77)
    dy = (torch.randn(m, n, generator=g) * 1e-3).to(torch.bfloat16)
    got = int8.column_sum(dy.to(dev))
    want = O.column_sum(bits(dy))
    assert np.array_equal(bits(got), want), mismatch(bits(got), want)


def test_column_sum_specials(dev):
    """NaN and infinities: a column holding a NaN, or both infinities, sums to
    NaN; one infinity sums to it -- whatever the order, as torch's sum does."""
    m, n = 100, 32
    dy = (torch.randn(m, n, generator=torch.Generator().manual_seed(9)) * 1e-3).to(torch.bfloat16)
    dy[7, 0] = float("nan")
    dy[3, 1] = float("inf")
    dy[90, 2] = float("-inf")
    dy[5, 3] = float("inf")
    dy[64, 3] = float("-inf")
    dy[40, 4] = float("nan")
    dy[41, 4] = float("inf")
    gb = bits(int8.column_sum(dy.to(dev)))
    got = torch.from_numpy(O.bf16_to_f32(gb).copy())
    want = O.column_sum(bits(dy))
    wnan = np.isnan(O.bf16_to_f32(want))
    # NaN payloads and signs are the hardware's own; the rest bit for bit
    assert np.array_equal(np.isnan(got.numpy()), wnan)
    assert np.array_equal(gb[~wnan], want[~wnan])
    ref = dy.sum(0).float()
    assert torch.equal(torch.isnan(got), torch.isnan(ref))
    assert torch.equal(torch.isinf(got), torch.isinf(ref))
    assert torch.isnan(got[[0, 3, 4]]).all() and got[1] == float("inf") and got[2] == float("-inf")
    fin = torch.isfinite(ref)
    assert torch.all((got[fin] - ref[fin]).abs() <= ref[fin].abs() * 2.0 ** -7 + 1e-30)


def test_column_sum_dirty_workspace(dev):
    """The workspace needs no clearing: a call on garbage partials equals one
    on zeros."""
    lib = L._lib()
    m, n = 300, 1040
    dy = (torch.randn(m, n, generator=torch.Generator().manual_seed(5))).to(torch.bfloat16).to(dev)
    nb = lib.xpuint8_column_sum_workspace_size(m, n)
    assert nb == ((m + 31) // 32) * n * 4
    outs = []
    for fill in (0, -1):
        work = torch.full((nb,), fill, device=dev, dtype=torch.int8)
        out = torch.empty(n, device=dev, dtype=torch.bfloat16)
        rc = lib.xpuint8_column_sum_stream(L._stream(dev), L._ptr(dy), L._ptr(out), m, n,
                                           L._ptr(work), nb)
        assert rc == 0, lib.xpuint8_last_error()
        outs.append(bits(out))
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(outs[0], O.column_sum(bits(dy)))


def test_int8_linear_bias_grad_int8_mode(dev):
    """int8_linear(mode="int8") at config 5's shape: dbias from the column-sum
    pass (bit for bit the oracle), dx from linear_dx_int8 (bit for bit)."""
    m, n, k = 4096, 5120, 1280
    x = activation(m, k, seed=41).to(dev).requires_grad_(True)
    w8, ws = int8.prepare_weight(weight(n, k, seed=42).to(dev))
    bias = torch.zeros(n, device=dev, dtype=torch.bfloat16, requires_grad=True)
    dy = (torch.randn(m, n, generator=torch.Generator().manual_seed(43)) * 1e-3).to(torch.bfloat16)
    y = int8.int8_linear(x, w8, ws, bias, mode="int8")
    y.backward(dy.to(dev))
    assert np.array_equal(bits(bias.grad), O.column_sum(bits(dy)))
    want = O.linear_dx_int8(bits(dy), w8.cpu().numpy(), ws.cpu().numpy())
    assert np.array_equal(bits(x.grad), want), mismatch(bits(x.grad), want)
