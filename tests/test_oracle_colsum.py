"""Pins for the oracle's column sum (the bias gradient dy.sum(dim=0) of the
reference's backward, python/xpu_kernels/int8/ops.py:276).

Independent checks, each failing for a plausible mistake (the wrong axis, a
dropped row or chunk, a second rounding):
* the float64 exact column sums, within the float32 summation bound of the
  build's chunked order plus half a bf16 ulp;
* closed forms: a constant column of v sums to M * v exactly; columns of
  +v / -v pairs sum to zero;
* torch's own dy.sum(dim=0) on bf16 (CPU), within one bf16 ulp.
"""

import numpy as np
import pytest
import torch

import oracle as O


def _bits(rng, m, n, scale=1e-3):
    return O.f32_to_bf16((rng.standard_normal((m, n)) * scale).astype(np.float32))


@pytest.mark.parametrize("m,n", [(1, 16), (31, 48), (33, 16), (200, 272), (1000, 96), (4096, 64)])
def test_column_sum_float64_bound(m, n):
    rng = np.random.default_rng(m * 31 + n)
    x = _bits(rng, m, n)
    got = O.bf16_to_f32(O.column_sum(x)).astype(np.float64)
    xf = O.bf16_to_f32(x).astype(np.float64)
    exact = xf.sum(axis=0)
    depth = (O.COL_CHUNK - 1) + (m + O.COL_CHUNK - 1) // O.COL_CHUNK + 8
    fp32_err = depth * 2.0 ** -24 * np.abs(xf).sum(axis=0)
    half_ulp = np.maximum(np.abs(exact) + fp32_err, 1e-38) * 2.0 ** -8
    assert np.all(np.abs(got - exact) <= fp32_err + half_ulp)
    # the wrong axis or a dropped row is far outside the bound
    assert not np.allclose(got[: min(n, m)], xf.sum(axis=1)[: min(n, m)])


def test_column_sum_closed_forms():
    m, n = 4096, 32
    v = O.f32_to_bf16(np.array([0.15625, -3.0, 1e-3, 7.5], dtype=np.float32))
    x = np.tile(np.repeat(v, 8), (m, 1))                      # constant columns
    want = O.f32_to_bf16(O.bf16_to_f32(np.repeat(v, 8)) * np.float32(m))
    assert np.array_equal(O.column_sum(x), want)
    y = x.copy()
    y[1::2] ^= np.uint16(0x8000)                               # +v, -v, +v, ...
    assert np.all(O.bf16_to_f32(O.column_sum(y)) == 0.0)


def test_column_sum_torch_chain():
    rng = np.random.default_rng(7)
    x = _bits(rng, 777, 160, scale=0.5)
    t = torch.from_numpy(x.view(np.int16).copy()).view(torch.bfloat16)
    ref = t.sum(dim=0).float().numpy()
    got = O.bf16_to_f32(O.column_sum(x))
    ulp = np.abs(ref) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - ref) <= ulp)
