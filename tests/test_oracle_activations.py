"""Pins for the oracle's activations (oracle/activations.py) and the library's
host-side activation tables, over all 65536 bf16 inputs.

* GELU-erf against torch's CPU ``F.gelu(approximate='none')`` -- the function
  the reference proved bit-identical to its kernel (debug/probe_gelu_torch.py):
  identical on every normal input with |x| <= 3; below -3 torch's fp32 erf
  loses accuracy in 1 + erf (cancellation), and there the oracle is the one
  within a bf16 ulp of the float64 GELU.
* every activation within one bf16 ulp of its float64 closed form (away from
  subnormal and overflow ranges);
* the tables the library uploads (xpuint8_activation_table, computed in C++
  from the same fp32 formulas) equal the oracle exactly, NaN for NaN.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle as O

BITS = np.arange(65536, dtype=np.uint32).astype(np.uint16)
X = O.bf16_to_f32(BITS)
E = (BITS.astype(np.int32) >> 7) & 0xFF
NORMAL = (E > 0) & (E < 255)


def _ulp_diff(a, b):
    """Distance in bf16 ulps between two bf16 bit patterns of the same sign."""
    ia, ib = a.astype(np.int32), b.astype(np.int32)
    sa = np.where(ia & 0x8000, -(ia & 0x7FFF), ia & 0x7FFF)
    sb = np.where(ib & 0x8000, -(ib & 0x7FFF), ib & 0x7FFF)
    return np.abs(sa - sb)


def _gelu_oracle():
    with np.errstate(all="ignore"):
        return O.f32_to_bf16(O.gelu_erf_f32(X))


def test_gelu_matches_torch_where_torch_is_accurate():
    ours = _gelu_oracle()
    t = torch.from_numpy(BITS.view(np.int16).copy()).view(torch.bfloat16)
    theirs = torch.nn.functional.gelu(t, approximate="none").view(torch.int16).numpy().view(np.uint16)
    sel = NORMAL & (np.abs(X) <= 3.0) & (np.abs(X) >= 1e-30)
    assert np.array_equal(ours[sel], theirs[sel])
    # below -3 the two may differ; the oracle is the accurate one
    bad = NORMAL & (ours != theirs) & (np.abs(X) < 1e30) & (np.abs(X) >= 1e-30)
    exact = 0.5 * X.astype(np.float64) * torch.special.erfc(
        torch.from_numpy(-X.astype(np.float64) / np.sqrt(2.0))).numpy()
    assert np.all(X[bad] < -3.0)
    err_ours = np.abs(O.bf16_to_f32(ours[bad]) - exact[bad])
    err_torch = np.abs(O.bf16_to_f32(theirs[bad]) - exact[bad])
    assert np.all(err_ours <= err_torch)


def _exact(fn):
    with np.errstate(all="ignore"):
        return fn(X.astype(np.float64))


@pytest.mark.parametrize("name", ["gelu_erf", "gelu_tanh", "silu", "sigmoid"])
def test_activations_within_one_ulp_of_float64(name):
    erf = lambda z: torch.special.erf(torch.from_numpy(z)).numpy()
    exact = {
        "gelu_erf": lambda x: 0.5 * x * (1.0 + erf(x / np.sqrt(2.0))),
        "gelu_tanh": lambda x: 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * x * (1 + 0.044715 * x * x))),
        "silu": lambda x: x / (1.0 + np.exp(-x)),
        "sigmoid": lambda x: 1.0 / (1.0 + np.exp(-x)),
    }[name]
    with np.errstate(all="ignore"):
        ours = {
            "gelu_erf": lambda: O.f32_to_bf16(O.gelu_erf_f32(X)),
            "gelu_tanh": lambda: O.f32_to_bf16(O.gelu_tanh_f32(X)),
            "silu": lambda: O.f32_to_bf16(X / (np.float32(1) + O.exp_f32(-X))),
            "sigmoid": lambda: O.f32_to_bf16(np.float32(1) / (np.float32(1) + O.exp_f32(-X))),
        }[name]()
    ref = O.f32_to_bf16(_exact(exact).astype(np.float32))
    sel = NORMAL & (np.abs(X) >= 2.0 ** -60) & (np.abs(X) <= 2.0 ** 60)
    if name in ("gelu_erf", "gelu_tanh"):
        # 1 + erf (1 + tanh) cancels below about -3: there the fp32 formula keeps
        # only the absolute accuracy of erf (2^-25), many bf16 ulps of a tiny result
        sel &= X > -3.0
    fin = sel & np.isfinite(O.bf16_to_f32(ref)) & (np.abs(O.bf16_to_f32(ref)) > 2.0 ** -120)
    assert np.max(_ulp_diff(ours[fin], ref[fin])) <= 1


def _lib():
    from xpu_kernels.int8 import _lib as L
    path = L.library_path()
    if path is None:
        pytest.skip("libxpuint8.so not built")
    return L.open_library(path)


def _table(lib, i):
    out = np.zeros(65536, dtype=np.uint16)
    assert lib.xpuint8_activation_table(i, out.ctypes.data_as(ctypes.c_void_p)) == 0
    return out


def test_library_tables_equal_the_oracle():
    lib = _lib()
    with np.errstate(all="ignore"):
        want = {
            0: O.f32_to_bf16(O.gelu_erf_f32(X)),
            1: O.f32_to_bf16(O.gelu_tanh_f32(X)),
            2: O.f32_to_bf16(X / (np.float32(1) + O.exp_f32(-X))),
            3: O.f32_to_bf16(O.tanh_fast_f32(O.bf16_round(X / np.float32(4)))),
            4: O.f32_to_bf16(np.float32(1) / (np.float32(1) + O.exp_f32(-X))),
            5: O.f32_to_bf16(O.tanh_fast_f32(O.bf16_round(X / np.float32(25)))),
        }
    for i, w in want.items():
        got = _table(lib, i)
        nan_g = (got & 0x7FFF) > 0x7F80
        nan_w = (w & 0x7FFF) > 0x7F80
        assert np.array_equal(nan_g, nan_w), i
        assert np.array_equal(got[~nan_g], w[~nan_w]), i


def test_library_situ_gate_table_is_situ_at_unit_hidden_factor():
    """Table 6 is situ's gate factor: with a hidden value whose factor
    tanh(bf16(h/25)) rounds to exactly 1, the oracle's whole situ activation
    of (h, g) is that table's entry for g, over every bf16 gate value."""
    lib = _lib()
    h = np.full_like(X, np.float32(1000.0))
    assert np.all(O.bf16_to_f32(O.f32_to_bf16(O.tanh_fast_f32(O.bf16_round(h / np.float32(25))))) == 1)
    with np.errstate(all="ignore"):
        want = O.f32_to_bf16(O.activate(3, h, X))
    got = _table(lib, 6)
    nan_g = (got & 0x7FFF) > 0x7F80
    nan_w = (want & 0x7FFF) > 0x7F80
    assert np.array_equal(nan_g, nan_w)
    assert np.array_equal(got[~nan_g], want[~nan_w])


def test_activate_composes_the_tables():
    """The paired activations are table lookups plus exact bf16 products."""
    rng = np.random.default_rng(0)
    a = O.bf16_round(rng.standard_normal(4096).astype(np.float32) * 3)
    b = O.bf16_round(rng.standard_normal(4096).astype(np.float32) * 3)
    y = O.bf16_round(O.gelu_erf_f32(b))
    assert np.array_equal(O.activate(4, a, b), O.bf16_round(a * y))
    assert np.array_equal(O.activate(5, a), O.bf16_round(O.gelu_erf_f32(a)))
    # products of two bf16 values are exact in fp32
    assert np.array_equal((a.astype(np.float64) * y).astype(np.float32).astype(np.float64),
                          a.astype(np.float64) * y)
