"""Pins for the oracle's quantizers, GEMM and epilogue.

Independent checks (not a retyping of the oracle's formulas):
* the float64 formula of the row quantizer (the reference's own check,
  tests/test_quantize.py:42-52) and its tie known-answer (:85-91);
* known answers derived from H: a constant row quantizes to +-127 everywhere;
  a zero row gives scale 1e-30 and zero codes;
* the reference's torch chains run literally in torch on the CPU
  (ops.py:94-99 prepare_weight, ops.py:327-330 quantize_row) on the oracle's
  rotated values: numpy float32 vs torch float32 semantics (division, round
  half even, clamp, bf16 conversion, the bf16 clamp floor);
* torch._int_mm on the CPU and brute-force int64 for the GEMM;
* the float64 dequant closed form (src/xpuint8.cpp:700-706) within a bf16 ulp;
* reference/convrot_linear.py's division-based chain against the kernel's
  reciprocal chain: code flips at most 1e-4 of elements.
"""

import numpy as np
import pytest
import torch

import oracle as O


def _bf16(rng, shape, scale=1.0, outliers=0):
    x = rng.standard_normal(shape).astype(np.float32) * np.float32(scale)
    if outliers:
        cols = rng.permutation(shape[-1])[:outliers]
        x[..., cols] *= np.float32(30.0)
    return O.f32_to_bf16(x)


def _t(bits):
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)


def _np(tbf16):
    return tbf16.contiguous().view(torch.int16).numpy().view(np.uint16)


# ----------------------------------------------------------------- bf16 / RNE
def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    f = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 7,
                        np.array([np.inf, -np.inf, 0.0, -0.0, 1e-40, 3.4e38], np.float32)])
    # include exact ties: low 16 bits == 0x8000
    ties = (rng.integers(0, 2**31, 2000).astype(np.uint32) & np.uint32(0xFFFF0000)) | np.uint32(0x8000)
    f = np.concatenate([f, ties.view(np.float32)])
    f = f[np.isfinite(f) | np.isinf(f)]
    want = _np(torch.from_numpy(f).to(torch.bfloat16))
    assert np.array_equal(O.f32_to_bf16(f), want)


# ------------------------------------------------------------- convrot quant
def test_convrot_quantize_against_float64_formula():
    rng = np.random.default_rng(1)
    x = _bf16(rng, (64, 1280), outliers=8)
    q, s = O.convrot_quantize(x)
    v = O.hadamard256(O.bf16_to_f32(x)).astype(np.float64)
    s64 = np.maximum(np.abs(v).max(axis=1) / 127.0, 1e-30)
    assert np.array_equal(s, s64.astype(np.float32))       # one correct rounding
    want = np.clip(np.round(v / s64[:, None]), -127, 127)
    d = np.abs(q.astype(np.float64) - want)
    assert d.max() <= 1 and (d > 0).mean() < 1e-3
    assert q.min() >= -127 and q.max() <= 127


def test_constant_and_zero_rows():
    x = np.zeros((3, 512), dtype=np.float32)
    x[0] = 0.5
    x[1] = -3.0
    q, s = O.convrot_quantize(O.f32_to_bf16(x))
    assert np.all(q[0] == 127) and np.all(q[1] == -127) and np.all(q[2] == 0)
    assert s[0] == np.float32(0.5) / np.float32(127) and s[1] == np.float32(3.0) / np.float32(127)
    assert s[2] == np.float32(1e-30)


def test_reciprocal_vs_division_flip_rate():
    """The kernel quantizer rint(v*(1/s)) against reference/convrot_linear.py's
    round(v/s): only rounding-boundary flips, by one unit, rarely."""
    rng = np.random.default_rng(2)
    x = _bf16(rng, (1024, 1280), outliers=8)
    v = O.hadamard256(O.bf16_to_f32(x))
    q, s = O.quantize_from_rotated(v)
    qd = np.clip(np.rint(v / s[:, None]), -127, 127).astype(np.int8)
    d = np.abs(q.astype(np.int16) - qd.astype(np.int16))
    assert d.max() <= 1 and (d > 0).mean() <= 1e-4


# --------------------------------------------------------------- quantize_row
def test_quantize_row_float64_formula():
    # the reference's own data recipe (tests/test_quantize.py:37-39, 42-52):
    # equal to the float64 formula everywhere
    g = torch.Generator().manual_seed(0)
    x = _np((torch.randn(8, 64, generator=g) * 0.4).to(torch.bfloat16))
    q, s = O.quantize_row(x)
    xf = O.bf16_to_f32(x).astype(np.float64)
    s64 = np.maximum(np.abs(xf).max(axis=1, keepdims=True) / 127.0, 1e-30)
    assert np.array_equal(q.astype(np.float64), np.clip(np.round(xf / s64), -127, 127))
    # on other data an exact float64 tie (x/s = k + 0.5) can round the other way
    # in fp32: at most one unit, rarely
    rng = np.random.default_rng(3)
    x = _bf16(rng, (64, 1024), scale=0.4)
    q, s = O.quantize_row(x)
    xf = O.bf16_to_f32(x).astype(np.float64)
    s64 = np.maximum(np.abs(xf).max(axis=1, keepdims=True) / 127.0, 1e-30)
    d = np.abs(q - np.clip(np.round(xf / s64), -127, 127))
    assert d.max() <= 1 and (d > 0).mean() < 1e-3


def test_quantize_row_ties_round_to_even():
    tie = O.f32_to_bf16(np.array([[127.0, 254.0, -254.0, 63.0]], dtype=np.float32))
    q, s = O.quantize_row(tie)
    assert q[0].tolist() == [64, 127, -127, 32] and s[0] == np.float32(2.0)


def test_quantize_row_matches_the_torch_chain():
    rng = np.random.default_rng(4)
    x = _bf16(rng, (256, 5120), scale=1e-3)
    x[7] = 0                                               # a zero row
    q, s = O.quantize_row(x)
    xt = _t(x).float()                                     # ops.py:327-330, verbatim
    st = (xt.abs().amax(dim=-1, keepdim=True) / 127.0).clamp_min(1e-30)
    qt = torch.round(xt / st).clamp_(-127, 127).to(torch.int8)
    assert np.array_equal(q, qt.numpy()) and np.array_equal(s, st.squeeze(-1).numpy())


# -------------------------------------------------------------- prepare_weight
def test_prepare_weight_matches_the_torch_chain():
    rng = np.random.default_rng(5)
    w = _bf16(rng, (96, 1280), scale=0.02)
    w[3] = 0                                               # zero row -> the bf16 floor
    w[4] = O.f32_to_bf16(np.full(1280, 1e-31, np.float32))  # below the floor
    q, s = O.prepare_weight(w)
    wr = _t(O.rotate_bf16(w))                              # ops.py:94-99, verbatim
    amax = wr.abs().amax(dim=1).clamp_min(1e-30)
    st = amax.float() / 127.0
    qt = torch.round(wr / st[:, None]).clamp_(-127, 127).to(torch.int8)
    assert np.array_equal(q, qt.numpy())
    assert np.array_equal(s.view(np.uint32), st.numpy().view(np.uint32))


def test_prepare_weight_fused_differs_only_in_last_bits():
    rng = np.random.default_rng(6)
    w = _bf16(rng, (64, 1024), scale=0.02)
    q1, s1 = O.prepare_weight(w)
    q2, s2 = O.prepare_weight_fused(w)
    assert np.max(np.abs(q1.astype(int) - q2.astype(int))) <= 1
    assert np.allclose(s1, s2, rtol=1e-2)


def test_rotate_bf16_roundtrip_is_close():
    rng = np.random.default_rng(7)
    x = _bf16(rng, (32, 512))
    back = O.bf16_to_f32(O.rotate_bf16(O.rotate_bf16(x))).reshape(32, 2, 256)
    xf = O.bf16_to_f32(x).reshape(32, 2, 256)
    # two bf16 roundings of rotated values: error ~ a bf16 ulp of the group's size
    rms = np.sqrt((xf.astype(np.float64) ** 2).mean(axis=-1, keepdims=True))
    assert np.max(np.abs(back - xf) / rms) < 2.0 ** -6


# --------------------------------------------------------------------- GEMM
def test_int_mm_matches_torch_and_brute_force():
    rng = np.random.default_rng(8)
    a = rng.integers(-127, 128, (33, 272), dtype=np.int8)
    b = rng.integers(-127, 128, (48, 272), dtype=np.int8)
    got = O.int_mm(a, b)
    want = torch._int_mm(torch.from_numpy(a), torch.from_numpy(b).t().contiguous()).numpy()
    assert np.array_equal(got, want)
    brute = np.einsum("mk,nk->mn", a.astype(np.int64), b.astype(np.int64))
    assert np.array_equal(got.astype(np.int64), brute)
    extreme = np.full((2, 4096), -127, np.int8)
    assert O.int_mm(extreme, extreme)[0, 0] == 127 * 127 * 4096


# ------------------------------------------------------------------- dequant
def test_dequant_closed_form_and_torch_chain():
    rng = np.random.default_rng(9)
    acc = rng.integers(-2**24, 2**24, (40, 64)).astype(np.int32)
    xs = rng.uniform(1e-3, 1e-1, 40).astype(np.float32)
    ws = rng.uniform(1e-4, 1e-2, 64).astype(np.float32)
    bias = rng.standard_normal(64).astype(np.float32)
    for b in (None, bias):
        got = O.dequant(acc, xs, ws, b)
        t = torch.from_numpy(acc).float() * (torch.from_numpy(ws)[None, :] * torch.from_numpy(xs)[:, None])
        if b is not None:
            t = t + torch.from_numpy(b)[None, :]
        assert np.array_equal(got, _np(t.to(torch.bfloat16)))
        exact = acc.astype(np.float64) * ws[None, :].astype(np.float64) * xs[:, None]
        if b is not None:
            exact = exact + b[None, :]
        g = O.bf16_to_f32(got).astype(np.float64)
        assert np.all(np.abs(g - exact) <= np.abs(exact) * 2.0 ** -8 + 1e-30)


def test_expand_scale():
    assert np.array_equal(O.expand_scale(np.float32(0.25), 5), np.full(5, 0.25, np.float32))
    col = np.arange(4, dtype=np.float32).reshape(4, 1)
    assert np.array_equal(O.expand_scale(col, 4), col.reshape(-1))
    with pytest.raises(ValueError):
        O.expand_scale(np.zeros(3, np.float32), 4)


# -------------------------------------------------------------------- linear
def test_linear_chain_against_float64_and_the_reference_oracle():
    """C1-like shape, scaled down: the kernel chain vs x @ W^T in float64, and
    vs the restated reference/convrot_linear.py fed the rotated activation."""
    rng = np.random.default_rng(10)
    x = _bf16(rng, (256, 1280), outliers=8)
    w = _bf16(rng, (384, 1280), scale=0.02)
    bias = _bf16(rng, (384,), scale=0.01)
    w8, ws = O.prepare_weight(w)
    y = O.bf16_to_f32(O.linear(x, w8, ws, O.bf16_to_f32(bias))).astype(np.float64)
    exact = (O.bf16_to_f32(x).astype(np.float64) @ O.bf16_to_f32(w).astype(np.float64).T
             + O.bf16_to_f32(bias))
    rel = np.linalg.norm(y - exact) / np.linalg.norm(exact)
    assert rel < 0.02
    ref = O.bf16_to_f32(O.convrot_int8_linear(O.hadamard256(O.bf16_to_f32(x)), w8, ws, bias))
    rel2 = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel2 < 1e-2
