"""Seeded random shapes over the whole dispatch space of the linear, the FFN and
linear_dx_int8, each bit-exact against the oracle.

The GEMM a call takes depends on M, N and K: the skinny kernel (M <= 64;
M <= 256 for the FFN's paired up-projection, in 128-row chunks above 128),
K slices on the skinny, the 128 x 128 or the split-K kernel for outputs too
small to fill the chip (then a dequant pass that adds the slices), the
split-K and the persistent kernels on the activation in MFMA-block order,
and the two-block kernel.  The fixed-shape tests sit on each side of every
threshold; these draw shapes between them (ragged M, N any multiple of 16, K
any multiple of 256), so that no combination of tile remainders and slice
counts goes untested.  Shapes are drawn once from fixed seeds and appear in
the test ids.
"""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import activation, bits, mismatch, npy, weight
from xpu_kernels import int8

pytestmark = pytest.mark.gpu


def _draw_m(rng):
    band = int(rng.integers(0, 4))
    lo, hi = [(1, 65), (65, 129), (129, 513), (513, 2600)][band]
    return int(rng.integers(lo, hi))


def _linear_shapes(count, seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        m = _draw_m(rng)
        n = 16 * int(rng.integers(1, 385))            # 16 .. 6144
        k = 256 * int(rng.integers(1, 33))            # 256 .. 8192
        if m * n * k <= 8e9:
            out.append((m, n, k))
    return out


def _ffn_shapes(count, seed=20261203):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        m = _draw_m(rng)
        k = 256 * int(rng.integers(1, 9))             # model width 256 .. 2048
        inner = 256 * int(rng.integers(1, 17))        # 256 .. 4096
        act = int(rng.choice([3, 4, 5]))
        if m * inner * k <= 3e9:
            out.append((m, k, inner, act))
    return out


def _dx_shapes(count, seed=20261204):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        m = _draw_m(rng)
        n = 16 * int(rng.integers(1, 385))            # contraction 16 .. 6144
        k = 256 * int(rng.integers(1, 21))            # output width 256 .. 5120
        if m * n * k <= 4e9:
            out.append((m, n, k))
    return out


LINEAR = _linear_shapes(30)
FFN = _ffn_shapes(10)
DX = _dx_shapes(10)


@pytest.mark.parametrize("m,n,k", LINEAR, ids=[f"{m}x{n}x{k}" for m, n, k in LINEAR])
def test_linear_random_shapes_exact(dev, m, n, k):
    x = activation(m, k, seed=m + 7 * n + k, n_out=3, mult=25.0)
    w8, ws = int8.prepare_weight(weight(n, k, seed=n + k).to(dev))
    bias = weight(1, n, seed=n + 3 * k, std=0.01)[0]
    y = int8.linear(x.to(dev), w8, ws, bias.to(dev))
    want = O.linear(bits(x), npy(w8), npy(ws), O.bf16_to_f32(bits(bias)))
    assert np.array_equal(bits(y), want), mismatch(bits(y), want)


@pytest.mark.parametrize("m,k,inner,act", FFN,
                         ids=[f"{m}x{k}x{inner}-act{a}" for m, k, inner, a in FFN])
def test_ffn_random_shapes_exact(dev, m, k, inner, act):
    name = {3: "situ", 4: "geglu_erf", 5: "gelu_erf"}[act]
    rows = 2 * inner if act in O.PAIRED else inner
    x = activation(m, k, seed=m + k + inner)
    up8, ups = int8.prepare_weight(weight(rows, k, seed=inner + 1).to(dev))
    dn8, dns = int8.prepare_weight(weight(k, inner, seed=inner + 2).to(dev))
    db = weight(1, k, seed=k + 5, std=0.01)[0]
    y = int8.ffn(x.to(dev), up8, ups, dn8, dns, db.to(dev), act=name)
    want = O.ffn(bits(x), npy(up8), npy(ups), npy(dn8), npy(dns), O.bf16_to_f32(bits(db)),
                 act=act)
    assert np.array_equal(bits(y), want), mismatch(bits(y), want)


@pytest.mark.parametrize("m,n,k", DX, ids=[f"{m}x{n}x{k}" for m, n, k in DX])
def test_linear_dx_int8_random_shapes_exact(dev, m, n, k):
    dy = activation(m, n, seed=m + n + 2 * k, scale=1e-3, n_out=0)
    w8, ws = int8.prepare_weight(weight(n, k, seed=k + n).to(dev))
    dx = int8.linear_dx_int8(dy.to(dev), w8, ws)
    want = O.linear_dx_int8(bits(dy), npy(w8), npy(ws))
    assert np.array_equal(bits(dx), want), mismatch(bits(dx), want)


# ------------------------------------------------------------ row kernels
# The row kernels pick their launch shape from K: rows per block (4, 2 or 1
# for K = 256-2048, longer rows), one or two groups per lane (K up to 16384
# or 32768), the two-pass kernel beyond; the quantize_row one also takes any
# N % 16 (a partial last group).

def _row_shapes(count, seed, kmax_groups, elems=3e7):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        g = int(rng.integers(1, kmax_groups + 1))
        m = int(rng.integers(1, 3000))
        if m * 256 * g <= elems:
            out.append((m, 256 * g))
    return out


QUANT = _row_shapes(12, 20261205, 280)
ACTQ = [(m, k, a) for (m, k), a in zip(_row_shapes(10, 20261206, 40, 1e7),
                                       np.random.default_rng(7).integers(1, 6, 10).tolist())]
QROW = [(m, 16 * int(n)) for m, n in zip(np.random.default_rng(8).integers(1, 2500, 10).tolist(),
                                        np.random.default_rng(9).integers(1, 1200, 10).tolist())]
WPREP = _row_shapes(6, 20261207, 40, 2e7)


@pytest.mark.parametrize("m,k", QUANT, ids=[f"{m}x{k}" for m, k in QUANT])
def test_quantize_and_rotate_random_shapes_exact(dev, m, k):
    x = activation(m, k, seed=m + k)
    q, s = int8.quantize(x.to(dev))
    wq, ws = O.convrot_quantize(bits(x))
    assert np.array_equal(npy(s).view(np.uint32), ws.view(np.uint32)), mismatch(npy(s), ws)
    assert np.array_equal(npy(q), wq), mismatch(npy(q), wq)
    got = bits(int8.rotate(x.to(dev)))
    want = O.rotate_bf16(bits(x))
    assert np.array_equal(got, want), mismatch(got, want)


@pytest.mark.parametrize("m,k,act", ACTQ, ids=[f"{m}x{k}-act{a}" for m, k, a in ACTQ])
def test_quantize_act_random_shapes_exact(dev, m, k, act):
    name = {v: kk for kk, v in int8.ACTIVATIONS.items()}[act]
    width = 2 * k if act in O.PAIRED else k
    x = activation(m, width, seed=act + m + k, scale=1.5)
    q, s = int8.quantize_act(x.to(dev), name)
    wq, ws = O.quantize_act(bits(x), act)
    assert np.array_equal(npy(s), ws), mismatch(npy(s), ws)
    assert np.array_equal(npy(q), wq), mismatch(npy(q), wq)
    if act in (3, 4, 5):
        # the same activation from an int32 accumulator
        rng = np.random.default_rng(m + k)
        acc = rng.integers(-300000, 300000, (m, width)).astype(np.int32)
        xs = rng.uniform(1e-3, 3e-2, m).astype(np.float32)
        wsc = rng.uniform(1e-4, 1e-3, width).astype(np.float32)
        t = lambda a: torch.from_numpy(a).to(dev)
        q2, s2 = int8.dequant_act_quantize(t(acc), t(xs), t(wsc), name)
        wq2, ws2 = O.dequant_act_quantize(acc, xs, wsc, act)
        assert np.array_equal(npy(s2), ws2) and np.array_equal(npy(q2), wq2), \
            mismatch(npy(q2), wq2)


@pytest.mark.parametrize("m,n", QROW, ids=[f"{m}x{n}" for m, n in QROW])
def test_quantize_row_random_shapes_exact(dev, m, n):
    dy = activation(m, n, seed=m + n, scale=1e-3, n_out=0)
    q, s = int8.quantize_row(dy.to(dev))
    wq, ws = O.quantize_row(bits(dy))
    assert np.array_equal(npy(s).view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(npy(q), wq), mismatch(npy(q), wq)


@pytest.mark.parametrize("n,k", WPREP, ids=[f"{n}x{k}" for n, k in WPREP])
def test_prepare_and_dequant_weight_random_shapes_exact(dev, n, k):
    w = weight(n, k, seed=n + k)
    q, s = int8.prepare_weight(w.to(dev))
    wq, ws = O.prepare_weight(bits(w))
    assert np.array_equal(npy(s).view(np.uint32), ws.view(np.uint32)), mismatch(npy(s), ws)
    assert np.array_equal(npy(q), wq), mismatch(npy(q), wq)
    got = bits(int8.dequant_weight(q, s))
    want = O.dequant_weight(wq, ws)
    assert np.array_equal(got, want), mismatch(got, want)


# ------------------------------------------------------- bf16 dense GEMMs
# linear_dx (dy @ w) and linear_dw (dy^T @ x) in bf16: the split-K kernel,
# K slices for small batches, the 128 x 128 TN / NN kernels for the shapes
# the split-K kernel does not take (dims % 16 only).  Bar: each element
# within one bf16 rounding of the float64 product plus the fp32 accumulation
# error, 2^-8 |ref| + 2^-14 sum |a||b|.

def _dense_shapes(count, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        m = _draw_m(rng)
        n = 16 * int(rng.integers(1, 320))
        k = 16 * int(rng.integers(1, 320))
        if m * n * k <= 4e9:
            out.append((m, n, k))
    return out


DENSE = _dense_shapes(12, 20261208)


def _bound_ok(got_bits, ref, mag):
    got = O.bf16_to_f32(got_bits).astype(np.float64)
    bound = 2.0 ** -8 * np.abs(ref) + 2.0 ** -14 * mag
    err = np.abs(got - ref)
    return bool(np.all(err <= bound)), float(np.max(err / np.maximum(bound, 1e-300)))


@pytest.mark.parametrize("m,n,k", DENSE, ids=[f"{m}x{n}x{k}" for m, n, k in DENSE])
def test_linear_dx_dw_random_shapes(dev, m, n, k):
    g = torch.Generator().manual_seed(m + 3 * n + k)
    dy = (torch.randn(m, n, generator=g) * 1e-3).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    a_dy = np.abs(O.bf16_to_f32(bits(dy)).astype(np.float64))
    dx = int8.linear_dx(dy.to(dev), w.to(dev))
    ok, worst = _bound_ok(bits(dx), O.linear_dx(bits(dy), bits(w)),
                          a_dy @ np.abs(O.bf16_to_f32(bits(w)).astype(np.float64)))
    assert ok, ("dx", worst)
    dw = int8.linear_dw(dy.to(dev), x.to(dev))
    ok, worst = _bound_ok(bits(dw), O.linear_dw(bits(dy), bits(x)),
                          a_dy.T @ np.abs(O.bf16_to_f32(bits(x)).astype(np.float64)))
    assert ok, ("dw", worst)
