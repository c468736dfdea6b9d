"""Parity of every HIP entry point with the CPU oracle, on the GPU.

Bar: bit-exact for integer, int8 and index results and for the int32
accumulators; bit-exact for bf16 outputs too (the kernels reproduce the
oracle's fp32 operation order), with the reference's own tolerances checked
separately against reference/convrot_linear.py's chain (int8 code flips
<= 1e-4 of elements, bf16 rel-err <= 1e-2).  Shapes cover tiny, ragged, the
two-pass long-row path, and the benchmark configurations at full size.
"""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import activation, bits, from_bits, mismatch, npy, weight
from xpu_kernels import int8
from xpu_kernels.int8 import _lib as L

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------ GEMM
@pytest.mark.parametrize("m,n,k", [(1, 16, 256), (32, 32, 64), (33, 48, 272), (128, 128, 1280),
                                   (300, 1040, 1280), (77, 4096, 4096)])
def test_int8_gemm_exact(dev, m, n, k):
    rng = np.random.default_rng(m * 7 + n + k)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    got = npy(int8.int_mm(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev).t()))
    want = O.int_mm(a, b)
    assert np.array_equal(got, want), mismatch(got, want)


def test_int8_gemm_extremes(dev):
    k = 8192
    a = np.full((64, k), -127, np.int8)
    b = np.full((64, k), -127, np.int8)
    b[1::2] = 127
    got = npy(int8.int_mm(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev).t()))
    assert np.array_equal(got, O.int_mm(a, b))


@pytest.mark.parametrize("m,n,k", [(40, 48, 96), (256, 512, 1280)])
def test_int8_gemm_nn_exact(dev, m, n, k):
    rng = np.random.default_rng(5)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (k, n), dtype=np.int8)          # row-major [K, N]
    got = npy(int8.int_mm(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)))
    assert np.array_equal(got, O.int_mm(a, np.ascontiguousarray(b.T)))


def test_int8_gemm_full_size_c3(dev):
    rng = np.random.default_rng(11)
    a = rng.integers(-127, 128, (4096, 1280), dtype=np.int8)
    b = rng.integers(-127, 128, (10240, 1280), dtype=np.int8)
    got = npy(int8.int_mm(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev).t()))
    assert np.array_equal(got, O.int_mm(a, b))


@pytest.mark.parametrize("m,n,k", [(2100, 10000, 1040), (4300, 6000, 272), (4352, 5120, 128),
                                   (4352, 5120, 192), (4096, 15360, 320)])
def test_persistent_tiles_exact(dev, m, n, k):
    """Shapes that take the persistent 256x320 kernel (one block per CU
    looping over tiles): ragged last row and column tiles, K not a multiple of
    64, and 288 / 323 / 272 tiles, so some blocks run two tiles and others
    one; two K steps (the next tile's loads issued between the tiles) and
    three (all of them issued from the previous tile's loop); 768 tiles of
    five K steps, three per block, so the LDS ring starts each tile at a
    different slot.  The int32 product, then the dequant epilogue (fp32
    bias, then bf16 bias) on the same operands."""
    rng = np.random.default_rng(m + n + k)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    want32 = O.int_mm(a, b)
    ta, tb = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    got = npy(int8.int_mm(ta, tb.t()))
    assert np.array_equal(got, want32), mismatch(got, want32)
    xs = rng.uniform(1e-3, 5e-2, m).astype(np.float32)
    ws = rng.uniform(1e-5, 1e-3, n).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float32)
    bias16 = O.f32_to_bf16(bias)
    lib = L._lib()
    t = lambda v: torch.from_numpy(v).to(dev)
    txs, tws = t(xs), t(ws)
    for bvec, kind, bref in ((t(bias), 0, bias), (t(bias16.view(np.int16)), 1, O.bf16_to_f32(bias16))):
        out = torch.empty((m, n), device=dev, dtype=torch.bfloat16)
        rc = lib.xpuint8_linear_gemm_stream(L._stream(dev), L._ptr(ta), L._ptr(txs), L._ptr(tb),
                                            L._ptr(tws), L._ptr(bvec), kind, L._ptr(out), m, n, k)
        assert rc == 0, lib.xpuint8_last_error()
        want = O.dequant(want32, xs, ws, bref)
        assert np.array_equal(bits(out), want), mismatch(bits(out), want)


@pytest.mark.parametrize("m,n,k", [(4096, 10240, 1280), (1000, 9728, 1152), (2560, 4112, 1104),
                                   (4352, 7808, 2560)])
def test_dequant_gemm_tiles_exact(dev, m, n, k):
    """The dequant GEMM entry (xpuint8_linear_gemm_stream) with no bias, an
    fp32 bias and a bf16 bias on: config 3; 232 rows in the last row tile and
    K = 1152; a 16-column last column tile and K = 1104 (zeros past K in the
    last step); 40 K steps over 4352 x 7808.  Each bit-exact against the
    oracle's dequant of the exact product."""
    rng = np.random.default_rng(m + 3 * n + k)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    want32 = O.int_mm(a, b)
    xs = rng.uniform(1e-3, 5e-2, m).astype(np.float32)
    ws = rng.uniform(1e-5, 1e-3, n).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float32)
    bias16 = O.f32_to_bf16(bias)
    lib = L._lib()
    t = lambda v: torch.from_numpy(v).to(dev)
    ta, tb, txs, tws = t(a), t(b), t(xs), t(ws)
    cases = ((None, 0, None), (t(bias), 0, bias),
             (t(bias16.view(np.int16)), 1, O.bf16_to_f32(bias16)))
    for bvec, kind, bref in cases:
        out = torch.full((m, n), -1, device=dev, dtype=torch.int16).view(torch.bfloat16)
        rc = lib.xpuint8_linear_gemm_stream(L._stream(dev), L._ptr(ta), L._ptr(txs), L._ptr(tb),
                                            L._ptr(tws), L._ptr(bvec) if bvec is not None else None,
                                            kind, L._ptr(out), m, n, k)
        assert rc == 0, lib.xpuint8_last_error()
        want = O.dequant(want32, xs, ws, bref)
        assert np.array_equal(bits(out), want), (kind, mismatch(bits(out), want))


# ------------------------------------------------------- rotate / quantize
QSHAPES = [(1, 256), (7, 1280), (64, 5120), (33, 8192), (5, 3072), (3, 10240), (2, 16384),
           (5, 4352), (3, 16896), (2, 32768), (2, 33792), (2, 66560), (3, 16640)]


@pytest.mark.parametrize("m,k", QSHAPES)
def test_convrot_quantize_exact(dev, m, k):
    x = activation(m, k, seed=m + k)
    q, s = int8.quantize(x.to(dev))
    wq, ws = O.convrot_quantize(bits(x))
    assert np.array_equal(npy(s).view(np.uint32), ws.view(np.uint32)), mismatch(npy(s), ws)
    assert np.array_equal(npy(q), wq), mismatch(npy(q), wq)


def test_convrot_quantize_full_size_c2(dev):
    x = activation(4096, 5120, seed=0)
    q, s = int8.quantize(x.to(dev))
    wq, ws = O.convrot_quantize(bits(x))
    assert np.array_equal(npy(s).view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(npy(q), wq), mismatch(npy(q), wq)
    # against the reference oracle's division chain: tie flips only
    v = O.hadamard256(O.bf16_to_f32(bits(x)))
    qd = np.clip(np.rint(v / ws[:, None]), -127, 127).astype(np.int8)
    d = np.abs(npy(q).astype(np.int16) - qd)
    assert d.max() <= 1 and (d > 0).mean() <= 1e-4


def test_quantize_special_rows(dev):
    x = np.zeros((4, 512), dtype=np.float32)
    x[1] = 0.5
    x[2] = -3.0
    x[3, 7] = 1e-35                       # a lone tiny value
    xb = O.f32_to_bf16(x)
    q, s = int8.quantize(from_bits(xb, dev))
    wq, ws = O.convrot_quantize(xb)
    assert np.array_equal(npy(q), wq) and np.array_equal(npy(s), ws)


def _huge_rows(k, seed=7):
    """bf16 rows at the top of the range, where the Hadamard's unscaled sums
    would overflow (max |x| in [2^120, 2^128)), mixed with ordinary rows and
    groups: a constant 2^124 row (a fixed point of the reference's chain),
    random signs and exponents in [120, 127), one huge group in an ordinary
    row (so the waves of one row take different transforms), a single spike
    of 2^127, values next to the bf16 maximum (the reference itself overflows
    on some outputs), an inf, and an ordinary row."""
    rng = np.random.default_rng(seed)
    sg = lambda: rng.choice([-1.0, 1.0], k)
    rows = [np.full(k, 2.0 ** 124), np.full(k, -2.0 ** 121),
            sg() * rng.uniform(1, 2, k) * 2.0 ** rng.integers(120, 127, k),
            sg() * rng.uniform(1, 2, k) * 2.0 ** rng.integers(110, 121, k)]
    r = rng.standard_normal(k)
    r[256:512] = sg()[:256] * 2.0 ** 125
    rows.append(r)
    r = np.zeros(k)
    r[5] = 2.0 ** 127
    rows.append(r)
    rows.append(sg() * 3.38e38)
    r = rng.standard_normal(k)
    r[3] = np.inf
    rows.append(r)
    rows.append(rng.standard_normal(k))
    return O.f32_to_bf16(np.array(rows, dtype=np.float32))


def _bf16_equal(a, b):
    """Bit equality of bf16 arrays, any NaN equal to any NaN (IEEE leaves the
    sign of an inf - inf NaN open, and x86 and the GPU differ on it)."""
    a, b = np.asarray(a, np.uint16), np.asarray(b, np.uint16)
    nan = lambda x: (x & 0x7FFF) > 0x7F80
    return bool(np.all((a == b) | (nan(a) & nan(b))))


def _finite_rows(xb):
    """The rows whose rotation the reference computes without overflow."""
    with np.errstate(over="ignore", invalid="ignore"):
        r = O.hadamard256(O.bf16_to_f32(xb))
    return np.isfinite(r).all(axis=1)


@pytest.mark.parametrize("k", [1280, 5120])
def test_rotate_huge_rows(dev, k):
    xb = _huge_rows(k)
    got = bits(int8.rotate(from_bits(xb, dev)))
    with np.errstate(over="ignore", invalid="ignore"):
        want = O.rotate_bf16(xb)
    assert _bf16_equal(got, want), mismatch(got, want)
    assert np.isinf(O.bf16_to_f32(want)).any()          # the reference's own overflow is covered


@pytest.mark.parametrize("k", [1280, 5120, 16896, 33024])
def test_quantize_huge_rows(dev, k):
    """The ConvRot quantizer on rows the reference rotates without overflow,
    through the one-group (k <= 64 groups), two-group (16896) and two-pass
    (33024 = 129 groups) row kernels."""
    xb = _huge_rows(k)[_finite_rows(_huge_rows(k))]
    assert len(xb) >= 4
    q, s = int8.quantize(from_bits(xb, dev))
    wq, ws = O.convrot_quantize(xb)
    assert np.array_equal(npy(s).view(np.uint32), ws.view(np.uint32)), mismatch(npy(s), ws)
    assert np.array_equal(npy(q), wq), mismatch(npy(q), wq)


@pytest.mark.parametrize("k", [1280, 5120])
def test_prepare_weight_huge_rows(dev, k):
    wb = _huge_rows(k, seed=8)
    wb = wb[_finite_rows(wb)]
    q, s = int8.prepare_weight(from_bits(wb, dev))
    wq, ws = O.prepare_weight(wb)
    assert np.array_equal(npy(s).view(np.uint32), ws.view(np.uint32)), mismatch(npy(s), ws)
    assert np.array_equal(npy(q), wq), mismatch(npy(q), wq)


@pytest.mark.parametrize("act", [4, 5])
def test_quantize_act_huge_rows(dev, act):
    """gelu_erf keeps a huge positive input (x * Phi(x) = x) and GEGLU multiplies
    a huge hidden value by gelu(gate): the activation's output reaches the
    scaled transform's range."""
    k = 1280
    h = _huge_rows(k, seed=9)
    h = h[_finite_rows(h)]
    rows = len(h)
    if act == 4:
        gate = np.abs(O.bf16_to_f32(bits(activation(rows, k, seed=10, n_out=0)))) + np.float32(0.5)
        x = np.concatenate([h, O.f32_to_bf16(gate)], axis=1)
    else:
        x = O.f32_to_bf16(np.abs(O.bf16_to_f32(h)))
    name = {v: kk for kk, v in int8.ACTIVATIONS.items()}[act]
    xb = np.ascontiguousarray(x)
    with np.errstate(over="ignore", invalid="ignore"):
        wq, ws = O.quantize_act(xb, act)
    keep = np.isfinite(ws) & (ws > 0)
    q, s = int8.quantize_act(from_bits(xb, dev), name)
    assert np.array_equal(npy(s)[keep].view(np.uint32), ws[keep].view(np.uint32)), mismatch(npy(s), ws)
    assert np.array_equal(npy(q)[keep], wq[keep]), mismatch(npy(q)[keep], wq[keep])
    assert keep.sum() >= 3


@pytest.mark.parametrize("act", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("m,k", [(9, 1280), (16, 5120)])
def test_quantize_act_exact(dev, act, m, k):
    name = {v: kk for kk, v in int8.ACTIVATIONS.items()}[act]
    width = 2 * k if act in O.PAIRED else k
    x = activation(m, width, seed=act * 100 + m, scale=1.5)
    q, s = int8.quantize_act(x.to(dev), name)
    wq, ws = O.quantize_act(bits(x), act)
    assert np.array_equal(npy(s), ws), mismatch(npy(s), ws)
    assert np.array_equal(npy(q), wq), mismatch(npy(q), wq)


# bf16 bit patterns on both sides of the table windows the activation
# quantizers read from LDS (|x| in [2^-20, 256)): zeros, denormals, the largest
# value below 2^-20, 2^-20, values around 2^-12 and 16 (the GEMM epilogue's
# window edges), the largest value below 256, 256, and values far outside
WINDOW_EDGES = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x357F, 0xB57F, 0x3580, 0xB580,
                         0x397F, 0xB97F, 0x3980, 0xB980, 0x417F, 0xC17F, 0x4180, 0xC180,
                         0x437F, 0xC37F, 0x4380, 0xC380, 0x447A, 0xC47A, 0x3F80, 0xBF80],
                        np.uint16)


@pytest.mark.parametrize("act", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("m,k", [(7, 1280), (2, 20480)])
def test_quantize_act_window_edges(dev, act, m, k):
    """Every lookup operand on a window edge or outside it, mixed into ordinary
    rows: the LDS lookups, the global-table fallback of a partly missing wave,
    and (k = 20480, two groups per lane) the kernel without the window."""
    name = {v: kk for kk, v in int8.ACTIVATIONS.items()}[act]
    width = 2 * k if act in O.PAIRED else k
    x = bits(activation(m, width, seed=act + k, scale=1.5))
    rng = np.random.default_rng(act * 7 + m)
    pick = rng.random((m, width)) < 0.3
    x[pick] = rng.choice(WINDOW_EDGES, int(pick.sum()))
    x[0, :len(WINDOW_EDGES)] = WINDOW_EDGES                  # one lane's values all on edges
    q, s = int8.quantize_act(from_bits(x, dev), name)
    wq, ws = O.quantize_act(x, act)
    assert np.array_equal(npy(s), ws), mismatch(npy(s), ws)
    assert np.array_equal(npy(q), wq), mismatch(npy(q), wq)


@pytest.mark.parametrize("act", [3, 4, 5])
@pytest.mark.parametrize("k", [1280, 20480])
def test_dequant_act_quantize_window_edges(dev, act, k):
    """Dequantized values on the window edges: with both scales 2^-10 the
    value is bf16(acc * 2^-20), so acc = 1 gives 2^-20, 256 gives 2^-12, 255
    the largest value below it, 2^24 gives 16, 2^28 gives 256 and 2^28 - 2^20
    the largest value below it; rows with x_scale 2^-14 take acc * 2^-24,
    where 15 falls below 2^-20 and 16 is on it."""
    m = 6
    n = 2 * k if act in O.PAIRED else k
    rng = np.random.default_rng(act + k)
    edges = np.array([0, 1, -1, 15, -15, 16, -16, 255, -255, 256, -256, 2 ** 24 - 2 ** 16,
                      -(2 ** 24 - 2 ** 16), 2 ** 24, -(2 ** 24), 2 ** 28 - 2 ** 20,
                      -(2 ** 28 - 2 ** 20), 2 ** 28, -(2 ** 28), 2 ** 30, -(2 ** 30), 2 ** 20,
                      -(2 ** 20)], np.int64)
    acc = rng.integers(-2 ** 22, 2 ** 22, (m, n))
    pick = rng.random((m, n)) < 0.4
    acc[pick] = rng.choice(edges, int(pick.sum()))
    acc = acc.astype(np.int32)
    xs = np.where(np.arange(m) % 2 == 0, 2.0 ** -10, 2.0 ** -14).astype(np.float32)
    ws = np.full(n, 2.0 ** -10, np.float32)
    name = {v: kk for kk, v in int8.ACTIVATIONS.items()}[act]
    t = lambda a: torch.from_numpy(a).to(dev)
    q, s = int8.dequant_act_quantize(t(acc), t(xs), t(ws), name)
    wq, wsc = O.dequant_act_quantize(acc, xs, ws, act)
    assert np.array_equal(npy(s), wsc), mismatch(npy(s), wsc)
    assert np.array_equal(npy(q), wq), mismatch(npy(q), wq)


@pytest.mark.parametrize("m,k", [(1, 256), (13, 1280), (64, 5120), (3, 20480)])
def test_rotate_exact(dev, m, k):
    x = activation(m, k, seed=k)
    got = bits(int8.rotate(x.to(dev)))
    want = O.rotate_bf16(bits(x))
    assert np.array_equal(got, want), mismatch(got, want)


@pytest.mark.parametrize("n,k", [(16, 256), (48, 1280), (10240, 1280)])
def test_prepare_weight_exact(dev, n, k):
    w = weight(n, k, seed=n)
    if n == 48:
        w[3] = 0
        w[5] = 1e-31
    q, s = int8.prepare_weight(w.to(dev))
    wq, ws = O.prepare_weight(bits(w))
    assert np.array_equal(npy(s).view(np.uint32), ws.view(np.uint32)), mismatch(npy(s), ws)
    assert np.array_equal(npy(q), wq), mismatch(npy(q), wq)


def test_prepare_weight_fused_is_the_quantizer(dev):
    w = weight(64, 1280)
    q, s = int8.prepare_weight_fused(w.to(dev))
    wq, ws = O.prepare_weight_fused(bits(w))
    assert np.array_equal(npy(q), wq) and np.array_equal(npy(s), ws)


@pytest.mark.parametrize("n,k", [(32, 512), (5120, 1280)])
def test_dequant_weight_exact(dev, n, k):
    w8, ws = O.prepare_weight(bits(weight(n, k)))
    got = bits(int8.dequant_weight(torch.from_numpy(w8).to(dev), torch.from_numpy(ws).to(dev)))
    want = O.dequant_weight(w8, ws)
    assert np.array_equal(got, want), mismatch(got, want)


@pytest.mark.parametrize("m,n", [(1, 16), (8, 64), (33, 1040), (4096, 5120), (3, 100), (1, 4)])
def test_quantize_row_exact(dev, m, n):
    dy = activation(m, n, seed=m, scale=1e-3, n_out=0)
    q, s = int8.quantize_row(dy.to(dev))
    wq, ws = O.quantize_row(bits(dy))
    assert np.array_equal(npy(s).view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(npy(q), wq), mismatch(npy(q), wq)
    # torch's chain run *on the GPU* divides by the python scalar 127 through a
    # reciprocal, so its scale can be one ulp off the CPU chain (the oracle):
    # agreement there is to within that ulp and one code unit
    qt, st = int8.quantize_row_torch(dy.to(dev))
    ds = np.abs(npy(s).view(np.int32).astype(np.int64) - npy(st).view(np.int32))
    assert ds.max() <= 1
    assert (npy(q).astype(np.int16) - npy(qt)).__abs__().max() <= 1


def test_quantize_row_ties(dev):
    tie = torch.tensor([[127.0, 254.0, -254.0, 63.0] + [0.0] * 12], dtype=torch.bfloat16)
    q, s = int8.quantize_row(tie.to(dev))
    assert npy(q)[0, :4].tolist() == [64, 127, -127, 32] and float(s[0]) == 2.0


def test_quantize_row_column_scaled(dev):
    dy = activation(64, 1280, seed=9, scale=1e-3, n_out=0)
    wsc = (torch.rand(1280, generator=torch.Generator().manual_seed(3)) * 1e-3).float()
    q, s = int8.quantize_row(dy.to(dev), wsc.to(dev))
    d = O.f32_to_bf16(O.bf16_to_f32(bits(dy)) * O.bf16_round(npy(wsc))[None, :])
    wq, ws = O.quantize_row(d)
    assert np.array_equal(npy(q), wq) and np.array_equal(npy(s), ws)


@pytest.mark.parametrize("m,n", [(1, 16), (3, 48), (5, 1040), (7, 5120), (33, 16384),
                                 (2, 16400)])
def test_quantize_row_column_scaled_edges(dev, m, n):
    """The column-scaled quantizer at its edges: one row, odd row counts (a
    row pair's second row past M), widths that leave the last wave partly
    idle, the widest row one block of lanes takes (16384) and one past it
    (the segmented kernel); a row of zeros takes the scale floor."""
    dy = activation(m, n, seed=m + n, scale=1e-3, n_out=0)
    dy[m // 2] = 0
    wsc = (torch.rand(n, generator=torch.Generator().manual_seed(n)) * 1e-3).float()
    q, s = int8.quantize_row(dy.to(dev), wsc.to(dev))
    d = O.f32_to_bf16(O.bf16_to_f32(bits(dy)) * O.bf16_round(npy(wsc))[None, :])
    wq, ws = O.quantize_row(d)
    assert np.array_equal(npy(s).view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(npy(q), wq), mismatch(npy(q), wq)


# ------------------------------------------------------------- epilogues
def test_dequant_rounding_edge_cases(dev):
    """The bf16 conversion at its edges, through the dequant epilogue: exact
    ties (acc = 2^8 + odd, unit scales: RNE to even), values past the bf16
    maximum (round to inf), fp32 denormal results, infinities and NaNs of
    either sign in the column scale (quiet NaN with the sign kept)."""
    rng = np.random.default_rng(5)
    n = 64
    ties = np.array([257, 259, 261, 263, -257, -259, 513, 515], np.int32)
    acc = np.stack([np.resize(ties, n),
                    rng.integers(-2 ** 30, 2 ** 30, n),
                    rng.integers(-2 ** 20, 2 ** 20, n),
                    rng.integers(1, 2 ** 8, n)]).astype(np.int32)
    xs = np.array([1.0, 2.0 ** 100, 2.0 ** -120, 1.0], np.float32)
    ws = np.ones(n, np.float32)
    ws[8:16] = 2.0 ** 27                     # row 1: |acc| * 2^127 -> past bf16 max
    ws[16:24] = np.float32(3.0e-8)           # row 2: denormal products
    ws[24:28] = [np.inf, -np.inf, np.nan, -np.nan]
    t = lambda a: torch.from_numpy(a).to(dev)
    got = bits(int8.dequant(t(acc), t(xs), t(ws)))
    want = O.dequant(acc, xs, ws)
    assert np.array_equal(got, want), mismatch(got, want)


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("m,n", [(37, 96), (5, 1040), (3, 2064), (9, 4112), (2, 10240)])
def test_dequant_and_slice_exact(dev, bias, m, n):
    """Row widths on both sides of the kernel's 1024-column slot and
    2048-column block boundaries; the slice is read from a wider row."""
    rng = np.random.default_rng(2 + n)
    acc = rng.integers(-2**22, 2**22, (m, n)).astype(np.int32)
    xs = rng.uniform(1e-3, 1e-1, m).astype(np.float32)
    ws = rng.uniform(1e-4, 1e-2, n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32) if bias else None
    t = lambda a: torch.from_numpy(a).to(dev)
    got = bits(int8.dequant(t(acc), t(xs), t(ws), None if b is None else t(b)))
    want = O.dequant(acc, xs, ws, b)
    assert np.array_equal(got, want), mismatch(got, want)
    wide = t(np.concatenate([acc, acc[:, :32]], axis=1))
    sl = bits(int8.dequant_slice(wide[:, :n], t(xs), t(ws), None if b is None else t(b)))
    assert np.array_equal(sl, want)


@pytest.mark.parametrize("act", [3, 4, 5])
def test_dequant_act_quantize_exact(dev, act):
    m, k = 24, 1280
    n = 2 * k if act in O.PAIRED else k
    rng = np.random.default_rng(act)
    acc = rng.integers(-300000, 300000, (m, n)).astype(np.int32)
    xs = rng.uniform(1e-3, 3e-2, m).astype(np.float32)
    ws = rng.uniform(1e-4, 1e-3, n).astype(np.float32)
    name = {v: kk for kk, v in int8.ACTIVATIONS.items()}[act]
    t = lambda a: torch.from_numpy(a).to(dev)
    q, s = int8.dequant_act_quantize(t(acc), t(xs), t(ws), name)
    wq, wsc = O.dequant_act_quantize(acc, xs, ws, act)
    assert np.array_equal(npy(s), wsc) and np.array_equal(npy(q), wq), mismatch(npy(q), wq)


# -------------------------------------------------------- linear / ffn / dx
def test_linear_exact_c1(dev):
    """Config 1's shapes and recipe (8 outlier channels x20)."""
    x = activation(1024, 1280, seed=0, n_out=8, mult=20.0)
    w = weight(1280, 1280, seed=1)
    bias = weight(1, 1280, seed=2, std=0.01)[0]
    w8, ws = int8.prepare_weight(w.to(dev))
    y = int8.linear(x.to(dev), w8, ws, bias.to(dev))
    want = O.linear(bits(x), npy(w8), npy(ws), O.bf16_to_f32(bits(bias)))
    assert np.array_equal(bits(y), want), mismatch(bits(y), want)
    # a bf16 bias is read by the epilogue directly, an fp32 one as it is: same bits
    y32 = int8.linear(x.to(dev), w8, ws, bias.float().to(dev))
    assert np.array_equal(bits(y32), want)
    # the reference oracle (reference/convrot_linear.py) fed the rotated activation
    ref = O.convrot_int8_linear(O.hadamard256(O.bf16_to_f32(bits(x))), npy(w8), npy(ws),
                                bits(bias))
    yf, rf = O.bf16_to_f32(bits(y)).astype(np.float64), O.bf16_to_f32(ref).astype(np.float64)
    assert np.linalg.norm(yf - rf) / np.linalg.norm(rf) < 1e-2


def test_linear_full_size_c3(dev):
    x = activation(4096, 1280, seed=0)
    w = weight(10240, 1280, seed=1)
    bias = weight(1, 10240, seed=2, std=0.01)[0]
    w8, ws = int8.prepare_weight(w.to(dev))
    y = int8.linear(x.to(dev), w8, ws, bias.to(dev))
    want = O.linear(bits(x), npy(w8), npy(ws), O.bf16_to_f32(bits(bias)))
    assert np.array_equal(bits(y), want), mismatch(bits(y), want)
    acc, xs = int8.linear_acc(x.to(dev), w8, ws)
    same = int8.dequant(acc, xs, ws, bias.to(dev))
    assert torch.equal(same.view(torch.int16), y.view(torch.int16))


@pytest.mark.parametrize("m,n,k", [(2100, 1280, 5120), (4096, 1296, 2304), (300, 1040, 1280)])
def test_linear_one_call_exact(dev, m, n, k):
    """xpuint8_linear_stream (quantize and GEMM in one call, the quantized
    activation in its workspace): bit-exact against the oracle's linear with
    an fp32 and a bf16 bias and with none.  The first two shapes take the
    split-K kernel, which reads the activation in the MFMA block layout
    written by the quantizer (ragged last row block, a 16-column last column
    tile, K = 2304); the third a row-major activation."""
    x = activation(m, k, seed=m, n_out=8, mult=20.0)
    w = weight(n, k, seed=n)
    bias = weight(1, n, seed=k, std=0.01)[0]
    w8, ws = int8.prepare_weight(w.to(dev))
    lib = L._lib()
    need = lib.xpuint8_linear_workspace_size(m, n, k)
    assert need > 0
    work = torch.empty(need, device=dev, dtype=torch.uint8)
    xd = x.to(dev)
    for bvec, kind, bref in ((None, 0, None), (bias.float(), 0, O.bf16_to_f32(bits(bias))),
                             (bias, 1, O.bf16_to_f32(bits(bias)))):
        out = torch.empty((m, n), device=dev, dtype=torch.bfloat16)
        bd = bvec.to(dev) if bvec is not None else None
        rc = lib.xpuint8_linear_stream(L._stream(dev), L._ptr(xd), L._ptr(w8), L._ptr(ws),
                                       L._ptr(bd) if bd is not None else None, kind, L._ptr(out),
                                       m, n, k, L._ptr(work), need)
        assert rc == 0, lib.xpuint8_last_error()
        want = O.linear(bits(x), npy(w8), npy(ws), bref)
        assert np.array_equal(bits(out), want), (kind, mismatch(bits(out), want))


# one shape per kernel the plain linear dispatches to (M <= 64: the skinny
# kernel; few tiles: the 128 x 128 kernel; more: the two-block 256 x 160
# kernel; a 256 x 320 tile per CU: the persistent kernel; narrow output with
# a long K: split K over the block-layout activation), with ragged rows and
# columns
@pytest.mark.parametrize("m,n,k", [(16, 528, 768), (64, 2048, 1024), (65, 1040, 512),
                                   (2000, 4000, 512), (4100, 5120, 256), (1500, 1920, 2048),
                                   (2050, 1296, 3072)])
def test_linear_dispatch_sweep(dev, m, n, k):
    """int8.linear through each GEMM kernel, bit-exact against the oracle."""
    x = activation(m, k, seed=m + k, n_out=4, mult=25.0)
    w = weight(n, k, seed=n + 1)
    bias = weight(1, n, seed=n + k, std=0.01)[0]
    w8, ws = int8.prepare_weight(w.to(dev))
    y = int8.linear(x.to(dev), w8, ws, bias.to(dev))
    want = O.linear(bits(x), npy(w8), npy(ws), O.bf16_to_f32(bits(bias)))
    assert np.array_equal(bits(y), want), mismatch(bits(y), want)


# Too few 128 x 160 output tiles for the chip: the product split in K across
# blocks (4, 4 and 4 slices through the split-K kernel; 32 and 2 through the
# 128 x 128 kernel for M <= 256; 2, 4, 4 and 2 through the skinny kernel for
# 33 <= M <= 128, with 8, 4, 7 and 3 row blocks), the int32 partial sums
# added by the dequant pass; ragged row and column tiles (1296 columns: a
# half-empty last pair of weight blocks); with a bf16 bias, an fp32 bias and
# none
@pytest.mark.parametrize("m,n,k", [(1024, 1280, 5120), (2048, 640, 5120), (1000, 1296, 4096),
                                   (200, 160, 16384), (128, 4096, 4096), (65, 4080, 1024),
                                   (64, 1280, 5120), (100, 1296, 5120), (33, 1040, 2048)])
def test_linear_k_slices_exact(dev, m, n, k):
    x = activation(m, k, seed=m + 2 * k, n_out=4, mult=25.0)
    w = weight(n, k, seed=n + 3)
    bias = weight(1, n, seed=n + k + 1, std=0.01)[0]
    w8, ws = int8.prepare_weight(w.to(dev))
    acc, xs = O.linear_acc(bits(x), npy(w8))              # the oracle's linear, shared
    for b in (bias.to(dev), bias.float().to(dev), None):
        y = int8.linear(x.to(dev), w8, ws, b)
        bref = None if b is None else O.bf16_to_f32(bits(bias))
        want = O.dequant(acc, xs, npy(ws), bref)
        assert np.array_equal(bits(y), want), (None if b is None else b.dtype,
                                               mismatch(bits(y), want))


# Each side of every threshold of the linear's GEMM choice: M = 32 / 33
# (skinny kernel / K slices on it), N = 2048 / 2032 at M = 64 (the skinny
# kernel whole / in K slices), M = 64 / 65 at N = 2048 (skinny kernel / K
# slices on it), M = 128 / 129 (slices on the skinny / 128 x 128 kernel), no
# skinny slice of 1024 at M = 128, N = 5120, K = 1280 (slices on the 128 x 128
# kernel), M = 256 / 257 (slices on the 128 x 128 / split-K kernel), 104 tiles
# of 128 x 160 (slices), exactly 128 tiles (the split-K kernel) at K = 1024,
# 1280 and 2048, and 17 tiles with K = 1280 (too short to split: the
# 128 x 128 kernel); ragged N
@pytest.mark.parametrize("m,n,k", [(32, 1280, 2048), (33, 1280, 2048), (64, 2048, 2048),
                                   (64, 2032, 2048), (65, 2048, 2048), (128, 1280, 4096),
                                   (129, 1280, 4096), (128, 5120, 1280),
                                   (64, 1280, 2048), (65, 1280, 2048), (256, 2560, 1024),
                                   (257, 2560, 2048), (1016, 2032, 2048), (1024, 2560, 1024),
                                   (1024, 2560, 2048), (2048, 1264, 1280), (2048, 1264, 1024),
                                   (2176, 160, 1280)])
def test_linear_dispatch_boundaries(dev, m, n, k):
    x = activation(m, k, seed=3 * m + k, n_out=4, mult=25.0)
    w = weight(n, k, seed=n + 5)
    bias = weight(1, n, seed=n + k + 2, std=0.01)[0]
    w8, ws = int8.prepare_weight(w.to(dev))
    y = int8.linear(x.to(dev), w8, ws, bias.to(dev))
    want = O.linear(bits(x), npy(w8), npy(ws), O.bf16_to_f32(bits(bias)))
    assert np.array_equal(bits(y), want), mismatch(bits(y), want)


def test_linear_shapes_and_dtypes(dev):
    x = activation(2 * 3 * 5, 512, seed=3).reshape(2, 3, 5, 512)
    w = weight(48, 512)
    w8, ws = int8.prepare_weight(w.to(dev))
    y = int8.linear(x.to(dev), w8, ws)
    assert y.shape == (2, 3, 5, 48) and y.dtype == torch.bfloat16
    y32 = int8.linear(x.float().to(dev), w8, ws)
    assert y32.dtype == torch.float32 and torch.equal(y32, y.float())
    want = O.linear(bits(x.reshape(30, 512)), npy(w8), npy(ws))
    assert np.array_equal(bits(y.reshape(30, 48)), want)


def test_ffn_geglu_exact(dev):
    m, k, inner = 512, 1280, 1280
    x = activation(m, k, seed=4)
    up8, ups = int8.prepare_weight(weight(2 * inner, k, seed=5).to(dev))
    dn8, dns = int8.prepare_weight(weight(k, inner, seed=6).to(dev))
    db = weight(1, k, seed=7, std=0.01)[0].float()
    y = int8.ffn(x.to(dev), up8, ups, dn8, dns, db.to(dev), act="geglu_erf")
    want = O.ffn(bits(x), npy(up8), npy(ups), npy(dn8), npy(dns), npy(db), act=4)
    assert np.array_equal(bits(y), want), mismatch(bits(y), want)


@pytest.mark.parametrize("m", [1, 64, 128, 200, 1024])
def test_ffn_small_batch_k_slices_exact(dev, m):
    """An FFN whose down-projection (K = 5120, N = 1280) has too few output
    tiles to fill the chip: the product is split in K across blocks (4 slices
    on the skinny kernel at M = 64 and 128, 8 on the 128 x 128 kernel at
    M = 200, 4 on the split-K kernel at M = 1024; the skinny kernel whole at
    M = 1).  Up to M = 128 the up-projection takes the skinny kernel with the
    hidden and gate rows in one block."""
    k, inner = 1280, 5120
    x = activation(m, k, seed=11 + m)
    up8, ups = int8.prepare_weight(weight(2 * inner, k, seed=12).to(dev))
    dn8, dns = int8.prepare_weight(weight(k, inner, seed=13).to(dev))
    db = weight(1, k, seed=14, std=0.01)[0].float()
    y = int8.ffn(x.to(dev), up8, ups, dn8, dns, db.to(dev), act="geglu_erf")
    want = O.ffn(bits(x), npy(up8), npy(ups), npy(dn8), npy(dns), npy(db), act=4)
    assert np.array_equal(bits(y), want), mismatch(bits(y), want)


def test_ffn_stream_dirty_workspace_exact(dev):
    """xpuint8_ffn_stream through the C ABI on a workspace full of 0xFF, with a
    bf16 bias, then again on the same (now used) workspace with a smaller M.
    The down-projection is split in K across blocks in both (2 slices on the
    split-K kernel at M = 1000, 4 on the 128 x 128 kernel at M = 130); both
    equal the oracle."""
    k, inner = 1280, 2048
    up8, ups = int8.prepare_weight(weight(2 * inner, k, seed=21).to(dev))
    dn8, dns = int8.prepare_weight(weight(k, inner, seed=22).to(dev))
    db = weight(1, k, seed=23, std=0.01)[0].to(dev)
    lib = L._lib()
    need = lib.xpuint8_ffn_workspace_size(1000, inner, k, 4)
    work = torch.full((need,), 255, device=dev, dtype=torch.uint8)
    for m in (1000, 130):
        assert lib.xpuint8_ffn_workspace_size(m, inner, k, 4) <= need
        x = activation(m, k, seed=24 + m).to(dev)
        out = torch.empty((m, k), device=dev, dtype=torch.bfloat16)
        rc = lib.xpuint8_ffn_stream(L._stream(dev), L._ptr(x), L._ptr(up8), L._ptr(ups),
                                    L._ptr(dn8), L._ptr(dns), L._ptr(db), 1, L._ptr(out), m,
                                    inner, k, 4, L._ptr(work), need)
        assert rc == 0, lib.xpuint8_last_error()
        want = O.ffn(bits(x.cpu()), npy(up8), npy(ups), npy(dn8), npy(dns),
                     O.bf16_to_f32(bits(db.cpu())), act=4)
        assert np.array_equal(bits(out), want), (m, mismatch(bits(out), want))


@pytest.mark.parametrize("act", [3, 4, 5])
@pytest.mark.parametrize("m,inner,k", [(300, 512, 1280), (64, 1280, 1040), (512, 256, 256),
                                       (1, 512, 1280), (17, 768, 256), (40, 256, 4096),
                                       (100, 512, 1280), (128, 768, 1040), (50, 784, 512),
                                       (200, 512, 1280), (256, 784, 1040)])
def test_ffn_up_epilogue_exact(dev, act, m, inner, k):
    """The up-projection GEMM's activation epilogue against the oracle's
    dequant_act of the int32 product (ragged M, a partial last column tile,
    K not a multiple of 64).  M <= 64 (M <= 256 for the paired activations)
    takes the weight-streaming skinny kernel: for the paired ones two output
    column blocks (hidden and gate rows of each) per block, 4 waves, the last
    block half past the end at 784 columns, above 128 rows in 128-row chunks
    over grid.y (72 and 128 rows in the second chunk); for GELU one block of
    16 rows, 4 waves, 16 at K = 4096."""
    check_ffn_up(dev, act, m, inner, k)


@pytest.mark.parametrize("act", [4, 5])
def test_ffn_up_persistent_tiles_exact(dev, act):
    """The same through the persistent 256x320 kernel: 578 paired tiles
    (GEGLU) or 289 plain ones (GELU), ragged in both dimensions, K % 64 != 0."""
    check_ffn_up(dev, act, 4100, 5200, 1040)


@pytest.mark.parametrize("act", [4, 5])
def test_ffn_up_wide_range_exact(dev, act):
    """The persistent kernel reads the GELU (erf) table through a window in LDS
    that holds the inputs with |g| in [2^-12, 16), and the table in global
    memory for the others: column scales spread over twelve decades put the
    activation's inputs on both sides of the window, both signs, in every
    wave."""
    check_ffn_up(dev, act, 4100, 5200, 1040, wide=True)


def check_ffn_up(dev, act, m, inner, k, wide=False):
    rng = np.random.default_rng(act * 100 + m)
    rows = 2 * inner if act in O.PAIRED else inner
    xq = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w8 = rng.integers(-127, 128, (rows, k), dtype=np.int8)
    xs = rng.uniform(0.01, 0.05, m).astype(np.float32)
    if wide:
        ws = (10.0 ** rng.uniform(-11, 1, rows)).astype(np.float32)
    else:
        ws = rng.uniform(1e-5, 1e-4, rows).astype(np.float32)
    out = torch.empty((m, inner), device=dev, dtype=torch.bfloat16)
    lib = L._lib()
    t = [torch.from_numpy(a).to(dev) for a in (xq, xs, w8, ws)]
    rc = lib.xpuint8_ffn_up_stream(L._stream(dev), L._ptr(t[0]), L._ptr(t[1]), L._ptr(t[2]),
                                   L._ptr(t[3]), L._ptr(out), m, inner, k, act)
    assert rc == 0, lib.xpuint8_last_error()
    want = O.f32_to_bf16(O.dequant_act(O.int_mm(xq, w8), xs, ws, act))
    assert np.array_equal(bits(out), want), mismatch(bits(out), want)


@pytest.mark.parametrize("act", ["situ", "gelu_erf"])
def test_ffn_other_activations_exact(dev, act):
    m, k, inner = 272, 1280, 768
    x = activation(m, k, seed=12)
    rows = 2 * inner if act == "situ" else inner
    up8, ups = int8.prepare_weight(weight(rows, k, seed=13).to(dev))
    dn8, dns = int8.prepare_weight(weight(k, inner, seed=14).to(dev))
    y = int8.ffn(x.to(dev), up8, ups, dn8, dns, None, act=act)
    want = O.ffn(bits(x), npy(up8), npy(ups), npy(dn8), npy(dns), None,
                 act=int8.ACTIVATIONS[act])
    assert np.array_equal(bits(y), want), mismatch(bits(y), want)


def test_ffn_full_size_c4(dev):
    """Config 4: x [4096,1280] -> GEGLU [4096,5120] -> [4096,1280]."""
    x = activation(4096, 1280, seed=3)
    up8, ups = int8.prepare_weight(weight(10240, 1280, seed=4).to(dev))
    dn8, dns = int8.prepare_weight(weight(1280, 5120, seed=5).to(dev))
    db = weight(1, 1280, seed=6, std=0.01)[0]
    y = int8.ffn(x.to(dev), up8, ups, dn8, dns, db.to(dev), act="geglu_erf")
    want = O.ffn(bits(x), npy(up8), npy(ups), npy(dn8), npy(dns), O.bf16_to_f32(bits(db)), act=4)
    assert np.array_equal(bits(y), want), mismatch(bits(y), want)


# (2080, 3000, 1200) and (2048, 4000, 1280) take the split-K kernel with
# ragged output rows and columns, the first with an odd number of 32-row
# contraction steps
@pytest.mark.parametrize("m,n,k", [(4096, 5120, 1280), (1000, 272, 208), (1, 16, 16),
                                   (77, 1280, 4096), (300, 2000, 2000), (33, 2400, 1600),
                                   (2080, 3000, 1200), (2048, 4000, 1280)])
def test_linear_dw(dev, m, n, k):
    """dL/dW = dy^T x through the bf16 MFMA kernel, against float64: each
    element within one bf16 rounding of the exact value plus the fp32
    accumulation error (bounded by 2^-14 * sum |dy| |x|)."""
    g = torch.Generator().manual_seed(m + n + k)
    dy = (torch.randn(m, n, generator=g) * 1e-3).to(torch.bfloat16)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    dw = int8.linear_dw(dy.to(dev), x.to(dev))
    assert dw.dtype == torch.bfloat16 and tuple(dw.shape) == (n, k)
    ref = O.linear_dw(bits(dy), bits(x))
    mag = np.abs(O.bf16_to_f32(bits(dy)).astype(np.float64)).T @ \
        np.abs(O.bf16_to_f32(bits(x)).astype(np.float64))
    got = O.bf16_to_f32(bits(dw)).astype(np.float64)
    err = np.abs(got - ref)
    assert np.all(err <= 2.0 ** -8 * np.abs(ref) + 2.0 ** -14 * mag), float(
        np.max(err / (2.0 ** -8 * np.abs(ref) + 2.0 ** -14 * mag)))


@pytest.mark.parametrize("m,n,k", [(16, 4096, 4096), (64, 1024, 1280), (50, 160, 4112), (1, 32, 48),
                                   (17, 256, 8192)])
def test_skinny_gemm_exact(dev, m, n, k):
    """M <= 64 takes the weight-streaming kernel: int32 and fused-dequant forms."""
    rng = np.random.default_rng(m * 7 + n)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    acc = npy(int8.int_mm(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev).t()))
    want = O.int_mm(a, b)
    assert np.array_equal(acc, want)
    xs = rng.uniform(0.01, 0.05, m).astype(np.float32)
    ws = rng.uniform(1e-5, 1e-4, n).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32) * 0.01
    t = [torch.from_numpy(v).to(dev) for v in (a, xs, b, ws, bias)]
    out = torch.empty((m, n), device=dev, dtype=torch.bfloat16)
    lib = L._lib()
    rc = lib.xpuint8_linear_gemm_stream(L._stream(dev), L._ptr(t[0]), L._ptr(t[1]), L._ptr(t[2]),
                                        L._ptr(t[3]), L._ptr(t[4]), 0, L._ptr(out), m, n, k)
    assert rc == 0, lib.xpuint8_last_error()
    assert np.array_equal(bits(out), O.dequant(want, xs, ws, bias))


@pytest.mark.parametrize("m,n,k", [(2100, 1296, 2064), (4096, 1280, 5120)])
def test_split_k_gemm_exact(dev, m, n, k):
    """Narrow output, long K: the split-K kernel (ragged M and N tiles, K not a
    multiple of 64), through the fused-dequant entry point."""
    rng = np.random.default_rng(m + k)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    xs = rng.uniform(0.01, 0.05, m).astype(np.float32)
    ws = rng.uniform(1e-5, 1e-4, n).astype(np.float32)
    t = [torch.from_numpy(v).to(dev) for v in (a, xs, b, ws)]
    out = torch.empty((m, n), device=dev, dtype=torch.bfloat16)
    lib = L._lib()
    rc = lib.xpuint8_linear_gemm_stream(L._stream(dev), L._ptr(t[0]), L._ptr(t[1]), L._ptr(t[2]),
                                        L._ptr(t[3]), None, 0, L._ptr(out), m, n, k)
    assert rc == 0, lib.xpuint8_last_error()
    want = O.dequant(O.int_mm(a, b), xs, ws)
    assert np.array_equal(bits(out), want), mismatch(bits(out), want)


def test_linear_dx_int8_full_size_c5(dev):
    dy = activation(4096, 5120, seed=8, scale=1e-3, n_out=0)
    w8, ws = int8.prepare_weight(weight(5120, 1280, seed=9).to(dev))
    dx = int8.linear_dx_int8(dy.to(dev), w8, ws)
    want = O.linear_dx_int8(bits(dy), npy(w8), npy(ws))
    assert np.array_equal(bits(dx), want), mismatch(bits(dx), want)


@pytest.mark.parametrize("m,n,k", [(2048, 2080, 1280), (4096, 4096, 768), (1024, 2048, 1280)])
def test_linear_dx_int8_split_k_shapes(dev, m, n, k):
    """Shapes where dx's GEMM reads the weight as stored (the split-K kernel's
    transposing LDS reads): a contraction that is not a multiple of 64
    (2080, zero-filled tail), output columns that leave a partial 160-wide
    tile (768), and a short one (2048)."""
    dy = activation(m, n, seed=n, scale=1e-3, n_out=0)
    w8, ws = int8.prepare_weight(weight(n, k, seed=k).to(dev))
    dx = int8.linear_dx_int8(dy.to(dev), w8, ws)
    want = O.linear_dx_int8(bits(dy), npy(w8), npy(ws))
    assert np.array_equal(bits(dx), want), mismatch(bits(dx), want)


@pytest.mark.parametrize("m,n,k", [(200, 5120, 1280), (1024, 5120, 1280), (300, 2560, 1024),
                                   (64, 5120, 1280), (100, 5120, 1280)])
def test_linear_dx_int8_k_slices_exact(dev, m, n, k):
    """Small batches, too few output tiles for the chip: the contraction is
    split across blocks (8 slices on the 128 x 128 kernel through the
    transposed weight at M = 200; 4 and 2 slices on the split-K kernel
    reading the weight as stored, the last with a ragged 160-column tile; 4
    slices on the skinny kernel through the transposed weight at M = 64 and
    100)."""
    dy = activation(m, n, seed=m + n, scale=1e-3, n_out=0)
    w8, ws = int8.prepare_weight(weight(n, k, seed=k + 1).to(dev))
    dx = int8.linear_dx_int8(dy.to(dev), w8, ws)
    want = O.linear_dx_int8(bits(dy), npy(w8), npy(ws))
    assert np.array_equal(bits(dx), want), mismatch(bits(dx), want)


def test_linear_dx_int8_exact(dev):
    m, n, k = 512, 1280, 1280
    dy = activation(m, n, seed=8, scale=1e-3, n_out=0)
    w8, ws = int8.prepare_weight(weight(n, k, seed=9).to(dev))
    dx = int8.linear_dx_int8(dy.to(dev), w8, ws)
    want = O.linear_dx_int8(bits(dy), npy(w8), npy(ws))
    assert np.array_equal(bits(dx), want), mismatch(bits(dx), want)


def test_int8_linear_autograd(dev):
    x = activation(256, 512, seed=10).to(dev).float().requires_grad_(True)
    w = weight(64, 512, seed=11).to(dev)
    bias = torch.zeros(64, device=dev, requires_grad=True)
    w8, ws = int8.prepare_weight(w)
    dy = torch.randn(256, 64, generator=torch.Generator().manual_seed(0)).to(dev)
    for mode in ("int8", "dense"):
        x.grad = None
        bias.grad = None
        y = int8.int8_linear(x, w8, ws, bias, mode=mode)
        y.backward(dy)
        exact = dy @ w.float()
        rel = ((x.grad - exact).norm() / exact.norm()).item()
        assert rel < 0.05, (mode, rel)
        assert torch.allclose(bias.grad, dy.sum(0))
