"""Pins for the oracle's composite chains (oracle/convrot.py, oracle/activations.py)
that the Hadamard/quantizer tests do not already cover: dequant_weight,
linear_dx_int8, the activations feeding quantize_act / dequant_act, the fused
dequant+activation+quantize and the FFN.

Each is checked two independent ways:

* against the reference's own torch chain, re-run here with torch on the CPU
  (python/xpu_kernels/int8/ops.py: dequant_weight 103-?, linear_dx_int8
  353-377, ffn 649-719; the eager activations the C kernels reproduce,
  src/xpuint8.cpp:120-160, 186-220), where torch computes every step in its
  own code (bf16 tensors, torch._int_mm);
* against float64 mathematics (the FFN and both backward paths must
  approximate the unquantized operator within the INT8 error), which a wrong
  operand, a missing rotation or a transposed weight cannot pass.
"""

import numpy as np
import torch
import torch.nn.functional as F

import oracle as O


def _bf16_tensor(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _ulps(a, b):
    ia, ib = a.astype(np.int32), b.astype(np.int32)
    sa = np.where(ia & 0x8000, -(ia & 0x7FFF), ia & 0x7FFF)
    sb = np.where(ib & 0x8000, -(ib & 0x7FFF), ib & 0x7FFF)
    return np.abs(sa - sb)


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / np.linalg.norm(b)


def _weights(n, k, seed):
    rng = np.random.default_rng(seed)
    w = O.f32_to_bf16((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    w8, ws = O.prepare_weight(w)
    return w, w8, ws


def _act_input(m, k, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((m, k)) * scale).astype(np.float32)
    x[:, rng.permutation(k)[: max(1, k // 100)]] *= 30
    return O.f32_to_bf16(x)


# ------------------------------------------------------------ dequant_weight
def test_dequant_weight_scaling_is_the_torch_chain_and_round_trips():
    w, w8, ws = _weights(64, 512, seed=1)
    # the scaling step against torch: (w8.float() * s[:, None]).to(bf16)
    t = (torch.from_numpy(w8).float() * torch.from_numpy(ws)[:, None]).to(torch.bfloat16)
    assert np.array_equal(O.dequant_weight(w8, ws), O.rotate_bf16(_bits(t)))
    # and it undoes prepare_weight: W within the int8 step (about 1 %)
    back = O.bf16_to_f32(O.dequant_weight(w8, ws))
    assert _rel(back, O.bf16_to_f32(w)) < 0.02


# ------------------------------------------------------------ linear_dx_int8
def test_linear_dx_int8_is_the_torch_chain():
    """ops.py:366-377 re-run with torch: d = dy.bf16 * ws.bf16, the row
    quantizer (pinned separately), torch._int_mm(q, w8), the dequant with unit
    column scales, the rotation."""
    w, w8, ws = _weights(128, 256, seed=2)
    rng = np.random.default_rng(3)
    dy = O.f32_to_bf16((rng.standard_normal((32, 128)) * 1e-3).astype(np.float32))
    d = _bf16_tensor(dy) * torch.from_numpy(ws).to(torch.bfloat16)
    q, a = O.quantize_row(_bits(d))
    acc = torch._int_mm(torch.from_numpy(q), torch.from_numpy(w8)).numpy()
    dx = O.dequant(acc, a, np.ones(acc.shape[1], np.float32))
    assert np.array_equal(O.linear_dx_int8(dy, w8, ws), O.rotate_bf16(dx))


def test_linear_dx_int8_approximates_dy_times_w():
    """dx = dy @ W for the unrotated weight: a missing rotation, a transposed
    weight or a wrong scale axis is off by O(1), the INT8 error is ~1 %."""
    w, w8, ws = _weights(256, 512, seed=4)
    rng = np.random.default_rng(5)
    dy = O.f32_to_bf16(rng.standard_normal((64, 256)).astype(np.float32))
    exact = O.bf16_to_f32(dy).astype(np.float64) @ O.bf16_to_f32(w).astype(np.float64)
    assert _rel(O.bf16_to_f32(O.linear_dx_int8(dy, w8, ws)), exact) < 0.03


def test_linear_dx_is_torch_matmul():
    """dy @ w (reference ops.py:204) in float64, and the transposed-operand
    identity dy @ w == (w^T dy^T)^T == linear_dw(w, dy^T)^T, which a swapped
    operand or a dropped transpose would break."""
    g = torch.Generator().manual_seed(7)
    dy = (torch.randn(33, 48, generator=g) * 1e-2).to(torch.bfloat16)
    w = (torch.randn(48, 80, generator=g) * 0.05).to(torch.bfloat16)
    b = lambda t: t.view(torch.int16).numpy().view(np.uint16)
    want = (dy.double() @ w.double()).numpy()
    assert np.allclose(O.linear_dx(b(dy), b(w)), want, rtol=0, atol=1e-12)
    assert O.linear_dx(b(dy), b(w)).shape == (33, 80)
    via_dw = O.linear_dw(np.ascontiguousarray(b(w)), np.ascontiguousarray(b(dy).T)).T
    assert np.allclose(O.linear_dx(b(dy), b(w)), via_dw, rtol=0, atol=1e-12)


def test_linear_dw_is_torch_matmul():
    rng = np.random.default_rng(6)
    dy = O.f32_to_bf16(rng.standard_normal((64, 48)).astype(np.float32))
    x = O.f32_to_bf16(rng.standard_normal((64, 32)).astype(np.float32))
    t = _bf16_tensor(dy).double().t() @ _bf16_tensor(x).double()
    assert np.allclose(O.linear_dw(dy, x), t.numpy(), rtol=0, atol=1e-12)


# --------------------------------------------------------------- activations
def _torch_act(act, first, second=None):
    """The eager bf16 chains the C activations reproduce (src/xpuint8.cpp:
    190-220, 150-160), on bf16 CPU tensors: every op rounds to bf16."""
    a = _bf16_tensor(first)
    b = None if second is None else _bf16_tensor(second)
    if act == 1:
        return F.gelu(a, approximate="tanh")
    if act == 2:                               # gate first, up second
        return F.silu(a) * b
    if act == 3:                               # hidden first, gate second
        return torch.tanh(b / 4.0) * torch.sigmoid(b) * torch.tanh(a / 25.0)
    if act == 4:                               # hidden * gelu(gate)
        return a * F.gelu(b, approximate="none")
    if act == 5:
        return F.gelu(a, approximate="none")
    raise ValueError(act)


def _pair(seed, m=64, k=512, scale=2.0):
    rng = np.random.default_rng(seed)
    h = O.f32_to_bf16((rng.standard_normal((m, k)) * scale).astype(np.float32))
    g = O.f32_to_bf16((rng.standard_normal((m, k)) * scale).astype(np.float32))
    return h, g


def test_activations_match_the_torch_chains():
    for act in (1, 2, 3, 4, 5):
        h, g = _pair(10 + act)
        second = g if act in O.PAIRED else None
        ours = O.f32_to_bf16(O.activate(act, O.bf16_to_f32(h),
                                        None if second is None else O.bf16_to_f32(second)))
        theirs = _bits(_torch_act(act, h, second))
        # torch's fp32 transcendentals are not correctly rounded: after the
        # bf16 rounding the two agree except on rare ties, by one bf16 ulp.
        # Where a GELU's argument is below -3, torch's 1 + erf / 1 + tanh
        # cancels and torch is the inaccurate one (the float64 pins above
        # cover the oracle there), so those elements are left out.
        arg = O.bf16_to_f32(second if act == 4 else h)
        sel = arg > -3.0 if act in (1, 4, 5) else np.ones(arg.shape, bool)
        d = _ulps(ours[sel], theirs[sel])
        assert d.max() <= 1 and (d > 0).mean() < 5e-3, (act, d.max(), (d > 0).mean())


def test_tanh_fast_is_tanh():
    """situ's tanh, expm1(2|z|) / (expm1(2|z|) + 2) with the sign or-ed back
    (src/xpuint8.cpp:128-148), within one bf16 ulp of float64 tanh on every
    bf16 input."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = O.bf16_to_f32(bits)
    e = (bits.astype(np.int32) >> 7) & 0xFF
    sel = (e > 0) & (e < 255) & (np.abs(x) > 2.0 ** -60)
    with np.errstate(all="ignore"):
        ours = O.f32_to_bf16(O.tanh_fast_f32(x))
    ref = O.f32_to_bf16(np.tanh(x.astype(np.float64)).astype(np.float32))
    assert _ulps(ours[sel], ref[sel]).max() <= 1


def _rows_equal(a, b):
    return np.all(a == b, axis=1)


def test_quantize_act_is_quantize_of_the_activation():
    """The pairing layout ([.., 2K] -> first half / second half) and the
    activation's place before the rotation: on every row where the torch
    chain's activation equals the oracle's bit for bit, quantize_act's codes
    and scale are convrot_quantize of that activation."""
    for act in (1, 2, 3, 4, 5):
        h, g = _pair(20 + act, m=48, k=512)
        # inside the range where torch's GELU is accurate (see above)
        h = O.f32_to_bf16(np.maximum(O.bf16_to_f32(h), -2.9))
        g = O.f32_to_bf16(np.maximum(O.bf16_to_f32(g), -2.9))
        x = np.concatenate([h, g], axis=1) if act in O.PAIRED else h
        q, s = O.quantize_act(x, act)
        v = _bits(_torch_act(act, h, g if act in O.PAIRED else None))
        ours = O.f32_to_bf16(O.activate(act, O.bf16_to_f32(h),
                                        O.bf16_to_f32(g) if act in O.PAIRED else None))
        same = _rows_equal(v, ours)
        assert same.mean() > 0.5, act
        wq, ws = O.convrot_quantize(v)
        assert np.array_equal(q[same], wq[same]) and np.array_equal(s[same], ws[same]), act


def test_dequant_act_is_the_torch_chain():
    """dequant_act: h = bf16(float(acc) * (ws * xs)) per half
    (src/xpuint8.cpp:238-261), then the activation -- against torch."""
    rng = np.random.default_rng(30)
    m, k = 32, 512
    acc = rng.integers(-25000, 25000, (m, 2 * k), dtype=np.int32)   # |h|, |g| < 2.5
    xs = rng.uniform(0.01, 0.1, m).astype(np.float32)
    ws = rng.uniform(1e-4, 1e-3, 2 * k).astype(np.float32)
    d = (torch.from_numpy(acc).float() * (torch.from_numpy(ws)[None, :] * torch.from_numpy(xs)[:, None]))
    d = d.to(torch.bfloat16)
    for act in (3, 4):
        theirs = _bits(_torch_act(act, _bits(d[:, :k]), _bits(d[:, k:])))
        ours = O.f32_to_bf16(O.dequant_act(acc, xs, ws, act))
        u = _ulps(ours, theirs)
        assert u.max() <= 1 and (u > 0).mean() < 2e-3, act
        same = _rows_equal(ours, theirs)
        q, s = O.dequant_act_quantize(acc, xs, ws, act)
        wq, wsc = O.convrot_quantize(theirs)
        assert np.array_equal(q[same], wq[same]) and np.array_equal(s[same], wsc[same])


def test_ffn_approximates_the_float64_block():
    """ffn = down(geglu(up(x))) + bias with the unquantized weights, in float64:
    wiring errors (halves swapped, rotation missing, a transposed weight) are
    O(1) off; the INT8 error of two quantized GEMMs is a few percent."""
    m, k, inner = 64, 256, 512
    x = _act_input(m, k, seed=40)
    up, up8, ups = _weights(2 * inner, k, seed=41)
    dn, dn8, dns = _weights(k, inner, seed=42)
    rng = np.random.default_rng(43)
    bias = (rng.standard_normal(k) * 0.01).astype(np.float32)
    got = O.bf16_to_f32(O.ffn(x, up8, ups, dn8, dns, bias, act=4)).astype(np.float64)
    xf = O.bf16_to_f32(x).astype(np.float64)
    hg = xf @ O.bf16_to_f32(up).astype(np.float64).T
    h, g = hg[:, :inner], hg[:, inner:]
    gelu = 0.5 * g * (1.0 + torch.special.erf(torch.from_numpy(g / np.sqrt(2.0))).numpy())
    want = (h * gelu) @ O.bf16_to_f32(dn).astype(np.float64).T + bias
    assert _rel(got, want) < 0.05
