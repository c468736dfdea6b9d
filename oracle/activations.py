"""numpy restatement of the reference's fused activations and the FFN chain
(test oracle; see the package docstring).

The reference evaluates every activation in fp32 and rounds to bf16 where the
eager torch chain would (src/xpuint8.cpp:119-261).  The transcendental
functions (erf, tanh, exp, expm1) are taken here as the *correctly rounded*
fp32 value: the float64 result rounded once to float32.  That is the
specification the HIP kernels are held to; the reference's own device library
(SYCL ``erf``) is not available to compare with, and torch's CPU ``gelu`` is
compared separately (it agrees except on a handful of bf16 inputs, each by at
most one bf16 ulp: tests/test_oracle_activations.py).
"""

from __future__ import annotations

import numpy as np
from scipy import special as _sp

from .convrot import (
    bf16_round, bf16_to_f32, expand_scale, f32_to_bf16, hadamard256, int_mm,
    convrot_quantize, dequant, quantize_from_rotated,
)

__all__ = [
    "ACTIVATIONS", "PAIRED", "erf_f32", "tanh_f32", "exp_f32", "expm1_f32",
    "gelu_erf_f32", "gelu_tanh_f32", "tanh_fast_f32", "activate", "quantize_act",
    "dequant_act", "dequant_act_quantize", "ffn",
]

#: activation ids of the C API (include/xpu_kernels/convrot.h:51-59)
ACTIVATIONS = {"gelu_tanh": 1, "swiglu": 2, "situ": 3, "geglu_erf": 4, "gelu_erf": 5}
#: the ids that read two halves (src/xpuint8.cpp:188)
PAIRED = (2, 3, 4)

_F = np.float32


def _cr(fn, x):
    """Correctly rounded fp32 value of a float64 function of an fp32 argument."""
    return fn(np.asarray(x, dtype=np.float32).astype(np.float64)).astype(np.float32)


def erf_f32(x):
    return _cr(_sp.erf, x)


def tanh_f32(x):
    return _cr(np.tanh, x)


def exp_f32(x):
    return _cr(np.exp, x)


def expm1_f32(x):
    return _cr(np.expm1, x)


def gelu_erf_f32(x):
    """``0.5f * x * (1.0f + erf(x * 0.7071067811865476f))`` in fp32, before the
    bf16 round (src/xpuint8.cpp:175-177)."""
    x = np.asarray(x, dtype=np.float32)
    return (_F(0.5) * x) * (_F(1.0) + erf_f32(x * _F(0.7071067811865476)))


def gelu_tanh_f32(x):
    """GELU with the tanh approximation, fp32 (src/xpuint8.cpp:195-197)."""
    x = np.asarray(x, dtype=np.float32)
    x2 = x * x
    inner = (_F(0.7978845608028654) * x) * (_F(1.0) + _F(0.044715) * x2)
    return (_F(0.5) * x) * (_F(1.0) + tanh_f32(inner))


def tanh_fast_f32(z):
    """The reference's tanh: ``expm1(2a) / (expm1(2a) + 2)`` with ``a = min(|z|, 20)``
    and the sign of ``z`` put back (src/xpuint8.cpp:142-148)."""
    z = np.asarray(z, dtype=np.float32)
    a = np.fmin(np.abs(z), _F(20.0))          # C fmin: a NaN argument is dropped
    m = expm1_f32(_F(2.0) * a)
    r = m / (m + _F(2.0))
    bits = r.view(np.uint32) | (z.view(np.uint32) & np.uint32(0x80000000))
    return bits.view(np.float32)


def _situ(h, g):
    """MossImage's situ on bf16-valued fp32 inputs (src/xpuint8.cpp:150-160)."""
    tg = bf16_round(tanh_fast_f32(bf16_round(g / _F(4.0))))
    sg = bf16_round(_F(1.0) / (_F(1.0) + exp_f32(-g)))
    th = bf16_round(tanh_fast_f32(bf16_round(h / _F(25.0))))
    p = bf16_round(tg * sg)
    return bf16_round(p * th)


def activate(act: int, first, second=None):
    """One activation on bf16-valued fp32 inputs, result bf16-valued fp32
    (``load_activated_reg<ACT>``, src/xpuint8.cpp:190-220)."""
    a = np.asarray(first, dtype=np.float32)
    if act == 0:
        return a
    if act == 1:
        return bf16_round(gelu_tanh_f32(a))
    if act == 2:            # swiglu: gate first, up second
        g, u = a, np.asarray(second, dtype=np.float32)
        silu = bf16_round(g / (_F(1.0) + exp_f32(-g)))
        return bf16_round(silu * u)
    if act == 3:            # situ: hidden first, gate second
        return _situ(a, np.asarray(second, dtype=np.float32))
    if act == 4:            # geglu_erf: hidden * gelu(gate)
        y = bf16_round(gelu_erf_f32(np.asarray(second, dtype=np.float32)))
        return bf16_round(a * y)
    if act == 5:
        return bf16_round(gelu_erf_f32(a))
    raise ValueError(f"unknown activation id {act}")


def quantize_act(x_bf16, act: int):
    """Activation fused into the rotate+quantize load
    (src/xpuint8.cpp:809-838 with ``load_activated_reg``).  A paired activation
    reads bf16 [M, 2K] and produces int8 [M, K]."""
    x = bf16_to_f32(x_bf16)
    if act in PAIRED:
        k = x.shape[-1] // 2
        v = activate(act, x[..., :k], x[..., k:])
    else:
        v = activate(act, x)
    return quantize_from_rotated(hadamard256(v))


def dequant_act(acc, x_scale, w_scale, act: int):
    """The activation input rebuilt from the up-projection accumulator:
    ``bf16(float(acc) * (ws * xs))`` per half, then the activation
    (src/xpuint8.cpp:238-261).  Returns bf16-valued fp32 [M, K]."""
    acc = np.asarray(acc, dtype=np.int32)
    m, n = acc.shape
    xs = expand_scale(x_scale, m)[:, None]
    ws = expand_scale(w_scale, n)[None, :]
    d = bf16_round(acc.astype(np.float32) * (ws * xs))
    if act in PAIRED:
        k = n // 2
        return activate(act, d[:, :k], d[:, k:])
    return activate(act, d)


def dequant_act_quantize(acc, x_scale, w_scale, act: int = 4):
    """Dequant + activation + rotate + quantize (src/xpuint8.cpp:517-573)."""
    return quantize_from_rotated(hadamard256(dequant_act(acc, x_scale, w_scale, act)))


def ffn(x_bf16, up_w8, up_scale, down_w8, down_scale, down_bias=None, act: int = 4):
    """``act(up(x)) @ down.T`` (python/xpu_kernels/int8/ops.py:705-719).
    Returns bf16 bits [M, K]."""
    q, xs = convrot_quantize(x_bf16)
    acc = int_mm(q, up_w8)
    q2, xs2 = dequant_act_quantize(acc, xs, up_scale, act)
    acc2 = int_mm(q2, down_w8)
    return dequant(acc2, xs2, down_scale, down_bias)

