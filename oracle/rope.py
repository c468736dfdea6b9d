"""RMSNorm + rotary embedding of a dequantized int32 accumulator -- TEST
INFRASTRUCTURE ONLY (see the package docstring).

Restates the reference's fused q/k consumer of a quantized qkv projection,
``_rms_rope_rows_dq_kernel`` (okolenmi/oko-xpu-kernels
python/xpu_kernels/triton/rope.py:149-222) and the torch chain it is checked
against (python/xpu_kernels/triton/reference.py:60-99):

    x   = bf16(float(acc) * (w_scale * x_scale))            rope.py:196-198
    y   = bf16(x * rsqrt(mean(x^2) + eps) * scale)           reference.py:60-70
    out = bf16(F00 * y0 + F01 * y1), bf16(F10 * y0 + F11 * y1)  reference.py:84-93

The reference verifies its kernel against that chain with a tolerance
(``SAME_ARITHMETIC_REL = 1e-3``, reference.py:43-51): the order of the row sum
(and the rsqrt) differ between implementations.  Here the mean of squares is
formed in float64 and rounded once; the rest is fp32 with each step rounded.
"""

import numpy as np

from .convrot import bf16_round

__all__ = ["rms_rope_dequant", "rms_rope_bf16"]

_F = np.float32


def _planes(freqs):
    """freqs_cis [FB, FS, 1, D/2, 2, 2] -> four [FB, FS, 1, D/2] planes
    (reference.py:73-81)."""
    f = np.asarray(freqs, dtype=_F)
    return f[..., 0, 0], f[..., 0, 1], f[..., 1, 0], f[..., 1, 1]


def rms_rope_bf16(x, freqs, scale, eps=1e-6, split_half=True):
    """x: bf16-valued fp32 [B, S, H, D] -> bf16-valued fp32 [B, S, H, D]
    (reference.py:60-99: rms_norm then rope_split_half; split_half=False pairs
    (2p, 2p+1) as the kernel's interleaved mode, rope.py:187-192)."""
    x = np.asarray(x, dtype=_F)
    D = x.shape[-1]
    ms = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(_F)
    inv = (_F(1.0) / np.sqrt(ms + _F(eps))).astype(_F)
    y = bf16_round((x * inv).astype(_F) * np.asarray(scale, dtype=_F))
    if split_half:
        y0, y1 = y[..., : D // 2], y[..., D // 2:]
    else:
        y0, y1 = y[..., 0::2], y[..., 1::2]
    f00, f01, f10, f11 = _planes(freqs)
    o0 = bf16_round((f00 * y0).astype(_F) + (f01 * y1).astype(_F))
    o1 = bf16_round((f10 * y0).astype(_F) + (f11 * y1).astype(_F))
    out = np.empty_like(y)
    if split_half:
        out[..., : D // 2], out[..., D // 2:] = o0, o1
    else:
        out[..., 0::2], out[..., 1::2] = o0, o1
    return out


def rms_rope_dequant(acc, x_scale, w_scale, freqs, scale, eps=1e-6, split_half=True):
    """acc int32 [B, S, H, D], x_scale [B, S], w_scale [H*D] -> bf16-valued fp32
    [B, S, H, D] (rope.py:196-222)."""
    acc = np.asarray(acc)
    B, S, H, D = acc.shape
    ws = np.asarray(w_scale, dtype=_F).reshape(H, D)
    xs = np.asarray(x_scale, dtype=_F).reshape(B, S)
    x = bf16_round(acc.astype(_F) * (ws[None, None] * xs[:, :, None, None]).astype(_F))
    return rms_rope_bf16(x, freqs, scale, eps, split_half)
