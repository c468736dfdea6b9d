"""RMSNorm + rotary embedding of q/k read from the int8 GEMM's accumulator.

The fused consumer of a quantized qkv projection
(okolenmi/oko-xpu-kernels ``python/xpu_kernels/triton/rope.py:378-405, 643-652``,
``_rows_dq`` and ``rms_rope_split_half_dequant``): the int32 accumulator slice
of q (or k), [B, S, H, D], is dequantized with the epilogue's expression and
bf16 rounding, RMS-normalized per head row, scaled, and rotated pairwise by
``freqs_cis`` [FB, FS, 1, D/2, 2, 2] in one HIP kernel
(``xpuint8_rms_rope_dequant_stream``).  The reference runs a Triton kernel
behind a self-test gate; here the HIP kernel is the only path.
"""

from __future__ import annotations

import torch

from .int8 import _lib as L

__all__ = ["rms_rope_split_half_dequant", "rows_dq"]


def _f32(t, name):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.dtype != torch.float32:
        t = t.to(torch.float32)
    return t


def rows_dq(acc, freqs_cis, scale, epsilon, x_scale, w_scale, split_half=True):
    """RMSNorm + rope of one [B, S, H, D] int32 accumulator slice -> bf16
    [B, S, H, D] (rope.py:378-405).

    ``acc``'s head dim must be contiguous (a column slice of a wider qkv
    accumulator is fine); ``x_scale`` is the quantizer's per-row scale, [B, S]
    (or [B*S]); ``w_scale`` the projection's per-column scale of this slice,
    [H*D]; ``scale`` the per-dim norm weight, [D]."""
    if not isinstance(acc, torch.Tensor) or acc.dtype != torch.int32 or acc.dim() != 4:
        raise TypeError("acc must be an int32 [B, S, H, D] tensor")
    if acc.device.type != "cuda":
        raise TypeError(f"expected a GPU (ROCm) tensor, got {acc.device}")
    B, S, H, D = acc.shape
    if acc.stride(3) != 1:
        raise ValueError("acc's head dimension must be contiguous")
    f = _f32(freqs_cis, "freqs_cis")
    if f.dim() != 6 or tuple(f.shape[3:]) != (D // 2, 2, 2) or f.shape[2] != 1:
        raise ValueError(f"freqs_cis must be [B or 1, S or 1, 1, {D // 2}, 2, 2], "
                         f"got {tuple(f.shape)}")
    if f.shape[0] not in (1, B) or f.shape[1] not in (1, S):
        raise ValueError(f"freqs_cis {tuple(f.shape)} does not broadcast over B={B}, S={S}")
    sc = _f32(scale, "scale").contiguous()
    if sc.numel() != D:
        raise ValueError(f"scale must have D={D} values")
    xs = _f32(x_scale, "x_scale")
    if xs.numel() != B * S:
        raise ValueError(f"x_scale must have B*S={B * S} values")
    xs = xs.reshape(B, S)
    ws = _f32(w_scale, "w_scale").contiguous()
    if ws.numel() != H * D:
        raise ValueError("w_scale must cover H * D columns")
    for t, name in ((f, "freqs_cis"), (sc, "scale"), (xs, "x_scale"), (ws, "w_scale")):
        if t.device != acc.device:
            raise TypeError(f"{name} is on {t.device} but acc is on {acc.device}")
    out = torch.empty((B, S, H, D), dtype=torch.bfloat16, device=acc.device)
    lib = L._lib()
    rc = lib.xpuint8_rms_rope_dequant_stream(
        L._stream(acc.device), L._ptr(acc), acc.stride(0), acc.stride(1), acc.stride(2),
        L._ptr(xs), xs.stride(0), xs.stride(1), L._ptr(ws), L._ptr(f),
        f.stride(0), f.stride(1), f.stride(3), f.stride(4), f.stride(5), f.shape[0], f.shape[1],
        L._ptr(sc), L._ptr(out), B, S, H, D, float(epsilon), 1 if split_half else 0)
    if rc != 0:
        L._err(lib, "rms_rope_dequant")
    return out


def rms_rope_split_half_dequant(q_acc, k_acc, freqs_cis, q_w, k_w, x_scale, q_scale,
                                k_scale=None, epsilon=1e-6, split_half=True):
    """``rms_rope_split_half`` with the INT8 dequant folded into the load
    (rope.py:643-652): returns (q, k) bf16 [B, S, H, D]."""
    if k_scale is None:
        k_scale = q_scale
    if k_w is None:
        k_w = q_w
    return (rows_dq(q_acc, freqs_cis, q_scale, epsilon, x_scale, q_w, split_half),
            rows_dq(k_acc, freqs_cis, k_scale, epsilon, x_scale, k_w, split_half))
