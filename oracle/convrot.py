"""numpy restatement of the reference's ConvRot INT8 arithmetic (test oracle).

Test infrastructure only: see the package docstring.  All floating-point work is
float32 numpy arithmetic, one IEEE rounding per operation and no fused
multiply-add, in the operation order of the reference code cited per function.
bf16 tensors are carried as ``uint16`` bit patterns.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "GS", "H4", "bf16_to_f32", "f32_to_bf16", "bf16_round", "hadamard256",
    "hadamard256_matrix", "rotate_bf16", "convrot_quantize", "quantize_from_rotated",
    "prepare_weight", "prepare_weight_fused", "quantize_row", "int_mm", "dequant",
    "linear_acc", "linear", "dequant_weight", "linear_dx_int8", "linear_dx", "linear_dw",
    "convrot_int8_linear", "expand_scale", "column_sum", "COL_CHUNK",
]

#: rows per fp32 partial sum of column_sum (the build's fixed order)
COL_CHUNK = 32

#: the ConvRot group size (src/xpuint8.cpp:71)
GS = 256

#: the 4-point factor of the Kronecker Hadamard (src/xpuint8.cpp:75)
H4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float32)

_F = np.float32
_HALF = _F(0.5)


# --------------------------------------------------------------------------- bf16

def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    """bf16 bits -> float32, exact (src/xpuint8.cpp:109-117, ``load_reg``)."""
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN.

    This is the conversion the reference's stores use (``BF(x)``,
    src/xpuint8.cpp:628, 705) and torch's ``.to(torch.bfloat16)``.
    """
    f = np.ascontiguousarray(f, dtype=np.float32)
    u = f.view(np.uint32)
    rounded = (u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))) >> np.uint32(16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    out = np.where(nan, (u >> np.uint32(16)) | np.uint32(0x40), rounded)
    return out.astype(np.uint16)


def bf16_round(f: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16, returned as float32."""
    return bf16_to_f32(f32_to_bf16(f))


# ----------------------------------------------------------------------- Hadamard

def _c_vec(by_digit1: bool, c: int) -> np.ndarray:
    """0.5*H4 column ``c`` spread over the 16 positions of a register
    (src/xpuint8.cpp:78-83, ``h4_col``)."""
    t = np.arange(16)
    row = ((t >> 2) & 3) if by_digit1 else (t & 3)
    return (_HALF * H4[row, c]).astype(np.float32)


_C = [_c_vec(False, c) for c in range(4)]
_D = [_c_vec(True, c) for c in range(4)]
# the broadcast-swizzle source positions of ``inreg`` (src/xpuint8.cpp:292-299)
_SW0 = [np.array([(t & ~3) + c for t in range(16)]) for c in range(4)]
_SW1 = [np.array([(t & 3) + 4 * c for t in range(16)]) for c in range(4)]


def _bfly4(a0, a1, a2, a3):
    """(H4/2) butterfly across four registers (src/xpuint8.cpp:279-285)."""
    p = a0 + a1
    m = a0 - a1
    q = a2 + a3
    n = a2 - a3
    return (p + n) * _HALF, (p - n) * _HALF, (m + q) * _HALF, (q - m) * _HALF


def hadamard256(v: np.ndarray) -> np.ndarray:
    """The 256-point block Hadamard along the last axis, float32 in and out.

    ``H = kron(H4, H4, H4, H4) / 16`` applied to every 256-element group with the
    reference's exact operation order: element ``i = 16*w + q`` of a group sits
    in register ``w`` at position ``q``; axes 0 and 1 (the base-4 digits of
    ``q``) are the in-register accumulation chains of ``inreg``
    (src/xpuint8.cpp:290-301), axis 2 (``w & 3``) and axis 3 (``w >> 2``) are
    ``bfly4`` across registers (src/xpuint8.cpp:279-285, 328-336), which the
    sub-group kernel computes bit-identically as ``bfly_xor`` over lanes xor 1,2
    and xor 4,8 (src/xpuint8.cpp:441-448, 474-477).
    """
    v = np.asarray(v, dtype=np.float32)
    k = v.shape[-1]
    if k % GS:
        raise ValueError(f"K={k} is not a multiple of {GS}")
    lead = v.shape[:-1]
    r = v.reshape(-1, k // GS, 16, 4, 4)               # [rows, group, w, q1, q0]
    # axis 0 (digit q0): output position q0=o is the chain
    #   t = c0[o]*v[q0=0] ; t += c1[o]*v[q0=1] ; t += c2[o]*v[q0=2] ; t += c3[o]*v[q0=3]
    # with c_c[o] = 0.5*H4[o][c] -- the same values as _C / _SW0 above
    t = np.empty_like(r)
    for o in range(4):
        acc = _HALF * H4[o, 0] * r[..., 0]
        for c in range(1, 4):
            acc = acc + (_HALF * H4[o, c]) * r[..., c]
        t[..., o] = acc
    # axis 1 (digit q1), the same chain on t (_D / _SW1)
    u = np.empty_like(t)
    for o in range(4):
        acc = _HALF * H4[o, 0] * t[..., 0, :]
        for c in range(1, 4):
            acc = acc + (_HALF * H4[o, c]) * t[..., c, :]
        u[..., o, :] = acc
    # axis 2: registers {4g..4g+3}; axis 3: registers {c, c+4, c+8, c+12}
    w = u.reshape(-1, k // GS, 4, 4, 16)               # [rows, group, w3, w2, q]
    a = _bfly4(w[:, :, :, 0], w[:, :, :, 1], w[:, :, :, 2], w[:, :, :, 3])
    w = np.stack(a, axis=3)
    a = _bfly4(w[:, :, 0], w[:, :, 1], w[:, :, 2], w[:, :, 3])
    w = np.stack(a, axis=2)
    return w.reshape(*lead, k)


def hadamard256_matrix() -> np.ndarray:
    """The explicit float64 matrix ``kron(H4,H4,H4,H4)/16`` (docs/architecture.md:29-35)."""
    h = np.ones((1, 1))
    for _ in range(4):
        h = np.kron(h, H4.astype(np.float64))
    return h / 16.0


# ---------------------------------------------------------------- quantizers

def quantize_from_rotated(v: np.ndarray):
    """Row absmax -> scale -> int8 of already-rotated fp32 values.

    ``s = fmax(rowmax / 127.0f, 1e-30f)``, ``q = clamp(rint(v * (1/s)), +-127)``
    (src/xpuint8.cpp:264-276, 494-498).
    """
    v = np.asarray(v, dtype=np.float32)
    rowmax = np.abs(v).max(axis=-1)
    s = np.maximum(rowmax / _F(127.0), _F(1e-30)).astype(np.float32)
    inv = (_F(1.0) / s).astype(np.float32)
    q = np.clip(np.rint(v * inv[..., None]), -127, 127).astype(np.int8)
    return q, s


def convrot_quantize(x_bf16: np.ndarray):
    """Rotate + per-row int8 quantize: bf16 [M,K] -> (int8 [M,K], fp32 [M]).

    src/xpuint8.cpp:450-502 (``launch_convrot_quant_warp<0>``).
    """
    return quantize_from_rotated(hadamard256(bf16_to_f32(x_bf16)))


def rotate_bf16(x_bf16: np.ndarray) -> np.ndarray:
    """bf16 -> Hadamard -> bf16 RNE (src/xpuint8.cpp:588-635)."""
    return f32_to_bf16(hadamard256(bf16_to_f32(x_bf16)))


def prepare_weight(w_bf16: np.ndarray):
    """The torch chain of ``prepare_weight`` (python/xpu_kernels/int8/ops.py:91-100).

    ``wr = rotate(w)`` in bf16; ``amax = |wr|.amax(1).clamp_min(1e-30)`` in bf16
    (so the floor is ``bf16(1e-30)``); ``s = amax.float() / 127``;
    ``q = round(wr / s)`` with an IEEE division, clamped to +-127.
    """
    wr = bf16_to_f32(rotate_bf16(w_bf16))
    amax = np.abs(wr).max(axis=-1)
    # torch converts the clamp's scalar to the tensor's dtype first
    floor = bf16_round(np.array([1e-30], dtype=np.float32))[0]
    amax = np.maximum(amax, floor).astype(np.float32)
    s = (amax / _F(127.0)).astype(np.float32)
    q = np.clip(np.rint(wr / s[..., None]), -127, 127).astype(np.int8)
    return q, s


def prepare_weight_fused(w_bf16: np.ndarray):
    """``prepare_weight_fused`` = the ConvRot quantizer on the weight
    (python/xpu_kernels/int8/ops.py:103-124)."""
    return convrot_quantize(w_bf16)


def quantize_row(x_bf16: np.ndarray):
    """Per-row symmetric int8, no rotation (python/xpu_kernels/int8/ops.py:320-330).

    ``s = (amax / 127).clamp_min(1e-30)``; ``q = round(x / s)`` (IEEE division),
    clamped to +-127.
    """
    xf = bf16_to_f32(x_bf16)
    s = np.maximum(np.abs(xf).max(axis=-1) / _F(127.0), _F(1e-30)).astype(np.float32)
    q = np.clip(np.rint(xf / s[..., None]), -127, 127).astype(np.int8)
    return q, s


# --------------------------------------------------------------------- GEMM + epilogue

def int_mm(a: np.ndarray, b_nk: np.ndarray) -> np.ndarray:
    """``torch._int_mm(a, b.t())``: int8 [M,K] x int8 [N,K]^T -> int32 [M,N].

    The reference calls it at python/xpu_kernels/int8/ops.py:587, 634, 714, 716.
    Computed as a float64 matmul, which is exact: every partial sum is an
    integer of magnitude <= 127*127*K < 2**53.
    """
    a = np.asarray(a, dtype=np.int8)
    b_nk = np.asarray(b_nk, dtype=np.int8)
    if a.shape[1] >= (1 << 53) // (127 * 127):
        raise ValueError("K too large for an exact float64 product")
    return (a.astype(np.float64) @ b_nk.astype(np.float64).T).astype(np.int32)


def expand_scale(scale, n: int) -> np.ndarray:
    """A flat fp32 [n] vector from a scalar / [n] / [n,1] scale
    (python/xpu_kernels/int8/ops.py:380-408)."""
    s = np.asarray(scale, dtype=np.float32).reshape(-1)
    if s.size == 1 and n != 1:
        s = np.full((n,), s[0], dtype=np.float32)
    if s.size != n:
        raise ValueError(f"scale has {s.size} values, expected {n}")
    return s


def dequant(acc: np.ndarray, x_scale, w_scale, bias=None) -> np.ndarray:
    """``bf16(float(acc) * (ws[n] * xs[m]) + bias[n])`` -> bf16 bits
    (src/xpuint8.cpp:692-710; bias fp32, python/xpu_kernels/int8/ops.py:489)."""
    acc = np.asarray(acc, dtype=np.int32)
    m, n = acc.shape
    xs = expand_scale(x_scale, m)
    ws = expand_scale(w_scale, n)
    v = acc.astype(np.float32) * (ws[None, :] * xs[:, None])
    if bias is not None:
        v = v + expand_scale(bias, n)[None, :]
    return f32_to_bf16(v)


def linear_acc(x_bf16, w8):
    """quantize -> int_mm (python/xpu_kernels/int8/ops.py:571-588)."""
    q, xs = convrot_quantize(x_bf16)
    return int_mm(q, w8), xs


def linear(x_bf16, w8, w_scale, bias=None):
    """The forward chain: quantize -> int_mm -> dequant
    (python/xpu_kernels/int8/ops.py:622-638).  ``bias`` is fp32 values."""
    acc, xs = linear_acc(x_bf16, w8)
    return dequant(acc, xs, w_scale, bias)


def dequant_weight(w8, w_scale) -> np.ndarray:
    """``rotate(bf16(w8 * s))`` (python/xpu_kernels/int8/ops.py:169-191)."""
    w = np.asarray(w8, dtype=np.int8).astype(np.float32) * expand_scale(
        w_scale, np.asarray(w8).shape[0])[:, None]
    return rotate_bf16(f32_to_bf16(w))


def linear_dx_int8(dy_bf16, w8, w_scale) -> np.ndarray:
    """dL/dx with the weight kept in int8 (python/xpu_kernels/int8/ops.py:353-377).

    ``d = bf16(dy) * bf16(ws)`` (one bf16 rounding of an exact product);
    ``(q, a) = quantize_row(d)``; ``acc = q @ w8`` (int32, contraction over N);
    ``dx = bf16(float(acc) * (1.0 * a[m]))``; then the rotation is undone.
    """
    ws = expand_scale(w_scale, np.asarray(w8).shape[0])
    d = f32_to_bf16(bf16_to_f32(dy_bf16) * bf16_round(ws)[None, :])
    q, a = quantize_row(d)
    acc = int_mm(q, np.ascontiguousarray(np.asarray(w8, dtype=np.int8).T))
    dx = dequant(acc, a, np.ones(acc.shape[1], dtype=np.float32))
    return rotate_bf16(dx)


def linear_dx(dy_bf16, w_bf16) -> np.ndarray:
    """``dy @ w`` in float64 (python/xpu_kernels/int8/ops.py:194-204, the
    dense-mode dL/dx against an unrotated bf16 weight); the build's bf16 GEMM
    is compared to this within a bf16 tolerance."""
    dy = bf16_to_f32(dy_bf16).astype(np.float64).reshape(-1, np.asarray(dy_bf16).shape[-1])
    w = bf16_to_f32(w_bf16).astype(np.float64)
    return dy @ w


def linear_dw(dy_bf16, x_bf16) -> np.ndarray:
    """``dy^T @ x`` in float64 (python/xpu_kernels/int8/ops.py:233-238); the
    build's bf16 GEMM is compared to this within a bf16 tolerance."""
    dy = bf16_to_f32(dy_bf16).astype(np.float64).reshape(-1, np.asarray(dy_bf16).shape[-1])
    x = bf16_to_f32(x_bf16).astype(np.float64).reshape(-1, np.asarray(x_bf16).shape[-1])
    return dy.T @ x


def column_sum(x_bf16: np.ndarray) -> np.ndarray:
    """``dy.sum(dim=0)`` of a bf16 [M, N] matrix, the bias gradient of the
    reference's backward (python/xpu_kernels/int8/ops.py:276, 821), in the
    build's fixed order: float32 sums of ``COL_CHUNK`` consecutive rows, each
    in row order; then eight running sums, sum w over chunks w, w + 8,
    w + 16, ... in order; then those eight added in order w = 0..7; one
    rounding to bf16.  (torch's own reduction order is unspecified; both are
    within the float32 summation bound of the exact sum before the one bf16
    rounding.)  Returns bf16 bits."""
    x = bf16_to_f32(x_bf16)
    m, n = x.shape
    # Vectorised over chunks (and then over the eight lanes): every running
    # sum starts at +0 and only ever adds, so it is never -0, and the +0 rows
    # and chunks that pad the last chunk and the last group of eight leave it
    # unchanged -- the same sums as the per-row loop.
    nc = -(-m // COL_CHUNK)
    xp = np.zeros((nc * COL_CHUNK, n), dtype=np.float32)
    xp[:m] = x
    xp = xp.reshape(nc, COL_CHUNK, n)
    chunks = np.zeros((nc, n), dtype=np.float32)
    for r in range(COL_CHUNK):
        chunks = (chunks + xp[:, r, :]).astype(np.float32)
    ng = -(-nc // 8)
    cp = np.zeros((ng * 8, n), dtype=np.float32)
    cp[:nc] = chunks
    cp = cp.reshape(ng, 8, n)
    lanes = np.zeros((8, n), dtype=np.float32)
    for i in range(ng):
        lanes = (lanes + cp[i]).astype(np.float32)
    tot = lanes[0]
    for w in range(1, 8):
        tot = (tot + lanes[w]).astype(np.float32)
    return f32_to_bf16(tot)


def convrot_int8_linear(x_rot_f32, weight, weight_scale, bias_bf16=None) -> np.ndarray:
    """Restatement of reference/convrot_linear.py:5-23, 2-D input only.

    The reference's rotation is the identity (``torch.eye``, line 11), so it is
    fed the already-rotated fp32 activation.  It quantizes with an IEEE division
    (line 17), dequantizes as ``(acc * xs) * ws`` (line 19), rounds to bf16
    (line 20) and adds the bias in bf16 (line 22).  Returns bf16 bits.
    """
    xr = np.asarray(x_rot_f32, dtype=np.float32)
    amax = np.abs(xr).max(axis=-1, keepdims=True)
    xs = np.maximum(amax / _F(127.0), _F(1e-30)).astype(np.float32)
    xq = np.clip(np.rint(xr / xs), -127, 127).astype(np.int8)
    acc = int_mm(xq, weight)
    ws = np.asarray(weight_scale, dtype=np.float32).reshape(1, -1)
    res = (acc.astype(np.float32) * xs) * ws
    out = f32_to_bf16(res)
    if bias_bf16 is not None:
        out = f32_to_bf16(bf16_to_f32(out) + bf16_to_f32(bias_bf16)[None, :])
    return out
