"""The INT8 API on ROCm tensors: weight preparation, the linear, the accumulator
paths, the FFN and the backward.

The counterpart of the reference's ``python/xpu_kernels/int8/ops.py`` (line
numbers cited per function): the same names, arguments, error types and
message substrings, with every kernel -- including the GEMMs and the chains the
reference left to torch -- running in ``libxpuint8.so`` on the caller's
current HIP stream.  Nothing here synchronises, and nothing falls back to a
CPU implementation: without the library every kernel call raises.

Two functions keep a torch path, for inputs the bf16 kernels do not take:
:func:`linear_dx` and :func:`linear_dw` compute ``dy @ w`` and ``dy^T @ x``
with torch's matmul (as the reference always does) when an operand is not a
bf16 GPU tensor (an fp32 training model) or a dimension is not a multiple of
16.  Every bf16 backward of the INT8 layers takes the kernels.
"""

from __future__ import annotations

from typing import Optional

import torch

from .._capture import is_capturing
from ._lib import (
    ACTIVATIONS,
    PAIRED_ACTIVATIONS,
    _c,
    _err,
    _flat2d,
    _lib,
    _ptr,
    _stream,
    load,
)

_NULL = None                 # a null c_void_p argument


def _opt(t):
    return _NULL if t is None else _ptr(t)


# ------------------------------------------------------------ packed weights
# A prepared weight can carry a packed copy: the same int8 codes in the MFMA
# block layout (xpuint8_pack_weight_stream), which the GEMMs that stream the
# weight through LDS load as whole cache lines, with the same results.  The
# copy is keyed by the weight's storage, so that aliases (``detach()``, an
# Int8Linear buffer) find it; it is used only while the weight's in-place
# version counter holds the value it was packed at, and it is dropped when
# the storage is.  Writes the version counter does not see (through
# ``.data``, DLPack or raw pointers) need a new :func:`pack_weight`.
# storage data_ptr -> [weakref to the storage, version, shape, packed, packed_nn]
# (packed_nn: the form linear_dx_int8's product reads, made at its first use)
_PACKED = {}


def _pack_key(w8):
    """The registry key of a weight that can carry a packed copy, else None:
    a CUDA int8 [N, K] tensor (N, K multiples of 16) that starts its storage,
    is contiguous and 16-byte aligned, and has a version counter (not an
    inference tensor)."""
    if not isinstance(w8, torch.Tensor) or w8.dtype != torch.int8 or w8.dim() != 2:
        return None
    if not w8.is_cuda or w8.is_inference() or w8.storage_offset() != 0:
        return None
    n, k = w8.shape
    if n == 0 or n % 16 or k == 0 or k % 16 or not w8.is_contiguous() or w8.data_ptr() % 16:
        return None
    return w8.untyped_storage().data_ptr()


def _drop_packed(key, ref):
    e = _PACKED.get(key)
    if e is not None and e[0] is ref:
        del _PACKED[key]


def pack_weight(w8):
    """Give the prepared weight ``w8`` (int8 [N, K]) a packed copy, read by
    :func:`linear`, :func:`int8_linear` and :func:`ffn` in place of ``w8``
    (bit-identical results, faster weight loads).  :func:`prepare_weight`
    calls it; call it again after writing ``w8`` in a way its version
    counter does not record.  Returns True if the copy is attached; a weight
    that cannot be tracked (see ``_pack_key``) gets none and is read as it is.
    Not during a device-graph capture (the copy would be captured and
    recomputed on every replay)."""
    key = _pack_key(w8)
    if key is None:
        return False
    if is_capturing():
        raise RuntimeError("pack_weight() allocates and writes the packed copy of a weight; "
                           "inside a device-graph capture it would be recomputed on every "
                           "replay. Call it before capturing.")
    import weakref
    lib = _lib()
    n, k = w8.shape
    need = lib.xpuint8_packed_weight_bytes(n, k)
    if need < 0:
        return False
    packed = torch.empty(int(need), device=w8.device, dtype=torch.int8)
    rc = lib.xpuint8_pack_weight_stream(_stream(w8.device), _ptr(w8), _ptr(packed), n, k)
    if rc != 0:
        _err(lib, "pack_weight")
    st = w8.untyped_storage()
    old = _PACKED.get(key)
    if old is not None and old[0]() is st:
        ref = old[0]
    else:
        ref = weakref.ref(st)
        weakref.finalize(st, _drop_packed, key, ref)
    _PACKED[key] = [ref, w8._version, (n, k), packed, None]
    return True


def _packed_entry(w8):
    """The registry entry of ``w8`` if its packed copy is still valid, else None."""
    if not _PACKED:
        return None
    key = _pack_key(w8)
    e = _PACKED.get(key) if key is not None else None
    if e is None:
        return None
    ref, version, shape = e[0], e[1], e[2]
    if ref() is not w8.untyped_storage() or tuple(w8.shape) != shape or w8._version != version:
        return None
    return e


def _packed_for(w8):
    """The packed copy attached to ``w8`` if it is still valid, else None."""
    e = _packed_entry(w8)
    return None if e is None else e[3]


def _packed_nn_for(w8):
    """The second packed form of a weight with a valid packed copy (the order
    in which linear_dx_int8's split-K product reads w8 [N, K] as its right
    operand), made at the first call outside a graph capture; else None."""
    e = _packed_entry(w8)
    if e is None:
        return None
    if e[4] is None and not is_capturing():
        lib = _lib()
        n, k = e[2]
        need = lib.xpuint8_packed_weight_nn_bytes(n, k)
        if need < 0:
            return None
        nn = torch.empty(int(need), device=w8.device, dtype=torch.int8)
        rc = lib.xpuint8_pack_weight_nn_stream(_stream(w8.device), _ptr(w8), _ptr(nn), n, k)
        if rc != 0:
            _err(lib, "pack_weight")
        e[4] = nn
    return e[4]


def rotate(x):
    """ConvRot rotation only: bf16 [.., K] in, bf16 [.., K] out (ops.py:26-37)."""
    lib = _lib()
    x2, shape = _flat2d(x)
    out = torch.empty_like(x2)
    m, k = x2.shape
    rc = lib.xpuint8_convrot_rotate_bf16_stream(_stream(x.device), _ptr(x2), _ptr(out), m, k)
    if rc != 0:
        _err(lib, "rotate")
    return out.reshape(shape)


def quantize(x):
    """Rotate and quantize an activation: bf16 [.., K] -> (int8 [.., K], fp32 [..])
    (ops.py:40-52)."""
    lib = _lib()
    x2, shape = _flat2d(x)
    m, k = x2.shape
    q = torch.empty((m, k), device=x.device, dtype=torch.int8)
    scale = torch.empty((m,), device=x.device, dtype=torch.float32)
    rc = lib.xpuint8_convrot_quantize_stream(_stream(x.device), _ptr(x2), _ptr(q), _ptr(scale),
                                             m, k)
    if rc != 0:
        _err(lib, "quantize")
    return q.reshape(*shape[:-1], k), scale.reshape(shape[:-1])


def quantize_act(x, activation: str):
    """Rotate+quantize with an activation fused into the load (ops.py:55-80).

    ``gelu_tanh``/``gelu_erf`` consume [.., K]; ``swiglu``, ``situ`` and
    ``geglu_erf`` consume [.., 2K]; the result is [.., K].
    """
    lib = _lib()
    x2, shape = _flat2d(x)
    m, k2 = x2.shape
    act = ACTIVATIONS[activation]
    k = k2 // 2 if activation in PAIRED_ACTIVATIONS else k2
    q = torch.empty((m, k), device=x.device, dtype=torch.int8)
    scale = torch.empty((m,), device=x.device, dtype=torch.float32)
    rc = lib.xpuint8_convrot_quantize_act_stream(_stream(x.device), _ptr(x2), _ptr(q),
                                                 _ptr(scale), m, k, act)
    if rc != 0:
        _err(lib, "quantize_act")
    return q.reshape(*shape[:-1], k), scale.reshape(shape[:-1])


def prepare_weight(w, group: int = 256, *, pack: bool = True):
    """Prepare an INT8 weight for :func:`linear` (ops.py:83-100).

    ``w`` is bf16 or fp32 [N, K] in the unrotated orientation.  Returns
    ``(int8 [N, K], fp32 [N])``.  One kernel, bit-identical to the reference's
    torch chain: rotate to bf16, the bf16 row absmax floored at bf16(1e-30),
    ``s = amax / 127`` and ``round(wr / s)`` with an IEEE division.  With
    ``pack`` (outside a device-graph capture) the codes also get a packed copy
    (:func:`pack_weight`), another N*K bytes of device memory.
    """
    if w.shape[1] % group:
        raise ValueError(f"K={w.shape[1]} is not a multiple of the group size {group}")
    lib = _lib()
    w2 = _c(w.detach().to(device=w.device, dtype=torch.bfloat16))
    n, k = w2.shape
    q = torch.empty((n, k), device=w.device, dtype=torch.int8)
    scale = torch.empty((n,), device=w.device, dtype=torch.float32)
    rc = lib.xpuint8_prepare_weight_stream(_stream(w.device), _ptr(w2), _ptr(q), _ptr(scale), n, k)
    if rc != 0:
        _err(lib, "prepare_weight")
    if pack and not is_capturing():
        pack_weight(q)
    return q, scale


def prepare_weight_fused(w, group: int = 256):
    """The ConvRot quantizer applied to the weight (ops.py:103-124): the rotated
    values stay fp32 (no bf16 round before the absmax), so it differs from
    :func:`prepare_weight` in the last bit of some codes -- a different function
    on purpose."""
    if w.shape[1] % group:
        raise ValueError(f"K={w.shape[1]} is not a multiple of the group size {group}")
    return quantize(w.detach().to(device=w.device, dtype=torch.bfloat16).contiguous())


def dequant_weight(w8, w_scale):
    """The unrotated bf16 weight behind an INT8 ConvRot weight (ops.py:127-166):
    ``rotate(bf16(w8 * s))`` in one kernel, bit-identical to
    :func:`dequant_weight_torch`."""
    if w8.dtype != torch.int8:
        raise TypeError(f"w8 must be int8, got {w8.dtype}")
    if w8.dim() != 2 or w8.shape[1] % 256 or w_scale.numel() not in (1, w8.shape[0]):
        raise TypeError(f"w8 must be int8 [N, K] with K % 256 == 0 and a [N] or scalar "
                        f"scale; got {tuple(w8.shape)} and {w_scale.numel()} scales")
    lib = _lib()
    w8c = _c(w8)
    scale = expand_scale(w_scale.detach(), w8.shape[0], w8.device)
    out = torch.empty(w8.shape, dtype=torch.bfloat16, device=w8.device)
    rc = lib.xpuint8_dequant_weight_stream(_stream(w8.device), _ptr(w8c), _ptr(scale), _ptr(out),
                                           w8.shape[0], w8.shape[1])
    if rc != 0:
        _err(lib, "dequant_weight")
    return out


def dequant_weight_torch(w8, w_scale):
    """The weight dequantization as a torch chain -- the definition
    (ops.py:169-191): fp32 multiply, bf16 round, then the rotation undone."""
    if w8.dtype != torch.int8:
        raise TypeError(f"w8 must be int8, got {w8.dtype}")
    if is_capturing():
        raise RuntimeError(
            "dequant_weight() materializes a full-precision copy of the weight; inside a "
            "device-graph capture it would be captured and re-computed on every replay. "
            "Call it before capturing, or use the int8 backward "
            "(xpu_kernels.int8_linear(..., mode='int8')), which needs no copy at all.")
    w = w8.to(torch.float32) * w_scale.to(torch.float32).reshape(-1, 1)
    return rotate(w.to(torch.bfloat16))


def linear_dx(dy, w):
    """``dL/dx = dy [.., N] @ w [N, K]`` for an unrotated weight (ops.py:194-204).

    bf16 operands on the GPU with N and K multiples of 16 take the bf16 MFMA
    kernel (fp32 accumulation, one rounding, like the matmul it replaces);
    other dtypes and shapes are torch's matmul in their dtype, the
    reference's own computation."""
    if dy.shape[-1] != w.shape[0]:
        raise ValueError(f"dy has {dy.shape[-1]} columns but w has {w.shape[0]} rows")
    n, k = int(w.shape[0]), int(w.shape[1])
    if (dy.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and dy.is_cuda
            and w.device == dy.device and w.dim() == 2 and n % 16 == 0 and k % 16 == 0):
        lib = _lib()
        dy2, w2 = _c(dy.reshape(-1, n)), _c(w)
        m = dy2.shape[0]
        dx = torch.empty((m, k), device=dy.device, dtype=torch.bfloat16)
        if m:
            # a small batch splits the contraction across blocks (fp32
            # partials in the workspace)
            need = int(lib.xpuint8_linear_dx_workspace_size(m, n, k))
            work = torch.empty(need, device=dy.device, dtype=torch.uint8) if need > 0 else None
            rc = lib.xpuint8_linear_dx_stream(_stream(dy.device), _ptr(dy2), _ptr(w2), _ptr(dx),
                                              m, n, k, _opt(work), max(need, 0))
            if rc != 0:
                _err(lib, "linear_dx")
        return dx.reshape(*dy.shape[:-1], k)
    return dy @ w


def linear_dw(dy, x):
    """``dL/dW = dy [.., N]^T @ x [.., K] -> [N, K]`` (ops.py:207-238).

    The contraction runs over the batch (token) dimension, so the batch dims
    must agree.
    """
    if dy.shape[-2] != x.shape[-2]:
        raise ValueError(
            f"dy has {dy.shape[-2]} rows but x has {x.shape[-2]}: the batch "
            f"dims must match for dy^T @ x")
    dy2 = dy.reshape(-1, dy.shape[-1])
    x2 = x.reshape(-1, x.shape[-1])
    n, k = dy2.shape[1], x2.shape[1]
    if (dy2.dtype == torch.bfloat16 and x2.dtype == torch.bfloat16 and dy2.is_cuda
            and x2.device == dy2.device and n % 16 == 0 and k % 16 == 0):
        # the hand-written bf16 MFMA kernel (fp32 accumulation, like the
        # matmul it replaces)
        lib = _lib()
        dy2, x2 = _c(dy2), _c(x2)
        dw = torch.empty((n, k), device=dy2.device, dtype=torch.bfloat16)
        rc = lib.xpuint8_linear_dw_stream(_stream(dy2.device), _ptr(dy2), _ptr(x2), _ptr(dw),
                                          dy2.shape[0], n, k)
        if rc != 0:
            _err(lib, "linear_dw")
        return dw
    # other dtypes and shapes: the product the reference computes, in their dtype
    return dy2.transpose(0, 1) @ x2


def column_sum(dy):
    """``dy.sum(dim=0)``, the bias gradient of the reference's backward
    (ops.py:276, 821).  A 2-D bf16 ``dy`` on the GPU (columns a multiple of
    16) takes one HIP column-sum pass (fp32 sums of 32-row chunks in row
    order, then the chunks in order, one bf16 rounding) instead of torch's
    reduction, whose order is its own; anything else is torch's sum."""
    if (isinstance(dy, torch.Tensor) and dy.dim() == 2 and dy.dtype == torch.bfloat16
            and dy.is_cuda and dy.shape[0] > 0 and dy.shape[1] % 16 == 0):
        lib = _lib()
        m, n = int(dy.shape[0]), int(dy.shape[1])
        d2 = _c(dy)
        nbytes = lib.xpuint8_column_sum_workspace_size(m, n)
        if nbytes < 0:
            _err(lib, "column_sum")
        work = torch.empty((max(nbytes, 16),), device=dy.device, dtype=torch.int8)
        out = torch.empty((n,), device=dy.device, dtype=torch.bfloat16)
        rc = lib.xpuint8_column_sum_stream(_stream(dy.device), _ptr(d2), _ptr(out), m, n,
                                           _ptr(work), nbytes)
        if rc != 0:
            _err(lib, "column_sum")
        return out
    return dy.sum(dim=0)


def _backward_one_call(dy, w8):
    """Whether the int8-mode backward can run as one library call: a 2-D bf16
    CUDA ``dy`` [M, N] against an int8 [N, K] weight of the shape contract
    (the cases where column_sum and linear_dx_int8 both take the kernels)."""
    return (isinstance(dy, torch.Tensor) and dy.is_cuda and dy.dtype == torch.bfloat16
            and dy.dim() == 2 and dy.shape[0] > 0 and w8.dtype == torch.int8
            and w8.dim() == 2 and w8.device == dy.device and dy.shape[1] == w8.shape[0]
            and w8.shape[0] % 16 == 0 and w8.shape[1] % 256 == 0)


def _linear_backward(dy, w8, w_scale, want_dbias, bias_dtype, mode):
    """The backward of _Int8LinearFn in one library call, bit for bit: dx =
    linear_dx_int8(dy, w8, w_scale) (mode "int8",
    xpuint8_linear_backward_int8_stream) or linear_dx(dy, dequant_weight(w8,
    w_scale)) (mode "dense", xpuint8_linear_backward_dense_stream), and, if
    wanted, the bias gradient column_sum(dy).  The bias gradient comes out in
    the bias's dtype when that is fp32 (each bf16 sum widened, exactly what
    autograd's cast would give) or bf16; otherwise bf16, which autograd casts
    as before."""
    lib = _lib()
    m, n = int(dy.shape[0]), int(dy.shape[1])
    k = int(w8.shape[1])
    d2 = _c(dy)
    ws = expand_scale(w_scale, n, dy.device)
    w8c = _c(w8)
    size = (lib.xpuint8_linear_backward_int8_workspace_size if mode == "int8"
            else lib.xpuint8_linear_backward_dense_workspace_size)
    what = "linear_dx_int8" if mode == "int8" else "linear_dx"
    nbytes = size(m, n, k)
    if nbytes < 0:
        _err(lib, what)
    work = torch.empty((nbytes,), device=dy.device, dtype=torch.int8)
    dx = torch.empty((m, k), device=dy.device, dtype=torch.bfloat16)
    dbias, f32 = None, 0
    if want_dbias:
        f32 = 1 if bias_dtype == torch.float32 else 0
        dbias = torch.empty((n,), device=dy.device, dtype=torch.float32 if f32 else torch.bfloat16)
    if mode == "int8":
        rc = lib.xpuint8_linear_backward_int8_stream(
            _stream(dy.device), _ptr(d2), _ptr(ws), _ptr(w8c), _opt(_packed_nn_for(w8c)),
            _ptr(dx), _opt(dbias), f32, m, n, k, _ptr(work), nbytes)
    else:
        rc = lib.xpuint8_linear_backward_dense_stream(
            _stream(dy.device), _ptr(d2), _ptr(w8c), _ptr(ws), _ptr(dx), _opt(dbias), f32, m, n,
            k, _ptr(work), nbytes)
    if rc != 0:
        _err(lib, what)
    return dx, dbias


class _Int8LinearFn(torch.autograd.Function):
    """The INT8 linear as an autograd op (ops.py:241-289): forward is
    :func:`linear`; backward is dbias plus dx through :func:`linear_dx_int8`
    (``mode="int8"``) or :func:`linear_dx` on the dequantized weight
    (``mode="dense"``).  The frozen int8 weight gets no gradient."""

    @staticmethod
    def forward(ctx, x, w8, w_scale, bias, mode):
        ctx.save_for_backward(w8, w_scale)
        ctx.mode = mode
        ctx.input_dtype = x.dtype
        ctx.bias_dtype = None if bias is None else bias.dtype
        return linear(x, w8, w_scale, bias)

    @staticmethod
    def backward(ctx, dy):
        w8, w_scale = ctx.saved_tensors
        if ctx.mode in ("int8", "dense") and _backward_one_call(dy, w8) and \
                w_scale.numel() in (1, w8.shape[0]):
            dx, dbias = _linear_backward(dy, w8, w_scale, ctx.needs_input_grad[3],
                                         ctx.bias_dtype, ctx.mode)
            return dx.to(ctx.input_dtype), None, None, dbias, None
        dbias = column_sum(dy) if ctx.needs_input_grad[3] else None
        dy = dy.to(torch.bfloat16)
        if ctx.mode == "int8":
            dx = linear_dx_int8(dy, w8, w_scale)
        elif ctx.mode == "dense":
            dx = linear_dx(dy, dequant_weight(w8, w_scale))
        else:
            raise ValueError(f"unknown backward mode {ctx.mode!r}; use 'dense' or 'int8'")
        return dx.to(ctx.input_dtype), None, None, dbias, None


def int8_linear(x, w8, w_scale, bias=None, *, mode="dense"):
    """The INT8 linear, differentiable (ops.py:292-317).  ``mode`` is
    ``"dense"`` (dequantized weight in the backward) or ``"int8"`` (weight stays
    int8, ``dy`` is row-quantized)."""
    if mode not in ("dense", "int8"):
        raise ValueError(f"unknown backward mode {mode!r}; use 'dense' or 'int8'")
    return _Int8LinearFn.apply(x, w8, w_scale, bias, mode)


def quantize_row_torch(x):
    """The per-row quantizer as a torch chain -- the definition (ops.py:320-330)."""
    xf = x.to(torch.float32)
    scale = (xf.abs().amax(dim=-1, keepdim=True) / 127.0).clamp_min(1e-30)
    q = torch.round(xf / scale).clamp_(-127, 127).to(torch.int8)
    return q.contiguous(), scale.squeeze(-1).contiguous()


def quantize_row(x, col_scale=None):
    """Per-row symmetric int8 quantization, no rotation: bf16 [.., N] ->
    (int8 [.., N], fp32 [..]) (ops.py:333-350), bit-identical to
    :func:`quantize_row_torch`.  ``col_scale`` ([N], optional) first replaces
    the row by ``bf16(x * bf16(col_scale))``, the product linear_dx_int8 needs."""
    lib = _lib()
    x2, shape = _flat2d(x)
    m, n = x2.shape
    if n % 16:
        # the kernel reads rows in 16-element pieces: widths that are not a
        # multiple of 16 are zero-padded (zeros change neither a row's max nor
        # any code) and the padding is dropped afterwards
        n16 = (n + 15) // 16 * 16
        xp = torch.zeros((m, n16), device=x.device, dtype=torch.bfloat16)
        xp[:, :n] = x2
        csp = None
        if col_scale is not None:
            csp = torch.zeros(n16, device=x.device, dtype=torch.float32)
            csp[:n] = expand_scale(col_scale, n, x.device)
        q, scale = quantize_row(xp, csp)
        return (q[:, :n].contiguous().reshape(*shape[:-1], n),
                scale.reshape(shape[:-1]))
    cs = None if col_scale is None else expand_scale(col_scale, n, x.device)
    q = torch.empty((m, n), device=x.device, dtype=torch.int8)
    scale = torch.empty((m,), device=x.device, dtype=torch.float32)
    rc = lib.xpuint8_quantize_row_stream(_stream(x.device), _ptr(x2), _opt(cs), _ptr(q),
                                         _ptr(scale), m, n)
    if rc != 0:
        _err(lib, "quantize_row")
    return q.reshape(*shape[:-1], n), scale.reshape(shape[:-1])


def linear_dx_int8(dy, w8, w_scale):
    """``dL/dx`` against the weight still in int8 (ops.py:353-377):
    ``d = bf16(dy) * bf16(ws)``, row-quantized, ``acc = q @ w8`` (int32), then
    ``bf16(acc * a[m])`` and the rotation undone."""
    lib = _lib()
    n, k = int(w8.shape[0]), int(w8.shape[1])
    d2 = _c(dy.to(torch.bfloat16).reshape(-1, n))
    m = d2.shape[0]
    ws = expand_scale(w_scale, n, dy.device)
    w8c = _c(w8)
    nbytes = lib.xpuint8_linear_dx_int8_workspace_size(m, n, k)
    if nbytes < 0:
        _err(lib, "linear_dx_int8")
    work = torch.empty((nbytes,), device=dy.device, dtype=torch.int8)
    dx = torch.empty((m, k), device=dy.device, dtype=torch.bfloat16)
    nn = _packed_nn_for(w8c)
    if nn is not None:
        rc = lib.xpuint8_linear_dx_int8_packed_stream(_stream(dy.device), _ptr(d2), _ptr(ws),
                                                      _ptr(w8c), _ptr(nn), _ptr(dx), m, n, k,
                                                      _ptr(work), nbytes)
    else:
        rc = lib.xpuint8_linear_dx_int8_stream(_stream(dy.device), _ptr(d2), _ptr(ws),
                                               _ptr(w8c), _ptr(dx), m, n, k, _ptr(work), nbytes)
    if rc != 0:
        _err(lib, "linear_dx_int8")
    return dx.reshape(*dy.shape[:-1], k)


def expand_scale(scale, n, device=None):
    """A flat fp32 ``[n]`` scale, broadcasting a per-tensor scalar (ops.py:380-408).
    Returns ``scale`` itself when it already is a flat fp32 [n] tensor on the
    device."""
    if not isinstance(scale, torch.Tensor):
        if not isinstance(scale, (float, int)):
            raise TypeError(f"scale must be a tensor or a python float, "
                            f"got {type(scale).__name__}")
        if device is None:
            raise TypeError("a python-scalar scale needs an explicit device")
        return torch.full((n,), float(scale), device=device, dtype=torch.float32)
    if (scale.dtype == torch.float32 and scale.dim() == 1 and scale.numel() == n
            and scale.is_contiguous() and (device is None or scale.device == device)
            and scale.data_ptr() % 16 == 0):
        return scale
    s = scale.reshape(-1).to(device=device or scale.device, dtype=torch.float32)
    if s.numel() == 1 and n != 1:
        s = s.expand(n)
    return _c(s)


def _bias_arg(bias, n, device):
    """(tensor or None, bias_bf16 flag) for the fused GEMM epilogue: a flat
    contiguous bf16 [n] bias on the device goes in as it is (the kernel widens
    it exactly, as ``bias.float()`` does), anything else through
    ``expand_scale`` as fp32."""
    if bias is None:
        return None, 0
    if (isinstance(bias, torch.Tensor) and bias.dtype == torch.bfloat16 and bias.dim() == 1
            and bias.numel() == n and bias.is_contiguous() and bias.device == device
            and bias.data_ptr() % 16 == 0):
        return bias, 1
    return expand_scale(bias, n, device), 0


def _dims(x, w8, act):
    m = 1
    for d in x.shape[:-1]:
        m *= int(d)
    return m, int(w8.shape[0]), int(w8.shape[1])


def unsupported_reason(x, w8, w_scale, act=None):
    """Why this call cannot use the fused kernels, or ``None`` if it can
    (ops.py:418-476).  :func:`linear` raises exactly this message."""
    if not isinstance(x, torch.Tensor) or not isinstance(w8, torch.Tensor):
        return "activation and weight must be torch tensors"
    if x.dtype not in (torch.bfloat16, torch.float32):
        return (f"activation dtype {x.dtype} is not bfloat16 or float32 "
                f"(the kernels consume bf16)")
    if w8.dtype != torch.int8 or w8.dim() != 2:
        return f"weight must be an int8 [N, K] tensor, got {w8.dtype} {tuple(w8.shape)}"
    if act is not None and act not in ACTIVATIONS:
        return (f"unknown activation {act!r}; expected None or one of "
                f"{', '.join(sorted(ACTIVATIONS))}")
    k = int(w8.shape[1])
    want = k * 2 if act in PAIRED_ACTIVATIONS else k
    if x.shape[-1] != want:
        return (f"activation has {x.shape[-1]} columns but this weight wants "
                f"{want} (K={k}{' with two halves' if want != k else ''})")
    if k % 256:
        return f"K={k} is not a multiple of the ConvRot group size (256)"
    if w8.shape[0] % 16:
        return (f"N={w8.shape[0]} is not a multiple of 16; the dequant epilogue "
                f"reads the output 16 columns at a time and would drop the tail")
    if isinstance(w_scale, torch.Tensor):
        if not w_scale.is_floating_point():
            return (f"weight scale dtype {w_scale.dtype} is not floating point; "
                    f"a per-channel scale is amax/127")
        if w_scale.dim() > 2:
            return (f"weight scale has {w_scale.dim()} dims; expected a scalar, "
                    f"[N] or [N, 1]")
        if w_scale.numel() not in (1, w8.shape[0]):
            return (f"weight scale has {w_scale.numel()} values; expected 1 or "
                    f"N={w8.shape[0]}")
    elif not isinstance(w_scale, (float, int)):
        return "weight scale must be a tensor or a python float"
    if load() is None:
        return "libxpuint8.so is not available (see xpu_kernels.int8._lib)"
    if x.device.type != "cuda":
        return f"activation is on {x.device}; the kernels need a GPU (ROCm) tensor"
    if w8.device != x.device:
        return (f"weight is on {w8.device} but the activation is on {x.device}; "
                f"the kernels take raw pointers into one stream")
    return None


def int_mm(a, b):
    """``torch._int_mm`` semantics on the library's MFMA GEMM: int8 a [M, K] @
    int8 b [K, N] -> int32 [M, N].  ``b`` given as ``w8.t()`` (a transposed view
    of a contiguous [N, K] weight) takes the NT kernel directly; a contiguous
    [K, N] ``b`` is transposed into a scratch buffer first."""
    lib = _lib()
    if a.dtype != torch.int8 or b.dtype != torch.int8 or a.dim() != 2 or b.dim() != 2:
        raise TypeError("int_mm takes two 2-D int8 tensors")
    m, k = a.shape
    if b.shape[0] != k:
        raise ValueError(f"K mismatch: a has {k} columns, b has {b.shape[0]} rows")
    n = b.shape[1]
    a = _c(a)
    c = torch.empty((m, n), device=a.device, dtype=torch.int32)
    st = _stream(a.device)
    if b.t().is_contiguous() and b.data_ptr() % 16 == 0:
        rc = lib.xpuint8_int8_gemm_stream(st, _ptr(a), _ptr(b.t()), _ptr(c), m, n, k)
    else:
        b = _c(b)
        work = torch.empty((k * n,), device=a.device, dtype=torch.int8)
        rc = lib.xpuint8_int8_gemm_nn_stream(st, _ptr(a), _ptr(b), _ptr(c), m, n, k, _ptr(work))
    if rc != 0:
        _err(lib, "int_mm")
    return c


def dequant(acc, x_scale, w_scale, bias=None):
    """bf16 dequant of an int32 [M, N] accumulator (ops.py:479-497)."""
    lib = _lib()
    if acc.dim() != 2 or acc.dtype != torch.int32:
        raise TypeError("acc must be an int32 [M, N] tensor")
    m, n = acc.shape
    acc = _c(acc)
    out = torch.empty((m, n), device=acc.device, dtype=torch.bfloat16)
    xs, ws = expand_scale(x_scale, m, acc.device), expand_scale(w_scale, n, acc.device)
    b = None if bias is None else expand_scale(bias, n, acc.device)
    rc = lib.xpuint8_dequant_epilogue_stream(_stream(acc.device), _ptr(acc), _ptr(out), _ptr(xs),
                                             _ptr(ws), _opt(b), m, n)
    if rc != 0:
        _err(lib, "dequant")
    return out


def dequant_slice(acc, x_scale, w_scale, bias=None):
    """As :func:`dequant`, for a [M, N] column slice of a wider accumulator,
    read in place through its row stride (ops.py:500-525)."""
    lib = _lib()
    if acc.dim() != 2 or acc.dtype != torch.int32:
        raise TypeError("acc must be an int32 [M, N] tensor")
    if acc.stride(1) != 1 or acc.stride(0) % 4 or acc.data_ptr() % 16:
        acc = acc.contiguous() if acc.stride(1) != 1 else acc
        if acc.stride(0) % 4 or acc.data_ptr() % 16:
            acc = acc.clone()
    m, n = acc.shape
    out = torch.empty((m, n), device=acc.device, dtype=torch.bfloat16)
    xs, ws = expand_scale(x_scale, m, acc.device), expand_scale(w_scale, n, acc.device)
    b = None if bias is None else expand_scale(bias, n, acc.device)
    rc = lib.xpuint8_dequant_epilogue_slice_stream(_stream(acc.device), _ptr(acc), _ptr(out),
                                                   _ptr(xs), _ptr(ws), _opt(b), m, n,
                                                   acc.stride(0))
    if rc != 0:
        _err(lib, "dequant_slice")
    return out


def dequant_act_quantize(acc, x_scale, w_scale, activation="situ"):
    """Dequant, activate, rotate and quantize an up-projection accumulator
    (ops.py:528-568): int32 [M, 2K] (paired) or [M, K] -> (int8 [M, K], fp32 [M])."""
    lib = _lib()
    act_id = ACTIVATIONS[activation]
    paired = activation in PAIRED_ACTIVATIONS
    if acc.dim() != 2 or acc.dtype != torch.int32:
        raise TypeError("acc must be an int32 [M, N] tensor")
    m, n = acc.shape
    if paired:
        if n % 2:
            raise TypeError(f"acc must be an int32 [M, 2K] tensor for {activation}, "
                            f"got {n} columns")
        k = n // 2
    else:
        k = n
    acc = _c(acc)
    q = torch.empty((m, k), device=acc.device, dtype=torch.int8)
    scale = torch.empty((m,), device=acc.device, dtype=torch.float32)
    xs = expand_scale(x_scale, m, acc.device)
    ws = expand_scale(w_scale, n, acc.device)
    rc = lib.xpuint8_dequant_act_quantize_stream(_stream(acc.device), _ptr(acc), _ptr(q),
                                                 _ptr(scale), _ptr(xs), _ptr(ws), m, k, act_id)
    if rc != 0:
        _err(lib, "dequant_act_quantize")
    return q, scale


def linear_acc(x, w8, w_scale, act: Optional[str] = None):
    """The GEMM without the output dequant: ``(int32 [M, N], fp32 [M])``
    (ops.py:571-588)."""
    if act is None and _acc_one_call(x, w8):
        x2 = _c(x.reshape(-1, x.shape[-1]))
        return _linear_acc_bf16(_lib(), x2, _c(w8), x2.shape[0], w8.shape[0], w8.shape[1])
    if act is None:
        xq, xs = quantize(x)
    else:
        xq, xs = quantize_act(x, act)
    if w8.dtype != torch.int8 or w8.dim() != 2:
        raise TypeError("w8 must be an int8 [N, K] tensor")
    if xq.shape[-1] != w8.shape[1]:
        raise ValueError(f"K mismatch: activation {xq.shape[-1]} vs weight {w8.shape[1]}")
    acc = int_mm(xq.reshape(-1, xq.shape[-1]), w8.contiguous().t())
    return acc, xs.reshape(-1)


def _acc_one_call(x, w8):
    """Whether quantize + int32 GEMM can run as one library call: a bf16 CUDA
    activation and an int8 [N, K] weight of the shape contract."""
    return (isinstance(x, torch.Tensor) and x.is_cuda and x.dtype == torch.bfloat16
            and x.dim() >= 1 and isinstance(w8, torch.Tensor) and w8.dtype == torch.int8
            and w8.dim() == 2 and w8.device == x.device and x.shape[-1] == w8.shape[1]
            and w8.shape[1] % 256 == 0 and w8.shape[0] % 16 == 0 and x.numel() > 0)


def _linear_acc_bf16(lib, x2, w8c, m, n, k):
    """quantize + int32 GEMM of a bf16 [m, k] through one library call
    (xpuint8_linear_acc_packed_stream, with the weight's packed copy if it
    has one): ``(int32 [m, n], fp32 [m])``."""
    need = lib.xpuint8_linear_workspace_size(m, n, k)
    if need < 0:
        _err(lib, "linear_acc")
    work = torch.empty(int(need), device=x2.device, dtype=torch.uint8)
    acc = torch.empty((m, n), device=x2.device, dtype=torch.int32)
    xs = torch.empty((m,), device=x2.device, dtype=torch.float32)
    rc = lib.xpuint8_linear_acc_packed_stream(_stream(x2.device), _ptr(x2), _ptr(w8c),
                                              _opt(_packed_for(w8c)), _ptr(acc), _ptr(xs), m, n,
                                              k, _ptr(work), int(need))
    if rc != 0:
        _err(lib, "linear_acc")
    return acc, xs


def _linear_residual_bf16(lib, x2, w8c, ws, b, b16, res, rs, m, n, k):
    """quantize + GEMM + dequant + residual update of a bf16 [m, k] through one
    library call (xpuint8_linear_residual_packed_stream, with the weight's
    packed copy if it has one)."""
    need = lib.xpuint8_linear_workspace_size(m, n, k)
    if need < 0:
        _err(lib, "linear")
    work = torch.empty(int(need), device=x2.device, dtype=torch.uint8)
    out = torch.empty((m, n), device=x2.device, dtype=torch.bfloat16)
    rc = lib.xpuint8_linear_residual_packed_stream(
        _stream(x2.device), _ptr(x2), _ptr(w8c), _opt(_packed_for(w8c)), _ptr(ws), _opt(b), b16,
        _ptr(res), _ptr(rs), _ptr(out), m, n, k, _ptr(work), int(need))
    if rc != 0:
        _err(lib, "linear")
    return out


def linear(x, w8, w_scale, bias=None, act: Optional[str] = None, residual=None,
           residual_scale=None, return_acc: bool = False):
    """INT8 ConvRot linear: bf16/fp32 [.., K] -> bf16/fp32 [.., N] (ops.py:591-646).

    Two kernels: rotate+quantize of ``x`` (with ``act`` fused into its load),
    then the MFMA GEMM with the dequant (+bias) epilogue fused into its store;
    a product too small to fill the GPU is split in K across blocks, and a
    third kernel adds the slices' int32 sums and applies the dequant.  When
    ``w8`` carries a valid packed copy (:func:`prepare_weight`,
    :func:`pack_weight`) the GEMMs that take the block layout read it instead,
    with the same results.
    ``residual``/``residual_scale`` apply ``residual + residual_scale * out``;
    ``return_acc`` returns ``(int32 [M, N], fp32 [M], fp32 [N])`` instead.
    """
    reason = unsupported_reason(x, w8, w_scale, act)
    if reason is not None:
        raise TypeError(reason)
    if return_acc and (bias is not None or residual is not None):
        raise ValueError("return_acc skips the epilogue, so bias and residual "
                         "cannot be applied")
    m, n, k = _dims(x, w8, act)
    input_dtype = x.dtype
    x2 = x.reshape(m, -1)
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(dtype=torch.bfloat16)
    if not x2.is_contiguous():
        x2 = x2.contiguous()

    lib = _lib()
    w8c = _c(w8)
    rs = None if return_acc else _fused_residual_scale(residual, residual_scale, input_dtype, n,
                                                      x.device)
    if act is None and not return_acc and rs is None:
        # quantize and GEMM in one call, the quantized activation in a
        # workspace laid out for the GEMM that reads it
        ws = expand_scale(w_scale, n, x.device)
        b, b16 = _bias_arg(bias, n, x.device)
        out = _linear_bf16(lib, x2, w8c, ws, b, b16, m, n, k, _packed_for(w8c))
        return _residual_tail(out, residual, residual_scale, input_dtype, x.shape, m, n)
    if act is None and rs is not None:
        # the residual update in the GEMM's store, quantize and GEMM in one call
        ws = expand_scale(w_scale, n, x.device)
        b, b16 = _bias_arg(bias, n, x.device)
        res = _c(residual.reshape(m, n).to(torch.bfloat16))
        out = _linear_residual_bf16(lib, x2, w8c, ws, b, b16, res, rs, m, n, k)
        return out.reshape(*x.shape[:-1], n)
    if act is None and return_acc:
        acc, xs = _linear_acc_bf16(lib, x2, w8c, m, n, k)
        return acc, xs, expand_scale(w_scale, n, acc.device)
    if act is None:
        xq, xs = quantize(x2)
    else:
        xq, xs = quantize_act(x2, act)
    if return_acc:
        acc = int_mm(xq, w8c.t())
        return acc, xs.reshape(-1), expand_scale(w_scale, n, acc.device)

    ws = expand_scale(w_scale, n, x.device)
    b, b16 = _bias_arg(bias, n, x.device)
    out = torch.empty((m, n), device=x.device, dtype=torch.bfloat16)
    if rs is not None:
        # the residual update in the GEMM's store: bf16 activation, residual
        # and per-column scale, the case whose addcmul result is bf16
        res = _c(residual.reshape(m, n).to(torch.bfloat16))
        rc = lib.xpuint8_linear_gemm_residual_stream(
            _stream(x.device), _ptr(xq), _ptr(xs), _ptr(w8c), _ptr(ws), _opt(b), b16,
            _ptr(res), _ptr(rs), _ptr(out), m, n, k)
        if rc != 0:
            _err(lib, "linear")
        return out.reshape(*x.shape[:-1], n)
    rc = lib.xpuint8_linear_gemm_stream(_stream(x.device), _ptr(xq), _ptr(xs), _ptr(w8c),
                                        _ptr(ws), _opt(b), b16, _ptr(out), m, n, k)
    if rc != 0:
        _err(lib, "linear")
    return _residual_tail(out, residual, residual_scale, input_dtype, x.shape, m, n)


def _linear_bf16(lib, x2, w8c, ws, b, b16, m, n, k, packed=None):
    """quantize + GEMM + dequant of a bf16 [m, k] through one library call
    (xpuint8_linear_stream, or xpuint8_linear_packed_stream with the weight's
    packed copy) with its workspace."""
    need = lib.xpuint8_linear_workspace_size(m, n, k)
    if need < 0:
        _err(lib, "linear")
    work = torch.empty(int(need), device=x2.device, dtype=torch.uint8)
    out = torch.empty((m, n), device=x2.device, dtype=torch.bfloat16)
    if packed is not None:
        rc = lib.xpuint8_linear_packed_stream(_stream(x2.device), _ptr(x2), _ptr(w8c),
                                              _ptr(packed), _ptr(ws), _opt(b), b16, _ptr(out), m,
                                              n, k, _ptr(work), int(need))
        if rc != 0:
            _err(lib, "linear")
        return out
    rc = lib.xpuint8_linear_stream(_stream(x2.device), _ptr(x2), _ptr(w8c), _ptr(ws), _opt(b),
                                   b16, _ptr(out), m, n, k, _ptr(work), int(need))
    if rc != 0:
        _err(lib, "linear")
    return out


def _residual_tail(out, residual, residual_scale, input_dtype, shape, m, n):
    """ops.py:639-646 after the GEMM: a residual the store did not fuse (an
    fp32 model, a per-row or full-size scale, an fp32 scale whose addcmul
    promotes to fp32) through the reference's own torch chain, then the
    reshape and the cast back to the input dtype."""
    if residual is not None:
        residual = residual.reshape(m, n).to(
            out.dtype if input_dtype == torch.bfloat16 else input_dtype)
        if input_dtype != torch.bfloat16:
            out = out.to(dtype=input_dtype)
        out = torch.addcmul(residual, out, residual_scale)
    out = out.reshape(*shape[:-1], n)
    return out if input_dtype == torch.bfloat16 else out.to(dtype=input_dtype)


def _fused_residual_scale(residual, residual_scale, input_dtype, n, device):
    """The flat bf16 [n] residual scale when ``residual + residual_scale * out``
    can run in the GEMM's epilogue, else None: a bf16 activation, a residual
    tensor on the device, and a bf16 scale tensor that is one value or one per
    output column (shape [.., n] with every leading dim 1), so the reference's
    addcmul is bf16 and broadcasts the scale along rows only."""
    if residual is None or input_dtype != torch.bfloat16:
        return None
    if not isinstance(residual, torch.Tensor) or residual.device != device:
        return None
    s = residual_scale
    if not isinstance(s, torch.Tensor) or s.dtype != torch.bfloat16 or s.device != device:
        return None
    if residual.dtype not in (torch.bfloat16, torch.float32, torch.float16):
        return None
    if s.numel() == 1:
        return _c(s.reshape(1).expand(n))
    if s.dim() >= 1 and s.shape[-1] == n and s.numel() == n:
        return _c(s.reshape(n))
    return None


def ffn(x, up_w8, up_scale, down_w8, down_scale, down_bias=None, act="situ"):
    """``act(up(x)) @ down.T`` (ops.py:649-719).  ``up_w8`` is [2*ffn, K]
    (``[hidden | gate]``) for a paired activation and [ffn, K] for
    ``gelu_erf``; ``down_w8`` is [K, ffn].  The up projection is unbiased.

    One library call (xpuint8_ffn_stream) of four kernels: rotate+quantize of
    x; the up-projection GEMM whose epilogue dequantizes each half and
    applies the activation, writing the bf16 activation [M, ffn] (its hidden
    and gate columns are computed in the same lanes); rotate+quantize of
    that; the down-projection GEMM with the dequant (+bias) epilogue (at small
    M split in K across blocks, with one more kernel that adds the slices).
    The codes equal the reference's fused
    dequant+activation+quantize of the int32 accumulator bit for bit (the
    bf16 activation is exactly the value that kernel forms), without writing
    the [M, 2*ffn] int32 accumulator."""
    if act not in ACTIVATIONS:
        raise TypeError(f"unknown activation {act!r}; "
                        f"known: {', '.join(sorted(ACTIVATIONS))}")
    if act not in ("situ", "geglu_erf", "gelu_erf"):
        raise TypeError(f"the fused FFN supports situ, geglu_erf and gelu_erf, "
                        f"not {act!r}")
    paired = act in PAIRED_ACTIVATIONS
    reason = unsupported_reason(x, up_w8, up_scale, None)
    if reason is not None:
        raise TypeError(reason)
    m, n, k = _dims(x, up_w8, None)
    if paired and n % 2:
        raise TypeError(f"up-projection N={n} must be 2*ffn for the {act} activation")
    inner = n // 2 if paired else n
    if inner % 256 or inner % 16:
        raise TypeError(f"the FFN's inner width {inner} must be a multiple of "
                        f"256 (and of 16) for the fused {act} epilogue")
    if down_w8.dtype != torch.int8 or down_w8.dim() != 2:
        raise TypeError(f"down weight must be an int8 [K, ffn] tensor, got "
                        f"{down_w8.dtype} {tuple(down_w8.shape)}")
    if tuple(down_w8.shape) != (k, inner):
        raise TypeError(f"down weight is {tuple(down_w8.shape)}, expected {(k, inner)}")
    if down_w8.device != x.device:
        raise TypeError(f"down weight is on {down_w8.device} but the activation "
                        f"is on {x.device}")
    if isinstance(down_scale, torch.Tensor):
        if down_scale.dtype != torch.float32 or down_scale.dim() > 2:
            raise TypeError("down weight scale must be a float32 scalar or [K]")
        if down_scale.numel() not in (1, k):
            raise TypeError(f"down weight scale has {down_scale.numel()} values; "
                            f"expected 1 or K={k}")
    elif not isinstance(down_scale, (float, int)):
        raise TypeError("down weight scale must be a tensor or a python float")

    device = x.device
    input_dtype = x.dtype
    x2 = x.reshape(m, k)
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(dtype=torch.bfloat16)
    if not x2.is_contiguous():
        x2 = x2.contiguous()

    lib = _lib()
    uw8 = _c(up_w8)
    us = expand_scale(up_scale, n, device)
    dw8 = _c(down_w8)
    ds = expand_scale(down_scale, k, device)
    b, b16 = _bias_arg(down_bias, k, device)
    code = ACTIVATIONS[act]
    need = lib.xpuint8_ffn_workspace_size(m, inner, k, code)
    if need < 0:
        _err(lib, "ffn")
    # the four (five) kernels in one library call, the intermediates in `work`
    work = torch.empty(int(need), device=device, dtype=torch.uint8)
    out = torch.empty((m, k), device=device, dtype=torch.bfloat16)
    up_p, down_p = _packed_for(uw8), _packed_for(dw8)
    if up_p is not None or down_p is not None:
        rc = lib.xpuint8_ffn_packed_stream(_stream(device), _ptr(x2), _ptr(uw8), _opt(up_p),
                                           _ptr(us), _ptr(dw8), _opt(down_p), _ptr(ds), _opt(b),
                                           b16, _ptr(out), m, inner, k, code, _ptr(work),
                                           int(need))
    else:
        rc = lib.xpuint8_ffn_stream(_stream(device), _ptr(x2), _ptr(uw8), _ptr(us), _ptr(dw8),
                                    _ptr(ds), _opt(b), b16, _ptr(out), m, inner, k, code,
                                    _ptr(work), int(need))
    if rc != 0:
        _err(lib, "ffn")
    out = out.reshape(*x.shape[:-1], k)
    return out if input_dtype == torch.bfloat16 else out.to(dtype=input_dtype)


def ffn_situ(x, up_w8, up_scale, down_w8, down_scale, down_bias=None):
    """:func:`ffn` with MossImage's activation (ops.py:722-727)."""
    return ffn(x, up_w8, up_scale, down_w8, down_scale, down_bias, act="situ")


class TrainableInt8Linear(torch.nn.Module):
    """A linear whose bf16 parameter is quantized on every forward with
    :func:`prepare_weight_fused` (straight-through; ops.py:730-789)."""

    def __init__(self, weight, bias=None, *, backward="ste"):
        super().__init__()
        if weight.dtype not in (torch.bfloat16, torch.float32):
            raise TypeError(f"the weight must be bfloat16 or float32, got {weight.dtype}")
        if backward not in ("ste", "dense"):
            raise ValueError(f"unknown backward mode {backward!r}; use 'ste' or 'dense'")
        self.weight = torch.nn.Parameter(weight.detach())
        self.bias = None if bias is None else torch.nn.Parameter(
            bias.detach().to(self.weight.dtype))
        self.backward = backward

    @classmethod
    def from_linear(cls, mod, *, backward="ste"):
        return cls(mod.weight.detach(), getattr(mod, "bias", None), backward=backward)

    def forward(self, x):
        return _TrainableInt8LinearFn.apply(x, self.weight, self.bias, self.backward)

    def extra_repr(self):
        return (f"{tuple(self.weight.shape)}, backward={self.backward}, "
                f"bias={self.bias is not None}")


class _TrainableInt8LinearFn(torch.autograd.Function):
    """The autograd op behind :class:`TrainableInt8Linear` (ops.py:792-824)."""

    @staticmethod
    def forward(ctx, x, weight, bias, mode):
        w8, ws = prepare_weight_fused(weight)
        y = linear(x, w8, ws, bias)
        ctx.save_for_backward(x, weight, w8, ws)
        ctx.mode = mode
        ctx.has_bias = bias is not None
        return y

    @staticmethod
    def backward(ctx, dy):
        x, weight, w8, ws = ctx.saved_tensors
        dy = dy.reshape(-1, dy.shape[-1])
        x2 = x.reshape(-1, x.shape[-1])
        w = dequant_weight(w8, ws) if ctx.mode == "dense" else weight
        # the reference multiplies dy @ w as they are (ops.py:815-820); the
        # dense weight is bf16, so an fp32 dy is cast to it (where the
        # reference's matmul would refuse the mixed dtypes)
        dx = linear_dx(dy if dy.dtype == w.dtype else dy.to(w.dtype), w)
        dw = linear_dw(dy, x2)
        db = column_sum(dy) if ctx.has_bias else None
        if dw.dtype != weight.dtype:
            dw = dw.to(weight.dtype)
        return (dx.reshape(x.shape[:-1] + (dx.shape[-1],)), dw, db, None)


class Int8Linear(torch.nn.Module):
    """Drop-in ``nn.Linear`` replacement with prepared weights (ops.py:831-902)."""

    def __init__(self, w8, w_scale, bias=None, *, backward="dense", pack=True):
        super().__init__()
        self.register_buffer("w8", w8.detach())
        self.register_buffer("w_scale", w_scale.detach().to(torch.float32))
        self.bias = None if bias is None else torch.nn.Parameter(
            bias.detach().to(torch.float32), requires_grad=False)
        if backward not in ("dense", "int8"):
            raise ValueError(f"unknown backward mode {backward!r}; use 'dense' or 'int8'")
        self.backward = backward
        # keep a packed copy of the weight (pack_weight), made again when the
        # weight moves or is written; False reads w8 as it is
        self.pack = pack

    @classmethod
    def from_linear(cls, mod, *, backward="dense", pack=True):
        q, scale = prepare_weight(mod.weight.detach(), pack=pack)
        return cls(q, scale, getattr(mod, "bias", None), backward=backward, pack=pack)

    def forward(self, x):
        if (self.pack and _pack_key(self.w8) is not None and _packed_for(self.w8) is None
                and not is_capturing()):
            pack_weight(self.w8)
        return int8_linear(x, self.w8, self.w_scale, self.bias, mode=self.backward)

    def dense_weight(self, refresh=False):
        """The unrotated bf16 weight, dequantized once and cached; refused inside
        a device-graph capture (ops.py:868-894)."""
        cached = getattr(self, "_dense", None)
        if cached is None or refresh:
            if is_capturing():
                raise RuntimeError(
                    "Int8Linear.dense_weight() materializes a second, full-precision copy "
                    "of the weight; inside a device-graph capture it would be captured and "
                    "re-computed on every replay. Call it before capturing.")
            cached = dequant_weight(self.w8, self.w_scale)
            self._dense = cached
        return cached

    def dx(self, dy):
        return linear_dx(dy, self.dense_weight())

    def extra_repr(self):
        n, k = self.w8.shape
        return f"in_features={k}, out_features={n}, bias={self.bias is not None}"
