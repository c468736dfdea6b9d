"""ConvRot INT8 primitives for AMD Instinct MI355X (gfx950), on ROCm tensors.

A drop-in for the reference's ``xpu_kernels.int8`` (okolenmi/oko-xpu-kernels,
``python/xpu_kernels/int8/__init__.py:66-102``): the same names and contracts,
backed by ``libxpuint8.so`` -- hand-written HIP kernels for gfx950 -- loaded
through ctypes.

    bf16 [M,K] --rotate+quantize--------------------------> int8 [M,K] + fp32 [M]
    int8 [M,K] x int8 [N,K].T --MFMA GEMM, dequant fused--> bf16 [M,N]
                              --MFMA GEMM---------------> int32 [M,N]
    int32 [M,N] --dequant(+bias)--------------------------> bf16 [M,N]
                 --or dequant+activation+rotate+quantize--> int8 [M,K2] + fp32 [M]

Bit-exactness contract: ``dequant(linear_acc(x, w8, ws)[0], ...)`` is
bit-identical to ``linear(x, ...)``; the dequant arithmetic is
``float(acc) * (w_scale[n] * x_scale[m])`` (+ bias) rounded to bf16, in that
order.  K must be a multiple of 256 and N a multiple of 16.
"""

from __future__ import annotations

from ._lib import ACTIVATIONS, PAIRED_ACTIVATIONS, available, device_name, load
from .ops import (
    Int8Linear,
    TrainableInt8Linear,
    column_sum,
    dequant,
    dequant_act_quantize,
    dequant_slice,
    dequant_weight,
    dequant_weight_torch,
    expand_scale,
    ffn,
    ffn_situ,
    int8_linear,
    int_mm,
    linear,
    linear_acc,
    linear_dw,
    linear_dx,
    linear_dx_int8,
    pack_weight,
    prepare_weight,
    prepare_weight_fused,
    quantize,
    quantize_act,
    quantize_row,
    quantize_row_torch,
    rotate,
    unsupported_reason,
)
from .selftest import selftest

__all__ = [
    "ACTIVATIONS", "Int8Linear", "PAIRED_ACTIVATIONS", "TrainableInt8Linear", "available",
    "dequant", "dequant_act_quantize", "dequant_slice", "dequant_weight",
    "dequant_weight_torch", "device_name", "expand_scale", "ffn", "ffn_situ", "int8_linear",
    "int_mm", "linear", "linear_acc", "linear_dw", "linear_dx", "linear_dx_int8", "load",
    "pack_weight", "prepare_weight", "prepare_weight_fused", "quantize", "quantize_act", "quantize_row",
    "quantize_row_torch", "rotate", "selftest", "unsupported_reason",
]
