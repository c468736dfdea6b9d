"""torch-CPU restatement of the reference's oracle, reference/convrot_linear.py:5-23
-- TEST INFRASTRUCTURE AND CPU BASELINE ONLY.

The reference's function uses ``torch.eye`` as its rotation (line 11); this
restatement keeps every other operation of it (the fp32 row scale, the IEEE
division, ``round``, ``clamp``, ``torch._int_mm``, the ``(acc * xs) * ws``
dequant, the bf16 cast and the bf16 bias add) and puts the real ConvRot
rotation in the identity's place: an fp32 [256, 256] matmul by
kron(H4, H4, H4, H4) / 16, which costs what the reference's identity matmul
costs.  It is the CPU baseline that ``bench.py`` times on the GPU host, and
``tests/test_oracle_torch_chain.py`` pins it against the numpy oracle.
Nothing in the product path imports it.
"""

from __future__ import annotations

import torch

H4 = ((1, 1, 1, -1), (1, 1, -1, 1), (1, -1, 1, 1), (-1, 1, 1, 1))   # src/xpuint8.cpp:75


def hadamard_matrix(group: int = 256) -> torch.Tensor:
    """kron(H4, H4, H4, H4) / 16 as an fp32 [256, 256] tensor (exact)."""
    if group != 256:
        raise ValueError("the ConvRot group is 256")
    h4 = torch.tensor(H4, dtype=torch.float64)
    h = torch.ones(1, 1, dtype=torch.float64)
    for _ in range(4):
        h = torch.kron(h, h4)
    return (h / 16.0).to(torch.float32)


def quantized_linear_from_rotated(x_rot, weight, weight_scale, bias=None, out_dtype=torch.bfloat16):
    """reference/convrot_linear.py:15-23 on an already-rotated fp32 activation
    [M, K]: row scale, int8 codes, torch._int_mm, dequant, cast, bias."""
    abs_max = x_rot.abs().amax(dim=-1, keepdim=True)
    x_scale = (abs_max.float() / 127.0).clamp(min=1e-30)
    x_int8 = (x_rot.float() / x_scale).round().clamp(-127, 127).to(torch.int8)
    result = torch._int_mm(x_int8, weight.t().contiguous())
    result = (result.float() * x_scale) * weight_scale.view(1, -1)
    result = result.to(out_dtype)
    if bias is not None:
        result = result + bias
    return result


def convrot_int8_linear(x, weight, weight_scale, bias=None, h=None):
    """The reference oracle with the ConvRot rotation: bf16 x [M, K] (K % 256
    == 0), int8 prepared weight [N, K], fp32 scale [N], bf16 bias [N] ->
    bf16 [M, N].  ``h`` is hadamard_matrix(), passed in to keep it out of a
    timed region."""
    if h is None:
        h = hadamard_matrix()
    m, k = x.shape
    x_rot = (x.float().reshape(m, k // 256, 256) @ h).reshape(m, k)   # H is symmetric
    return quantized_linear_from_rotated(x_rot, weight, weight_scale, bias, x.dtype)
