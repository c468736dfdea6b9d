"""The split-K GEMM's two-team epilogue (each team finishes half of the
tile's rows; the row and column operands loaded before the main loop) with
every epilogue it serves, at ragged shapes where the last tiles are partly
outside the output: the dequant with a bf16 bias, an fp32 bias and none; the
fused residual update; and the GELU up-projection of an FFN whose inner width
is narrow.  Each is bit for bit the oracle's."""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import activation, bits, mismatch, npy, weight
from xpu_kernels import int8
from xpu_kernels.int8 import _lib as L

pytestmark = pytest.mark.gpu

# (M, N, K) that take the split-K kernel: fewer than 192 tiles of 256 x 160,
# at least 128 tiles of 128 x 160, K >= 1024.  2100 rows leave the last row
# tile 52 rows (its second wave row entirely outside), 1296 columns a last
# column tile of 16.
SHAPES = [(2100, 1296, 2048), (4096, 1280, 1024), (3000, 1120, 1280)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("bias_kind", ["bf16", "fp32", "none"])
def test_splitk_dequant_bias_forms_exact(dev, m, n, k, bias_kind):
    x = activation(m, k, seed=m + k)
    w8, ws = int8.prepare_weight(weight(n, k, seed=n + 3).to(dev))
    lib = L._lib()
    q = torch.empty((m, k), device=dev, dtype=torch.int8)
    s = torch.empty(m, device=dev, dtype=torch.float32)
    tx = x.to(dev)
    assert lib.xpuint8_convrot_quantize_stream(L._stream(dev), L._ptr(tx), L._ptr(q), L._ptr(s),
                                               m, k) == 0
    b16 = weight(1, n, seed=7, std=0.01)[0]
    if bias_kind == "bf16":
        barg, flag, bf = b16.to(dev), 1, O.bf16_to_f32(bits(b16))
    elif bias_kind == "fp32":
        b32 = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 0.01).float()
        barg, flag, bf = b32.to(dev), 0, b32.numpy()
    else:
        barg, flag, bf = None, 0, None
    out = torch.full((m, n), -1, device=dev, dtype=torch.int16).view(torch.bfloat16)
    rc = lib.xpuint8_linear_gemm_stream(L._stream(dev), L._ptr(q), L._ptr(s), L._ptr(w8),
                                        L._ptr(ws), None if barg is None else L._ptr(barg), flag,
                                        L._ptr(out), m, n, k)
    assert rc == 0, lib.xpuint8_last_error()
    want = O.dequant(O.int_mm(npy(q), npy(w8)), npy(s), npy(ws), bf)
    assert np.array_equal(bits(out), want), mismatch(bits(out), want)


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_splitk_residual_exact(dev, m, n, k):
    x = activation(m, k, seed=m + 2 * k)
    w8, ws = int8.prepare_weight(weight(n, k, seed=n + 5).to(dev))
    bias = weight(1, n, seed=9, std=0.01)[0]
    g = torch.Generator().manual_seed(m * n)
    res = torch.randn(m, n, generator=g).to(torch.bfloat16)
    rscale = (torch.rand(n, generator=g) * 2 - 0.5).to(torch.bfloat16)
    got = int8.linear(x.to(dev), w8, ws, bias.to(dev), residual=res.to(dev),
                      residual_scale=rscale.to(dev))
    d = O.linear(bits(x), npy(w8), npy(ws), O.bf16_to_f32(bits(bias)))
    f = O.bf16_to_f32
    want = O.f32_to_bf16(f(bits(res)) + f(d) * f(bits(rscale))[None, :])
    assert np.array_equal(bits(got), want), mismatch(bits(got), want)


@pytest.mark.parametrize("m,k,inner", [(4096, 2048, 1280), (2100, 1024, 1280)])
def test_splitk_gelu_up_projection_exact(dev, m, k, inner):
    """FFN with GELU (erf): the up-projection [m, inner] from K = k takes the
    split-K kernel with the activation epilogue."""
    x = activation(m, k, seed=m + inner)
    up8, ups = int8.prepare_weight(weight(inner, k, seed=inner + 1).to(dev))
    dn8, dns = int8.prepare_weight(weight(k, inner, seed=inner + 2).to(dev))
    db = weight(1, k, seed=k + 5, std=0.01)[0]
    y = int8.ffn(x.to(dev), up8, ups, dn8, dns, db.to(dev), act="gelu_erf")
    want = O.ffn(bits(x), npy(up8), npy(ups), npy(dn8), npy(dns), O.bf16_to_f32(bits(db)),
                 act=5)
    assert np.array_equal(bits(y), want), mismatch(bits(y), want)
