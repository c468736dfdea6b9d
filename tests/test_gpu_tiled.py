"""The MFMA block layout of the quantized activation, on the GPU.

``xpuint8_convrot_quantize_tiled_stream`` must hold exactly the codes of the
row-major quantizer (pinned to the oracle elsewhere), placed by the layout the
header documents, and ``xpuint8_linear_gemm_tiled_stream`` on them must equal
``xpuint8_linear_gemm_stream`` on the row-major codes bit for bit: the
persistent ping-pong kernel (X in that layout) against the same kernel with
row-major X, and the split-K kernel's tiled form, at ragged and full shapes.
"""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import activation, bits, mismatch, weight
from xpu_kernels import int8
from xpu_kernels.int8 import _lib as L

pytestmark = pytest.mark.gpu


def untile(buf, m, k):
    """Row-major [m, k] codes from the block layout (the header's formula)."""
    kb = (k + 63) // 64
    blocks = buf[: ((m + 15) // 16) * kb * 1024].reshape(-1, kb, 16, 4, 16)
    r = np.arange(16)[:, None]
    c = np.arange(4)[None, :]
    pos = c ^ ((r >> 1) & 3)                                  # chunk c of row r sits at pos
    rows = blocks[:, :, r, pos, :]                            # [rg, kb, 16, 4, 16] logical order
    full = rows.transpose(0, 2, 1, 3, 4).reshape(-1, kb * 64)
    return full[:m, :k]


def quantize_both(dev, x, m, k):
    lib = L._lib()
    tx = x.to(dev)
    q = torch.empty((m, k), device=dev, dtype=torch.int8)
    s = torch.empty(m, device=dev, dtype=torch.float32)
    rc = lib.xpuint8_convrot_quantize_stream(L._stream(dev), L._ptr(tx), L._ptr(q), L._ptr(s), m, k)
    assert rc == 0, lib.xpuint8_last_error()
    tb = ((m + 15) // 16) * ((k + 63) // 64) * 1024
    qt = torch.full((tb,), 99, device=dev, dtype=torch.int8)
    st = torch.empty(m, device=dev, dtype=torch.float32)
    rc = lib.xpuint8_convrot_quantize_tiled_stream(L._stream(dev), L._ptr(tx), L._ptr(qt),
                                                   L._ptr(st), m, k)
    assert rc == 0, lib.xpuint8_last_error()
    return q, s, qt, st


@pytest.mark.parametrize("m,k", [(1, 256), (37, 1280), (4100, 1280), (64, 5120), (9, 20480)])
def test_quantize_tiled_is_the_quantizer(dev, m, k):
    x = activation(m, k, seed=m + k)
    q, s, qt, st = quantize_both(dev, x, m, k)
    torch.cuda.synchronize()
    assert torch.equal(s, st)
    got = untile(qt.cpu().numpy(), m, k)
    want = q.cpu().numpy()
    assert np.array_equal(got, want), mismatch(got, want)


@pytest.mark.parametrize("m,n,k", [(4096, 10240, 1280), (4100, 10240, 1280), (2304, 9600, 2560),
                                   (4352, 7808, 768), (4096, 1280, 5120), (2100, 1296, 2048)])
def test_linear_gemm_tiled_matches_row_major(dev, m, n, k):
    """The persistent kernel on tiled X (config 3; 4 rows in a last partial
    16-row block; 30 tiles of 9 x 2560 ... ; 12 K steps) and the split-K kernel
    on tiled X (the last two shapes), against the row-major entry point and
    the oracle's dequant of the exact product."""
    g = torch.Generator().manual_seed(m + n + k)
    x = activation(m, k, seed=m + 7 * k)
    w = weight(n, k, seed=n + k)
    w8, ws = int8.prepare_weight(w.to(dev))
    q, s, qt, st = quantize_both(dev, x, m, k)
    bias = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16).to(dev)
    lib = L._lib()
    outs = []
    for fn, xq in (("xpuint8_linear_gemm_stream", q), ("xpuint8_linear_gemm_tiled_stream", qt)):
        out = torch.full((m, n), -1, device=dev, dtype=torch.int16).view(torch.bfloat16)
        rc = getattr(lib, fn)(L._stream(dev), L._ptr(xq), L._ptr(s), L._ptr(w8), L._ptr(ws),
                              L._ptr(bias), 1, L._ptr(out), m, n, k)
        assert rc == 0, (fn, lib.xpuint8_last_error())
        outs.append(bits(out))
    assert np.array_equal(outs[1], outs[0]), mismatch(outs[1], outs[0])
    want = O.dequant(O.int_mm(q.cpu().numpy(), w8.cpu().numpy()), s.cpu().numpy(),
                     ws.cpu().numpy(), O.bf16_to_f32(bits(bias)))
    assert np.array_equal(outs[0], want), mismatch(outs[0], want)


@pytest.mark.parametrize("m,n,k", [(4096, 10240, 1280), (2100, 1296, 2048)])
@pytest.mark.parametrize("bias_kind", ["fp32", "none"])
def test_linear_gemm_tiled_bias_forms(dev, m, n, k, bias_kind):
    """The tiled entry point with an fp32 bias and with none (persistent and
    split-K kernels), against the oracle's dequant of the exact product."""
    x = activation(m, k, seed=m + 11 * k)
    w8, ws = int8.prepare_weight(weight(n, k, seed=n + 2 * k).to(dev))
    q, s, qt, st = quantize_both(dev, x, m, k)
    if bias_kind == "fp32":
        b = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 0.01).float()
        barg, bf = b.to(dev), b.numpy()
    else:
        barg, bf = None, None
    lib = L._lib()
    out = torch.full((m, n), -1, device=dev, dtype=torch.int16).view(torch.bfloat16)
    rc = lib.xpuint8_linear_gemm_tiled_stream(L._stream(dev), L._ptr(qt), L._ptr(st), L._ptr(w8),
                                              L._ptr(ws), None if barg is None else L._ptr(barg),
                                              0, L._ptr(out), m, n, k)
    assert rc == 0, lib.xpuint8_last_error()
    want = O.dequant(O.int_mm(q.cpu().numpy(), w8.cpu().numpy()), s.cpu().numpy(),
                     ws.cpu().numpy(), bf)
    assert np.array_equal(bits(out), want), mismatch(bits(out), want)


def test_linear_gemm_tiled_rejects_other_shapes(dev):
    lib = L._lib()
    p = torch.empty(16, device=dev, dtype=torch.int8)
    rc = lib.xpuint8_linear_gemm_tiled_stream(L._stream(dev), L._ptr(p), L._ptr(p), L._ptr(p),
                                              L._ptr(p), None, 0, L._ptr(p), 300, 1040, 1280)
    assert rc == 2
    assert b"block layout" in lib.xpuint8_last_error()
