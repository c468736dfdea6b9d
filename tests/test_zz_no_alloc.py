"""The no-allocation entry point, xpuint8_linear_dx_int8_noalloc_stream,
against the workspace entry point it mirrors (xpuint8_linear_dx_int8_stream),
through the C ABI: bit-identical dx on two calls in a row, the second smaller
than the first (the library's fixed scratch keeps the first call's contents,
which the second must not depend on), and the size limit reported as an
error before any device work."""

import numpy as np
import pytest
import torch

from gpu_util import activation, bits, mismatch, weight
from xpu_kernels import int8
from xpu_kernels.int8 import _lib as L

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20


def _inputs(dev, m, n, k, seed):
    w8, ws = int8.prepare_weight(weight(n, k, seed=seed).to(dev))
    dy = (activation(m, n, seed=seed + 1, n_out=0).float() * 1e-3).to(torch.bfloat16).to(dev)
    return dy, w8, ws


def _with_workspace(lib, dev, dy, w8, ws, m, n, k):
    nbytes = lib.xpuint8_linear_dx_int8_workspace_size(m, n, k)
    assert nbytes > 0
    work = torch.empty((nbytes,), device=dev, dtype=torch.int8)
    out = torch.empty((m, k), device=dev, dtype=torch.bfloat16)
    rc = lib.xpuint8_linear_dx_int8_stream(L._stream(dev), L._ptr(dy), L._ptr(ws), L._ptr(w8),
                                           L._ptr(out), m, n, k, L._ptr(work), nbytes)
    assert rc == 0, lib.xpuint8_last_error()
    return out


def _no_alloc(lib, dev, dy, w8, ws, m, n, k):
    out = torch.empty((m, k), device=dev, dtype=torch.bfloat16)
    rc = lib.xpuint8_linear_dx_int8_noalloc_stream(L._stream(dev), L._ptr(dy), L._ptr(ws),
                                                   L._ptr(w8), L._ptr(out), m, n, k)
    assert rc == 0, lib.xpuint8_last_error()
    return out


def test_no_alloc_matches_the_workspace_entry_point(dev):
    lib = L._lib()
    # config 5's dx (38 MB of scratch), then a smaller, ragged-in-M call
    for m, n, k, seed in ((4096, 5120, 1280, 20), (77, 1024, 512, 30)):
        print(f"no_alloc: dx M={m} N={n} K={k} seed={seed}", flush=True)
        dy, w8, ws = _inputs(dev, m, n, k, seed)
        got = _no_alloc(lib, dev, dy, w8, ws, m, n, k)
        want = _with_workspace(lib, dev, dy, w8, ws, m, n, k)
        torch.cuda.synchronize()
        assert np.array_equal(bits(got), bits(want)), mismatch(bits(got), bits(want))


def test_no_alloc_rejects_shapes_beyond_the_scratch(dev):
    lib = L._lib()
    m, n, k = 16384, 5120, 1280
    assert lib.xpuint8_linear_dx_int8_workspace_size(m, n, k) > SCRATCH_BYTES
    p = L._ptr(torch.empty(16, device=dev, dtype=torch.int8))
    rc = lib.xpuint8_linear_dx_int8_noalloc_stream(L._stream(dev), p, p, p, p, m, n, k)
    assert rc == 4 and "64 MiB" in lib.xpuint8_last_error().decode()
