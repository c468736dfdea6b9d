"""The library from plain C, with no Python or torch in the process:
tests/c_abi/linear_consumer.c (built by the library's Makefile) allocates with
hipMalloc, prepares the weight and runs the one-call INT8 linear on a stream
of its own through include/xpuint8.h, and checks that a K off the group size
and a short workspace are refused.  Its outputs must equal the oracle's bit
for bit: the split-K shape (N = 1280), a 128 x 128-tile shape and a ragged
one."""

import os
import subprocess

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_abi", "linear_consumer")


@pytest.mark.parametrize("m,n,k", [(4096, 1280, 1280), (512, 2048, 2048), (300, 1040, 1280)])
def test_c_consumer_linear_exact(tmp_path, m, n, k):
    assert os.path.exists(BIN), "tests/c_abi/linear_consumer is not built (run build())"
    rng = np.random.default_rng(m + 3 * n + 7 * k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, rng.choice(k, k // 100, replace=False)] *= 30.0
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    b = (rng.standard_normal(n) * 0.01).astype(np.float32)
    xb, wb, bb = O.f32_to_bf16(x), O.f32_to_bf16(w), O.f32_to_bf16(b)
    xb.tofile(tmp_path / "x.bin")
    wb.tofile(tmp_path / "w.bin")
    bb.tofile(tmp_path / "b.bin")
    print(f"c consumer {m}x{n}x{k}", flush=True)
    r = subprocess.run([BIN, str(tmp_path), str(m), str(n), str(k)], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("ok")
    w8 = np.fromfile(tmp_path / "w8.bin", dtype=np.int8).reshape(n, k)
    ws = np.fromfile(tmp_path / "ws.bin", dtype=np.float32)
    y = np.fromfile(tmp_path / "y.bin", dtype=np.uint16).reshape(m, n)
    ow8, ows = O.prepare_weight(wb)
    assert np.array_equal(w8, ow8) and np.array_equal(ws, ows)
    want = O.linear(xb, ow8, ows, O.bf16_to_f32(bb))
    assert np.array_equal(y, want), f"{int((y != want).sum())} elements differ"
