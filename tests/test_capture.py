"""Capture readiness (the reference's tests/test_capture.py:1-175, for the
gates this build has): the contract -- what raises, what is reported -- on the
CPU, and a real HIP-graph capture of the hot path on the GPU, replayed several
times with eager work in between, every replay checked bit for bit against the
eager call."""

from unittest import mock

import numpy as np
import pytest
import torch

import xpu_kernels
from xpu_kernels import capture, int8


def _model():
    """A model with one INT8 linear in it, built by hand (no device needed)."""
    w8 = torch.randint(-127, 128, (32, 512), dtype=torch.int8)
    scale = torch.full((32,), 0.01, dtype=torch.float32)
    mod = torch.nn.Module()
    mod.proj = int8.Int8Linear(w8, scale)
    return mod


def test_is_capturing_is_false_and_never_raises():
    assert xpu_kernels.is_capturing() is False


def test_unknown_gate_names_are_rejected():
    with pytest.raises(ValueError) as exc:
        capture.capture_status(need=("int9",))
    assert "int8" in str(exc.value)


def test_status_reports_a_missing_dense_weight():
    problems = capture.capture_status(need=(), model=_model())
    assert any("dense weight" in p for p in problems)


def test_prepare_materializes_the_dense_weight():
    model = _model()

    def fake_dequant(w8, w_scale):
        return torch.zeros((w8.shape[0], w8.shape[1]), dtype=torch.bfloat16)

    with mock.patch("xpu_kernels.int8.ops.dequant_weight", fake_dequant):
        summary = capture.prepare_for_capture(model, need=())
    assert summary["dense_weights"] == 1
    assert not [p for p in capture.capture_status(need=(), model=model) if "dense weight" in p]


def test_dense_weight_refuses_to_allocate_inside_a_capture():
    model = _model()
    with mock.patch("xpu_kernels.int8.ops.is_capturing", return_value=True):
        with pytest.raises(RuntimeError) as exc:
            model.proj.dense_weight()
    assert "capture" in str(exc.value)


def test_the_gate_refuses_to_probe_inside_a_capture():
    gate = capture.gates()["int8"]
    saved = (gate.verified, gate.reason)
    gate.reset()
    try:
        with mock.patch("xpu_kernels.capture.is_capturing", return_value=True):
            with pytest.raises(RuntimeError) as exc:
                gate.ok()
            assert "capture" in str(exc.value)
            assert gate.verified is None
            # and the report says unverified instead of probing
            problems = capture.capture_status(need=("int8",))
        assert any("unverified" in p for p in problems)
    finally:
        gate.verified, gate.reason = saved


def test_the_dense_weight_is_only_demanded_where_it_is_needed():
    model = torch.nn.Module()
    model.dense = int8.Int8Linear(torch.zeros(4, 256, dtype=torch.int8),
                                  torch.ones(4, dtype=torch.float32), backward="dense")
    model.cheap = int8.Int8Linear(torch.zeros(4, 256, dtype=torch.int8),
                                  torch.ones(4, dtype=torch.float32), backward="int8")
    problems = capture.capture_status(need=(), model=model)
    assert any(p.startswith("dense:") for p in problems)
    assert not any(p.startswith("cheap:") for p in problems)


def test_require_raises_with_the_problems():
    with pytest.raises(RuntimeError) as exc:
        capture.require_capture_ready(need=(), model=_model())
    assert "dense weight" in str(exc.value)


# ------------------------------------------------------------------ GPU
def _graph(fn, warm):
    """Capture ``fn()`` into a HIP graph (after warm-up on a side stream)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warm):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def _bits(t):
    return t.detach().contiguous().cpu().view(torch.int16).numpy()


@pytest.mark.gpu
def test_hot_path_replays_exactly(dev):
    """linear, the GEGLU FFN and the int8 backward (dx) captured once and
    replayed on fresh inputs: each replay equals the eager call bit for bit."""
    summary = capture.prepare_for_capture(need=("int8",))
    assert summary["verified"] == ["int8"], summary
    g = torch.Generator().manual_seed(11)
    M, K, N, F = 256, 1280, 1024, 512

    def rnd(*shape, s=1.0):
        return (torch.randn(*shape, generator=g) * s).to(torch.bfloat16).to(dev)

    w8, ws = int8.prepare_weight(rnd(N, K, s=0.02))
    bias = rnd(N, s=0.01)
    up8, ups = int8.prepare_weight(rnd(2 * F, K, s=0.02))
    dn8, dns = int8.prepare_weight(rnd(K, F, s=0.02))
    x = rnd(M, K)
    dy = rnd(M, N, s=1e-3)
    calls = {
        "linear": lambda: int8.linear(x, w8, ws, bias),
        "ffn": lambda: int8.ffn(x, up8, ups, dn8, dns, bias[:K] if K <= N else None,
                                act="geglu_erf"),
        "dx": lambda: int8.linear_dx_int8(dy, w8, ws),
    }
    graphs = {name: _graph(fn, warm=2) for name, fn in calls.items()}
    for rep in range(3):
        # fresh inputs in place, eager references, then the replays
        x.copy_(rnd(M, K, s=1.0 + rep))
        dy.copy_(rnd(M, N, s=1e-3 * (rep + 1)))
        want = {name: fn() for name, fn in calls.items()}
        torch.cuda.synchronize()
        for name, (graph, out) in graphs.items():
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(_bits(out), _bits(want[name])), (name, rep)
