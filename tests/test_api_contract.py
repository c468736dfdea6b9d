"""The device-free part of the INT8 operator contract, as one table.

Callers of the reference's ``xpu_kernels.int8`` branch on *which* check fails
(ComfyUI falls back per layer on ``unsupported_reason``), so the order of the
checks, the exception types and the message fragments are API.  Each row below
names a call, what it must produce, and the reference line that fixes it
(paths under okolenmi/oko-xpu-kernels ``python/xpu_kernels/int8/ops.py``
unless stated).  The rows run without a GPU: every check they exercise happens
before the library or a device is touched.

A row's ``expect`` is either ``("reason", fragments)`` -- ``unsupported_reason``
returns a message containing every fragment -- or ``(exception type(s),
fragments)`` -- the call raises such an exception with those fragments in its
text.
"device-only" marks calls that pass every argument check, so the only reason
left is the missing device or library.
"""

import pytest
import torch

from xpu_kernels import int8

I8, BF16, F32 = torch.int8, torch.bfloat16, torch.float32


def w8(n=32, k=512):
    return torch.zeros((n, k), dtype=I8)


def act(m=4, k=512, dtype=BF16):
    return torch.zeros((m, k), dtype=dtype)


def per_channel(n=32):
    return torch.full((n,), 0.01, dtype=F32)


def reason(*args, **kw):
    return lambda: int8.unsupported_reason(*args, **kw)


DEVICE_ONLY = ("device-only", ())

# (id, call, expect, reference line)
CASES = [
    ("valid-call", reason(act(), w8(), per_channel()), DEVICE_ONLY, "ops.py:469-476"),
    ("fp16-activation", reason(act(dtype=torch.float16), w8(), per_channel()),
     ("reason", ("float16",)), "ops.py:435-437"),
    ("float-weight", reason(act(), w8().float(), per_channel()), ("reason", ("int8",)),
     "ops.py:438-439"),
    ("1d-weight", reason(act(), w8()[0], per_channel()), ("reason", ("int8",)), "ops.py:438-439"),
    ("unknown-act", reason(act(), w8(), per_channel(), act="silu"), ("reason", ("silu", "situ")),
     "ops.py:440-442"),
    ("k-mismatch", reason(act(k=512), w8(k=1024), per_channel()), ("reason", ("512", "1024")),
     "ops.py:443-447"),
    ("paired-act-wants-2k", reason(act(k=512), w8(k=512), per_channel(), act="situ"),
     ("reason", ("1024",)), "ops.py:444-447"),
    ("paired-act-2k-ok", reason(act(k=1024), w8(k=512), per_channel(), act="situ"), DEVICE_ONLY,
     "ops.py:444-447"),
    ("geglu-wants-2k", reason(act(k=512), w8(k=512), per_channel(), act="geglu_erf"),
     ("reason", ("1024",)), "ops.py:444-447"),
    ("gelu-erf-unpaired", reason(act(k=512), w8(k=512), per_channel(), act="gelu_erf"),
     DEVICE_ONLY, "ops.py:444-447"),
    ("group-size", reason(act(k=384), w8(k=384), per_channel()), ("reason", ("256",)),
     "ops.py:449-450"),
    ("n-multiple-of-16", reason(act(), w8(n=24), per_channel(24)), ("reason", ("24", "16")),
     "ops.py:451-453"),
    ("int-scale", reason(act(), w8(), torch.zeros(32, dtype=torch.int32)),
     ("reason", ("floating point",)), "ops.py:457-459"),
    ("3d-scale", reason(act(), w8(), torch.zeros((2, 2, 8))), ("reason", ("dims",)),
     "ops.py:461-463"),
    ("scale-count", reason(act(), w8(), torch.zeros(7)), ("reason", ("values",)),
     "ops.py:464-466"),
    ("string-scale", reason(act(), w8(), "0.01"), ("reason", ("tensor or a python float",)),
     "ops.py:467-468"),
    ("scalar-tensor-scale", reason(act(), w8(), torch.zeros(1)), DEVICE_ONLY, "ops.py:464"),
    ("column-scale", reason(act(), w8(), torch.zeros(32, 1)), DEVICE_ONLY,
     "tests/test_int8_api.py:148-150"),
    ("float-scale", reason(act(), w8(), 0.01), DEVICE_ONLY, "ops.py:467"),
    ("linear-raises-the-reason", lambda: int8.linear(act(k=384), w8(k=384), per_channel()),
     (TypeError, ("256",)), "ops.py:616-618"),
    ("prepare-weight-group", lambda: int8.prepare_weight(torch.zeros((32, 384), dtype=BF16)),
     (ValueError, ("384", "256")), "ops.py:91-92"),
    ("prepare-weight-fused-group",
     lambda: int8.prepare_weight_fused(torch.zeros((32, 384), dtype=BF16)),
     (ValueError, ("384", "256")), "ops.py:122-123"),
    ("ffn-unknown-act", lambda: int8.ffn(act(), w8(), per_channel(), w8(), per_channel(), act="silu"),
     (TypeError, ("silu",)), "ops.py:669-671"),
    ("ffn-unfused-act",
     lambda: int8.ffn(act(), w8(), per_channel(), w8(), per_channel(), act="swiglu"),
     (TypeError, ("swiglu",)), "ops.py:672-674"),
    ("int8-linear-mode",
     lambda: int8.int8_linear(act(2, 4), w8(4, 4), torch.ones(4), mode="nope"),
     (ValueError, ("nope",)), "ops.py:315-316"),
    ("int8-module-mode", lambda: int8.Int8Linear(w8(4, 4), torch.ones(4), backward="nope"),
     (ValueError, ("nope",)), "ops.py:844-846"),
    ("trainable-mode",
     lambda: int8.TrainableInt8Linear(torch.zeros((32, 512), dtype=BF16), backward="exact"),
     (ValueError, ("exact",)), "ops.py:768-770"),
    ("trainable-dtype", lambda: int8.TrainableInt8Linear(torch.zeros((32, 512), dtype=torch.float16)),
     (TypeError, ("bfloat16",)), "ops.py:766-767"),
    ("linear-dx-shapes", lambda: int8.linear_dx(act(4, 16), torch.zeros((8, 32), dtype=BF16)),
     (ValueError, ("16", "8")), "ops.py:202-203"),
    ("linear-dw-batches",
     lambda: int8.linear_dw(torch.zeros(8, 16, dtype=BF16), torch.zeros(4, 32, dtype=BF16)),
     (ValueError, ("rows",)), "ops.py:233-236"),
    ("expand-scale-needs-device", lambda: int8.expand_scale(0.5, 3), (TypeError, ("device",)),
     "ops.py:399-400"),
    ("expand-scale-type", lambda: int8.expand_scale("0.5", 3, torch.device("cpu")),
     (TypeError, ("tensor or a python float",)), "ops.py:396-398"),
    # no silent CPU fallback: without the library (or on a CPU tensor) a kernel
    # call raises
    ("quantize-cpu-tensor", lambda: int8.quantize(act()), ((TypeError, RuntimeError), ()),
     "_lib.py:161-184"),
    ("rotate-cpu-tensor", lambda: int8.rotate(act()), ((TypeError, RuntimeError), ()),
     "_lib.py:161-184"),
]


def _no_device_reason(msg):
    """A message that only says the library or the device is missing."""
    return msg is None or "libxpuint8" in msg or "GPU" in msg


@pytest.mark.parametrize("call,expect,where", [c[1:] for c in CASES], ids=[c[0] for c in CASES])
def test_contract(call, expect, where):
    kind, fragments = expect
    if kind == "device-only":
        assert _no_device_reason(call()), where
    elif kind == "reason":
        msg = call()
        assert msg is not None and all(f in msg for f in fragments), (where, msg)
    else:
        with pytest.raises(kind) as exc:
            call()
        assert all(f in str(exc.value) for f in fragments), (where, str(exc.value))


def test_linear_raises_exactly_the_reason():
    """ops.py:616-618: the TypeError text *is* unsupported_reason's string."""
    x, w, s = act(k=384), w8(k=384), per_channel()
    with pytest.raises(TypeError) as exc:
        int8.linear(x, w, s)
    assert str(exc.value) == int8.unsupported_reason(x, w, s)


def test_activation_registry():
    """ops.py / _lib.py: the activation names and which read two halves."""
    assert set(int8.ACTIVATIONS) >= {"gelu_tanh", "swiglu", "situ", "geglu_erf", "gelu_erf"}
    assert set(int8.PAIRED_ACTIVATIONS) == {"swiglu", "situ", "geglu_erf"}


def test_expand_scale_forms():
    """ops.py:380-408: a flat fp32 [n] scale passes through untouched (no copy on
    the hot path); a one-element scale is broadcast; [N, 1] is flattened; a
    python float is materialised on the given device."""
    flat = per_channel(32)
    assert int8.expand_scale(flat, 32, flat.device) is flat
    assert torch.equal(int8.expand_scale(torch.tensor(0.25), 5, torch.device("cpu")),
                       torch.full((5,), 0.25))
    col = torch.arange(4, dtype=F32).reshape(4, 1)
    assert torch.equal(int8.expand_scale(col, 4, col.device), col.reshape(-1))
    got = int8.expand_scale(0.5, 3, torch.device("cpu"))
    assert got.dtype == F32 and got.shape == (3,)


def test_linear_dw_on_cpu_is_the_plain_product():
    """ops.py:237-238: dW = dy^T x with the batch as the contraction, leading
    dims flattened (on the CPU it is torch's own matmul)."""
    g = torch.Generator().manual_seed(0)
    dy = torch.randn(2, 3, 8, 16, generator=g).to(BF16)
    x = torch.randn(2, 3, 8, 32, generator=g).to(BF16)
    dw = int8.linear_dw(dy, x)
    assert dw.shape == (16, 32)
    assert torch.equal(dw, dy.reshape(-1, 16).t() @ x.reshape(-1, 32))
