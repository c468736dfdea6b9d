"""Capture readiness: what must be true before a step is captured into a HIP
graph (the reference's ``python/xpu_kernels/capture.py:1-182``).

A captured region is replayed as recorded.  On this path two things can be
wrong inside one, both quietly:

1. **The library's one-time set-up.**  ``libxpuint8.so`` uploads its
   activation tables on first use (a synchronous copy, illegal during a
   capture), and the package's self-test synchronizes and reads values back.
   Both must happen before the capture starts; the gate named ``"int8"``
   runs them once and latches the verdict.

2. **The INT8 backward's dequantized weight.**  ``Int8Linear`` in ``"dense"``
   backward mode needs the weight in bf16, a second full-precision copy of it.
   Made inside a capture, the copy would be re-computed on every replay, so
   ``Int8Linear.dense_weight()`` refuses to run inside one and
   :func:`prepare_for_capture` makes it beforehand.

The reference's gates are its Triton kernels (rms_rope, rms_adaln); this
build's hot path has one gate, ``"int8"``.  Everything here is called
*outside* a capture.
"""

from __future__ import annotations

from typing import Iterable

from ._capture import is_capturing

__all__ = ["capture_status", "gates", "is_capturing", "prepare_for_capture",
           "require_capture_ready"]


class _Int8Gate:
    """The library's readiness: loaded, initialised on the device (tables
    uploaded) and self-tested -- probed once, outside a capture."""

    def __init__(self):
        self.verified = None          # None: not probed yet; else True/False
        self.reason = ""

    def reset(self):
        self.verified, self.reason = None, ""

    def ok(self) -> bool:
        if self.verified is None:
            if is_capturing():
                raise RuntimeError(
                    "int8: the library's set-up and self-test synchronize and cannot "
                    "run inside a capture; call prepare_for_capture() before capturing")
            from .int8 import _lib as L
            from .int8.selftest import selftest
            if not L.available():
                self.verified, self.reason = False, f"library unavailable: {L._ERR}"
            else:
                lib = L.load()
                rc = lib.xpuint8_init()
                if rc != 0:
                    self.verified, self.reason = False, f"xpuint8_init failed ({rc})"
                elif not selftest(verbose=False):
                    self.verified, self.reason = False, "the self-test failed"
                else:
                    self.verified, self.reason = True, ""
        return bool(self.verified)

    def describe(self) -> str:
        if self.verified is None:
            return "unverified"
        return "verified" if self.verified else self.reason


_GATES = {"int8": _Int8Gate()}


def gates() -> dict:
    """The package's gates by name."""
    return _GATES


def _wanted(need):
    if need is None:
        return list(_GATES)
    wanted = list(need)
    unknown = [n for n in wanted if n not in _GATES]
    if unknown:
        # a typo must not read as "everything is fine"
        raise ValueError(f"unknown kernel(s) {unknown!r}; this package has {sorted(_GATES)}")
    return wanted


def _int8_modules(model):
    """Every ``Int8Linear`` in a model, by dotted name."""
    from .int8 import Int8Linear

    if model is None:
        return []
    if isinstance(model, Int8Linear):
        return [(getattr(model, "_name", "int8_linear"), model)]
    return [(name, m) for name, m in model.named_modules() if isinstance(m, Int8Linear)]


def capture_status(need: Iterable[str] | None = None, model=None) -> list[str]:
    """Everything that would make a captured step wrong or wasteful, as a list
    of problem strings (empty: ready).  ``need`` names the gates the step
    relies on (``None``: all); ``model`` is an optional module whose
    ``Int8Linear`` layers in ``"dense"`` backward mode are checked for a
    materialized dense weight.  Inside a capture an unprobed gate is reported
    as unverified instead of being probed."""
    problems: list[str] = []
    capturing = is_capturing()
    for name in _wanted(need):
        gate = _GATES[name]
        if gate.verified is None and capturing:
            problems.append(f"{name}: unverified -- the self-test cannot run inside a "
                            f"capture; call prepare_for_capture() before capturing")
            continue
        if not gate.ok():
            problems.append(f"{name}: {gate.describe()}")
    for name, module in _int8_modules(model):
        # "int8" mode never leaves int8, so it never needs the dense copy
        if getattr(module, "backward", "dense") != "dense":
            continue
        if getattr(module, "_dense", None) is None:
            problems.append(
                f"{name}: the dense weight is not materialized -- the dequant would be "
                f"captured and re-run on every replay; call prepare_for_capture(model) first")
    return problems


def require_capture_ready(need: Iterable[str] | None = None, model=None) -> None:
    """Raise ``RuntimeError`` unless the step is ready to be captured."""
    problems = capture_status(need=need, model=model)
    if problems:
        raise RuntimeError("not ready to capture a step:\n  " + "\n  ".join(problems))


def prepare_for_capture(model=None, need: Iterable[str] | None = None) -> dict:
    """Get a step ready to be captured: probe the gates in ``need`` (library
    set-up and self-test) and materialize the dense weight of every
    ``"dense"``-mode ``Int8Linear`` in ``model``.  Returns a summary dict."""
    wanted = _wanted(need)
    verified = [name for name in wanted if _GATES[name].ok()]
    materialized = 0
    for _name, module in _int8_modules(model):
        if getattr(module, "backward", "dense") != "dense":
            continue
        module.dense_weight()
        materialized += 1
    return {"verified": verified, "dense_weights": materialized,
            "problems": capture_status(need=wanted, model=model)}
