"""xpu_kernels for MI355X: the ConvRot INT8 linear on gfx950.

Mirrors the INT8 half of the reference package's flat namespace
(``python/xpu_kernels/__init__.py:33-85``), so ``import xpu_kernels`` and
``from xpu_kernels import int8`` work as they do there, with the capture
readiness checks (``capture_status``, ``is_capturing``,
``prepare_for_capture``, ``require_capture_ready``) and the accumulator
consumer ``rope.rms_rope_split_half_dequant`` beside them.
"""

from . import int8
from .int8 import *  # noqa: F401,F403
from .int8 import __all__ as _int8_all
from . import capture, rope
from .capture import capture_status, is_capturing, prepare_for_capture, require_capture_ready

__version__ = "0.1.0"
__all__ = ["capture", "capture_status", "int8", "is_capturing", "prepare_for_capture",
           "require_capture_ready", "rope", *_int8_all]
