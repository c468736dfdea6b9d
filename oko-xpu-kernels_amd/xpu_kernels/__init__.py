"""xpu_kernels for MI355X: the ConvRot INT8 linear on gfx950.

Mirrors the INT8 half of the reference package's flat namespace
(``python/xpu_kernels/__init__.py:33-85``), so ``import xpu_kernels`` and
``from xpu_kernels import int8`` work as they do there.
"""

from . import int8
from .int8 import *  # noqa: F401,F403
from .int8 import __all__ as _int8_all

__version__ = "0.1.0"
__all__ = ["int8", *_int8_all]
