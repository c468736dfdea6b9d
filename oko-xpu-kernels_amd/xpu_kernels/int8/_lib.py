"""Loading and calling ``libxpuint8.so`` (gfx950): the ctypes surface, nothing else.

The counterpart of the reference's ``python/xpu_kernels/int8/_lib.py:74-191``:
the same discovery order (environment override, the package directory, the
repository's ``build/`` and ``lib/``, ``sys.prefix``), argtypes declared for
every symbol (a ctypes default ``int`` would truncate 64-bit pointers), and
the library initialised once.  The stream handed to the library is the HIP
stream behind ``torch.cuda.current_stream(device)``.
"""

from __future__ import annotations

import ctypes
import os
import sys
import threading
from typing import Optional

import torch

_LIB = None
_TRIED = False
_PATH = None
_ERR = None
_LOCK = threading.Lock()

LIBNAME = "libxpuint8.so"


def _candidate_paths():
    for var in ("XPU_KERNELS_LIB", "XPU_INT8_LIB"):
        env = os.environ.get(var)
        if env:
            yield env
    here = os.path.dirname(os.path.abspath(__file__))       # .../xpu_kernels/int8
    pkg = os.path.dirname(here)                             # .../xpu_kernels
    for base in (here, pkg):
        yield os.path.join(base, LIBNAME)
    root = os.path.dirname(pkg)
    yield os.path.join(root, "build", LIBNAME)
    yield os.path.join(root, "lib", LIBNAME)
    yield os.path.join(sys.prefix, "lib", LIBNAME)


#: every exported symbol: name -> (argtypes, restype).  Mirrors include/xpuint8.h.
def _signatures():
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    c_int, c_str = ctypes.c_int, ctypes.c_char_p
    return {
        "xpuint8_init": ([], c_int),
        "xpuint8_device_name": ([], c_str),
        "xpuint8_convrot_groupsize": ([], c_int),
        "xpuint8_last_error": ([], c_str),
        "xpuint8_convrot_quantize": ([vp] * 3 + [i64] * 2, c_int),
        "xpuint8_convrot_quantize_stream": ([vp] * 4 + [i64] * 2, c_int),
        "xpuint8_convrot_quantize_tiled_stream": ([vp] * 4 + [i64] * 2, c_int),
        "xpuint8_convrot_quantize_act": ([vp] * 3 + [i64] * 2 + [i32], c_int),
        "xpuint8_convrot_quantize_act_stream": ([vp] * 4 + [i64] * 2 + [i32], c_int),
        "xpuint8_dequant_weight": ([vp] * 3 + [i64] * 2, c_int),
        "xpuint8_dequant_weight_stream": ([vp] * 4 + [i64] * 2, c_int),
        "xpuint8_convrot_rotate_bf16": ([vp] * 2 + [i64] * 2, c_int),
        "xpuint8_convrot_rotate_bf16_stream": ([vp] * 3 + [i64] * 2, c_int),
        "xpuint8_dequant_epilogue": ([vp] * 5 + [i64] * 2, c_int),
        "xpuint8_dequant_epilogue_stream": ([vp] * 6 + [i64] * 2, c_int),
        "xpuint8_dequant_epilogue_slice": ([vp] * 5 + [i64] * 3, c_int),
        "xpuint8_dequant_epilogue_slice_stream": ([vp] * 6 + [i64] * 3, c_int),
        "xpuint8_dequant_act_quantize": ([vp] * 5 + [i64] * 2 + [i32], c_int),
        "xpuint8_dequant_act_quantize_stream": ([vp] * 6 + [i64] * 2 + [i32], c_int),
        "xpuint8_int8_gemm_stream": ([vp] * 4 + [i64] * 3, c_int),
        "xpuint8_int8_gemm_nn_stream": ([vp] * 4 + [i64] * 3 + [vp], c_int),
        "xpuint8_linear_gemm_stream": ([vp] * 6 + [i32, vp] + [i64] * 3, c_int),
        "xpuint8_linear_gemm_tiled_stream": ([vp] * 6 + [i32, vp] + [i64] * 3, c_int),
        "xpuint8_linear_stream": ([vp] * 5 + [i32, vp] + [i64] * 3 + [vp, i64], c_int),
        "xpuint8_linear_workspace_size": ([i64] * 3, i64),
        "xpuint8_linear_gemm_residual_stream": ([vp] * 6 + [i32] + [vp] * 3 + [i64] * 3, c_int),
        "xpuint8_ffn_up_stream": ([vp] * 6 + [i64] * 3 + [i32], c_int),
        "xpuint8_ffn_stream": ([vp] * 7 + [i32, vp] + [i64] * 3 + [i32, vp, i64], c_int),
        "xpuint8_ffn_workspace_size": ([i64] * 3 + [i32], i64),
        "xpuint8_packed_weight_bytes": ([i64] * 2, i64),
        "xpuint8_pack_weight_stream": ([vp] * 3 + [i64] * 2, c_int),
        "xpuint8_linear_packed_stream": ([vp] * 6 + [i32, vp] + [i64] * 3 + [vp, i64], c_int),
        "xpuint8_linear_gemm_packed_stream": ([vp] * 6 + [i32, vp] + [i64] * 3, c_int),
        "xpuint8_linear_residual_packed_stream": ([vp] * 6 + [i32] + [vp] * 3 + [i64] * 3
                                                  + [vp, i64], c_int),
        "xpuint8_linear_acc_packed_stream": ([vp] * 6 + [i64] * 3 + [vp, i64], c_int),
        "xpuint8_ffn_packed_stream": ([vp] * 9 + [i32, vp] + [i64] * 3 + [i32, vp, i64], c_int),
        "xpuint8_packed_weight_nn_bytes": ([i64] * 2, i64),
        "xpuint8_pack_weight_nn_stream": ([vp] * 3 + [i64] * 2, c_int),
        "xpuint8_linear_dx_int8_packed_stream": ([vp] * 6 + [i64] * 3 + [vp, i64], c_int),
        "xpuint8_linear_backward_int8_workspace_size": ([i64] * 3, i64),
        "xpuint8_linear_backward_int8_stream": ([vp] * 7 + [i32] + [i64] * 3 + [vp, i64], c_int),
        "xpuint8_linear_backward_dense_workspace_size": ([i64] * 3, i64),
        "xpuint8_linear_backward_dense_stream": ([vp] * 6 + [i32] + [i64] * 3 + [vp, i64], c_int),
        "xpuint8_dx_gemm_stream": ([vp] * 5 + [i64] * 3 + [vp], c_int),
        "xpuint8_linear_dx_int8_stream": ([vp] * 5 + [i64] * 3 + [vp, i64], c_int),
        "xpuint8_column_sum_stream": ([vp] * 3 + [i64] * 2 + [vp, i64], c_int),
        "xpuint8_column_sum_workspace_size": ([i64] * 2, i64),
        "xpuint8_linear_dx_int8_workspace_size": ([i64] * 3, i64),
        "xpuint8_linear_dx_int8_noalloc_stream": ([vp] * 5 + [i64] * 3, c_int),
        "xpuint8_prepare_weight_stream": ([vp] * 4 + [i64] * 2, c_int),
        "xpuint8_quantize_row_stream": ([vp] * 5 + [i64] * 2, c_int),
        "xpuint8_linear_dw_stream": ([vp] * 4 + [i64] * 3, c_int),
        "xpuint8_linear_dx_stream": ([vp] * 4 + [i64] * 3 + [vp, i64], c_int),
        "xpuint8_linear_dx_workspace_size": ([i64] * 3, i64),
        "xpuint8_rms_rope_dequant_stream": ([vp, vp] + [i64] * 3 + [vp] + [i64] * 2 + [vp, vp]
                                            + [i64] * 7 + [vp, vp] + [i64] * 4
                                            + [ctypes.c_float, i32], c_int),
        "xpuint8_activation_table": ([i32, vp], c_int),
    }


def open_library(path: str):
    """``ctypes.CDLL`` of one candidate with every argtype declared; no device
    call.  Raises ``OSError``/``AttributeError`` when the file is unusable."""
    lib = ctypes.CDLL(path)
    for name, (args, res) in _signatures().items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


def library_path() -> Optional[str]:
    """The first candidate that exists, without loading it."""
    for path in _candidate_paths():
        if path and os.path.exists(path):
            return path
    return None


def load():
    """Load, bind and initialise the library.  Returns the ctypes handle or None."""
    global _LIB, _TRIED, _PATH, _ERR
    if _LIB is not None or _TRIED:
        return _LIB
    with _LOCK:
        if _LIB is not None or _TRIED:
            return _LIB
        _TRIED = True
        for path in _candidate_paths():
            if not path or not os.path.exists(path):
                continue
            try:
                lib = open_library(path)
            except (OSError, AttributeError) as exc:
                _ERR = f"{path}: {exc}"
                continue
            if lib.xpuint8_init() != 0:
                _ERR = f"{path}: {lib.xpuint8_last_error()!r}"
                continue
            _LIB, _PATH = lib, path
            return lib
        if _ERR is None:
            tried = ", ".join(p for p in _candidate_paths() if p)
            _ERR = (f"no {LIBNAME} found (tried: {tried}); build it with "
                    f"`make -C oko-xpu-kernels_amd/csrc`")
        return None


def available() -> bool:
    """True when the library loaded and initialised on this machine."""
    return load() is not None


def device_name() -> Optional[str]:
    lib = load()
    if lib is None:
        return None
    name = lib.xpuint8_device_name()
    return name.decode() if name else None


def _lib():
    lib = load()
    if lib is None:
        raise RuntimeError(f"libxpuint8 unavailable: {_ERR or 'not found'}")
    return lib


def _err(lib, what):
    raise RuntimeError(f"{what}: {lib.xpuint8_last_error()!r}")


# torch's accessor of the current stream's raw handle (0.1 us against 2 us for
# building a torch.cuda.Stream per call; a private name, so the public form
# stays as the fallback)
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device):
    """The HIP stream behind torch's current stream on ``device``, as the
    integer handle (ctypes passes it as the ``c_void_p`` argument)."""
    if _RAW_STREAM is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _RAW_STREAM(index)
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t):
    """A tensor's device address as an integer (a ``c_void_p`` argument)."""
    return t.data_ptr()


def _fp32(t):
    return t.reshape(-1).to(dtype=torch.float32).contiguous()


def _c(t):
    """``t`` contiguous with a 16-byte aligned start (the library reads and
    writes every buffer with 16-byte vector accesses); copies only if needed."""
    if not t.is_contiguous():
        t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _flat2d(x):
    if x.dtype != torch.bfloat16:
        raise TypeError(f"expected bfloat16, got {x.dtype}")
    if x.device.type != "cuda":
        raise TypeError(f"expected a GPU (ROCm) tensor, got {x.device}")
    x = _c(x)
    return x.reshape(-1, x.shape[-1]), x.shape


ACTIVATIONS = {"gelu_tanh": 1, "swiglu": 2, "situ": 3, "geglu_erf": 4, "gelu_erf": 5}

#: The activations that read a *pair* of halves (``[hidden, gate]`` or
#: ``[gate, up]``) rather than a single tensor.
PAIRED_ACTIVATIONS = ("swiglu", "situ", "geglu_erf")
