"""Is the current stream being captured into a HIP graph?

The counterpart of the reference's ``python/xpu_kernels/_capture.py:15-34``:
kernels that would materialise a full-precision copy of a weight refuse to run
inside a capture, because a captured copy is re-made on every replay.
"""

import torch


def is_capturing() -> bool:
    try:
        return bool(torch.cuda.is_available() and torch.cuda.is_current_stream_capturing())
    except Exception:  # noqa: BLE001 - no device runtime means no capture
        return False
