"""Per-device scratch for split-K GEMV partials and their completion counters.

The MM8 kernels leave their counters at zero after every call, so one
zero-initialised buffer per device can be reused by every call issued on one
stream.  Calls that run concurrently on different streams of the same device
must not share it (the decode step issues all of them on one stream).
Grow it before graph capture (``reserve``); growing replaces the buffer.
"""
from __future__ import annotations

import threading

import torch

_lock = threading.Lock()
_buffers: dict[int, torch.Tensor] = {}


def reserve(device: torch.device, nbytes: int) -> torch.Tensor:
    """Return the device's workspace, growing it (zero-filled) to ``nbytes``."""
    idx = torch.device(device).index
    if idx is None:
        idx = torch.cuda.current_device()
    with _lock:
        buf = _buffers.get(idx)
        if buf is None or buf.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    "rwkv7mi workspace must be reserved before graph capture "
                    f"(need {nbytes} bytes on cuda:{idx})"
                )
            size = max(int(nbytes), 1 << 20)
            if buf is not None:
                size = max(size, 2 * buf.numel())
            buf = torch.zeros(size, dtype=torch.uint8, device=torch.device("cuda", idx))
            _buffers[idx] = buf
        return buf


__all__ = ["reserve"]
