"""Per-device scratch buffers, one per named slot.

Slot ``"mm8"`` holds the row-major MM8 kernel's split-K partials and
completion counters; the kernel leaves its counters at zero after every call,
so one zero-initialised buffer per device can be reused by every call issued
on one stream.  Slot ``"mm8g"`` holds the many-row MM8 GEMM's x', row sums and
split partials (each call writes them before reading).  Slot ``"lora"`` holds
the LoRA kernels' fp32 partials.  Slots
never share memory, so one kernel family cannot disturb another's counters.
Calls that run concurrently on different streams of the same device must not
share a slot (the decode step issues all of them on one stream).  Grow a slot
before graph capture (``reserve``); growing replaces the buffer.
"""
from __future__ import annotations

import threading

import torch

_lock = threading.Lock()
_buffers: dict[tuple[int, str], torch.Tensor] = {}


def reserve(device: torch.device, nbytes: int, slot: str = "mm8") -> torch.Tensor:
    """Return the device's buffer for ``slot``, growing it (zero-filled) to ``nbytes``."""
    idx = torch.device(device).index
    if idx is None:
        idx = torch.cuda.current_device()
    key = (idx, slot)
    with _lock:
        buf = _buffers.get(key)
        if buf is None or buf.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    f"rwkv7mi workspace '{slot}' must be reserved before graph capture "
                    f"(need {nbytes} bytes on cuda:{idx})"
                )
            size = max(int(nbytes), 1 << 20)
            if buf is not None:
                size = max(size, 2 * buf.numel())
            buf = torch.zeros(size, dtype=torch.uint8, device=torch.device("cuda", idx))
            _buffers[key] = buf
        return buf


__all__ = ["reserve"]
