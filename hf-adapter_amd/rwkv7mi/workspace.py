"""Per-device scratch buffers, one per named slot.

Slot ``"mm8"`` holds the row-major MM8 kernel's split-K partials and
completion counters; the kernel leaves its counters at zero after every call,
so one zero-initialised buffer per device can be reused by every call issued
on one stream.  Slot ``"mm8t"`` holds the blocked GEMV's split-K partials
(written before they are read).  Slot ``"mm8g"`` holds the many-row MM8 GEMM's x', row sums and
split partials (each call writes them before reading).  Slot ``"lora"`` holds
the LoRA kernels' fp32 partials.  Slot ``"mm8p"`` holds the prefill GEMM's
fp16 dequantised weights (each call writes them before reading).  Slots never share memory, so one kernel
family cannot disturb another's counters.  Calls that run concurrently on
different streams of the same device must not share a slot (the decode step
issues all of them on one stream).

Growth and captured graphs: a hipGraph captured while a slot had one buffer
keeps that buffer's address in its kernel nodes.  ``reserve`` therefore never
frees a buffer it replaces: the old buffer moves to a retired list and stays
allocated until the process ends (or ``release_retired`` is called by a
caller that has dropped every graph), so an older graph that replays after a
slot has grown still reads and writes memory that nothing else owns.  Slots
grow by doubling, so the retired buffers of a slot total less than its live
one.  Grow a slot before graph capture: growing during capture raises.
"""
from __future__ import annotations

import threading

import torch

_lock = threading.Lock()
_buffers: dict[tuple[int, str], torch.Tensor] = {}
_retired: dict[tuple[int, str], list[torch.Tensor]] = {}
_generation: dict[tuple[int, str], int] = {}


def _key(device, slot):
    idx = torch.device(device).index
    if idx is None:
        idx = torch.cuda.current_device()
    return (idx, slot)


def reserve(device: torch.device, nbytes: int, slot: str = "mm8") -> torch.Tensor:
    """Return the device's buffer for ``slot``, growing it (zero-filled) to ``nbytes``."""
    key = _key(device, slot)
    with _lock:
        buf = _buffers.get(key)
        if buf is None or buf.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    f"rwkv7mi workspace '{slot}' must be reserved before graph capture "
                    f"(need {nbytes} bytes on cuda:{key[0]})"
                )
            size = max(int(nbytes), 1 << 20)
            if buf is not None:
                size = max(size, 2 * buf.numel())
                # a captured graph may still hold this buffer's address
                _retired.setdefault(key, []).append(buf)
            buf = torch.zeros(size, dtype=torch.uint8, device=torch.device("cuda", key[0]))
            _buffers[key] = buf
            _generation[key] = _generation.get(key, 0) + 1
        return buf


def generation(device: torch.device, slot: str) -> int:
    """How many buffers ``slot`` has had on ``device`` (0 before the first reserve)."""
    return _generation.get(_key(device, slot), 0)


def retired_bytes(device: torch.device | None = None) -> int:
    """Bytes held by replaced buffers (all devices when ``device`` is None)."""
    with _lock:
        return sum(int(b.numel()) for (idx, _), bs in _retired.items() for b in bs
                   if device is None or idx == _key(device, "")[0])


def release_retired() -> None:
    """Free the replaced buffers.  Only safe once every graph captured before the
    last growth has been dropped."""
    with _lock:
        _retired.clear()


__all__ = ["reserve", "generation", "retired_bytes", "release_retired"]
