"""Chunked DPLR prefill with the reference's names and signatures.

Mirrors ``self_chunk_rwkv7`` (rwkv7_hf/self_chunk_rwkv7.py:33) and
``dplr_chunk_scan`` (rwkv7_hf/dplr_prefill.py:505).  Both run the gfx950 WY
chunk kernel (chunk 16, bf16x3 MFMA products, fp32 state in registers).
``self_chunk_rwkv7`` keeps the reference's argument checks (N = 64, T
divisible by chunk_size, chunk_size in {16, 32, 64}); ``dplr_chunk_scan``
accepts any T like the reference's pure-torch oracle.  The kernel always uses
16-token chunks internally (one workgroup of four state waves and four chunk
producer waves per (batch, head)); ``chunk_size`` does not change the result
beyond rounding.
"""
from __future__ import annotations

from typing import Any

import torch

from . import _lib
from .fused_recurrent_update import _as_bthn, _check_state, _same_dtype, _state_dst


def self_chunk_rwkv7_available() -> bool:
    try:
        _lib.load()
    except RuntimeError:
        return False
    return torch.cuda.is_available()


def _aligned16(x: torch.Tensor) -> torch.Tensor:
    """The kernel reads 16-byte channel runs; a view at an odd offset is copied."""
    return x if x.data_ptr() % 16 == 0 else x.clone()


def _run_chunk(r4, w4, k4, v4, kk4, a4, state, *, w_is_log: int, chunk: int,
               state_out=None, out=None):
    """The chunk kernel; ``w_is_log``: 0 decay, 1 natural-log decay, 2 raw
    pre-activation (decay ``exp(-0.606531 sigmoid(w))`` formed in-kernel)."""
    B, T, H, N = (int(s) for s in r4.shape)
    r4, w4, k4, v4, kk4, a4 = (_aligned16(x) for x in (r4, w4, k4, v4, kk4, a4))
    _lib.require_gpu(r4, w4, k4, v4, kk4, a4, state, name="wkv7 chunk prefill")
    st = state.contiguous()
    final = _state_dst(st, state_out)
    y = out if out is not None else torch.empty((B, T, H, N), device=r4.device, dtype=r4.dtype)
    _lib.call(
        "rwkv7mi_wkv7_chunk_prefill",
        _lib.ptr(r4), _lib.ptr(w4), _lib.ptr(k4), _lib.ptr(v4), _lib.ptr(kk4), _lib.ptr(a4),
        _lib.ptr(st), _lib.ptr(final), _lib.ptr(y), B, T, H, N, int(chunk), int(w_is_log),
        _lib.dtype_code(r4), _lib.dtype_code(w4), _lib.stream_of(r4),
    )
    return y, final


def self_chunk_rwkv7(r, w_decay, k, v, kk, a_gate, state_native, *, chunk_size: int = 16,
                     w_is_log: bool = False, safe_gate: bool | None = None,
                     h_tiles: tuple[int, int] | None = None, state_out: torch.Tensor | None = None):
    """Return ``(recurrent_output [B,T,H,N], final_native_state [B,H,V,K])``.

    ``w_decay`` is the per-step decay (or its natural log when ``w_is_log``);
    the DPLR pair is ``(-kk, kk * a_gate)`` as in the reference.
    """
    if not self_chunk_rwkv7_available():
        raise RuntimeError("self chunk RWKV-7 requires the rwkv7mi HIP library and a GPU")
    if int(chunk_size) not in {16, 32, 64}:
        raise ValueError("self chunk RWKV-7 chunk_size must be 16, 32, or 64")
    if r.dim() != 4 or any(tuple(x.shape) != tuple(r.shape) for x in (w_decay, k, v, kk, a_gate)):
        raise ValueError("self chunk inputs must share [B,T,H,N]")
    B, T, H, N = (int(x) for x in r.shape)
    if N != 64 or T % int(chunk_size):
        raise ValueError("self chunk RWKV-7 requires head_dim=64 and T divisible by chunk_size")
    _check_state(state_native)
    _same_dtype(r, k, v, kk, a_gate, name="self_chunk_rwkv7")
    return _run_chunk(r.contiguous(), w_decay.contiguous(), k.contiguous(), v.contiguous(), kk.contiguous(),
                      a_gate.contiguous(), state_native, w_is_log=int(bool(w_is_log)), chunk=int(chunk_size),
                      state_out=state_out)


def dplr_chunk_scan(r: Any, w: Any, k: Any, v: Any, kk: Any, a: Any, state: Any, *, chunk_size: int = 64,
                    algorithm: str | None = None, force_fallback: bool = False,
                    state_out: torch.Tensor | None = None):
    """Chunked scan over ``[B,T,H,N]`` or ``[B,T,H*N]`` inputs, any T (ragged tail)."""
    B, H, N = _check_state(state)
    if int(chunk_size) <= 0:
        raise ValueError("chunk_size must be positive")
    r4, flat = _as_bthn(r, H, N, name="r")
    w4, _ = _as_bthn(w, H, N, name="w")
    k4, _ = _as_bthn(k, H, N, name="k")
    v4, _ = _as_bthn(v, H, N, name="v")
    kk4, _ = _as_bthn(kk, H, N, name="kk")
    a4, _ = _as_bthn(a, H, N, name="a")
    if int(r4.shape[0]) != B:
        raise ValueError("r/w/k/v/kk/a batch size must match state")
    _same_dtype(r4, k4, v4, kk4, a4, name="dplr_chunk_scan")
    y, final = _run_chunk(r4, w4, k4, v4, kk4, a4, state, w_is_log=0, chunk=16, state_out=state_out)
    if flat:
        return y.reshape(B, int(r4.shape[1]), H * N), final
    return y, final


CHUNK_STATUS_TIMEOUT = 1  # a bounded wait between the kernel's waves gave up: that call's output is void
CHUNK_STATUS_CLAMPED = 2  # a chunk's log2-decay span exceeded 252; gate factors were clamped


def wkv7_chunk_status(clear: bool = True) -> int:
    """The chunk kernel's sticky status bits on the current device since the
    last clear (synchronises the device)."""
    import ctypes

    v = ctypes.c_int(0)
    _lib.call("rwkv7mi_wkv7_chunk_status", int(bool(clear)), ctypes.byref(v))
    return int(v.value)


def check_wkv7_chunk_status() -> None:
    """Raise RuntimeError if a chunk-kernel wait gave up since the last check."""
    st = wkv7_chunk_status(clear=True)
    if st & CHUNK_STATUS_TIMEOUT:
        raise RuntimeError("wkv7 chunk kernel: a bounded wait between its waves timed out; outputs are void")


__all__ = ["self_chunk_rwkv7", "self_chunk_rwkv7_available", "dplr_chunk_scan", "wkv7_chunk_status",
           "check_wkv7_chunk_status", "CHUNK_STATUS_TIMEOUT", "CHUNK_STATUS_CLAMPED"]
