"""Prefill state preparation with the reference's API.

Mirrors ``fused_prefill_state_prep`` (rwkv7_hf/fused_prefill.py:184): returns
``(w, k_adjusted, v_interpolated, kk_normalized)``.  ``w_transform="decay"``
returns the decay ``exp(-0.606531 sigmoid(w_raw))`` in fp32 (as the
reference); ``w_transform="log"`` returns its natural log, the form the
chunked scan consumes directly (``w_is_log=True``).
"""
from __future__ import annotations

import torch

from . import _lib


def fused_prefill_state_prep(w_raw, k_raw, v_raw, a, k_k, k_a, *, v_first=None, v_gate=None, num_heads: int,
                             head_dim: int, w_out_dtype: str = "fp32", w_transform: str = "decay",
                             a_is_raw: bool = False, v_gate_is_raw: bool = False, force_fallback: bool = False,
                             v_mode: int | None = None):
    if w_out_dtype not in {"fp32", "input"}:
        raise ValueError("w_out_dtype must be 'fp32' or 'input'")
    if w_transform not in {"decay", "log"}:
        raise ValueError("w_transform must be 'decay' or 'log'")
    H, N = int(num_heads), int(head_dim)
    A = H * N
    shape = tuple(k_raw.shape)
    kr = k_raw.reshape(-1, A).contiguous()
    rows = int(kr.shape[0])
    aa = a.reshape(rows, A)
    if a_is_raw:
        aa = torch.sigmoid(aa)
    aa = aa.contiguous()
    wr = w_raw.reshape(rows, A).contiguous()
    v = v_raw.reshape(rows, A).contiguous().clone()
    if v_mode is None:
        v_mode = 2 if v_gate is not None else 0
    vf = None if v_first is None else v_first.reshape(rows, A)
    vg = None
    if v_mode == 2:
        if vf is None or v_gate is None:
            raise ValueError("V interpolation needs v_first and v_gate")
        vg = v_gate.reshape(rows, A)
        if v_gate_is_raw:
            vg = torch.sigmoid(vg)
        vg = vg.contiguous()
        vf = vf.contiguous()
    kk_out = torch.empty_like(kr)
    k_out = torch.empty_like(kr)
    logw = torch.empty((rows, A), device=kr.device, dtype=torch.float32)
    kks = k_k.reshape(A).contiguous()
    kas = k_a.reshape(A).to(kks.dtype).contiguous()
    _lib.require_gpu(kr, aa, wr, v, kks, name="fused_prefill_state_prep")
    _lib.call("rwkv7mi_state_prep", _lib.ptr(kr), _lib.ptr(aa), _lib.ptr(wr), _lib.ptr(v), _lib.ptr(vf),
              _lib.ptr(vg), _lib.ptr(kks), _lib.ptr(kas), _lib.ptr(kk_out), _lib.ptr(k_out), _lib.ptr(logw), rows,
              H, N, int(v_mode), _lib.dtype_code(kr), _lib.dtype_code(kks), _lib.stream_of(kr))
    w = logw if w_transform == "log" else torch.exp(logw)
    if w_out_dtype == "input":
        w = w.to(kr.dtype)
    return w.reshape(shape), k_out.reshape(shape), v.reshape(shape), kk_out.reshape(shape)


__all__ = ["fused_prefill_state_prep"]
