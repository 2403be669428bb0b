"""Prefill state preparation with the reference's API.

Mirrors ``fused_prefill_state_prep`` (rwkv7_hf/fused_prefill.py:184-322):
returns ``(w, k_adjusted, v_interpolated, kk_normalized)`` in the input's
``[B, T, H*N]`` or ``[rows, H*N]`` layout.  ``w_transform="decay"`` returns
the decay ``exp(-0.606531 sigmoid(w_raw))``, ``"log_decay"`` its natural log
(the form the chunked scan consumes with ``w_is_log=True``; ``"log"`` is
accepted as an alias); ``w_out_dtype`` picks fp32 or the input dtype.  The
V interpolation runs when both ``v_first`` and ``v_gate`` are given, as in
the reference; ``a_is_raw`` / ``v_gate_is_raw`` apply the sigmoid in-kernel.
Everything is one HIP launch (``rwkv7mi_state_prep``); the inputs are not
modified.

``v_mode`` (this build's keyword) selects the V handling explicitly: 0 pass
through, 1 layer 0 (``v_first`` receives V), 2 interpolate.
"""
from __future__ import annotations

import torch

from . import _lib


def _flat(x, A, name):
    if x.dim() < 2 or int(x.numel()) % A:
        raise ValueError(f"{name} must be [..., {A}] or [..., H, N] with H * N = {A}")
    return x.reshape(-1, A)


def fused_prefill_state_prep(w_raw, k_raw, v_raw, a, k_k, k_a, *, v_first=None, v_gate=None, num_heads: int,
                             head_dim: int, w_out_dtype: str = "fp32", w_transform: str = "decay",
                             a_is_raw: bool = False, v_gate_is_raw: bool = False, force_fallback: bool = False,
                             v_mode: int | None = None, v_out=None):
    if w_out_dtype not in {"fp32", "input"}:
        raise ValueError(f"w_out_dtype must be 'fp32' or 'input'; got {w_out_dtype!r}")
    if w_transform not in {"decay", "log_decay", "log"}:
        raise ValueError(f"w_transform must be 'decay' or 'log_decay'; got {w_transform!r}")
    H, N = int(num_heads), int(head_dim)
    A = H * N
    shape = tuple(k_raw.shape)
    kr = _flat(k_raw, A, "k_raw").contiguous()
    rows = int(kr.shape[0])
    if any(tuple(t.shape) != shape for t in (w_raw, v_raw, a)):
        raise ValueError("w_raw, k_raw, v_raw and a must have identical layouts")
    if int(k_k.numel()) != A or int(k_a.numel()) != A:
        raise ValueError(f"k_k and k_a must have {A} elements")
    dt = kr.dtype
    aa = a.reshape(rows, A).to(dt).contiguous()
    wr = w_raw.reshape(rows, A).to(dt).contiguous()
    vr = v_raw.reshape(rows, A).to(dt).contiguous()
    if v_mode is None:
        v_mode = 2 if (v_first is not None and v_gate is not None) else 0
    vf = vg = None
    if v_mode:
        if v_first is None:
            raise ValueError("the V handling needs v_first")
        vf = v_first.reshape(rows, A)
        if not vf.is_contiguous() or vf.dtype != dt:
            raise ValueError("v_first must be contiguous in the activation dtype")
    if v_mode == 2:
        if v_gate is None:
            raise ValueError("V interpolation needs v_first and v_gate")
        vg = v_gate.reshape(rows, A).to(dt).contiguous()
    if v_out is None:
        v_out = torch.empty_like(vr)
    elif tuple(v_out.shape) != tuple(vr.shape) or not v_out.is_contiguous() or v_out.dtype != dt:
        raise ValueError("v_out must be a contiguous tensor shaped and typed like v_raw")
    kk_out = torch.empty_like(kr)
    k_out = torch.empty_like(kr)
    wdt = torch.float32 if w_out_dtype == "fp32" else dt
    w_out = torch.empty((rows, A), device=kr.device, dtype=wdt)
    kks = k_k.reshape(A).contiguous()
    kas = k_a.reshape(A).to(kks.dtype).contiguous()
    flags = ((_lib.PREP_A_RAW if a_is_raw else 0) | (_lib.PREP_VGATE_RAW if v_gate_is_raw else 0)
             | (_lib.PREP_W_DECAY if w_transform == "decay" else 0))
    _lib.require_gpu(kr, aa, wr, vr, kks, name="fused_prefill_state_prep")
    _lib.call("rwkv7mi_state_prep", _lib.ptr(kr), _lib.ptr(aa), _lib.ptr(wr), _lib.ptr(vr), _lib.ptr(v_out),
              _lib.ptr(vf), _lib.ptr(vg), _lib.ptr(kks), _lib.ptr(kas), _lib.ptr(kk_out), _lib.ptr(k_out),
              _lib.ptr(w_out), rows, H, N, int(v_mode), int(flags), _lib.dtype_code(kr), _lib.dtype_code(kks),
              _lib.dtype_code(w_out), _lib.stream_of(kr))
    return w_out.reshape(shape), k_out.reshape(shape), v_out.reshape(shape), kk_out.reshape(shape)


__all__ = ["fused_prefill_state_prep"]
