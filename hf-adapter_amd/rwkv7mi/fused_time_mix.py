"""Sequence token-shift mixes with the reference's API.

Mirrors ``fused_attn_sequence_shift_mix`` / ``fused_ffn_sequence_shift_mix``
(rwkv7_hf/fused_time_mix.py:413-515): ``x [B, T, C]`` is the already
normalised hidden sequence, ``prev_t = x_{t-1}`` (``initial_prev`` for
``t = 0``) and ``out_i = x + (prev - x) * mix_i``; the return value is
``(*mixed, x[:, -1])``.  The six attention mixes come back in the logical
order r, w, k, v, a, g; a ``workspace [6, B, T, C]`` is filled in the
reference's physical order r, k, v, w, a, g (R/K/V adjacent,
rwkv7_hf/fused_time_mix.py:441-453).

This build's own extension (keyword only): ``norm_weight`` / ``norm_bias``
fold the LayerNorm into the same kernel, so ``x`` is the raw residual stream
and the last element of the result is ``LayerNorm(x)[:, -1]`` (the next
token's shift state).  ``prev_out`` receives that last row in place.
"""
from __future__ import annotations

import torch

from . import _lib

# logical mix index (r, w, k, v, a, g) -> slot of the reference's workspace
_ATTN_SLOT = (0, 3, 1, 2, 4, 5)


def _flat_mix(m, D, dtype):
    m = m.reshape(-1)
    if int(m.numel()) != D:
        raise ValueError(f"mix vectors must contain {D} values")
    return m.to(dtype).contiguous()


def _seq_mix(x, initial_prev, mixes, norm_weight, norm_bias, eps, outs=None, prev_out=None):
    if x.dim() != 3:
        raise ValueError("x must be [B, T, C]")
    if (norm_weight is None) != (norm_bias is None):
        raise ValueError("pass both norm_weight and norm_bias, or neither")
    B, T, D = (int(s) for s in x.shape)
    xs = x.contiguous()
    pdt = norm_weight.dtype if norm_weight is not None else x.dtype
    w = b = None
    if norm_weight is not None:
        w = norm_weight.reshape(-1).contiguous()
        b = norm_bias.reshape(-1).to(pdt).contiguous()
        if int(w.numel()) != D or int(b.numel()) != D:
            raise ValueError(f"norm_weight / norm_bias must contain {D} values")
    ms = [_flat_mix(m, D, pdt) for m in mixes]
    prev_in = initial_prev.reshape(B, D)
    if prev_in.dtype != x.dtype:
        prev_in = prev_in.to(x.dtype)
    prev_in = prev_in.contiguous()
    new_prev = prev_out if prev_out is not None else torch.empty((B, D), device=x.device, dtype=x.dtype)
    if new_prev.data_ptr() == prev_in.data_ptr():
        raise ValueError("prev_out must not alias initial_prev")
    if outs is None:
        outs = [torch.empty((B, T, D), device=x.device, dtype=x.dtype) for _ in ms]
    _lib.require_gpu(xs, prev_in, name="sequence_shift_mix")
    _lib.call("rwkv7mi_seq_norm_mix", _lib.ptr(xs), _lib.ptr(prev_in), _lib.ptr(new_prev), _lib.ptr(w), _lib.ptr(b),
              _lib.ptr_array(ms), _lib.ptr_array(outs), len(ms), B, T, D, float(eps), _lib.dtype_code(xs),
              _lib.dtype_code(ms[0]), _lib.stream_of(xs))
    return outs, new_prev


def _workspace_ok(ws, shape, x):
    return (ws is not None and tuple(ws.shape) == shape and ws.device == x.device and ws.dtype == x.dtype
            and ws.is_contiguous())


def fused_attn_sequence_shift_mix(x, initial_prev, *mixes, block_size: int = 256, num_warps: int = 4,
                                  workspace=None, strict_fp16_rounding: bool = False, norm_weight=None,
                                  norm_bias=None, eps: float = 1e-5, prev_out=None):
    """Six mixes r, w, k, v, a, g of ``x`` against its one-token shift; returns
    ``(xr, xw, xk, xv, xa, xg, next_prev)``.  ``block_size``, ``num_warps`` and
    ``strict_fp16_rounding`` are accepted for the reference's signature (the
    kernel mixes in fp32 and rounds once)."""
    if len(mixes) != 6:
        raise ValueError("fused_attn_sequence_shift_mix requires six mix vectors")
    if x.dim() != 3:
        raise ValueError("x must be [B, T, C]")
    B, T, D = (int(s) for s in x.shape)
    store = workspace if _workspace_ok(workspace, (6, B, T, D), x) else torch.empty(
        (6, B, T, D), device=x.device, dtype=x.dtype)
    slots = store.unbind(0)
    outs = [slots[_ATTN_SLOT[i]] for i in range(6)]
    outs, new_prev = _seq_mix(x, initial_prev, mixes, norm_weight, norm_bias, eps, outs=outs, prev_out=prev_out)
    return (*outs, new_prev)


def fused_ffn_sequence_shift_mix(x, initial_prev, mix, block_size: int = 256, num_warps: int = 4, workspace=None,
                                 strict_fp16_rounding: bool = False, *, norm_weight=None, norm_bias=None,
                                 eps: float = 1e-5, out=None, prev_out=None):
    """FFN key mix ``x + (prev - x) * mix``; returns ``(mixed, next_prev)``."""
    if x.dim() != 3:
        raise ValueError("x must be [B, T, C]")
    target = out if out is not None else workspace
    outs = [target] if _workspace_ok(target, tuple(x.shape), x) else None
    outs, new_prev = _seq_mix(x, initial_prev, [mix], norm_weight, norm_bias, eps, outs=outs, prev_out=prev_out)
    return outs[0], new_prev


__all__ = ["fused_attn_sequence_shift_mix", "fused_ffn_sequence_shift_mix"]
