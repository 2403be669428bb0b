"""Sequence token-shift mixes with the reference's API.

Mirrors ``fused_attn_sequence_shift_mix`` / ``fused_ffn_sequence_shift_mix``
(rwkv7_hf/fused_time_mix.py:413, :470).  Unlike the reference (which expects an
already normalised ``x``), the optional ``norm_weight``/``norm_bias`` keywords
fold the LayerNorm of each row into the same kernel; without them ``x`` is
mixed as given (the kernel then applies an identity-affine LayerNorm only when
asked to).  Returns ``(*mixed, last_row)`` like the reference.
"""
from __future__ import annotations

import torch

from . import _lib


def _seq_mix(x, initial_prev, mixes, norm_weight, norm_bias, eps, out=None, prev_out=None):
    if x.dim() != 3:
        raise ValueError("x must be [B, T, C]")
    B, T, D = (int(s) for s in x.shape)
    if norm_weight is None:
        raise ValueError("rwkv7mi sequence mixes normalise in-kernel: pass norm_weight/norm_bias")
    xs = x.contiguous()
    w = norm_weight.reshape(-1).contiguous()
    b = norm_bias.reshape(-1).to(w.dtype).contiguous()
    ms = [m.reshape(-1).to(w.dtype).contiguous() for m in mixes]
    for m in ms:
        if int(m.numel()) != D:
            raise ValueError(f"mix vectors must contain {D} values")
    prev_in = initial_prev.reshape(B, D).contiguous()
    new_prev = prev_out if prev_out is not None else torch.empty((B, D), device=x.device, dtype=x.dtype)
    if new_prev.data_ptr() == prev_in.data_ptr():
        raise ValueError("prev_out must not alias initial_prev")
    stacked = out if out is not None else torch.empty((len(ms), B, T, D), device=x.device, dtype=x.dtype)
    outs = [stacked[i] for i in range(len(ms))]
    _lib.require_gpu(xs, prev_in, w, name="sequence_shift_mix")
    _lib.call("rwkv7mi_seq_norm_mix", _lib.ptr(xs), _lib.ptr(prev_in), _lib.ptr(new_prev), _lib.ptr(w), _lib.ptr(b),
              _lib.ptr_array(ms), _lib.ptr_array(outs), len(ms), B, T, D, float(eps), _lib.dtype_code(xs),
              _lib.dtype_code(w), _lib.stream_of(xs))
    return (*outs, new_prev)


def fused_attn_sequence_shift_mix(x, initial_prev, *mixes, block_size: int = 256, num_warps: int = 4,
                                  workspace=None, strict_fp16_rounding: bool = False, norm_weight=None,
                                  norm_bias=None, eps: float = 1e-5, prev_out=None):
    """Six mixes r,w,k,v,a,g of LN(x) against its one-token shift; returns (*mixes, LN(x)[:, -1])."""
    if len(mixes) != 6:
        raise ValueError("fused_attn_sequence_shift_mix requires six mix vectors")
    return _seq_mix(x, initial_prev, mixes, norm_weight, norm_bias, eps, out=workspace, prev_out=prev_out)


def fused_ffn_sequence_shift_mix(x, initial_prev, mix, *, block_size: int = 256, num_warps: int = 4,
                                 norm_weight=None, norm_bias=None, eps: float = 1e-5, out=None, prev_out=None):
    """FFN key mix of LN(x); returns (mixed, LN(x)[:, -1])."""
    res = _seq_mix(x, initial_prev, [mix], norm_weight, norm_bias, eps,
                   out=None if out is None else out.reshape(1, *x.shape), prev_out=prev_out)
    return res[0], res[1]


__all__ = ["fused_attn_sequence_shift_mix", "fused_ffn_sequence_shift_mix"]
