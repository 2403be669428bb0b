"""Attention output preparation with the reference's API.

Mirrors ``fused_attn_output_prepare`` (rwkv7_hf/fused_output.py:190):
``(GroupNorm_H(recurrent_out) + (sum_head r*k*r_k) * v) * g`` before ``o_proj``.
"""
from __future__ import annotations

import torch

from . import _lib


def fused_attn_output_prepare(recurrent_out, r, k, v, g, r_k, group_norm_weight, group_norm_bias, *,
                              num_heads: int, head_dim: int, head_v_dim: int, eps: float,
                              force_fallback: bool = False, out=None):
    H, N = int(num_heads), int(head_dim)
    if int(head_v_dim) != N:
        raise ValueError("rwkv7mi output prep requires head_v_dim == head_dim")
    A = H * N
    shape = tuple(recurrent_out.shape)
    y2 = recurrent_out.reshape(-1, A).contiguous()
    rows = int(y2.shape[0])
    rr, kk, vv, gg = (t.reshape(rows, A).contiguous() for t in (r, k, v, g))
    rk = r_k.reshape(A).contiguous()
    gw = group_norm_weight.reshape(A).to(rk.dtype).contiguous()
    gb = group_norm_bias.reshape(A).to(rk.dtype).contiguous()
    o = out.reshape(rows, A) if out is not None else torch.empty_like(y2)
    _lib.require_gpu(y2, rr, kk, vv, gg, rk, name="fused_attn_output_prepare")
    _lib.call("rwkv7mi_output_prepare", _lib.ptr(y2), _lib.ptr(rr), _lib.ptr(kk), _lib.ptr(vv), _lib.ptr(gg),
              _lib.ptr(rk), _lib.ptr(gw), _lib.ptr(gb), _lib.ptr(o), rows, H, N, float(eps), _lib.dtype_code(y2),
              _lib.dtype_code(rk), _lib.stream_of(y2))
    return o.reshape(shape)


__all__ = ["fused_attn_output_prepare"]
