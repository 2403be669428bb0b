"""Decode LayerNorm + token-shift mixes with the reference's API.

Mirrors ``fused_attn_norm_mix6_decode`` (rwkv7_hf/fused_decode_norm_mix.py:161)
and ``fused_ffn_add_norm_mix_decode`` (:296): ``previous`` is updated in place
with the normalised row; outputs are new tensors (or caller buffers via
``out=``).  The ``stack_*`` options return views into one stacked allocation as
the reference does.  Runs the gfx950 kernel; GPU tensors only.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


def _rows(x, name):
    if x.dim() < 1:
        raise ValueError(f"{name} must have a hidden dimension")
    D = int(x.shape[-1])
    return x.reshape(-1, D), D


def _vec(t, D, name):
    t = t.reshape(-1)
    if int(t.numel()) != D:
        raise ValueError(f"{name} must contain {D} values, got {int(t.numel())}")
    return t.contiguous()


def fused_attn_norm_mix6_decode(x, previous, norm_weight, norm_bias, mix_r, mix_w, mix_k, mix_v, mix_a, mix_g,
                                *, eps: float = 1e-5, num_warps: int = 4, stack_rkv: bool = False,
                                stack_wav: bool = False, stack_rkv_wagv: bool = False,
                                force_fallback: bool = False, pre_norm_weight=None, pre_norm_bias=None,
                                out=None, residual_parts=None):
    """LayerNorm ``x``, update ``previous`` in place and return the six mixes (r,w,k,v,a,g).

    ``pre_norm_*`` (extension): layer-0 pre-norm applied to ``x`` first, written back into ``x``.
    ``out`` (extension): a ``[6, rows, D]`` buffer (order r,w,k,v,a,g) to write into.
    ``residual_parts`` (extension): ``[S, rows, D]`` fp32 split-K partials of the
    previous layer's FFN value (:func:`mm8_matmul_partials`, S <= 4); ``x`` first
    becomes ``round(sum_s part[s] + x)``, written back, as the split reduce would.
    """
    x2, D = _rows(x, "x")
    p2, Dp = _rows(previous, "previous")
    if Dp != D or p2.shape[0] != x2.shape[0]:
        raise ValueError("x and previous must have identical shapes")
    if not p2.is_contiguous() or p2.data_ptr() != previous.data_ptr():
        raise ValueError("previous must be contiguous (it is updated in place)")
    if x2.data_ptr() == p2.data_ptr():
        raise ValueError("x and previous must not alias")
    params = [_vec(t, D, n) for t, n in ((norm_weight, "norm_weight"), (norm_bias, "norm_bias"))]
    mixes = [_vec(t, D, n).to(params[0].dtype) for t, n in ((mix_r, "mix_r"), (mix_w, "mix_w"), (mix_k, "mix_k"),
                                                           (mix_v, "mix_v"), (mix_a, "mix_a"), (mix_g, "mix_g"))]
    pre = None
    if pre_norm_weight is not None:
        pre = (_vec(pre_norm_weight, D, "pre_norm_weight").to(params[0].dtype),
               _vec(pre_norm_bias, D, "pre_norm_bias").to(params[0].dtype))
        if x2.data_ptr() != x.data_ptr() or not x2.is_contiguous():
            raise ValueError("x must be contiguous when the pre-norm is written back")
    else:
        x2 = x2.contiguous()
    rows = int(x2.shape[0])
    _lib.require_gpu(x2, p2, *params, name="fused_attn_norm_mix6_decode")
    if out is None:
        stacked = torch.empty((6, rows, D), device=x2.device, dtype=x2.dtype)
    else:
        stacked = out.reshape(6, rows, D)
    outs = [stacked[i] for i in range(6)]
    if residual_parts is not None:
        if pre is not None:
            raise ValueError("residual_parts and the pre-norm do not combine")
        parts = residual_parts
        if (parts.dim() != 3 or tuple(parts.shape[1:]) != (rows, D) or parts.dtype != torch.float32
                or not parts.is_contiguous() or x2.data_ptr() != x.data_ptr()):
            raise ValueError("residual_parts: contiguous fp32 [S, rows, D] partials and a contiguous x")
        _lib.call("rwkv7mi_attn_norm_mix6_parts", _lib.ptr(x2), _lib.ptr(p2), _lib.ptr(params[0]),
                  _lib.ptr(params[1]), _lib.ptr_array(mixes), _lib.ptr_array(outs), 6, _lib.ptr(parts),
                  int(parts.shape[0]), rows * D, rows, D, float(eps), _lib.dtype_code(x2),
                  _lib.dtype_code(params[0]), _lib.stream_of(x2))
        shape = tuple(x.shape)
        return tuple(o.reshape(shape) for o in outs)
    _lib.call("rwkv7mi_attn_norm_mix6", _lib.ptr(x2), _lib.ptr(p2), _lib.ptr(params[0]), _lib.ptr(params[1]),
              _lib.ptr(pre[0] if pre else None), _lib.ptr(pre[1] if pre else None), _lib.ptr_array(mixes),
              _lib.ptr_array(outs), 6, rows, D, float(eps), _lib.dtype_code(x2), _lib.dtype_code(params[0]),
              _lib.stream_of(x2))
    shape = tuple(x.shape)
    return tuple(o.reshape(shape) for o in outs)


def fused_ffn_add_norm_mix_decode(residual, attn_out, previous, norm_weight, norm_bias, mix, *, eps: float = 1e-5,
                                  num_warps: int = 4, force_fallback: bool = False, residual_out=None, mixed=None):
    """``x = residual + attn_out``; ``h = LN(x)``; returns ``(x, h + (previous - h) * mix)``; ``previous <- h``.

    ``attn_out`` may be None (extension): then ``residual`` already holds the sum.
    """
    r2, D = _rows(residual, "residual")
    p2, _ = _rows(previous, "previous")
    if p2.data_ptr() != previous.data_ptr() or not p2.is_contiguous():
        raise ValueError("previous must be contiguous (it is updated in place)")
    a2 = None
    if attn_out is not None:
        a2, Da = _rows(attn_out, "attn_out")
        if Da != D or a2.shape[0] != r2.shape[0]:
            raise ValueError("residual, attn_out, and previous must have identical shapes")
        a2 = a2.contiguous()
    r2 = r2.contiguous()
    w = _vec(norm_weight, D, "norm_weight")
    b = _vec(norm_bias, D, "norm_bias").to(w.dtype)
    m = _vec(mix, D, "mix").to(w.dtype)
    rows = int(r2.shape[0])
    _lib.require_gpu(r2, p2, w, name="fused_ffn_add_norm_mix_decode")
    res_out = residual_out.reshape(rows, D) if residual_out is not None else (
        torch.empty_like(r2) if a2 is not None else r2)
    mix_out = mixed.reshape(rows, D) if mixed is not None else torch.empty_like(r2)
    _lib.call("rwkv7mi_ffn_add_norm_mix", _lib.ptr(r2), _lib.ptr(a2), _lib.ptr(p2), _lib.ptr(w), _lib.ptr(b),
              _lib.ptr(m), _lib.ptr(res_out if a2 is not None else None), _lib.ptr(mix_out), rows, D, float(eps),
              _lib.dtype_code(r2), _lib.dtype_code(w), _lib.stream_of(r2))
    shape = tuple(residual.shape)
    return res_out.reshape(shape), mix_out.reshape(shape)


def attn_mix_lora_chunks(D: int) -> int:
    """K-chunks :func:`attn_mix_lora_decode` splits width ``D`` into (0: unsupported)."""
    return int(_lib.load().rwkv7mi_attn_mix_lora_chunks(int(D)))


def attn_mix_lora_decode(x, previous, norm_weight, norm_bias, mixes, outs, lora_downs, lora_mix, part, *,
                         h_out, x_out=None, pre_norm_weight=None, pre_norm_bias=None, eps: float = 1e-5) -> int:
    """Decode attention-side entry for 1..8 fp16/bf16 rows in one launch:
    layer 0's pre-norm (the normalised row -> ``x_out``), ``h = LayerNorm``
    (-> ``h_out``), the r / k / v mixed rows of ``mixes`` (x_r, x_w, x_k, x_v,
    x_a, x_g) into ``outs``, and the LoRA down projections of the mixes
    ``lora_mix[q]`` as K-chunk partial sums in ``part`` (fp32
    ``[q][chunk][row][rank_q]``) -- fused_attn_norm_mix6_decode
    (rwkv7_hf/fused_decode_norm_mix.py:161) plus the down half of
    fused_wavg_lora (rwkv7_hf/fused_lora.py:706).  ``previous`` is read only.
    Returns the chunk count (the wkv kernel's ``lora_splits``)."""
    rows, D = int(_rows(x, "x")[0].shape[0]), int(x.shape[-1])
    ranks = [int(w.shape[0]) for w in lora_downs]
    chunks = attn_mix_lora_chunks(D)
    if not chunks or not 1 <= rows <= 8 or x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("attn_mix_lora_decode: 1..8 fp16/bf16 rows, D a multiple of 128 up to 4096")
    if len(mixes) != 6 or len(outs) != 3 or not 1 <= len(lora_downs) <= 4 or len(lora_mix) != len(lora_downs):
        raise ValueError("attn_mix_lora_decode: six mixes, three outputs, 1..4 LoRA problems")
    if (pre_norm_weight is None) != (x_out is None):
        raise ValueError("attn_mix_lora_decode: x_out goes with the pre-norm")
    for t in (x, h_out, previous, *outs) + ((x_out,) if x_out is not None else ()):
        if tuple(t.shape) != (rows, D) or not t.is_contiguous() or t.dtype != x.dtype:
            raise ValueError("attn_mix_lora_decode: rows must be contiguous [rows, D] in x's dtype")
    for w in lora_downs:
        if w.dim() != 2 or int(w.shape[1]) != D or w.dtype != x.dtype:
            raise ValueError("attn_mix_lora_decode: LoRA down weights are [rank, D] in x's dtype")
    if part.dtype != torch.float32 or not part.is_contiguous() or int(part.numel()) < chunks * rows * sum(ranks):
        raise ValueError("attn_mix_lora_decode: part must be contiguous fp32 with chunks * rows * sum(ranks) values")
    pdt = norm_weight.dtype
    vecs = [_vec(m, D, "mix") for m in mixes]
    if any(v.dtype != pdt for v in vecs) or norm_bias.dtype != pdt:
        raise ValueError("attn_mix_lora_decode: the mixes and LN parameters must share one dtype")
    _lib.require_gpu(x, previous, h_out, part, name="attn_mix_lora_decode")
    _lib.call(
        "rwkv7mi_attn_mix_lora", _lib.ptr(x), _lib.ptr(x_out), _lib.ptr(previous), _lib.ptr(h_out),
        _lib.ptr(_vec(norm_weight, D, "norm_weight")), _lib.ptr(_vec(norm_bias, D, "norm_bias")),
        _lib.ptr(None if pre_norm_weight is None else _vec(pre_norm_weight, D, "pre_norm_weight")),
        _lib.ptr(None if pre_norm_bias is None else _vec(pre_norm_bias, D, "pre_norm_bias")),
        _lib.ptr_array(vecs), _lib.ptr_array(list(outs)), len(lora_downs),
        _lib.ptr_array([w.contiguous() for w in lora_downs]), (ctypes.c_int64 * len(ranks))(*ranks),
        (ctypes.c_int * len(lora_mix))(*[int(i) for i in lora_mix]), _lib.ptr(part), rows, D, float(eps),
        _lib.dtype_code(x), _lib.dtype_code(norm_weight), _lib.stream_of(x))
    return chunks


def layer_norm(x, weight, bias, eps: float = 1e-5, out=None):
    """``F.layer_norm`` over the last dimension (HIP kernel)."""
    x2, D = _rows(x, "x")
    x2 = x2.contiguous()
    w = _vec(weight, D, "weight")
    b = _vec(bias, D, "bias").to(w.dtype)
    y = out.reshape(x2.shape) if out is not None else torch.empty_like(x2)
    _lib.require_gpu(x2, w, name="layer_norm")
    _lib.call("rwkv7mi_layer_norm", _lib.ptr(x2), _lib.ptr(y), _lib.ptr(w), _lib.ptr(b), int(x2.shape[0]), D,
              float(eps), _lib.dtype_code(x2), _lib.dtype_code(w), _lib.stream_of(x2))
    return y.reshape(x.shape)


__all__ = ["attn_mix_lora_chunks", "attn_mix_lora_decode", "fused_attn_norm_mix6_decode", "fused_ffn_add_norm_mix_decode", "layer_norm"]
