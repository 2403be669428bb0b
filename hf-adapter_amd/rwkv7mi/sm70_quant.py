"""Group-wise symmetric W4 (group 128/256) with the reference's API.

Mirrors ``quantize_w4_groupwise`` (rwkv7_hf/sm70_quant.py:502) and
``w4_groupwise_linear`` (:579).  The packer is a gfx950 kernel that reproduces
the reference's fp32 ops (amax/7, correctly rounded division, round half to
even) bit for bit; the linear is the fused HIP dequant GEMV/GEMM.  GPU tensors
only.
"""
from __future__ import annotations

import torch

from . import _lib


def quantize_w4_groupwise(weight: torch.Tensor, group_size: int = 128):
    """Symmetric row-major W4 with one scale per (output, group).

    Returns ``(packed [O, I/2] uint8, scales [O, I/group] weight.dtype, in_features)``.
    """
    group_size = int(group_size)
    if group_size not in {128, 256}:
        raise ValueError("sm70 groupwise W4 requires group_size=128 or 256")
    if weight.dim() != 2 or weight.shape[1] % group_size:
        raise ValueError("groupwise W4 requires rank-2 weight with K divisible by group_size")
    _lib.require_gpu(weight, name="quantize_w4_groupwise")
    w = weight.detach().contiguous()
    out_features, in_features = (int(s) for s in w.shape)
    packed = torch.empty((out_features, in_features // 2), device=w.device, dtype=torch.uint8)
    scales = torch.empty((out_features, in_features // group_size), device=w.device, dtype=w.dtype)
    _lib.call(
        "rwkv7mi_w4g_pack", _lib.ptr(w), out_features, in_features, group_size, _lib.dtype_code(w),
        _lib.ptr(packed), _lib.ptr(scales), _lib.stream_of(w),
    )
    return packed, scales, in_features


def w4_groupwise_linear_into(x2, q, scales, out2, *, group_size=128, bias=None, residual=None,
                             epilogue=_lib.EPI_NONE):
    rows, in_features = (int(s) for s in x2.shape)
    out_features = int(q.shape[0])
    _lib.require_gpu(x2, q, scales, out2, name="w4_groupwise_linear")
    if int(q.shape[1]) * 2 != in_features:
        raise ValueError(f"w4: packed {tuple(q.shape)} does not match in_features={in_features}")
    if tuple(out2.shape) != (rows, out_features) or not out2.is_contiguous() or out2.dtype != x2.dtype:
        raise ValueError("w4: out must be a contiguous [rows, out_features] tensor of x's dtype")
    if residual is not None:
        residual = residual.reshape(rows, out_features)
        if not residual.is_contiguous() or residual.dtype != x2.dtype:
            raise ValueError("w4: residual must be contiguous with x's dtype")
    _lib.call(
        "rwkv7mi_w4g_matmul", _lib.ptr(x2), _lib.ptr(q), _lib.ptr(scales), _lib.ptr(bias),
        _lib.ptr(residual), _lib.ptr(out2), rows, out_features, in_features, int(group_size),
        int(epilogue), _lib.dtype_code(x2), _lib.dtype_code(scales), _lib.stream_of(x2),
    )
    return out2


def w4_groupwise_linear(x, q, scales, out_features, in_features, *, group_size=128, out=None):
    """``y = x @ W^T`` with ``W[o,i] = (nib - 8) * scales[o, i // group_size]``."""
    group_size = int(group_size)
    if group_size not in {128, 256} or int(in_features) % group_size:
        raise ValueError("sm70 groupwise W4 requires group_size=128/256 and divisible K")
    if int(q.shape[0]) != int(out_features):
        raise ValueError("w4: out_features does not match packed rows")
    scalar = x.dim() == 1
    x2 = x.reshape(-1, x.shape[-1])
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous().clone() if x2.data_ptr() % 16 else x2.contiguous()
    rows = int(x2.shape[0])
    if out is not None:
        out2 = out.reshape(rows, int(out_features))
    else:
        out2 = torch.empty((rows, int(out_features)), device=x.device, dtype=x.dtype)
    w4_groupwise_linear_into(x2, q, scales, out2, group_size=group_size)
    if out is not None:
        return out
    return out2.reshape(int(out_features)) if scalar else out2.reshape(*x.shape[:-1], int(out_features))


def quantize_w4_affine_groupwise(weight: torch.Tensor, group_size: int = 128):
    """Asymmetric (min/max affine) W4 with a scale and a bias per (output, group):
    ``W[o, i] ~ q s + b``, ``q`` in [0, 15] (the group's minimum maps to 0, its
    maximum to 15).  The form of MLX's affine group quantisation, the
    reference's only asymmetric group format (rwkv7_hf/mlx_quant.py:258-290);
    parity with MLX itself is unpinned.

    Returns ``(packed [O, I/2] uint8, scales [O, I/group], biases [O, I/group], in_features)``.
    """
    group_size = int(group_size)
    if group_size not in {128, 256}:
        raise ValueError("affine groupwise W4 requires group_size=128 or 256")
    if weight.dim() != 2 or weight.shape[1] % group_size:
        raise ValueError("groupwise W4 requires rank-2 weight with K divisible by group_size")
    _lib.require_gpu(weight, name="quantize_w4_affine_groupwise")
    w = weight.detach().contiguous()
    out_features, in_features = (int(s) for s in w.shape)
    packed = torch.empty((out_features, in_features // 2), device=w.device, dtype=torch.uint8)
    scales = torch.empty((out_features, in_features // group_size), device=w.device, dtype=w.dtype)
    biases = torch.empty_like(scales)
    _lib.call("rwkv7mi_w4a_pack", _lib.ptr(w), out_features, in_features, group_size, _lib.dtype_code(w),
              _lib.ptr(packed), _lib.ptr(scales), _lib.ptr(biases), _lib.stream_of(w))
    return packed, scales, biases, in_features


def w4_affine_groupwise_linear(x, q, scales, biases, out_features, in_features, *, group_size=128, out=None,
                               bias=None):
    """``y = x @ W^T (+ bias)`` with ``W[o, i] = q[o, i] scales[o, g] + biases[o, g]``."""
    group_size = int(group_size)
    if group_size not in {128, 256} or int(in_features) % group_size:
        raise ValueError("affine groupwise W4 requires group_size=128/256 and divisible K")
    if int(q.shape[0]) != int(out_features) or int(q.shape[1]) * 2 != int(in_features):
        raise ValueError("w4a: packed shape does not match the features")
    if tuple(scales.shape) != tuple(biases.shape) or scales.dtype != biases.dtype:
        raise ValueError("w4a: scales and biases must share shape and dtype")
    x2 = x.reshape(-1, int(x.shape[-1]))
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous().clone() if x2.data_ptr() % 16 else x2.contiguous()
    rows = int(x2.shape[0])
    out2 = out.reshape(rows, int(out_features)) if out is not None else torch.empty(
        (rows, int(out_features)), device=x.device, dtype=x.dtype)
    _lib.require_gpu(x2, q, scales, biases, out2, name="w4_affine_groupwise_linear")
    _lib.call("rwkv7mi_w4a_matmul", _lib.ptr(x2), _lib.ptr(q), _lib.ptr(scales.contiguous()),
              _lib.ptr(biases.contiguous()), _lib.ptr(bias), None, _lib.ptr(out2), rows, int(out_features),
              int(in_features), group_size, int(_lib.EPI_NONE), _lib.dtype_code(x2), _lib.dtype_code(scales),
              _lib.stream_of(x2))
    if out is not None:
        return out
    return out2.reshape(*x.shape[:-1], int(out_features))


__all__ = ["quantize_w4_groupwise", "w4_groupwise_linear", "w4_groupwise_linear_into",
           "quantize_w4_affine_groupwise", "w4_affine_groupwise_linear"]
