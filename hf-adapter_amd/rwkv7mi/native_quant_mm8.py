"""Native MM8 (uint8 affine) quantization with the reference's API.

Mirrors rwkv7_hf/native_quant_mm8.py (rwkv-rs/hf-adapter 0.8.1):
``quantize_mm8`` (:62), ``mm8_matmul`` (:111), ``mm8_linear`` (:122),
``mm8_gemv_triton`` (:383), ``mm8_matmul_triton`` (:468), ``MM8Linear``
(:564) and ``quantize_model_mm8`` (:631).  Packing runs as a gfx950 kernel
that reproduces the reference's fp32 op sequence bit for bit; every matmul runs
the fused HIP dequant GEMV/GEMM (fp32 accumulation).  Inputs must be GPU
tensors: there is no CPU path.
"""
from __future__ import annotations

import ctypes
import types

import torch

from . import _lib
from . import workspace as _ws
from .native_quant_policy import normalize_native_mm_policy, should_quantize_linear


def quantize_mm8(weight: torch.Tensor):
    """Quantize ``weight: [N, M]`` to the rwkv fp16i8 format.

    Returns ``(w_u8 [N,M] uint8, mx [M], rx [M], my [N,1], ry [N,1])`` in
    ``weight.dtype``, identical to the reference packer.
    """
    if weight.dim() != 2:
        raise ValueError("quantize_mm8 expects a 2-D weight")
    _lib.require_gpu(weight, name="quantize_mm8")
    w = weight.contiguous()
    n, m = (int(s) for s in w.shape)
    dev, dt = w.device, w.dtype
    w_u8 = torch.empty((n, m), device=dev, dtype=torch.uint8)
    mx = torch.empty(m, device=dev, dtype=dt)
    rx = torch.empty(m, device=dev, dtype=dt)
    my = torch.empty((n, 1), device=dev, dtype=dt)
    ry = torch.empty((n, 1), device=dev, dtype=dt)
    ws = torch.empty(2 * n + 2 * m, device=dev, dtype=torch.float32)
    _lib.call(
        "rwkv7mi_mm8_pack", _lib.ptr(w), n, m, _lib.dtype_code(w), _lib.ptr(w_u8), _lib.ptr(mx),
        _lib.ptr(rx), _lib.ptr(my), _lib.ptr(ry), _lib.ptr(ws), _lib.stream_of(w),
    )
    return w_u8, mx, rx, my, ry


def quantize_mm8_outmajor(weight: torch.Tensor):
    """Quantize ``nn.Linear.weight: [M, N]`` (out, in) to the same format as
    ``quantize_mm8(weight.t())`` but with out-major byte storage.

    Returns ``(w_u8, mx, rx, my, ry)`` where ``w_u8`` is the ``[N, M]`` (in, out)
    transposed view of a contiguous ``[M, N]`` uint8 tensor; its values equal
    the reference packer's bit for bit.  This layout feeds the fused decode
    GEMV (``rwkv7mi_mm8t_matmul``).
    """
    if weight.dim() != 2:
        raise ValueError("quantize_mm8_outmajor expects a 2-D weight")
    _lib.require_gpu(weight, name="quantize_mm8_outmajor")
    w = weight.contiguous()
    m, n = (int(s) for s in w.shape)
    dev, dt = w.device, w.dtype
    w_t = torch.empty((m, n), device=dev, dtype=torch.uint8)
    mx = torch.empty(m, device=dev, dtype=dt)
    rx = torch.empty(m, device=dev, dtype=dt)
    my = torch.empty((n, 1), device=dev, dtype=dt)
    ry = torch.empty((n, 1), device=dev, dtype=dt)
    ws = torch.empty(2 * n + 2 * m, device=dev, dtype=torch.float32)
    _lib.call(
        "rwkv7mi_mm8_pack_t", _lib.ptr(w), n, m, _lib.dtype_code(w), _lib.ptr(w_t), _lib.ptr(mx),
        _lib.ptr(rx), _lib.ptr(my), _lib.ptr(ry), _lib.ptr(ws), _lib.stream_of(w),
    )
    return w_t.t(), mx, rx, my, ry


def mm8_block(w_u8: torch.Tensor) -> torch.Tensor:
    """The decode GEMV's blocked copy of ``w_u8 [in, out]`` (any strides):
    ``[ceil(out/16), ceil(in/128), 2048]`` uint8, tile ``(g, b)`` holding at
    byte ``1024 h + 16 (16 q + c) + e`` the weight of output ``16 g + c`` and
    input ``128 b + 64 h + 16 q + e``; edges padded with zeros.  A wave's
    128-input step of 16 outputs is one contiguous 2 KB run."""
    if w_u8.dim() != 2 or w_u8.dtype != torch.uint8:
        raise ValueError("mm8_block expects a 2-D uint8 [in, out] tensor")
    _lib.require_gpu(w_u8, name="mm8_block")
    n, m = (int(s) for s in w_u8.shape)
    out = torch.empty(((m + 15) // 16, (n + 127) // 128, 2048), device=w_u8.device, dtype=torch.uint8)
    # element (i, o) sits at i * stride(0) + o * stride(1)
    _lib.call("rwkv7mi_mm8t_block", _lib.ptr(w_u8), int(w_u8.stride(1)), int(w_u8.stride(0)), n, m, _lib.ptr(out),
              _lib.stream_of(w_u8))
    return out


def mm8_unblock(w_blk: torch.Tensor, in_features: int, out_features: int) -> torch.Tensor:
    """Inverse of :func:`mm8_block`: the reference's contiguous ``w_u8 [in, out]``."""
    if not is_blocked(w_blk):
        raise ValueError("mm8_unblock expects a blocked MM8 tensor")
    n, m = int(in_features), int(out_features)
    if tuple(w_blk.shape[:2]) != ((m + 15) // 16, (n + 127) // 128):
        raise ValueError(f"mm8_unblock: blocked shape {tuple(w_blk.shape)} does not match [{n}, {m}]")
    out = torch.empty((n, m), device=w_blk.device, dtype=torch.uint8)
    _lib.call("rwkv7mi_mm8t_unblock", _lib.ptr(w_blk), n, m, _lib.ptr(out), 1, m, _lib.stream_of(w_blk))
    return out


def mm8_block_shape(n: int, m: int) -> tuple:
    """Shape of the blocked copy of ``w_u8 [n, m]`` (see :func:`mm8_block`)."""
    return ((int(m) + 15) // 16, (int(n) + 127) // 128, 2048)


def is_blocked(w: torch.Tensor) -> bool:
    """True for the decode GEMV's blocked weight tensor (see :func:`mm8_block`)."""
    return (w.dim() == 3 and int(w.shape[2]) == 2048 and w.dtype == torch.uint8 and w.is_contiguous())


def quantize_mm8_blocked(weight: torch.Tensor):
    """``quantize_mm8_outmajor`` with the bytes in the blocked decode layout:
    ``(w_blk, mx, rx, my, ry)``."""
    w_u8, mx, rx, my, ry = quantize_mm8_outmajor(weight)
    w_blk = mm8_block(w_u8)
    del w_u8
    return w_blk, mx, rx, my, ry


def is_out_major(w_u8: torch.Tensor) -> bool:
    """True when ``w_u8 [N, M]`` is the transposed view of contiguous ``[M, N]`` bytes."""
    return (w_u8.dim() == 2 and not w_u8.is_contiguous() and w_u8.t().is_contiguous())


def mm8_workspace_bytes(rows: int, n: int, m: int) -> int:
    """Workspace of the row-major kernel (the ``"mm8"`` slot)."""
    return int(_lib.load().rwkv7mi_mm8_workspace_bytes(int(rows), int(n), int(m)))


def mm8_prefill_workspace_bytes(nprob: int, n: int, m: int) -> int:
    """Bytes of the ``"mm8p"`` slot a prefill GEMM of ``nprob`` ``[n -> m]``
    problems needs: their fp16 dequantised weights in MFMA operand order."""
    return int(_lib.load().rwkv7mi_mm8t_gemm_prefill_ws_bytes(int(nprob), int(n), int(m)))


def mm8t_workspace_bytes(nprob: int, rows: int, n: int, m: int) -> int:
    """Split-K partials the blocked GEMV needs for ``rows`` rows (the ``"mm8t"``
    slot); 0 when the rows' x' fits one LDS chunk."""
    return int(_lib.load().rwkv7mi_mm8t_matmul_workspace_bytes(int(nprob), int(rows), int(n), int(m)))


def _check_out(x2, m, out, residual):
    rows = int(x2.shape[0])
    if tuple(out.shape) != (rows, m) or not out.is_contiguous() or out.dtype != x2.dtype:
        raise ValueError("mm8: out must be a contiguous [rows, M] tensor of x's dtype")
    if residual is not None:
        residual = residual.reshape(rows, m)
        if not residual.is_contiguous() or residual.dtype != x2.dtype:
            raise ValueError("mm8: residual must be contiguous with x's dtype")
    return residual


# Blocked-weight routes by row count: the fused GEMV up to GEMV_ROWS rows, the
# 64-row MFMA tile GEMM up to GEMM_ROWS, the 256 x 256 prefill GEMM above.
GEMV_ROWS = 16
GEMM_ROWS = 256


def mm8_matmul_into(x2, w_u8, mx, rx, my, ry, out, *, bias=None, residual=None, epilogue=_lib.EPI_NONE):
    """``out[rows, M] = epilogue(x2[rows, N] @ dequant(W))``.

    ``w_u8`` is the blocked tensor of :func:`mm8_block` (the decode layout, no
    allocation), contiguous ``[N, M]`` (the reference's storage; its own
    kernel with a workspace slot) or the out-major view of
    :func:`quantize_mm8_outmajor` (blocked into a temporary first).
    """
    rows, n = (int(s) for s in x2.shape)
    _lib.require_gpu(x2, w_u8, out, name="mm8_matmul")
    if is_out_major(w_u8):
        if int(w_u8.shape[0]) != n:
            raise ValueError(f"mm8: x has {n} features but w_u8 is {tuple(w_u8.shape)}")
        w_u8 = mm8_block(w_u8)
    if is_blocked(w_u8):
        m = int(mx.numel())
        if tuple(w_u8.shape[:2]) != ((m + 15) // 16, (n + 127) // 128) or int(ry.numel()) != n:
            raise ValueError(f"mm8: blocked weights {tuple(w_u8.shape)} do not match [{n}, {m}]")
        residual = _check_out(x2, m, out, residual)
        mod = types.SimpleNamespace(w_blk=w_u8, mx=mx, rx=rx, my=my, ry=ry, bias=bias, in_features=n, out_features=m)
        if rows > GEMM_ROWS:
            mm8_gemm_prefill_multi_into([x2], [mod], [out], residuals=[residual], epilogues=[epilogue])
        elif rows > GEMV_ROWS:
            mm8_gemm_multi_into([x2], [mod], [out], residuals=[residual], epilogues=[epilogue])
        else:
            mm8_matmul_multi_into([x2], [mod], [out], residuals=[residual], epilogues=[epilogue])
        return out
    m = int(w_u8.shape[1])
    if int(w_u8.shape[0]) != n:
        raise ValueError(f"mm8: x has {n} features but w_u8 is {tuple(w_u8.shape)}")
    residual = _check_out(x2, m, out, residual)
    if not w_u8.is_contiguous():
        raise ValueError("mm8: w_u8 must be blocked, contiguous [N, M] or the out-major view")
    ws = _ws.reserve(x2.device, mm8_workspace_bytes(rows, n, m))
    _lib.call(
        "rwkv7mi_mm8_matmul", _lib.ptr(x2), _lib.ptr(w_u8), _lib.ptr(mx), _lib.ptr(rx), _lib.ptr(my),
        _lib.ptr(ry), _lib.ptr(bias), _lib.ptr(residual), _lib.ptr(out), rows, n, m, int(epilogue),
        _lib.dtype_code(x2), _lib.dtype_code(mx), _lib.ptr(ws), int(ws.numel()), _lib.stream_of(x2),
    )
    return out


def mm8_matmul_multi_into(xs, mods, outs, *, residuals=None, epilogues=None):
    """Up to four out-major ``MM8Linear`` products of one shape in a single launch.

    ``xs[p] [rows, N]`` -> ``outs[p] [rows, M]`` through ``mods[p]``.
    """
    k = len(mods)
    if not 1 <= k <= 4 or len(xs) != k or len(outs) != k:
        raise ValueError("mm8_matmul_multi_into: 1..4 problems")
    rows, n = (int(s) for s in xs[0].shape)
    m = int(mods[0].out_features)
    residuals = list(residuals) if residuals is not None else [None] * k
    epilogues = list(epilogues) if epilogues is not None else [_lib.EPI_NONE] * k
    for x2, mod, out, r in zip(xs, mods, outs, residuals):
        if tuple(x2.shape) != (rows, n) or not x2.is_contiguous() or x2.dtype != xs[0].dtype:
            raise ValueError("mm8_matmul_multi_into: inputs must share one contiguous shape and dtype")
        if mod.in_features != n or mod.out_features != m or not is_blocked(mod.w_blk):
            raise ValueError("mm8_matmul_multi_into: modules must be blocked MM8Linear of one shape")
        _check_out(x2, m, out, r)
    _lib.require_gpu(*xs, *outs, name="mm8_matmul_multi")
    arr = lambda ts: _lib.ptr_array(ts)
    eps = (ctypes.c_int * k)(*[int(e) for e in epilogues])
    need = mm8t_workspace_bytes(k, rows, n, m)
    ws = _ws.reserve(xs[0].device, need, slot="mm8t") if need else None
    _lib.call(
        "rwkv7mi_mm8t_matmul_multi_ws", k, arr(xs), arr([md.w_blk for md in mods]), arr([md.mx for md in mods]),
        arr([md.rx for md in mods]), arr([md.my for md in mods]), arr([md.ry for md in mods]),
        arr([md.bias for md in mods]), arr(residuals), arr(outs), eps,
        rows, n, m, _lib.dtype_code(xs[0]), _lib.dtype_code(mods[0].mx), _lib.ptr(ws),
        0 if ws is None else int(ws.numel()), _lib.stream_of(xs[0]),
    )
    return outs


def mm8_matmul_multi_lora_into(xs, mods, outs, lora_xs, lora_downs, lora_part, *, splits: int = 4):
    """:func:`mm8_matmul_multi_into` (at most 16 rows, no split K) or, for
    17..64 rows, :func:`mm8_gemm_multi_into`, with the decode LoRA down
    projections in the same launch, on the workgroups the products leave free:
    ``lora_part`` (fp32, contiguous) receives
    ``[p][z][row][n] = sum_{k in range z} lora_xs[p][row, k] lora_downs[p][n, k]``
    over ``splits`` K ranges, the layout the fused wkv decode kernel reads
    (``down_splits=splits``)."""
    k = len(mods)
    if not 1 <= k <= 4 or len(xs) != k or len(outs) != k:
        raise ValueError("mm8_matmul_multi_lora_into: 1..4 problems")
    rows, n = (int(s) for s in xs[0].shape)
    m = int(mods[0].out_features)
    kl = len(lora_xs)
    if not 1 <= kl <= 4 or len(lora_downs) != kl:
        raise ValueError("mm8_matmul_multi_lora_into: 1..4 LoRA problems")
    for x2, mod, out in zip(xs, mods, outs):
        if tuple(x2.shape) != (rows, n) or not x2.is_contiguous() or x2.dtype != xs[0].dtype:
            raise ValueError("mm8_matmul_multi_lora_into: inputs must share one contiguous shape and dtype")
        if mod.in_features != n or mod.out_features != m or not is_blocked(mod.w_blk):
            raise ValueError("mm8_matmul_multi_lora_into: modules must be blocked MM8Linear of one shape")
        _check_out(x2, m, out, None)
    for lx, wd in zip(lora_xs, lora_downs):
        if tuple(lx.shape) != (rows, n) or not lx.is_contiguous() or lx.dtype != xs[0].dtype:
            raise ValueError("mm8_matmul_multi_lora_into: LoRA inputs must match the products' rows, width and dtype")
        if wd.dim() != 2 or int(wd.shape[1]) != n or not wd.is_contiguous() or wd.dtype != xs[0].dtype:
            raise ValueError("mm8_matmul_multi_lora_into: LoRA down weights must be contiguous [rank, in]")
    ranks = [int(wd.shape[0]) for wd in lora_downs]
    need = int(splits) * rows * sum(ranks)
    if (lora_part.dtype != torch.float32 or not lora_part.is_contiguous() or int(lora_part.numel()) < need):
        raise ValueError("mm8_matmul_multi_lora_into: lora_part must be contiguous fp32 with "
                         "splits * rows * sum(ranks) values")
    _lib.require_gpu(*xs, *outs, *lora_xs, *lora_downs, lora_part, name="mm8_matmul_multi_lora")
    arr = lambda ts: _lib.ptr_array(ts)
    eps = (ctypes.c_int * k)(*([_lib.EPI_NONE] * k))
    if rows > GEMV_ROWS:
        ws = _ws.reserve(xs[0].device, mm8_gemm_workspace_bytes(k, rows, n, m, 0), slot="mm8g")
        _lib.call(
            "rwkv7mi_mm8t_gemm_multi_lora", k, arr(xs), arr([md.w_blk for md in mods]),
            arr([md.mx for md in mods]), arr([md.rx for md in mods]), arr([md.my for md in mods]),
            arr([md.ry for md in mods]), arr([md.bias for md in mods]), arr([None] * k), arr(outs), eps,
            rows, n, m, _lib.dtype_code(xs[0]), _lib.dtype_code(mods[0].mx), 0, _lib.ptr(ws), int(ws.numel()),
            kl, arr(lora_xs), arr(lora_downs), (ctypes.c_int64 * kl)(*ranks), int(splits), _lib.ptr(lora_part),
            int(lora_part.numel()) * 4, _lib.stream_of(xs[0]),
        )
        return outs
    _lib.call(
        "rwkv7mi_mm8t_matmul_multi_lora", k, arr(xs), arr([md.w_blk for md in mods]), arr([md.mx for md in mods]),
        arr([md.rx for md in mods]), arr([md.my for md in mods]), arr([md.ry for md in mods]),
        arr([md.bias for md in mods]), arr([None] * k), arr(outs), eps,
        rows, n, m, _lib.dtype_code(xs[0]), _lib.dtype_code(mods[0].mx), kl, arr(lora_xs), arr(lora_downs),
        (ctypes.c_int64 * kl)(*ranks), int(splits), _lib.ptr(lora_part), int(lora_part.numel()) * 4,
        _lib.stream_of(xs[0]),
    )
    return outs


def mm8_matmul_partials(x2, mod):
    """The split-K products of ``x2 [rows, N] @ mod`` left as fp32 partials for the
    consumer to add (no reduce launch): returns ``(part [S, rows, M], S)``, a view
    of the ``"mm8t"`` workspace slot valid until the next call that uses that
    slot; ``out = sum_s part[s] (+ bias)`` in split order.  Only for shapes the
    blocked GEMV splits (:func:`mm8t_workspace_bytes` > 0)."""
    rows, n = (int(s) for s in x2.shape)
    m = int(mod.out_features)
    if mod.in_features != n or not is_blocked(mod.w_blk) or not x2.is_contiguous():
        raise ValueError("mm8_matmul_partials: a contiguous x and a blocked MM8Linear of matching width")
    need = mm8t_workspace_bytes(1, rows, n, m)
    if not need:
        raise ValueError("mm8_matmul_partials: this shape does not split K")
    _lib.require_gpu(x2, name="mm8_matmul_partials")
    ws = _ws.reserve(x2.device, need, slot="mm8t")
    splits = ctypes.c_int(0)
    _lib.call("rwkv7mi_mm8t_matmul_partials", _lib.ptr(x2), _lib.ptr(mod.w_blk), _lib.ptr(mod.mx), _lib.ptr(mod.rx),
              _lib.ptr(mod.my), _lib.ptr(mod.ry), rows, n, m, _lib.dtype_code(x2), _lib.dtype_code(mod.mx),
              _lib.ptr(ws), int(ws.numel()), ctypes.byref(splits), _lib.stream_of(x2))
    S = int(splits.value)
    return ws[: S * rows * m * 4].view(torch.float32).view(S, rows, m), S


def mm8_gemm_workspace_bytes(nprob: int, rows: int, n: int, m: int, splits: int = 0) -> int:
    """Scratch bytes :func:`mm8_gemm_multi_into` needs: x' and row sums, plus the
    split-K partials when there is more than one split."""
    return int(_lib.load().rwkv7mi_mm8t_gemm_workspace_bytes(int(nprob), int(rows), int(n), int(m), int(splits)))


def mm8_gemm_multi_into(xs, mods, outs, *, residuals=None, epilogues=None, splits: int = 0):
    """Many-row (17..256) form of :func:`mm8_matmul_multi_into`: up to four
    blocked ``MM8Linear`` products of one shape on the MFMA tile kernel, the
    route ``mm8_matmul_triton`` takes through dequantisation for rows above
    ``fused_max_rows`` (rwkv7_hf/native_quant_mm8.py:468-507).  Split-K
    partials use the device's ``"mm8g"`` workspace slot (reserve it before
    graph capture)."""
    k = len(mods)
    if not 1 <= k <= 4 or len(xs) != k or len(outs) != k:
        raise ValueError("mm8_gemm_multi_into: 1..4 problems")
    rows, n = (int(s) for s in xs[0].shape)
    m = int(mods[0].out_features)
    residuals = list(residuals) if residuals is not None else [None] * k
    epilogues = list(epilogues) if epilogues is not None else [_lib.EPI_NONE] * k
    for x2, mod, out, r in zip(xs, mods, outs, residuals):
        if tuple(x2.shape) != (rows, n) or not x2.is_contiguous() or x2.dtype != xs[0].dtype:
            raise ValueError("mm8_gemm_multi_into: inputs must share one contiguous shape and dtype")
        if mod.in_features != n or mod.out_features != m or not is_blocked(mod.w_blk):
            raise ValueError("mm8_gemm_multi_into: modules must be blocked MM8Linear of one shape")
        _check_out(x2, m, out, r)
    _lib.require_gpu(*xs, *outs, name="mm8_gemm_multi")
    need = mm8_gemm_workspace_bytes(k, rows, n, m, splits)
    ws = _ws.reserve(xs[0].device, need, slot="mm8g")
    arr = lambda ts: _lib.ptr_array(ts)
    eps = (ctypes.c_int * k)(*[int(e) for e in epilogues])
    _lib.call(
        "rwkv7mi_mm8t_gemm_multi", k, arr(xs), arr([md.w_blk for md in mods]), arr([md.mx for md in mods]),
        arr([md.rx for md in mods]), arr([md.my for md in mods]), arr([md.ry for md in mods]),
        arr([md.bias for md in mods]), arr(residuals), arr(outs), eps, rows, n, m, _lib.dtype_code(xs[0]),
        _lib.dtype_code(mods[0].mx), int(splits), _lib.ptr(ws), int(ws.numel()),
        _lib.stream_of(xs[0]),
    )
    return outs


# x's buffer descriptor in the prefill GEMM spans rows * in_features * 2 bytes,
# below 2^31: longer inputs are split into row chunks
_PREFILL_MAX_BYTES = (1 << 31) - 1


def mm8_gemm_prefill_multi_into(xs, mods, outs, *, residuals=None, epilogues=None):
    """Prefill form (more than ``GEMM_ROWS`` rows) of :func:`mm8_matmul_multi_into`:
    up to four blocked ``MM8Linear`` products of one shape, the route
    ``mm8_matmul_triton`` takes for rows above ``fused_max_rows``
    (rwkv7_hf/native_quant_mm8.py:468-507): the fp16 dequantised weight is
    materialised (into the device's ``"mm8p"`` workspace slot, in MFMA operand
    order) and one fp16 MFMA GEMM with the epilogue fused runs over it, as in
    the prefill projections of rwkv7_hf/native_jit_prefill.py:542-631,
    955-1013.  fp16 or bf16 activations with metadata of the same type; fp32
    runs the 64-row tile GEMM over 256-row chunks (without a dequantised weight).
    Reserve the workspace (one eager call) before capturing a graph."""
    k = len(mods)
    if not 1 <= k <= 4 or len(xs) != k or len(outs) != k:
        raise ValueError("mm8_gemm_prefill_multi_into: 1..4 problems")
    rows, n = (int(s) for s in xs[0].shape)
    m = int(mods[0].out_features)
    residuals = list(residuals) if residuals is not None else [None] * k
    epilogues = list(epilogues) if epilogues is not None else [_lib.EPI_NONE] * k
    for x2, mod, out, r in zip(xs, mods, outs, residuals):
        if tuple(x2.shape) != (rows, n) or not x2.is_contiguous() or x2.dtype != xs[0].dtype:
            raise ValueError("mm8_gemm_prefill_multi_into: inputs must share one contiguous shape and dtype")
        if mod.in_features != n or mod.out_features != m or not is_blocked(mod.w_blk):
            raise ValueError("mm8_gemm_prefill_multi_into: modules must be blocked MM8Linear of one shape")
        _check_out(x2, m, out, r)
    _lib.require_gpu(*xs, *outs, name="mm8_gemm_prefill_multi")
    fast = xs[0].dtype in (torch.float16, torch.bfloat16) and all(md.mx.dtype == xs[0].dtype for md in mods)
    chunk = max(1, _PREFILL_MAX_BYTES // (2 * n)) if fast else GEMM_ROWS
    eps = (ctypes.c_int * k)(*[int(e) for e in epilogues])
    arr = lambda ts: _lib.ptr_array(ts)
    for r0 in range(0, rows, chunk):
        r1 = min(rows, r0 + chunk)
        xc = [x[r0:r1] for x in xs]
        oc = [o[r0:r1] for o in outs]
        rc = [None if r is None else r.reshape(rows, m)[r0:r1] for r in residuals]
        if not fast:
            if r1 - r0 > GEMV_ROWS:
                mm8_gemm_multi_into(xc, mods, oc, residuals=rc, epilogues=epilogues)
            else:
                mm8_matmul_multi_into(xc, mods, oc, residuals=rc, epilogues=epilogues)
            continue
        need = mm8_prefill_workspace_bytes(k, n, m)
        ws = _ws.reserve(xs[0].device, need, "mm8p")
        _lib.call(
            "rwkv7mi_mm8t_gemm_prefill_ws", k, arr(xc), arr([md.w_blk for md in mods]), arr([md.mx for md in mods]),
            arr([md.rx for md in mods]), arr([md.my for md in mods]), arr([md.ry for md in mods]),
            arr([md.bias for md in mods]), arr(rc), arr(oc), eps, r1 - r0, n, m, _lib.dtype_code(xs[0]),
            _lib.dtype_code(xs[0]), _lib.ptr(ws), need, _lib.stream_of(xs[0]),
        )
    return outs


def mm8_lnmix_multi_into(x, prev, ln_w, ln_b, eps: float, mixes, mods, outs, *, epilogues=None, h_out=None,
                         aux_mixes=(), aux_outs=(), lora_downs=None, lora_out=None):
    """Decode form of ``fused_attn_norm_mix6_decode`` / ``fused_ffn_add_norm_mix_decode``
    (rwkv7_hf/fused_decode_norm_mix.py:161, 296) followed by up to four out-major
    ``MM8Linear`` products, in one launch: ``h = LayerNorm(x)``,
    ``outs[p] = (h + (prev - h) * mixes[p]) @ W_p`` (the mixed input rounded to the
    activation dtype as the reference's tensor is).  Also writes ``h`` to ``h_out``
    (the next token's ``prev``; ``prev`` itself is only read) and
    ``aux_outs[a] = h + (prev - h) * aux_mixes[a]`` for other consumers.
    fp16 / bf16 only; rows <= 2 at in_features 4096 (the rows must fit one staging batch, which
    the row statistics are taken from; the library rejects larger calls).

    ``lora_downs`` (one ``[rank, in]`` weight per extra mix) adds the decode LoRA's
    down projections of the extra mixes (the first half of ``fused_wavg_lora``,
    rwkv7_hf/fused_lora.py:706), summed over K in fp32 into ``lora_out``
    (``rows * sum(ranks)`` values, problem-major), for
    :func:`fused_lora.fused_wavg_lora_output_prepare_raw`'s ``down_sums``.
    """
    k = len(mods)
    if not 1 <= k <= 4 or len(mixes) != k or len(outs) != k:
        raise ValueError("mm8_lnmix_multi_into: 1..4 problems")
    if len(aux_mixes) != len(aux_outs) or len(aux_mixes) > 4:
        raise ValueError("mm8_lnmix_multi_into: 0..4 extra mixes")
    rows, n = (int(s) for s in x.shape)
    m = int(mods[0].out_features)
    dt = x.dtype
    vecs = [t.reshape(-1) for t in (ln_w, ln_b, *mixes, *aux_mixes)]
    for t in (x, prev, *vecs, *outs, *aux_outs, *( [h_out] if h_out is not None else [])):
        if not t.is_contiguous() or t.dtype != dt:
            raise ValueError("mm8_lnmix_multi_into: tensors must be contiguous in the activation dtype")
    for t in vecs:
        if t.numel() != n:
            raise ValueError("mm8_lnmix_multi_into: LN parameters and mixes must have in_features values")
    for t in (prev, *aux_outs, *([h_out] if h_out is not None else [])):
        if tuple(t.shape) != (rows, n):
            raise ValueError("mm8_lnmix_multi_into: prev, h_out and extra outputs are [rows, in_features]")
    reads = {t.data_ptr() for t in (x, prev)}
    if any(t.data_ptr() in reads for t in (*outs, *aux_outs, *([h_out] if h_out is not None else []))):
        raise ValueError("mm8_lnmix_multi_into: outputs must not alias x or prev (every workgroup reads them)")
    for mod, out in zip(mods, outs):
        if mod.in_features != n or mod.out_features != m or not is_blocked(mod.w_blk) or mod.bias is not None:
            raise ValueError("mm8_lnmix_multi_into: blocked MM8Linear modules of one shape, without bias")
        if mod.mx.dtype != dt:
            raise ValueError("mm8_lnmix_multi_into: MM8 metadata must be in the activation dtype")
        _check_out(x, m, out, None)
    epilogues = list(epilogues) if epilogues is not None else [_lib.EPI_NONE] * k
    _lib.require_gpu(x, prev, *outs, name="mm8_lnmix_multi")
    arr = lambda ts: _lib.ptr_array(ts)
    na = len(aux_mixes)
    lw = lr = None
    if lora_downs is not None:
        if len(lora_downs) != na or lora_out is None:
            raise ValueError("mm8_lnmix_multi_into: one LoRA down weight per extra mix, and lora_out")
        for d in lora_downs:
            if d.dim() != 2 or int(d.shape[1]) != n or d.dtype != dt or not d.is_contiguous():
                raise ValueError("mm8_lnmix_multi_into: LoRA down weights are contiguous [rank, in] in x's dtype")
        ranks = [int(d.shape[0]) for d in lora_downs]
        if lora_out.dtype != torch.float32 or not lora_out.is_contiguous() or int(lora_out.numel()) < rows * sum(ranks):
            raise ValueError("mm8_lnmix_multi_into: lora_out must be contiguous fp32 with rows * sum(ranks) values")
        lw, lr = arr(list(lora_downs)), (ctypes.c_int64 * na)(*ranks)
    _lib.call(
        "rwkv7mi_mm8t_lnmix_multi", k, _lib.ptr(x), _lib.ptr(prev), _lib.ptr(vecs[0]), _lib.ptr(vecs[1]),
        float(eps), arr(vecs[2:2 + k]), arr([md.w_blk for md in mods]), arr([md.mx for md in mods]),
        arr([md.rx for md in mods]), arr([md.my for md in mods]), arr([md.ry for md in mods]), arr(outs),
        (ctypes.c_int * k)(*[int(e) for e in epilogues]), _lib.ptr(h_out), na, arr(vecs[2 + k:]), arr(list(aux_outs)),
        lw, lr, _lib.ptr(lora_out if lora_downs is not None else None), rows, n, m, _lib.dtype_code(x),
        _lib.stream_of(x),
    )
    return outs


def dequantize_mm8(w_u8, mx, rx, my, ry, out_dtype=None):
    """The dequantised weight ``[N, M]``: ``(w + 0.5) ry rx + my + mx`` in
    ``out_dtype`` (default: the metadata dtype), rwkv7_hf/native_quant_mm8.py:100-108.
    One HIP pass in fp32 with a single rounding.  ``w_u8`` is the reference's
    contiguous ``[N, M]`` bytes or the blocked decode layout (the result is then
    the ``[N, M]`` view of an ``[M, N]`` tensor)."""
    dt = out_dtype if out_dtype is not None else mx.dtype
    _lib.require_gpu(w_u8, mx, name="dequantize_mm8")
    if is_blocked(w_u8):
        n, m = int(ry.numel()), int(mx.numel())
        out = torch.empty((m, n), device=w_u8.device, dtype=dt)
        _lib.call("rwkv7mi_mm8t_dequant", _lib.ptr(w_u8), _lib.ptr(mx.reshape(-1)), _lib.ptr(rx.reshape(-1)),
                  _lib.ptr(my.reshape(-1).contiguous()), _lib.ptr(ry.reshape(-1).contiguous()), _lib.ptr(out), n, m,
                  _lib.dtype_code(mx), _lib.dtype_code(out), _lib.stream_of(w_u8))
        return out.t()
    if w_u8.dim() != 2 or not w_u8.is_contiguous():
        raise ValueError("dequantize_mm8 expects contiguous [N, M] bytes or the blocked layout")
    n, m = (int(s) for s in w_u8.shape)
    out = torch.empty((n, m), device=w_u8.device, dtype=dt)
    _lib.call("rwkv7mi_mm8_dequant", _lib.ptr(w_u8), _lib.ptr(mx.reshape(-1).contiguous()),
              _lib.ptr(rx.reshape(-1).contiguous()), _lib.ptr(my.reshape(-1).contiguous()),
              _lib.ptr(ry.reshape(-1).contiguous()), _lib.ptr(out), n, m, _lib.dtype_code(mx), _lib.dtype_code(out),
              _lib.stream_of(w_u8))
    return out


def _meta_1d(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    t = t.reshape(-1)
    if t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


def mm8_matmul(x, w_u8, mx, rx, my, ry):
    """``y = x @ dequant(W)`` for ``x: [..., N]`` -> ``[..., M]`` (fused HIP kernel)."""
    n, m = int(ry.numel()), int(mx.numel())
    lead = x.shape[:-1]
    x2 = x.reshape(-1, n).contiguous()
    mdt = mx.dtype
    out = torch.empty((x2.shape[0], m), device=x.device, dtype=x.dtype)
    mm8_matmul_into(x2, w_u8, _meta_1d(mx, mdt), _meta_1d(rx, mdt), _meta_1d(my, mdt), _meta_1d(ry, mdt), out)
    return out.reshape(*lead, m)


mm8_linear = mm8_matmul


def mm8_gemv_triton(x, w_u8, mx, rx, my, ry):
    """Reference name of the B=1 GEMV; runs the same HIP kernel."""
    return mm8_matmul(x, w_u8, mx, rx, my, ry)


def mm8_matmul_triton(x, w_u8, mx, rx, my, ry, *, max_gemv_rows: int | None = None):
    """Reference name of the routed matmul; one HIP kernel for every row count."""
    return mm8_matmul(x, w_u8, mx, rx, my, ry)


class MM8Linear(torch.nn.Module):
    """Drop-in for ``nn.Linear`` storing int8 (mm8) weights, dequantized on the fly.

    The state dict matches the reference module (rwkv7_hf/native_quant_mm8.py:583-589):
    ``w_u8 [in, out]``, ``mx, rx [out]``, ``my, ry [in, 1]`` and optional
    ``bias``, with the same values.  The bytes live in the decode GEMV's
    blocked layout (``w_blk``, see :func:`mm8_block`); ``state_dict`` writes
    them back as the reference's ``w_u8`` and ``load_state_dict`` accepts a
    reference ``w_u8`` (hooks below), and the ``w_u8`` attribute materialises
    the reference tensor.
    """

    def __init__(self, linear, *, fused=True):
        super().__init__()
        self.in_features, self.out_features = int(linear.weight.shape[1]), int(linear.weight.shape[0])
        w_blk, mx, rx, my, ry = quantize_mm8_blocked(linear.weight.data)
        self.register_buffer("w_blk", w_blk, persistent=False)
        self.register_buffer("mx", mx)
        self.register_buffer("rx", rx)
        self.register_buffer("my", my)
        self.register_buffer("ry", ry)
        if linear.bias is not None:
            self.register_buffer("bias", linear.bias.data.clone())
        else:
            self.bias = None
        self.fused = bool(fused)
        self.sm7x_rowwise = False
        self.register_state_dict_post_hook(MM8Linear._export_w_u8)
        self.register_load_state_dict_pre_hook(MM8Linear._import_w_u8)

    @classmethod
    def from_packed(cls, w_blk, mx, rx, my, ry, in_features: int, out_features: int, bias=None, *, fused=True):
        """A module from already packed tensors (a prepacked checkpoint): the
        blocked bytes ``w_blk`` (:func:`mm8_block_shape`) and the four scale
        vectors as :func:`quantize_mm8_blocked` returns them.  No quantisation."""
        n, m = int(in_features), int(out_features)
        if tuple(w_blk.shape) != mm8_block_shape(n, m) or w_blk.dtype != torch.uint8:
            raise ValueError(f"MM8Linear.from_packed: w_blk {w_blk.dtype} {tuple(w_blk.shape)} is not the blocked "
                             f"layout of [{n}, {m}]")
        if mx.numel() != m or rx.numel() != m or my.numel() != n or ry.numel() != n:
            raise ValueError("MM8Linear.from_packed: scale vectors do not match the features")
        self = cls.__new__(cls)
        torch.nn.Module.__init__(self)
        self.in_features, self.out_features = n, m
        self.register_buffer("w_blk", w_blk.contiguous(), persistent=False)
        self.register_buffer("mx", mx)
        self.register_buffer("rx", rx)
        self.register_buffer("my", my)
        self.register_buffer("ry", ry)
        if bias is not None:
            self.register_buffer("bias", bias)
        else:
            self.bias = None
        self.fused = bool(fused)
        self.sm7x_rowwise = False
        self.register_state_dict_post_hook(MM8Linear._export_w_u8)
        self.register_load_state_dict_pre_hook(MM8Linear._import_w_u8)
        return self

    @property
    def w_u8(self) -> torch.Tensor:
        """The reference's ``w_u8 [in, out]`` (a new contiguous tensor)."""
        return mm8_unblock(self.w_blk, self.in_features, self.out_features)

    @staticmethod
    def _export_w_u8(module, state_dict, prefix, local_metadata):
        state_dict[prefix + "w_u8"] = module.w_u8

    @staticmethod
    def _import_w_u8(module, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys, error_msgs):
        key = prefix + "w_u8"
        if key not in state_dict:
            if strict:
                missing_keys.append(key)
            return
        w = state_dict.pop(key)
        if tuple(w.shape) != (module.in_features, module.out_features) or w.dtype != torch.uint8:
            error_msgs.append(f"{key}: expected uint8 [{module.in_features}, {module.out_features}], "
                              f"got {w.dtype} {tuple(w.shape)}")
            return
        with torch.no_grad():
            module.w_blk.copy_(mm8_block(w.to(module.w_blk.device)))

    def _run(self, x, out=None, residual=None, epilogue=_lib.EPI_NONE):
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        rows = int(x2.shape[0])
        if out is None:
            out2 = torch.empty((rows, self.out_features), device=x.device, dtype=x.dtype)
        else:
            out2 = out.reshape(rows, self.out_features)
        mm8_matmul_into(x2, self.w_blk, self.mx, self.rx, self.my.reshape(-1), self.ry.reshape(-1), out2,
                        bias=self.bias, residual=residual, epilogue=epilogue)
        return out2.reshape(*lead, self.out_features) if out is None else out

    def forward(self, x):
        return self._run(x)

    def rwkv7_forward_into(self, x, out):
        return self._run(x, out=out)

    def rwkv7_forward_relu2(self, x):
        return self._run(x, epilogue=_lib.EPI_RELU2)

    def rwkv7_forward_add(self, x, residual):
        return self._run(x, residual=residual.contiguous(), epilogue=_lib.EPI_RESIDUAL)

    def rwkv7_forward_ffn(self, x, down, residual):
        """The FFN pair ``residual + down(relu(self(x))^2)`` in two fused launches
        (key with the relu^2 epilogue, value with the residual epilogue), the
        optional quantized-module hook of rwkv7_hf/native_jit_graph_dispatch.py:594-598
        and native_jit_prefill.py:964-973.  Returns a new tensor, or ``None`` (the
        caller's fallback) when ``down`` is not an MM8Linear of the matching shape."""
        if not isinstance(down, MM8Linear) or down.in_features != self.out_features:
            return None
        hidden = self._run(x, epilogue=_lib.EPI_RELU2)
        res = residual.reshape(*hidden.shape[:-1], down.out_features).contiguous()
        return down._run(hidden, residual=res, epilogue=_lib.EPI_RESIDUAL)

    def _workspace_slot(self, rows: int):
        rows = int(rows)
        if GEMV_ROWS < rows <= GEMM_ROWS:
            return "mm8g", mm8_gemm_workspace_bytes(1, rows, self.in_features, self.out_features)
        if 0 < rows <= GEMV_ROWS:
            return "mm8t", mm8t_workspace_bytes(1, rows, self.in_features, self.out_features)
        return None, 0

    def rwkv7_workspace_bytes(self, rows: int) -> int:
        """Scratch bytes a ``rows``-row call needs: the fused GEMV's split-K
        partials (``"mm8t"`` slot, only when the rows' x' exceeds one LDS chunk)
        up to GEMV_ROWS rows, the tile GEMM's x', row sums and split partials
        (``"mm8g"`` slot) from GEMV_ROWS + 1 to GEMM_ROWS rows."""
        return self._workspace_slot(rows)[1]

    def rwkv7_reserve_workspace(self, rows: int) -> None:
        """Grow the slot a ``rows``-row call uses (call before graph capture)."""
        slot, need = self._workspace_slot(rows)
        if need:
            _ws.reserve(self.w_blk.device, need, slot=slot)

    def extra_repr(self):
        return f"in={self.in_features}, out={self.out_features}, mm8(fused={self.fused}, hip=gfx950)"


def quantize_model_mm8(model, *, min_params: int = 8_000_000, fused: bool = True, policy: str = "memory") -> int:
    """Swap eligible ``nn.Linear`` modules for :class:`MM8Linear`; returns the count."""
    policy = normalize_native_mm_policy(policy)
    targets = [
        name for name, mod in model.named_modules()
        if isinstance(mod, torch.nn.Linear)
        and should_quantize_linear(name, int(mod.weight.numel()), min_params=min_params, policy=policy)
    ]
    for full_name in targets:
        parent_name, _, attr = full_name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, attr, MM8Linear(getattr(parent, attr), fused=fused))
    setattr(model, "_rwkv7_native_mm_quantization", "mm8")
    setattr(model, "_rwkv7_native_mm_replaced_modules", len(targets))
    setattr(model, "_rwkv7_native_mm_block_replaced_modules", sum(n.startswith("model.layers.") for n in targets))
    invalidate_model_caches(model)
    return len(targets)


# Attributes under which the reference model keeps operand packs and graph
# runners built from the modules being swapped (rwkv7_hf/native_quant_mm8.py:674-683,
# native_quant_mm4.py:820-829), plus this build's runner cache.
MODEL_CACHE_ATTRS = (
    "_rwkv7_native_jit_pack_cache",
    "_rwkv7_native_graph_pack_cache",
    "_rwkv7_native_graph_runner_cache",
    "_rwkv7_native_prefill_graph_runner_cache",
    "_rwkv7_native_prefill_graph_hot_runner",
    "_rwkv7_native_model_jit_pack_cache",
)


def invalidate_model_caches(model) -> None:
    """Drop the packs and graph runners a model built from its old modules."""
    for attr in MODEL_CACHE_ATTRS:
        if hasattr(model, attr):
            delattr(model, attr)
    for name in ("_graph_runners", "_prefill_graph_runners"):
        runners = getattr(model, name, None)
        if isinstance(runners, dict):
            runners.clear()


__all__ = ["mm8_gemm_prefill_multi_into", "mm8_block_shape",
    "quantize_mm8", "dequantize_mm8", "quantize_mm8_outmajor", "quantize_mm8_blocked", "mm8_block", "mm8_unblock", "is_blocked",
    "is_out_major", "mm8_matmul", "mm8_linear", "mm8_matmul_into",
    "mm8_matmul_multi_into", "mm8_gemm_multi_into", "mm8_gemm_workspace_bytes", "mm8_gemv_triton",
    "mm8_matmul_triton", "mm8_workspace_bytes", "mm8t_workspace_bytes", "MM8Linear", "quantize_model_mm8", "invalidate_model_caches",
]
