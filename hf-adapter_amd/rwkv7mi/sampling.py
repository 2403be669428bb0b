"""Greedy token selection on the GPU (``rwkv7mi_argmax_rows``): the argmax of
each logits row as the reference's greedy loop takes it with torch
(bench/bench_native_quant_e2e_decode.py:424-437), so a captured decode graph
can end with its next tokens."""
from __future__ import annotations

import torch

from . import _lib


def argmax_workspace_bytes(rows: int, n: int, dtype: torch.dtype) -> int:
    """Workspace bytes of the many-workgroup argmax of ``rows`` rows of ``n``."""
    return int(_lib.load().rwkv7mi_argmax_workspace_bytes(int(rows), int(n), _lib._DTYPE_CODE[dtype]))


def argmax_rows(logits: torch.Tensor, *, out: torch.Tensor | None = None,
                out2: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """``logits [rows, n]`` -> ``int64 [rows]``: the first index of each row's
    maximum (NaN counts as the maximum), written to ``out`` (and ``out2``)
    when given.  No host synchronisation; capturable.  Rows are split over
    many workgroups (two launches); ``workspace`` (a contiguous tensor of at
    least :func:`argmax_workspace_bytes` bytes) is allocated when not given."""
    if logits.dim() != 2:
        raise ValueError("argmax_rows: logits must be [rows, n]")
    _lib.require_gpu(logits, out, out2, name="argmax_rows")
    rows, n = (int(s) for s in logits.shape)
    if logits.stride(1) != 1 or logits.data_ptr() % 16 or (logits.stride(0) * logits.element_size()) % 16:
        logits = logits.contiguous()
        if logits.data_ptr() % 16 or (n * logits.element_size()) % 16:
            raise ValueError("argmax_rows: rows must be 16-byte aligned")
    for t in (out, out2):
        if t is not None and (t.dtype != torch.int64 or t.numel() != rows or not t.is_contiguous()):
            raise ValueError("argmax_rows: out must be a contiguous int64 tensor of one entry per row")
    if out is None:
        out = torch.empty(rows, device=logits.device, dtype=torch.int64)
    need = argmax_workspace_bytes(rows, n, logits.dtype)
    if workspace is None:
        workspace = torch.empty(need, device=logits.device, dtype=torch.uint8)
    elif (not workspace.is_contiguous() or workspace.numel() * workspace.element_size() < need
          or workspace.data_ptr() % 8):
        raise ValueError("argmax_rows: workspace must be contiguous, 8-byte aligned, "
                         "of at least argmax_workspace_bytes bytes")
    _lib.call("rwkv7mi_argmax_rows_ws", _lib.ptr(logits), rows, n, int(logits.stride(0)), _lib.dtype_code(logits),
              _lib.ptr(out), _lib.ptr(out2), _lib.ptr(workspace), workspace.numel() * workspace.element_size(),
              _lib.stream_of(logits))
    return out


__all__ = ["argmax_rows", "argmax_workspace_bytes"]
