"""wkv7 recurrence operators with the reference's names and signatures.

Mirrors rwkv7_hf/fused_recurrent_update.py (rwkv-rs/hf-adapter 0.8.1):
``fused_recurrent_update`` (:1214), ``fused_recurrent_output_prepare`` (:967),
``fused_recurrent_output_prepare_raw`` (:1089) and ``fused_recurrent_scan``
(:1299).  Shapes, validation messages (ValueError) and return conventions
follow the reference; Triton tuning keywords (``block_n``, ``block_m``,
``num_warps``) are validated the same way and otherwise ignored, and
``force_fallback`` is accepted for signature compatibility only — every call
runs the gfx950 HIP kernel (there is no torch/CPU fallback path).

Extra keyword arguments beyond the reference (``state_out``, ``out``) let the
caller provide destination buffers, e.g. to update the recurrent state in place
inside a captured decode graph.
"""
from __future__ import annotations

from typing import Any

import torch

from . import _lib


def _as_bhn(x: Any, H: int, N: int, *, name: str):
    if x.dim() == 3:
        if int(x.shape[1]) != H or int(x.shape[2]) != N:
            raise ValueError(f"{name} must be shaped [batch,{H},{N}] or [batch,{H * N}]; got {tuple(x.shape)}")
        return x.contiguous(), False
    if x.dim() == 2:
        if int(x.shape[1]) != H * N:
            raise ValueError(f"{name} must be shaped [batch,{H},{N}] or [batch,{H * N}]; got {tuple(x.shape)}")
        return x.reshape(int(x.shape[0]), H, N).contiguous(), True
    raise ValueError(f"{name} must be shaped [batch,{H},{N}] or [batch,{H * N}]")


def _as_bthn(x: Any, H: int, N: int, *, name: str):
    if x.dim() == 4:
        if int(x.shape[2]) != H or int(x.shape[3]) != N:
            raise ValueError(
                f"{name} must be shaped [batch,tokens,{H},{N}] or [batch,tokens,{H * N}]; got {tuple(x.shape)}"
            )
        return x.contiguous(), False
    if x.dim() == 3:
        if int(x.shape[2]) != H * N:
            raise ValueError(
                f"{name} must be shaped [batch,tokens,{H},{N}] or [batch,tokens,{H * N}]; got {tuple(x.shape)}"
            )
        return x.reshape(int(x.shape[0]), int(x.shape[1]), H, N).contiguous(), True
    raise ValueError(f"{name} must be shaped [batch,tokens,{H},{N}] or [batch,tokens,{H * N}]")


def _check_state(state):
    if state.dim() != 4:
        raise ValueError("state must be shaped [batch, heads, head_dim, head_dim]")
    B, H, N, N2 = (int(vv) for vv in state.shape)
    if N != N2:
        raise ValueError("state must be square in the last two dimensions")
    if state.dtype != torch.float32:
        raise ValueError("rwkv7mi keeps the recurrent state in float32")
    if N != 64:
        raise ValueError(f"rwkv7mi kernels require head_dim=64; got {N}")
    return B, H, N


def _state_dst(state: torch.Tensor, state_out: torch.Tensor | None) -> torch.Tensor:
    if state_out is None:
        return torch.empty_like(state)
    if state_out.shape != state.shape or state_out.dtype != torch.float32 or not state_out.is_contiguous():
        raise ValueError("state_out must be a contiguous float32 tensor shaped like state")
    return state_out


def _same_dtype(ref: torch.Tensor, *tensors: torch.Tensor, name: str) -> None:
    for t in tensors:
        if t.dtype != ref.dtype:
            raise ValueError(f"{name}: all vector inputs must share dtype {ref.dtype}; got {t.dtype}")


def fused_recurrent_update(
    r: Any, w: Any, k: Any, v: Any, kk: Any, a: Any, state: Any, *,
    block_n: int = 64, force_fallback: bool = False,
    state_out: torch.Tensor | None = None, out: torch.Tensor | None = None,
):
    """One-token RWKV-7 recurrent update; returns ``(out, new_state)``.

    ``state`` is not modified unless ``state_out is state`` (in-place update).
    """
    B, H, N = _check_state(state)
    if int(block_n) < N:
        raise ValueError(f"block_n must be >= head_dim={N}; got {block_n}")
    r3, flat = _as_bhn(r, H, N, name="r")
    w3, _ = _as_bhn(w, H, N, name="w")
    k3, _ = _as_bhn(k, H, N, name="k")
    v3, _ = _as_bhn(v, H, N, name="v")
    kk3, _ = _as_bhn(kk, H, N, name="kk")
    a3, _ = _as_bhn(a, H, N, name="a")
    if int(r3.shape[0]) != B:
        raise ValueError("r/w/k/v/kk/a batch size must match state")
    _same_dtype(r3, k3, v3, kk3, a3, name="fused_recurrent_update")
    _lib.require_gpu(r3, w3, k3, v3, kk3, a3, state, name="fused_recurrent_update")
    st = state.contiguous()
    new_state = _state_dst(st, state_out)
    y = out if out is not None else torch.empty((B, H, N), device=r3.device, dtype=r3.dtype)
    _lib.call(
        "rwkv7mi_wkv7_decode_update",
        _lib.ptr(r3), _lib.ptr(w3), _lib.ptr(k3), _lib.ptr(v3), _lib.ptr(kk3), _lib.ptr(a3),
        _lib.ptr(st), _lib.ptr(new_state), _lib.ptr(y), B, H, N,
        _lib.dtype_code(r3), _lib.dtype_code(w3), _lib.stream_of(r3),
    )
    if flat:
        return y.reshape(B, H * N), new_state
    return y, new_state


def fused_recurrent_output_prepare(
    r: Any, w: Any, k: Any, v: Any, kk: Any, a: Any, state: Any, g: Any, r_k: Any,
    group_norm_weight: Any, group_norm_bias: Any, *, eps: float, block_n: int = 64,
    num_warps: int = 8, force_fallback: bool = False,
    state_out: torch.Tensor | None = None, out: torch.Tensor | None = None,
):
    """Recurrent update + GroupNorm + bonus + gate; returns ``(prepared, new_state)``."""
    B, H, N = _check_state(state)
    if int(block_n) < N:
        raise ValueError(f"block_n must be >= head_dim={N}; got {block_n}")
    r3, flat = _as_bhn(r, H, N, name="r")
    w3, _ = _as_bhn(w, H, N, name="w")
    k3, _ = _as_bhn(k, H, N, name="k")
    v3, _ = _as_bhn(v, H, N, name="v")
    kk3, _ = _as_bhn(kk, H, N, name="kk")
    a3, _ = _as_bhn(a, H, N, name="a")
    g3, _ = _as_bhn(g, H, N, name="g")
    if r_k.numel() != H * N:
        raise ValueError(f"r_k must be [{H}, {N}], got {tuple(r_k.shape)}")
    if group_norm_weight.numel() != H * N:
        raise ValueError(f"group_norm_weight must be [{H * N}], got {tuple(group_norm_weight.shape)}")
    if group_norm_bias.numel() != H * N:
        raise ValueError(f"group_norm_bias must be [{H * N}], got {tuple(group_norm_bias.shape)}")
    _same_dtype(r3, k3, v3, kk3, a3, g3, name="fused_recurrent_output_prepare")
    rk = r_k.reshape(H * N).contiguous()
    gnw = group_norm_weight.reshape(H * N).to(rk.dtype).contiguous()
    gnb = group_norm_bias.reshape(H * N).to(rk.dtype).contiguous()
    _lib.require_gpu(r3, w3, k3, v3, kk3, a3, g3, state, rk, name="fused_recurrent_output_prepare")
    st = state.contiguous()
    new_state = _state_dst(st, state_out)
    y = out if out is not None else torch.empty((B, H, N), device=r3.device, dtype=r3.dtype)
    _lib.call(
        "rwkv7mi_wkv7_decode_output_prepare",
        _lib.ptr(r3), _lib.ptr(w3), _lib.ptr(k3), _lib.ptr(v3), _lib.ptr(kk3), _lib.ptr(a3),
        _lib.ptr(st), _lib.ptr(new_state), _lib.ptr(g3), _lib.ptr(rk), _lib.ptr(gnw), _lib.ptr(gnb),
        _lib.ptr(y), B, H, N, float(eps), _lib.dtype_code(r3), _lib.dtype_code(w3), _lib.dtype_code(rk),
        _lib.stream_of(r3),
    )
    if flat:
        return y.reshape(B, H * N), new_state
    return y, new_state


def fused_recurrent_output_prepare_raw(
    r: Any, w_raw: Any, k_raw: Any, v: Any, a: Any, state: Any, g: Any, k_k: Any, k_a: Any,
    r_k: Any, group_norm_weight: Any, group_norm_bias: Any, *, eps: float, block_n: int = 64,
    num_warps: int = 8, force_fallback: bool = False,
    state_out: torch.Tensor | None = None, out: torch.Tensor | None = None,
    v_first: torch.Tensor | None = None, v_gate: torch.Tensor | None = None, v_mode: int = 0,
):
    """Decode recurrence + output prep from raw W/K and sigmoid'd A.

    ``v_mode`` (extension): 0 = V used as given (reference behaviour);
    1 = layer 0, V is copied into ``v_first``; 2 = ``v + (v_first - v) * v_gate``
    is applied in-kernel before the update.
    """
    B, H, N = _check_state(state)
    if int(block_n) < N:
        raise ValueError(f"block_n must be >= head_dim={N}; got {block_n}")
    if int(num_warps) not in {1, 2, 4, 8}:
        raise ValueError(f"num_warps must be one of 1, 2, 4, or 8; got {num_warps}")
    r3, flat = _as_bhn(r, H, N, name="r")
    w3, _ = _as_bhn(w_raw, H, N, name="w_raw")
    k3, _ = _as_bhn(k_raw, H, N, name="k_raw")
    v3, _ = _as_bhn(v, H, N, name="v")
    a3, _ = _as_bhn(a, H, N, name="a")
    g3, _ = _as_bhn(g, H, N, name="g")
    hidden = H * N
    for value, name in ((k_k, "k_k"), (k_a, "k_a"), (r_k, "r_k"),
                        (group_norm_weight, "group_norm_weight"), (group_norm_bias, "group_norm_bias")):
        if int(value.numel()) != hidden:
            raise ValueError(f"{name} must contain {hidden} values")
    _same_dtype(r3, w3, k3, v3, a3, g3, name="fused_recurrent_output_prepare_raw")
    kk_s = k_k.reshape(hidden).contiguous()
    ka = k_a.reshape(hidden).to(kk_s.dtype).contiguous()
    rk = r_k.reshape(hidden).to(kk_s.dtype).contiguous()
    gnw = group_norm_weight.reshape(hidden).to(kk_s.dtype).contiguous()
    gnb = group_norm_bias.reshape(hidden).to(kk_s.dtype).contiguous()
    if v_mode not in (0, 1, 2):
        raise ValueError("v_mode must be 0, 1 or 2")
    if v_mode and (v_first is None or not v_first.is_contiguous() or v_first.numel() != B * hidden
                   or v_first.dtype != r3.dtype):
        raise ValueError("v_mode 1/2 needs a contiguous v_first [B, H*N] of the activation dtype")
    vg = None
    if v_mode == 2:
        if v_gate is None or v_gate.numel() != B * hidden:
            raise ValueError("v_mode 2 needs v_gate [B, H*N]")
        vg = v_gate.to(r3.dtype).contiguous()
    _lib.require_gpu(r3, w3, k3, v3, a3, g3, state, kk_s, v_first, vg, name="fused_recurrent_output_prepare_raw")
    st = state.contiguous()
    new_state = _state_dst(st, state_out)
    y = out if out is not None else torch.empty((B, H, N), device=r3.device, dtype=r3.dtype)
    _lib.call(
        "rwkv7mi_wkv7_decode_output_prepare_raw",
        _lib.ptr(r3), _lib.ptr(w3), _lib.ptr(k3), _lib.ptr(v3), _lib.ptr(a3), _lib.ptr(st),
        _lib.ptr(new_state), _lib.ptr(g3), _lib.ptr(kk_s), _lib.ptr(ka), _lib.ptr(rk), _lib.ptr(gnw),
        _lib.ptr(gnb), _lib.ptr(y), _lib.ptr(v_first), _lib.ptr(vg), int(v_mode), B, H, N, float(eps),
        _lib.dtype_code(r3), _lib.dtype_code(kk_s), _lib.stream_of(r3),
    )
    if flat:
        return y.reshape(B, hidden), new_state
    return y, new_state


def fused_recurrent_scan(
    r: Any, w: Any, k: Any, v: Any, kk: Any, a: Any, state: Any, *,
    block_n: int = 64, block_m: int | None = None, num_warps: int | None = None,
    force_fallback: bool = False, state_out: torch.Tensor | None = None,
):
    """Sequential multi-token scan; returns ``(out [B,T,H,N] or flat, final_state)``."""
    B, H, N = _check_state(state)
    if int(block_n) < N:
        raise ValueError(f"block_n must be >= head_dim={N}; got {block_n}")
    if block_m is not None and int(block_m) <= 0:
        raise ValueError(f"block_m must be positive; got {block_m}")
    if num_warps is not None and int(num_warps) not in {1, 2, 4, 8}:
        raise ValueError(f"num_warps must be one of 1, 2, 4, or 8; got {num_warps}")
    r4, flat = _as_bthn(r, H, N, name="r")
    w4, _ = _as_bthn(w, H, N, name="w")
    k4, _ = _as_bthn(k, H, N, name="k")
    v4, _ = _as_bthn(v, H, N, name="v")
    kk4, _ = _as_bthn(kk, H, N, name="kk")
    a4, _ = _as_bthn(a, H, N, name="a")
    if int(r4.shape[0]) != B:
        raise ValueError("r/w/k/v/kk/a batch size must match state")
    _same_dtype(r4, k4, v4, kk4, a4, name="fused_recurrent_scan")
    T = int(r4.shape[1])
    _lib.require_gpu(r4, w4, k4, v4, kk4, a4, state, name="fused_recurrent_scan")
    st = state.contiguous()
    final = _state_dst(st, state_out)
    y = torch.empty((B, T, H, N), device=r4.device, dtype=r4.dtype)
    _lib.call(
        "rwkv7mi_wkv7_scan",
        _lib.ptr(r4), _lib.ptr(w4), _lib.ptr(k4), _lib.ptr(v4), _lib.ptr(kk4), _lib.ptr(a4),
        _lib.ptr(st), _lib.ptr(final), _lib.ptr(y), B, T, H, N,
        _lib.dtype_code(r4), _lib.dtype_code(w4), _lib.stream_of(r4),
    )
    if flat:
        return y.reshape(B, T, H * N), final
    return y, final


def _scan_checks(state, block_n, block_m, num_warps):
    B, H, N = _check_state(state)
    if int(block_n) < N:
        raise ValueError(f"block_n must be >= head_dim={N}; got {block_n}")
    if block_m is not None and not 0 < int(block_m) <= N:
        raise ValueError(f"block_m must be in [1, head_dim={N}]; got {block_m}")
    if num_warps is not None and int(num_warps) not in {1, 2, 4, 8}:
        raise ValueError(f"num_warps must be one of 1, 2, 4, or 8; got {num_warps}")
    return B, H, N


def fused_recurrent_scan_clampw(
    r: Any, w_raw: Any, k: Any, v: Any, kk: Any, a: Any, state: Any, *,
    block_n: int = 64, block_m: int | None = None, num_warps: int | None = None,
    force_fallback: bool = False, state_out: torch.Tensor | None = None,
):
    """Scan over ``[B,T,H,N]`` (or flat) inputs with the raw W pre-activation:
    the decay ``exp(-0.606531 sigmoid(w_raw))`` is formed inside the chunk
    kernel, so no decay tensor is written (rwkv7_hf/fused_recurrent_update.py:1420-1538).
    Returns ``(out, final_state)``."""
    from .self_chunk_rwkv7 import _run_chunk

    B, H, N = _scan_checks(state, block_n, block_m, num_warps)
    r4, flat = _as_bthn(r, H, N, name="r")
    w4, _ = _as_bthn(w_raw, H, N, name="w_raw")
    k4, _ = _as_bthn(k, H, N, name="k")
    v4, _ = _as_bthn(v, H, N, name="v")
    kk4, _ = _as_bthn(kk, H, N, name="kk")
    a4, _ = _as_bthn(a, H, N, name="a")
    if int(r4.shape[0]) != B:
        raise ValueError("r/w/k/v/kk/a batch size must match state")
    _same_dtype(r4, w4, k4, v4, kk4, a4, name="fused_recurrent_scan_clampw")
    y, final = _run_chunk(r4, w4, k4, v4, kk4, a4, state, w_is_log=2, chunk=16, state_out=state_out)
    if flat:
        return y.reshape(B, int(r4.shape[1]), H * N), final
    return y, final


def fused_recurrent_scan_state_prep(
    r: Any, w_raw: Any, k_raw: Any, v_raw: Any, a: Any, state: Any, k_k: Any, k_a: Any, *,
    v_first: Any | None = None, v_gate: Any | None = None, block_n: int = 64,
    block_m: int | None = None, num_warps: int | None = None, force_fallback: bool = False,
    state_out: torch.Tensor | None = None,
):
    """State prep fused in front of the scan (rwkv7_hf/fused_recurrent_update.py:1541-1707):
    ``kk = normalize(k_raw * k_k)``, ``k = k_raw (1 + (a - 1) k_a)``,
    ``v = v_raw + (v_first - v_raw) v_gate`` when both are given, decay from
    ``w_raw`` — ``a`` and ``v_gate`` already sigmoid'd.  Two launches: the prep
    kernel (the log decay in fp32) and the chunk kernel.  Returns
    ``(out, final_state, k_adjusted, v_interpolated)`` in the input layout."""
    from .fused_prefill import fused_prefill_state_prep
    from .self_chunk_rwkv7 import _run_chunk

    B, H, N = _scan_checks(state, block_n, block_m, num_warps)
    r4, flat = _as_bthn(r, H, N, name="r")
    w4, _ = _as_bthn(w_raw, H, N, name="w_raw")
    k4, _ = _as_bthn(k_raw, H, N, name="k_raw")
    v4, _ = _as_bthn(v_raw, H, N, name="v_raw")
    a4, _ = _as_bthn(a, H, N, name="a")
    if int(r4.shape[0]) != B:
        raise ValueError("r/w/k/v/a batch size must match state")
    hidden = H * N
    if int(k_k.numel()) != hidden or int(k_a.numel()) != hidden:
        raise ValueError(f"k_k and k_a must have {hidden} elements")
    has_v_gate = v_first is not None and v_gate is not None
    vf = vg = None
    if has_v_gate:
        vf, _ = _as_bthn(v_first, H, N, name="v_first")
        vg, _ = _as_bthn(v_gate, H, N, name="v_gate")
    _same_dtype(r4, w4, k4, v4, a4, name="fused_recurrent_scan_state_prep")
    T = int(r4.shape[1])
    w_log, k_adj, v_adj, kk = fused_prefill_state_prep(
        w4, k4, v4, a4, k_k, k_a, v_first=None if vf is None else vf.to(r4.dtype).contiguous(), v_gate=vg,
        num_heads=H, head_dim=N, w_transform="log_decay", v_mode=2 if has_v_gate else 0)
    y, final = _run_chunk(r4, w_log, k_adj, v_adj, kk, a4, state, w_is_log=1, chunk=16, state_out=state_out)
    if flat:
        return (y.reshape(B, T, hidden), final, k_adj.reshape(B, T, hidden), v_adj.reshape(B, T, hidden))
    return y, final, k_adj, v_adj


def fused_recurrent_scan_output_prepare(
    r: Any, w: Any, k: Any, v: Any, kk: Any, a: Any, state: Any, g: Any, r_k: Any,
    group_norm_weight: Any, group_norm_bias: Any, *, eps: float, block_n: int = 64,
    force_fallback: bool = False, state_out: torch.Tensor | None = None,
):
    """Scan followed by the attention output prep (per-head GroupNorm, bonus
    ``(sum r k r_k) v`` and gate ``g``; rwkv7_hf/fused_recurrent_update.py:1710-1833).
    ``w`` is the decay in the activation dtype or fp32.  Two launches: the
    chunk kernel and the output-prep kernel.  Returns ``(prepared, final_state)``
    with ``prepared`` ready for ``o_proj``."""
    from .fused_output import fused_attn_output_prepare
    from .self_chunk_rwkv7 import _run_chunk

    B, H, N = _scan_checks(state, block_n, None, None)
    r4, flat = _as_bthn(r, H, N, name="r")
    w4, _ = _as_bthn(w, H, N, name="w")
    k4, _ = _as_bthn(k, H, N, name="k")
    v4, _ = _as_bthn(v, H, N, name="v")
    kk4, _ = _as_bthn(kk, H, N, name="kk")
    a4, _ = _as_bthn(a, H, N, name="a")
    g4, _ = _as_bthn(g, H, N, name="g")
    if int(r4.shape[0]) != B:
        raise ValueError("r/w/k/v/kk/a/g batch size must match state")
    if r_k.dim() != 2 or int(r_k.shape[0]) != H or int(r_k.shape[1]) != N:
        raise ValueError(f"r_k must be [{H}, {N}], got {tuple(r_k.shape)}")
    if group_norm_weight.dim() != 1 or int(group_norm_weight.shape[0]) != H * N:
        raise ValueError(f"group_norm_weight must be [{H * N}], got {tuple(group_norm_weight.shape)}")
    if group_norm_bias.dim() != 1 or int(group_norm_bias.shape[0]) != H * N:
        raise ValueError(f"group_norm_bias must be [{H * N}], got {tuple(group_norm_bias.shape)}")
    _same_dtype(r4, k4, v4, kk4, a4, g4, name="fused_recurrent_scan_output_prepare")
    if w4.dtype not in (r4.dtype, torch.float32):
        raise ValueError("w must be in the activation dtype or float32")
    T, A = int(r4.shape[1]), H * N
    y, final = _run_chunk(r4, w4, k4, v4, kk4, a4, state, w_is_log=0, chunk=16, state_out=state_out)
    prep = fused_attn_output_prepare(y.reshape(B * T, A), r4.reshape(B * T, A), k4.reshape(B * T, A),
                                     v4.reshape(B * T, A), g4.reshape(B * T, A), r_k, group_norm_weight,
                                     group_norm_bias, num_heads=H, head_dim=N, head_v_dim=N, eps=eps)
    if flat:
        return prep.reshape(B, T, A), final
    return prep.reshape(B, T, H, N), final


__all__ = [
    "fused_recurrent_update",
    "fused_recurrent_output_prepare",
    "fused_recurrent_output_prepare_raw",
    "fused_recurrent_scan",
    "fused_recurrent_scan_clampw",
    "fused_recurrent_scan_state_prep",
    "fused_recurrent_scan_output_prepare",
]
