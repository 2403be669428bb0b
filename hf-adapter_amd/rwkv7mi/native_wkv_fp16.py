"""Opt-in fp16-state recurrence with the reference's names and signatures.

Mirrors rwkv7_hf/native_wkv_fp16.py (rwkv-rs/hf-adapter 0.8.1):
``native_fp16_recurrent_should_use`` (:597), ``native_fp16_recurrent_available``
(:668), ``native_fp16_recurrent_build_error`` (:674),
``native_fp16_recurrent_output_prepare_raw`` (:678) and ``native_fp16_sequence``
(:756).  The default state of this package stays fp32; this lane runs only when
a caller holds an fp16 state of head size 64 and fp16 activations, as in the
reference.  Both operators run the gfx950 kernels of csrc/wkv7_f16.hip through
the C ABI (``rwkv7mi_wkv7_fp16_decode_output_prepare_raw``,
``rwkv7mi_wkv7_fp16_sequence``); there is no torch/CPU fallback.

Validation follows the reference: shape and dtype errors raise ValueError
before the library is touched, a missing library raises RuntimeError.  One
behavioural difference: the reference's decode kernel increments
``elapsed[b]`` from head 0's block while other heads of the same batch row may
still read it; here the increment is a second launch on the same stream, so
every head of a step sees the same phase.
"""
from __future__ import annotations

from typing import Any

import torch

from . import _lib

_BUILD_ERROR: str | None = None


def native_fp16_recurrent_should_use(*, state_dtype: Any, input_dtype: Any, head_dim: int) -> bool:
    return bool(state_dtype == torch.float16 and input_dtype == torch.float16 and int(head_dim) == 64)


def _load() -> Any | None:
    global _BUILD_ERROR
    try:
        return _lib.load()
    except RuntimeError as exc:
        _BUILD_ERROR = f"{type(exc).__name__}: {exc}"
        return None


def native_fp16_recurrent_available(*, build: bool = False) -> bool:
    if not torch.cuda.is_available():
        return False
    return _load() is not None if build else True


def native_fp16_recurrent_build_error() -> str | None:
    return _BUILD_ERROR


def _require_library(what: str) -> None:
    if _load() is None:
        raise RuntimeError(f"{what} extension is unavailable: {native_fp16_recurrent_build_error()}")


def native_fp16_recurrent_output_prepare_raw(
    r: Any, w_raw: Any, k_raw: Any, v: Any, a: Any, state: Any, g: Any, k_k: Any, k_a: Any, r_k: Any,
    norm_weight: Any, norm_bias: Any, elapsed: Any, *, advance_elapsed: bool, eps: float,
    out: Any | None = None, v_first: Any | None = None, v_gate: Any | None = None, v_mode: int = 0,
) -> Any:
    """One decode token on an fp16 state (updated in place); returns ``out`` shaped like ``r``.

    ``elapsed`` (int32 ``[B]``) feeds the decay dither's phase and moves by one
    when ``advance_elapsed`` is set.  Extensions beyond the reference: ``out``
    (a contiguous fp16 tensor with ``r``'s element count) receives the result
    instead of a new tensor, for callers that must not allocate (a captured
    decode graph); ``v_mode`` 1 copies ``v`` into ``v_first`` (layer 0), 2 uses
    ``v + (v_first - v) * v_gate`` in place of ``v``, rounded to fp16 after each
    operation as the reference's torch form before this call
    (rwkv7_hf/native_jit_decode.py:762-766).  ``v`` itself is not written.
    """
    if state.dim() != 4:
        raise ValueError("state must be [B,H,64,64]")
    if not native_fp16_recurrent_should_use(state_dtype=state.dtype, input_dtype=r.dtype,
                                            head_dim=int(state.shape[-1])):
        raise ValueError("native FP16 recurrence received an unsupported dtype or shape")
    _require_library("native FP16 recurrence")
    tensors = (r, w_raw, k_raw, v, a, state, g, k_k, k_a, r_k, norm_weight, norm_bias)
    if not all(t.is_cuda and t.dtype == torch.float16 and t.is_contiguous() for t in tensors):
        raise ValueError("native FP16 recurrence requires contiguous CUDA fp16 tensors")
    if not (elapsed.is_cuda and elapsed.dtype == torch.int32 and elapsed.is_contiguous()):
        raise ValueError("elapsed must be a contiguous CUDA int32 tensor")
    B, H, N, N2 = (int(x) for x in state.shape)
    if N2 != N:
        raise ValueError("state must be [B,H,64,64]")
    if int(r.numel()) != B * H * N:
        raise ValueError("r shape does not match state")
    for t in (w_raw, k_raw, v, a, g):
        if t.shape != r.shape:
            raise ValueError("token tensors must share shape")
    for t in (k_k, k_a, r_k, norm_weight, norm_bias):
        if int(t.numel()) != H * N:
            raise ValueError("per-channel tensor shape mismatch")
    if int(elapsed.numel()) != B:
        raise ValueError("elapsed must be contiguous CUDA int32 [B]")
    if out is None:
        out = torch.empty_like(r)
    elif not (out.is_cuda and out.dtype == torch.float16 and out.is_contiguous()
              and int(out.numel()) == int(r.numel())):
        raise ValueError("out must be a contiguous CUDA fp16 tensor with r's element count")
    if v_mode not in (0, 1, 2):
        raise ValueError("v_mode must be 0, 1 or 2")
    for t, name, need in ((v_first, "v_first", v_mode >= 1), (v_gate, "v_gate", v_mode == 2)):
        if need and (t is None or not (t.is_cuda and t.dtype == torch.float16 and t.is_contiguous()
                                       and int(t.numel()) == int(r.numel()))):
            raise ValueError(f"v_mode {v_mode} needs a contiguous CUDA fp16 {name} with r's element count")
    _lib.call(
        "rwkv7mi_wkv7_fp16_decode_output_prepare_raw",
        _lib.ptr(r), _lib.ptr(w_raw), _lib.ptr(k_raw), _lib.ptr(v), _lib.ptr(a), _lib.ptr(state), _lib.ptr(g),
        _lib.ptr(k_k), _lib.ptr(k_a), _lib.ptr(r_k), _lib.ptr(norm_weight), _lib.ptr(norm_bias),
        _lib.ptr(elapsed), int(bool(advance_elapsed)), _lib.ptr(out),
        _lib.ptr(v_first if v_mode >= 1 else None), _lib.ptr(v_gate if v_mode == 2 else None), int(v_mode),
        B, H, N, float(eps), _lib.stream_of(r),
    )
    return out


def native_fp16_sequence(
    r: Any, w: Any, k: Any, v: Any, neg_kk: Any, kka: Any, state: Any, elapsed: Any, *, w0: Any | None = None,
) -> Any:
    """The fixed-order fp16 recurrence over ``[B,T,H,64]``; returns y in the same layout.

    ``w`` holds the raw decay pre-activation; ``w0`` (``[H*64]``), when given,
    is added to it in fp32 before the decay is formed.  The state is updated in
    place; ``elapsed`` is read, not advanced.
    """
    if state.dim() != 4 or r.dim() != 4:
        raise ValueError("state and sequence tensors must be rank four")
    if not native_fp16_recurrent_should_use(state_dtype=state.dtype, input_dtype=r.dtype,
                                            head_dim=int(state.shape[-1])):
        raise ValueError("native FP16 sequence received an unsupported dtype or shape")
    _require_library("native FP16 sequence")
    tensors = (r, w, k, v, neg_kk, kka, state)
    if not all(t.is_cuda and t.dtype == torch.float16 and t.is_contiguous() for t in tensors):
        raise ValueError("native FP16 sequence requires contiguous CUDA fp16 tensors")
    if not (elapsed.is_cuda and elapsed.dtype == torch.int32 and elapsed.is_contiguous()
            and int(elapsed.numel()) == int(r.shape[0])):
        raise ValueError("elapsed must be a contiguous CUDA int32 [B] tensor")
    B, T, H, N = (int(x) for x in r.shape)
    if N != 64:
        raise ValueError("r must be [B,T,H,64]")
    if T <= 0:
        raise ValueError("sequence requires at least one token")
    if tuple(state.shape) != (B, H, N, N):
        raise ValueError("state batch/head shape does not match sequence")
    for t, name in ((w, "w"), (k, "k"), (v, "v"), (neg_kk, "neg_kk"), (kka, "kka")):
        if t.shape != r.shape:
            raise ValueError(f"{name} shape must match r")
    if w0 is not None:
        if not (w0.is_cuda and w0.dtype == torch.float16 and w0.is_contiguous()):
            raise ValueError("w0 must be contiguous CUDA fp16")
        if int(w0.numel()) != H * N:
            raise ValueError("w0 must have H*64 elements")
    out = torch.empty_like(r)
    _lib.call(
        "rwkv7mi_wkv7_fp16_sequence",
        _lib.ptr(r), _lib.ptr(w), _lib.ptr(w0), _lib.ptr(k), _lib.ptr(v), _lib.ptr(neg_kk), _lib.ptr(kka),
        _lib.ptr(state), _lib.ptr(elapsed), _lib.ptr(out), B, T, H, N, _lib.stream_of(r),
    )
    return out


__all__ = [
    "native_fp16_recurrent_available",
    "native_fp16_recurrent_build_error",
    "native_fp16_recurrent_output_prepare_raw",
    "native_fp16_recurrent_should_use",
    "native_fp16_sequence",
]
