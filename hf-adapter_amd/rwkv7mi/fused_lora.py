"""W/A/G/V LoRA projections with the reference's API.

Mirrors ``fused_wavg_lora`` (rwkv7_hf/fused_lora.py:706) and ``fused_wag_lora``
(:559): two grouped launches of the gfx950 LoRA kernels — the four down
projections split over K (tanh for W, sigmoid for G applied when the partials
are reduced) and the four up projections (bias, and the V-gate sigmoid fused).  Returns ``(w, a_pre, g, v_gate)``;
the caller applies the outer sigmoid to ``a_pre`` as in the reference.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import workspace as _ws

ACT_NONE, ACT_TANH, ACT_SIGMOID, ACT_RELU2 = 0, 1, 2, 3


def dense_multi(problems, rows: int):
    """problems: list of (x2 [rows,K], W [N,K], bias or None, y [rows,N], act)."""
    xs = [p[0] for p in problems]
    Ws = [p[1] for p in problems]
    bs = [p[2] for p in problems]
    ys = [p[3] for p in problems]
    k = len(problems)
    Ns = (ctypes.c_int64 * k)(*[int(p[1].shape[0]) for p in problems])
    Ks = (ctypes.c_int64 * k)(*[int(p[1].shape[1]) for p in problems])
    acts = (ctypes.c_int * k)(*[int(p[4]) for p in problems])
    _lib.require_gpu(*xs, *Ws, *ys, name="dense_multi")
    _lib.call("rwkv7mi_dense_multi", _lib.ptr_array(xs), _lib.ptr_array(Ws), _lib.ptr_array(bs), _lib.ptr_array(ys),
              Ns, Ks, acts, len(problems), int(rows), _lib.dtype_code(xs[0]), _lib.stream_of(xs[0]))


def lora_workspace_bytes(ranks, rows: int, D: int) -> int:
    arr = (ctypes.c_int64 * len(ranks))(*[int(r) for r in ranks])
    return int(_lib.load().rwkv7mi_lora_workspace_bytes(len(ranks), arr, int(rows), int(D)))


def lora_multi(xs, downs, ups, biases, outs, acts_down, acts_up):
    """Grouped LoRA: ``outs[i] = act_up(act_down(xs[i] @ downs[i].T) @ ups[i].T + biases[i])``.

    Up to 256 rows: two launches for up to four projections (split-K down
    kernel, up kernel that reduces the partials; the fp32 partials live in the
    per-device workspace).  More rows (prefills): one launch of the fused
    kernel, 64 rows per workgroup, no workspace.
    """
    k = len(xs)
    rows, D = (int(s) for s in xs[0].shape)
    A = int(ups[0].shape[0])
    ranks = [int(d.shape[0]) for d in downs]
    _lib.require_gpu(*xs, *downs, *ups, *outs, name="lora_multi")
    ws = _ws.reserve(xs[0].device, lora_workspace_bytes(ranks, rows, D), slot="lora")
    _lib.call("rwkv7mi_lora_multi", k, _lib.ptr_array(xs), _lib.ptr_array(downs), _lib.ptr_array(ups),
              _lib.ptr_array(biases), _lib.ptr_array(outs), (ctypes.c_int64 * k)(*ranks),
              (ctypes.c_int * k)(*[int(a) for a in acts_down]), (ctypes.c_int * k)(*[int(a) for a in acts_up]),
              rows, D, A, _lib.dtype_code(xs[0]), _lib.ptr(ws), int(ws.numel()), _lib.stream_of(xs[0]))
    return outs


def fused_lora_decode_supported(ranks, rows: int) -> bool:
    """Whether ``fused_wavg_lora_output_prepare_raw`` takes these shapes."""
    ranks = [int(r) for r in ranks]
    return 0 < int(rows) <= 64 and len(ranks) in (3, 4) and all(0 < r <= 128 and r % 8 == 0 for r in ranks)


def fused_wavg_lora_output_prepare_raw(r, k_raw, v, xs, downs, ups, biases, state, k_k, k_a, r_k,
                                       group_norm_weight, group_norm_bias, *, eps: float, out, state_out=None,
                                       v_first=None, v_mode: int = 0, down_sums=None, down_splits: int = 1,
                                       elapsed=None, advance_elapsed: bool = False):
    """``fused_wavg_lora`` (rwkv7_hf/fused_lora.py:706) followed by
    ``fused_recurrent_output_prepare_raw`` (fused_recurrent_update.py:1089) in two
    launches: the split-K down projections, then one decode kernel in which each
    (batch, head) workgroup computes its 64 channels of the W/A/G/V up projections
    before the state update.  ``xs``/``downs``/``ups``/``biases`` are in the order
    W, A, G[, V]; activations are the reference's (tanh/none, none/sigmoid,
    sigmoid/none, none/sigmoid).  Returns ``(out [B, H*N], new_state)``.

    ``down_sums`` (fp32, from :func:`native_quant_mm8.mm8_lnmix_multi_into` with
    ``lora_downs``, or :func:`fused_decode_norm_mix.attn_mix_lora_decode`): the
    down projections already summed over K, or over ``down_splits`` K-chunks
    (``[problem][split][row][rank]``); ``xs`` and the down launch are then
    skipped.

    An fp16 ``state`` (``[B, H, 64, 64]``, fp16 activations and parameters)
    runs the fp16-state kernel instead (the reference's fp16 decode,
    rwkv7_hf/native_jit_decode.py:762-784, with
    ``native_fp16_recurrent_output_prepare_raw``'s semantics): the state is
    updated in place (``state_out`` None or ``state`` itself), ``elapsed``
    (int32 ``[B]``) feeds the decay dither and moves by one when
    ``advance_elapsed`` is set."""
    k = len(xs)
    rows, D = (int(s) for s in xs[0].shape)
    ranks = [int(d.shape[0]) for d in downs]
    if not fused_lora_decode_supported(ranks, rows):
        raise ValueError("fused LoRA decode: rows <= 64, 3 or 4 ranks, multiples of 8 up to 128")
    B, H, N = (int(x) for x in state.shape[:3])
    if rows != B or int(r.numel()) != B * H * N:
        raise ValueError("fused LoRA decode: rows must match the state batch")
    acts_down = [ACT_TANH, ACT_NONE, ACT_SIGMOID, ACT_NONE][:k]
    acts_up = [ACT_NONE, ACT_SIGMOID, ACT_NONE, ACT_SIGMOID][:k]
    hidden = H * N
    f16 = state.dtype == torch.float16
    if f16:
        if not (r.dtype == k_raw.dtype == v.dtype == out.dtype == torch.float16 and int(N) == 64
                and int(state.shape[3]) == 64 and state.is_contiguous()):
            raise ValueError("fused LoRA decode on an fp16 state: fp16 activations, contiguous [B,H,64,64] state")
        if state_out is not None and state_out.data_ptr() != state.data_ptr():
            raise ValueError("fused LoRA decode on an fp16 state: the state is updated in place")
        if elapsed is None or not (elapsed.is_cuda and elapsed.dtype == torch.int32 and elapsed.is_contiguous()
                                   and int(elapsed.numel()) == B):
            raise ValueError("fused LoRA decode on an fp16 state: elapsed must be contiguous CUDA int32 [B]")
        if any(u.dtype != torch.float16 for u in ups) or any(
                b is not None and b.dtype != torch.float16 for b in biases):
            raise ValueError("fused LoRA decode on an fp16 state: fp16 up weights and biases")
        if v_mode and (v_first is None or v_first.dtype != torch.float16):
            raise ValueError("fused LoRA decode on an fp16 state: v_first must be fp16")
    pdt = torch.float16 if f16 else k_k.dtype
    kk_s, ka, rk, gnw, gnb = (t.reshape(hidden).to(pdt).contiguous()
                              for t in (k_k, k_a, r_k, group_norm_weight, group_norm_bias))
    _lib.require_gpu(r, k_raw, v, *xs, *downs, *ups, state, out, name="fused_wavg_lora_output_prepare_raw")
    s = _lib.stream_of(r)
    rk_arr = (ctypes.c_int64 * k)(*ranks)
    if down_sums is not None:
        if (down_sums.dtype != torch.float32 or not down_sums.is_contiguous()
                or int(down_splits) < 1 or int(down_sums.numel()) < int(down_splits) * rows * sum(ranks)):
            raise ValueError("fused LoRA decode: down_sums must be contiguous fp32 with "
                             "down_splits * rows * sum(ranks) values")
        ws, splits = down_sums, int(down_splits)
    else:
        ws = _ws.reserve(xs[0].device, lora_workspace_bytes(ranks, rows, D), slot="lora")
        splits = 0
        _lib.call("rwkv7mi_lora_down_multi", k, _lib.ptr_array(xs), _lib.ptr_array(downs), rk_arr,
                  (ctypes.c_int * k)(*acts_down), rows, D, _lib.dtype_code(xs[0]), _lib.ptr(ws), int(ws.numel()), s)
    if f16:
        _lib.call("rwkv7mi_wkv7_fp16_decode_lora_output_prepare",
                  _lib.ptr(r), _lib.ptr(k_raw), _lib.ptr(v), _lib.ptr(ws), k, rk_arr, _lib.ptr_array(ups),
                  _lib.ptr_array(biases), (ctypes.c_int * k)(*acts_down), (ctypes.c_int * k)(*acts_up), D, splits,
                  _lib.ptr(state), _lib.ptr(kk_s), _lib.ptr(ka), _lib.ptr(rk), _lib.ptr(gnw), _lib.ptr(gnb),
                  _lib.ptr(elapsed), int(bool(advance_elapsed)), _lib.ptr(out), _lib.ptr(v_first), int(v_mode),
                  B, H, N, float(eps), s)
        return out, state
    new_state = state if state_out is None else state_out
    _lib.call("rwkv7mi_wkv7_decode_lora_output_prepare",
              _lib.ptr(r), _lib.ptr(k_raw), _lib.ptr(v), _lib.ptr(ws), k, rk_arr, _lib.ptr_array(ups),
              _lib.ptr_array(biases), (ctypes.c_int * k)(*acts_down), (ctypes.c_int * k)(*acts_up), D, splits,
              _lib.ptr(state), _lib.ptr(new_state), _lib.ptr(kk_s), _lib.ptr(ka), _lib.ptr(rk), _lib.ptr(gnw),
              _lib.ptr(gnb), _lib.ptr(out), _lib.ptr(v_first), int(v_mode), B, H, N, float(eps),
              _lib.dtype_code(r), _lib.dtype_code(kk_s), s)
    return out, new_state


def _flat(x, name):
    had_seq = x.dim() == 3
    x2 = x.reshape(-1, int(x.shape[-1]))
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    return x2, had_seq


def _lin(w, dtype):
    w = w.to(dtype) if w.dtype != dtype else w
    return w.contiguous()


def fused_wavg_lora(xw, xa, xg, xv, w_down_weight, a_down_weight, g_down_weight, v_down_weight,
                    w_up_weight, a_up_weight, g_up_weight, v_up_weight, w_up_bias=None, a_up_bias=None,
                    g_up_bias=None, v_up_bias=None, *, block_m: int = 16, block_r: int = 64, block_k: int = 64,
                    num_warps: int = 4, force_fallback: bool = False, mids=None, outs=None):
    """W: tanh(xw W1^T) W2^T + b;  A: (xa A1^T) A2^T + b (pre-sigmoid);
    G: sigmoid(xg G1^T) G2^T;  V gate: sigmoid((xv V1^T) V2^T + b)."""
    x2s = [_flat(x, n) for x, n in ((xw, "xw"), (xa, "xa"), (xg, "xg"), (xv, "xv"))]
    had_seq = x2s[0][1]
    xs = [t[0] for t in x2s]
    rows, D = (int(s) for s in xs[0].shape)
    for x in xs[1:]:
        if tuple(x.shape) != (rows, D):
            raise ValueError("xw, xa, xg and xv must have identical flattened shapes")
    dt = xs[0].dtype
    downs = [_lin(w, dt) for w in (w_down_weight, a_down_weight, g_down_weight, v_down_weight)]
    ups = [_lin(w, dt) for w in (w_up_weight, a_up_weight, g_up_weight, v_up_weight)]
    biases = [None if b is None else _lin(b, dt) for b in (w_up_bias, a_up_bias, g_up_bias, v_up_bias)]
    out_dim = int(ups[0].shape[0])
    for d, u in zip(downs, ups):
        if int(d.shape[1]) != D or int(u.shape[1]) != int(d.shape[0]) or int(u.shape[0]) != out_dim:
            raise ValueError("LoRA weights do not match: down [R, D], up [out, R]")
    dev = xs[0].device
    if outs is None:
        outs = [torch.empty((rows, out_dim), device=dev, dtype=dt) for _ in range(4)]
    lora_multi(xs, downs, ups, biases, outs, [ACT_TANH, ACT_NONE, ACT_SIGMOID, ACT_NONE],
               [ACT_NONE, ACT_NONE, ACT_NONE, ACT_SIGMOID])
    if had_seq:
        return tuple(o.reshape(int(xw.shape[0]), int(xw.shape[1]), out_dim) for o in outs)
    return tuple(outs)


def fused_wag_lora(xw, xa, xg, w_down_weight, a_down_weight, g_down_weight, w_up_weight, a_up_weight, g_up_weight,
                   w_up_bias=None, a_up_bias=None, g_up_bias=None, **kwargs):
    """Layer-0 variant without the V gate; returns ``(w, a_pre, g)``."""
    x2s = [_flat(x, n)[0] for x, n in ((xw, "xw"), (xa, "xa"), (xg, "xg"))]
    rows = int(x2s[0].shape[0])
    dt = x2s[0].dtype
    downs = [_lin(w, dt) for w in (w_down_weight, a_down_weight, g_down_weight)]
    ups = [_lin(w, dt) for w in (w_up_weight, a_up_weight, g_up_weight)]
    biases = [None if b is None else _lin(b, dt) for b in (w_up_bias, a_up_bias, g_up_bias)]
    out_dim = int(ups[0].shape[0])
    dev = x2s[0].device
    for d, u in zip(downs, ups):
        if int(d.shape[1]) != int(x2s[0].shape[1]) or int(u.shape[1]) != int(d.shape[0]) or int(u.shape[0]) != out_dim:
            raise ValueError("LoRA weights do not match: down [R, D], up [out, R]")
    outs = [torch.empty((rows, out_dim), device=dev, dtype=dt) for _ in range(3)]
    lora_multi(x2s, downs, ups, biases, outs, [ACT_TANH, ACT_NONE, ACT_SIGMOID], [ACT_NONE] * 3)
    if xw.dim() == 3:
        return tuple(o.reshape(int(xw.shape[0]), int(xw.shape[1]), out_dim) for o in outs)
    return tuple(outs)


__all__ = ["fused_wavg_lora", "fused_wag_lora", "dense_multi", "lora_multi", "lora_workspace_bytes"]
