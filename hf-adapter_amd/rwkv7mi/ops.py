"""``torch.ops.rwkv7mi.*``: the hot-path operators registered as torch custom ops.

The reference loads its native kernels as torch extensions whose functions
take and return tensors (rwkv7_hf/sm70_quant.py:61-72, 440-478;
kernel_package.py:304-371).  This module gives the same seam a dispatcher
schema: each op below is defined in the ``rwkv7mi`` library namespace, with
in-place arguments marked ``Tensor(a!)`` so functionalisation and graph
capture see the mutation, a CUDA implementation that calls the gfx950 kernel
through the C ABI (``librwkv7mi.so``), a CPU implementation that raises
``RuntimeError`` (there is no CPU fallback) and a fake (meta) implementation
that gives output shapes without running anything, so the ops trace under
``torch.compile`` / ``torch.export``.

Out-of-place ops return new tensors; the ``*_`` ops update their marked
arguments and return nothing.  Importing ``rwkv7mi`` registers them once.
"""
from __future__ import annotations

import torch

LIB_NAME = "rwkv7mi"

# name -> schema (argument order follows the Python functions of the same name)
SCHEMAS = {
    "fused_recurrent_update":
        "fused_recurrent_update(Tensor r, Tensor w, Tensor k, Tensor v, Tensor kk, Tensor a, Tensor state)"
        " -> (Tensor, Tensor)",
    "fused_recurrent_update_":
        "fused_recurrent_update_(Tensor r, Tensor w, Tensor k, Tensor v, Tensor kk, Tensor a, Tensor(a!) state,"
        " Tensor(b!) out) -> ()",
    "fused_recurrent_output_prepare_raw":
        "fused_recurrent_output_prepare_raw(Tensor r, Tensor w_raw, Tensor k_raw, Tensor v, Tensor a, Tensor state,"
        " Tensor g, Tensor k_k, Tensor k_a, Tensor r_k, Tensor gn_w, Tensor gn_b, float eps) -> (Tensor, Tensor)",
    "fused_recurrent_output_prepare_raw_":
        "fused_recurrent_output_prepare_raw_(Tensor r, Tensor w_raw, Tensor k_raw, Tensor v, Tensor a,"
        " Tensor(a!) state, Tensor g, Tensor k_k, Tensor k_a, Tensor r_k, Tensor gn_w, Tensor gn_b, float eps,"
        " Tensor(b!) out) -> ()",
    "chunk_scan":
        "chunk_scan(Tensor r, Tensor w, Tensor k, Tensor v, Tensor kk, Tensor a, Tensor state, int w_mode)"
        " -> (Tensor, Tensor)",
    "chunk_scan_":
        "chunk_scan_(Tensor r, Tensor w, Tensor k, Tensor v, Tensor kk, Tensor a, Tensor(a!) state, int w_mode,"
        " Tensor(b!) y) -> ()",
    "mm8_matmul":
        "mm8_matmul(Tensor x, Tensor w_u8, Tensor mx, Tensor rx, Tensor my, Tensor ry) -> Tensor",
    "mm8_matmul_out":
        "mm8_matmul_out(Tensor x, Tensor w_u8, Tensor mx, Tensor rx, Tensor my, Tensor ry, Tensor(a!) out) -> ()",
    "quantize_mm8":
        "quantize_mm8(Tensor weight) -> (Tensor, Tensor, Tensor, Tensor, Tensor)",
    "w4_groupwise_linear":
        "w4_groupwise_linear(Tensor x, Tensor q, Tensor scales, int out_features, int in_features, int group_size)"
        " -> Tensor",
    "attn_norm_mix6_":
        "attn_norm_mix6_(Tensor x, Tensor(a!) previous, Tensor norm_weight, Tensor norm_bias, Tensor mix_r,"
        " Tensor mix_w, Tensor mix_k, Tensor mix_v, Tensor mix_a, Tensor mix_g, float eps, Tensor(b!) out) -> ()",
    "ffn_add_norm_mix_":
        "ffn_add_norm_mix_(Tensor(a!) x, Tensor attn_out, Tensor(b!) previous, Tensor norm_weight,"
        " Tensor norm_bias, Tensor mix, float eps, Tensor(c!) mixed) -> ()",
    "wavg_lora":
        "wavg_lora(Tensor xw, Tensor xa, Tensor xg, Tensor xv, Tensor w1, Tensor a1, Tensor g1, Tensor v1,"
        " Tensor w2, Tensor a2, Tensor g2, Tensor v2, Tensor? w0, Tensor? a0, Tensor? v0)"
        " -> (Tensor, Tensor, Tensor, Tensor)",
    "state_prep":
        "state_prep(Tensor w_raw, Tensor k_raw, Tensor v_raw, Tensor a, Tensor k_k, Tensor k_a, Tensor? v_first,"
        " Tensor? v_gate, int num_heads, int head_dim, bool log_decay) -> (Tensor, Tensor, Tensor, Tensor)",
    "output_prepare":
        "output_prepare(Tensor y, Tensor r, Tensor k, Tensor v, Tensor g, Tensor r_k, Tensor gn_w, Tensor gn_b,"
        " int num_heads, float eps) -> Tensor",
    "seq_shift_mix":
        "seq_shift_mix(Tensor x, Tensor initial_prev, Tensor[] mixes) -> Tensor[]",
}


def _cuda_impls():
    from . import fused_decode_norm_mix as fdm
    from . import fused_lora, fused_output, fused_prefill, fused_time_mix, native_quant_mm8, sm70_quant
    from .fused_recurrent_update import fused_recurrent_output_prepare_raw, fused_recurrent_update
    from .self_chunk_rwkv7 import _run_chunk
    from .fused_recurrent_update import _as_bthn, _check_state

    def update(r, w, k, v, kk, a, state):
        return fused_recurrent_update(r, w, k, v, kk, a, state)

    def update_(r, w, k, v, kk, a, state, out):
        fused_recurrent_update(r, w, k, v, kk, a, state, state_out=state, out=out)

    def prep_raw(r, w_raw, k_raw, v, a, state, g, k_k, k_a, r_k, gn_w, gn_b, eps):
        return fused_recurrent_output_prepare_raw(r, w_raw, k_raw, v, a, state, g, k_k, k_a, r_k, gn_w, gn_b, eps=eps)

    def prep_raw_(r, w_raw, k_raw, v, a, state, g, k_k, k_a, r_k, gn_w, gn_b, eps, out):
        fused_recurrent_output_prepare_raw(r, w_raw, k_raw, v, a, state, g, k_k, k_a, r_k, gn_w, gn_b, eps=eps,
                                           state_out=state, out=out)

    def _bthn(state, *xs):
        _, H, N = _check_state(state)
        return [_as_bthn(x, H, N, name="input")[0] for x in xs]

    def chunk(r, w, k, v, kk, a, state, w_mode):
        r4, w4, k4, v4, kk4, a4 = _bthn(state, r, w, k, v, kk, a)
        y, s = _run_chunk(r4, w4, k4, v4, kk4, a4, state, w_is_log=int(w_mode), chunk=16)
        return y.reshape(r.shape), s

    def chunk_(r, w, k, v, kk, a, state, w_mode, y):
        r4, w4, k4, v4, kk4, a4 = _bthn(state, r, w, k, v, kk, a)
        if not y.is_contiguous() or y.numel() != r4.numel() or y.dtype != r4.dtype:
            raise ValueError("chunk_scan_: y must be contiguous, shaped and typed like r")
        _run_chunk(r4, w4, k4, v4, kk4, a4, state, w_is_log=int(w_mode), chunk=16, state_out=state,
                   out=y.view(r4.shape))

    def mm8(x, w_u8, mx, rx, my, ry):
        return native_quant_mm8.mm8_matmul(x, w_u8, mx, rx, my, ry)

    def mm8_out(x, w_u8, mx, rx, my, ry, out):
        n, m = int(ry.numel()), int(mx.numel())
        if not out.is_contiguous() or out.dtype != x.dtype or out.numel() != x.numel() // n * m:
            raise ValueError("mm8_matmul_out: out must be contiguous [..., M] in x's dtype")
        meta = lambda t: t.reshape(-1).contiguous()
        native_quant_mm8.mm8_matmul_into(x.reshape(-1, n).contiguous(), w_u8, meta(mx), meta(rx), meta(my), meta(ry),
                                         out.view(-1, m))

    def quant8(weight):
        return native_quant_mm8.quantize_mm8(weight)

    def w4g(x, q, scales, out_features, in_features, group_size):
        return sm70_quant.w4_groupwise_linear(x, q, scales, out_features, in_features, group_size=group_size)

    def mix6_(x, previous, nw, nb, mr, mw, mk, mv, ma, mg, eps, out):
        fdm.fused_attn_norm_mix6_decode(x, previous, nw, nb, mr, mw, mk, mv, ma, mg, eps=eps, out=out)

    def ffn_mix_(x, attn_out, previous, nw, nb, mix, eps, mixed):
        fdm.fused_ffn_add_norm_mix_decode(x, attn_out, previous, nw, nb, mix, eps=eps, residual_out=x, mixed=mixed)

    def wavg(xw, xa, xg, xv, w1, a1, g1, v1, w2, a2, g2, v2, w0, a0, v0):
        return tuple(fused_lora.fused_wavg_lora(xw, xa, xg, xv, w1, a1, g1, v1, w2, a2, g2, v2, w0, a0, None, v0))

    def sprep(w_raw, k_raw, v_raw, a, k_k, k_a, v_first, v_gate, num_heads, head_dim, log_decay):
        return fused_prefill.fused_prefill_state_prep(
            w_raw, k_raw, v_raw, a, k_k, k_a, v_first=v_first, v_gate=v_gate, num_heads=num_heads,
            head_dim=head_dim, w_transform="log_decay" if log_decay else "decay")

    def oprep(y, r, k, v, g, r_k, gn_w, gn_b, num_heads, eps):
        N = int(y.shape[-1]) // int(num_heads) if y.dim() >= 2 else 64
        return fused_output.fused_attn_output_prepare(y, r, k, v, g, r_k, gn_w, gn_b, num_heads=num_heads,
                                                      head_dim=N, head_v_dim=N, eps=eps)

    def shift(x, initial_prev, mixes):
        outs, last = fused_time_mix._seq_mix(x, initial_prev, list(mixes), None, None, 0.0)
        return [*outs, last]

    return {
        "fused_recurrent_update": update, "fused_recurrent_update_": update_,
        "fused_recurrent_output_prepare_raw": prep_raw, "fused_recurrent_output_prepare_raw_": prep_raw_,
        "chunk_scan": chunk, "chunk_scan_": chunk_, "mm8_matmul": mm8, "mm8_matmul_out": mm8_out,
        "quantize_mm8": quant8, "w4_groupwise_linear": w4g, "attn_norm_mix6_": mix6_,
        "ffn_add_norm_mix_": ffn_mix_, "wavg_lora": wavg, "state_prep": sprep, "output_prepare": oprep,
        "seq_shift_mix": shift,
    }


def _fake_impls():
    def update(r, w, k, v, kk, a, state):
        return torch.empty_like(r), torch.empty_like(state)

    def none(*args):
        return None

    def prep_raw(r, w_raw, k_raw, v, a, state, g, k_k, k_a, r_k, gn_w, gn_b, eps):
        return torch.empty_like(r), torch.empty_like(state)

    def chunk(r, w, k, v, kk, a, state, w_mode):
        return torch.empty_like(r), torch.empty_like(state)

    def mm8(x, w_u8, mx, rx, my, ry):
        return x.new_empty((*x.shape[:-1], int(mx.numel())))

    def quant8(weight):
        n, m = (int(s) for s in weight.shape)
        return (weight.new_empty((n, m), dtype=torch.uint8), weight.new_empty(m), weight.new_empty(m),
                weight.new_empty((n, 1)), weight.new_empty((n, 1)))

    def w4g(x, q, scales, out_features, in_features, group_size):
        return x.new_empty((*x.shape[:-1], int(out_features)))

    def wavg(xw, xa, xg, xv, w1, a1, g1, v1, w2, a2, g2, v2, w0, a0, v0):
        rows = xw.shape[:-1]
        return tuple(xw.new_empty((*rows, int(u.shape[0]))) for u in (w2, a2, g2, v2))

    def sprep(w_raw, k_raw, v_raw, a, k_k, k_a, v_first, v_gate, num_heads, head_dim, log_decay):
        return (torch.empty_like(k_raw, dtype=torch.float32), torch.empty_like(k_raw), torch.empty_like(v_raw),
                torch.empty_like(k_raw))

    def oprep(y, r, k, v, g, r_k, gn_w, gn_b, num_heads, eps):
        return torch.empty_like(y)

    def shift(x, initial_prev, mixes):
        return [torch.empty_like(x) for _ in mixes] + [x.new_empty((x.shape[0], x.shape[2]))]

    return {
        "fused_recurrent_update": update, "fused_recurrent_update_": none,
        "fused_recurrent_output_prepare_raw": prep_raw, "fused_recurrent_output_prepare_raw_": none,
        "chunk_scan": chunk, "chunk_scan_": none, "mm8_matmul": mm8, "mm8_matmul_out": none,
        "quantize_mm8": quant8, "w4_groupwise_linear": w4g, "attn_norm_mix6_": none, "ffn_add_norm_mix_": none,
        "wavg_lora": wavg, "state_prep": sprep, "output_prepare": oprep, "seq_shift_mix": shift,
    }


def _cpu_refusal(name):
    def impl(*args, **kwargs):
        raise RuntimeError(f"torch.ops.rwkv7mi.{name}: rwkv7mi runs on the GPU only (there is no CPU fallback)")
    return impl


_registered = False
_lib_handle = None


def register() -> None:
    """Define the ``rwkv7mi`` ops (once per process)."""
    global _registered, _lib_handle
    if _registered:
        return
    lib = torch.library.Library(LIB_NAME, "DEF")
    cuda, fake = _cuda_impls(), _fake_impls()
    for name, schema in SCHEMAS.items():
        lib.define(schema)
        lib.impl(name, cuda[name], "CUDA")
        lib.impl(name, _cpu_refusal(name), "CPU")
        torch.library.register_fake(f"{LIB_NAME}::{name}", fake[name], lib=lib)
    _lib_handle = lib
    _registered = True


__all__ = ["SCHEMAS", "register", "LIB_NAME"]
