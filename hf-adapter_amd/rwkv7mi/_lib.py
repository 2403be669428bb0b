"""ctypes binding of librwkv7mi.so (the gfx950 C ABI declared in include/rwkv7mi.h).

The library is loaded after torch so that it binds to the HIP runtime torch
already mapped (both carry the soname libamdhip64.so.7).  There is no fallback:
if the library is missing every operator raises RuntimeError.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "librwkv7mi.so"

F32, F16, BF16 = 0, 1, 2
EPI_NONE, EPI_RELU2, EPI_RESIDUAL = 0, 1, 2
PREP_A_RAW, PREP_VGATE_RAW, PREP_W_DECAY = 1, 2, 4

_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_c_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/rwkv7mi.h
SIGNATURES = {
    "rwkv7mi_last_error": (ctypes.c_char_p, []),
    "rwkv7mi_abi_version": (_i32, []),
    "rwkv7mi_wkv7_decode_update": (_i32, [_c_p] * 8 + [_c_p, _i64, _i64, _i64, _i32, _i32, _c_p]),
    "rwkv7mi_wkv7_decode_output_prepare": (
        _i32,
        [_c_p] * 8 + [_c_p] * 5 + [_i64, _i64, _i64, _f32, _i32, _i32, _i32, _c_p],
    ),
    "rwkv7mi_wkv7_decode_output_prepare_raw": (
        _i32,
        [_c_p] * 7 + [_c_p] * 7 + [_c_p, _c_p, _i32, _i64, _i64, _i64, _f32, _i32, _i32, _c_p],
    ),
    "rwkv7mi_wkv7_scan": (_i32, [_c_p] * 9 + [_i64, _i64, _i64, _i64, _i32, _i32, _c_p]),
    "rwkv7mi_wkv7_chunk_prefill": (
        _i32,
        [_c_p] * 9 + [_i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _c_p],
    ),
    "rwkv7mi_wkv7_chunk_status": (_i32, [_i32, ctypes.POINTER(_i32)]),
    "rwkv7mi_wkv7_fp16_decode_output_prepare_raw": (
        _i32,
        [_c_p] * 12 + [_c_p, _i32, _c_p, _c_p, _c_p, _i32, _i64, _i64, _i64, _f32, _c_p],
    ),
    "rwkv7mi_wkv7_fp16_decode_lora_output_prepare": (
        _i32,
        [_c_p] * 4 + [_i64] + [_c_p] * 5 + [_i64, _i64] + [_c_p] * 7 + [_i32, _c_p, _c_p, _i32, _i64, _i64, _i64, _f32,
                                                                         _c_p],
    ),
    "rwkv7mi_wkv7_fp16_sequence": (_i32, [_c_p] * 10 + [_i64, _i64, _i64, _i64, _c_p]),
    "rwkv7mi_mm8_pack": (_i32, [_c_p, _i64, _i64, _i32, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p]),
    "rwkv7mi_mm8_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "rwkv7mi_mm8_matmul": (
        _i32,
        [_c_p] * 9 + [_i64, _i64, _i64, _i32, _i32, _i32, _c_p, _sz, _c_p],
    ),
    "rwkv7mi_mm8_dequant": (_i32, [_c_p] * 6 + [_i64, _i64, _i32, _i32, _c_p]),
    "rwkv7mi_mm8_pack_t": (_i32, [_c_p, _i64, _i64, _i32, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p]),
    "rwkv7mi_mm8t_matmul": (_i32, [_c_p] * 9 + [_i64, _i64, _i64, _i32, _i32, _i32, _c_p]),
    "rwkv7mi_mm8t_matmul_multi": (_i32, [_i32] + [_c_p] * 10 + [_i64, _i64, _i64, _i32, _i32, _c_p]),
    "rwkv7mi_mm8t_matmul_workspace_bytes": (_sz, [_i32, _i64, _i64, _i64]),
    "rwkv7mi_mm8t_matmul_multi_ws": (_i32, [_i32] + [_c_p] * 10 + [_i64, _i64, _i64, _i32, _i32, _c_p, _sz, _c_p]),
    "rwkv7mi_mm8t_gemm_multi_lora": (
        _i32, [_i32] + [_c_p] * 10 + [_i64, _i64, _i64, _i32, _i32, _i32, _c_p, _sz, _i64, _c_p, _c_p, _c_p, _i64,
                                      _c_p, _sz, _c_p]),
    "rwkv7mi_mm8t_matmul_multi_lora": (
        _i32, [_i32] + [_c_p] * 10 + [_i64, _i64, _i64, _i32, _i32, _i64, _c_p, _c_p, _c_p, _i64, _c_p, _sz, _c_p]),
    "rwkv7mi_mm8t_dequant": (_i32, [_c_p] * 6 + [_i64, _i64, _i32, _i32, _c_p]),
    "rwkv7mi_mm8t_gemm_workspace_bytes": (_sz, [_i32, _i64, _i64, _i64, _i32]),
    "rwkv7mi_mm8t_gemm_multi": (_i32, [_i32] + [_c_p] * 10 + [_i64, _i64, _i64, _i32, _i32, _i32, _c_p, _sz, _c_p]),
    "rwkv7mi_mm8t_gemm_multi_noalloc": (_i32, [_i32] + [_c_p] * 10 + [_i64, _i64, _i64, _i32, _i32, _i32, _c_p]),
    "rwkv7mi_mm8t_gemm_prefill": (_i32, [_i32] + [_c_p] * 10 + [_i64, _i64, _i64, _i32, _i32, _c_p]),
    "rwkv7mi_mm8t_gemm_prefill_ws": (_i32, [_i32] + [_c_p] * 10 + [_i64, _i64, _i64, _i32, _i32, _c_p, _i64, _c_p]),
    "rwkv7mi_mm8t_gemm_prefill_ws_bytes": (_i64, [_i32, _i64, _i64]),
    "rwkv7mi_dense_gemm_prefill_ws": (_i32, [_i32] + [_c_p] * 6 + [_i64, _i64, _i64, _i32, _c_p, _i64, _c_p]),
    "rwkv7mi_mm8t_blocked_bytes": (_sz, [_i64, _i64]),
    "rwkv7mi_mm8t_block": (_i32, [_c_p, _i64, _i64, _i64, _i64, _c_p, _c_p]),
    "rwkv7mi_mm8t_unblock": (_i32, [_c_p, _i64, _i64, _c_p, _i64, _i64, _c_p]),
    "rwkv7mi_mm8t_lnmix_multi": (
        _i32,
        [_i32] + [_c_p] * 4 + [_f32] + [_c_p] * 8 + [_c_p, _i32, _c_p, _c_p, _c_p, _c_p, _c_p]
        + [_i64, _i64, _i64, _i32, _c_p],
    ),
    "rwkv7mi_mm4_pack": (_i32, [_c_p, _i64, _i64, _i32, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p]),
    "rwkv7mi_mm4_pack_t": (_i32, [_c_p, _i64, _i64, _i32, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p]),
    "rwkv7mi_mm4t_matmul": (_i32, [_c_p] * 9 + [_i64, _i64, _i64, _i32, _i32, _i32, _c_p]),
    "rwkv7mi_mm4_dequant": (_i32, [_c_p] * 6 + [_i64, _i64, _i32, _i32, _c_p]),
    "rwkv7mi_mm4_matmul_workspace_bytes": (_sz, [_i64, _i64]),
    "rwkv7mi_mm4_matmul": (_i32, [_c_p] * 9 + [_i64, _i64, _i64, _i64, _i32, _i32, _i32, _c_p, _sz, _c_p]),
    "rwkv7mi_attn_mix_lora": (
        _i32, [_c_p] * 10 + [_i64, _c_p, _c_p, _c_p, _c_p, _i64, _i64, _f32, _i32, _i32, _c_p]),
    "rwkv7mi_attn_mix_lora_chunks": (_i32, [_i64]),
    "rwkv7mi_slot_copy": (_i32, [_c_p, _i64, _i64, _c_p, _c_p, _i64, _i64, _c_p, _c_p, _i64, _i64, _i64, _c_p]),
    "rwkv7mi_argmax_rows": (_i32, [_c_p, _i64, _i64, _i64, _i32, _c_p, _c_p, _c_p]),
    "rwkv7mi_argmax_workspace_bytes": (_sz, [_i64, _i64, _i32]),
    "rwkv7mi_argmax_rows_ws": (_i32, [_c_p, _i64, _i64, _i64, _i32, _c_p, _c_p, _c_p, _sz, _c_p]),
    "rwkv7mi_mm8t_matmul_partials": (_i32, [_c_p] * 6 + [_i64, _i64, _i64, _i32, _i32, _c_p, _sz, ctypes.POINTER(_i32), _c_p]),
    "rwkv7mi_attn_norm_mix6_parts": (_i32, [_c_p] * 6 + [_i64, _c_p, _i64, _i64, _i64, _i64, _f32, _i32, _i32, _c_p]),
    "rwkv7mi_lora_workspace_bytes": (_sz, [_i64, _c_p, _i64, _i64]),
    "rwkv7mi_lora_multi": (_i32, [_i64] + [_c_p] * 8 + [_i64, _i64, _i64, _i32, _c_p, _sz, _c_p]),
    "rwkv7mi_lora_down_multi": (_i32, [_i64] + [_c_p] * 4 + [_i64, _i64, _i32, _c_p, _sz, _c_p]),
    "rwkv7mi_wkv7_decode_lora_output_prepare": (
        _i32,
        [_c_p] * 4 + [_i64] + [_c_p] * 5 + [_i64, _i64] + [_c_p] * 9 + [_i32, _i64, _i64, _i64, _f32, _i32, _i32, _c_p],
    ),
    "rwkv7mi_w4g_pack": (_i32, [_c_p, _i64, _i64, _i64, _i32, _c_p, _c_p, _c_p]),
    "rwkv7mi_w4a_pack": (_i32, [_c_p, _i64, _i64, _i64, _i32, _c_p, _c_p, _c_p, _c_p]),
    "rwkv7mi_w4a_matmul": (_i32, [_c_p] * 7 + [_i64, _i64, _i64, _i64, _i32, _i32, _i32, _c_p]),
    "rwkv7mi_w4g_matmul": (
        _i32,
        [_c_p] * 6 + [_i64, _i64, _i64, _i64, _i32, _i32, _i32, _c_p],
    ),
    "rwkv7mi_attn_norm_mix6": (
        _i32, [_c_p] * 8 + [_i64, _i64, _i64, _f32, _i32, _i32, _c_p],
    ),
    "rwkv7mi_ffn_add_norm_mix": (_i32, [_c_p] * 8 + [_i64, _i64, _f32, _i32, _i32, _c_p]),
    "rwkv7mi_seq_norm_mix": (_i32, [_c_p] * 7 + [_i64, _i64, _i64, _i64, _f32, _i32, _i32, _c_p]),
    "rwkv7mi_layer_norm": (_i32, [_c_p] * 4 + [_i64, _i64, _f32, _i32, _i32, _c_p]),
    "rwkv7mi_dense_multi": (_i32, [_c_p] * 7 + [_i64, _i64, _i32, _c_p]),
    "rwkv7mi_state_prep": (_i32, [_c_p] * 12 + [_i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _c_p]),
    "rwkv7mi_output_prepare": (_i32, [_c_p] * 9 + [_i64, _i64, _i64, _f32, _i32, _i32, _c_p]),
}

_lock = threading.Lock()
_lib = None


def load():
    """Load and bind the library (once).  Raises RuntimeError if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"rwkv7mi native library not built: {LIB_PATH} is missing "
                "(run python hf-adapter_amd/build.py)"
            )
        lib = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def declared_symbols(header: Path) -> list[str]:
    """Names of the functions declared in include/rwkv7mi.h."""
    import re

    text = header.read_text()
    return sorted(set(re.findall(r"\b(rwkv7mi_[a-z0-9_]+)\s*\(", text)))


def call(name: str, *args):
    lib = load()
    fn = getattr(lib, name)
    rc = fn(*args)
    if rc != 0:
        msg = lib.rwkv7mi_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(f"{name}: {msg}")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def ptr_array(tensors) -> ctypes.Array:
    """A C array of device pointers (NULL for None)."""
    return (ctypes.c_void_p * len(tensors))(*[None if t is None else t.data_ptr() for t in tensors])


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}") from None


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(*tensors: torch.Tensor | None, name: str) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                f"{name}: rwkv7mi runs on the GPU only; got a {t.device} tensor "
                "(there is no CPU fallback)"
            )
    load()


__all__ = [
    "F32", "F16", "BF16", "EPI_NONE", "EPI_RELU2", "EPI_RESIDUAL", "LIB_PATH", "SIGNATURES",
    "load", "call", "dtype_code", "ptr", "stream_of", "require_gpu", "declared_symbols",
]
