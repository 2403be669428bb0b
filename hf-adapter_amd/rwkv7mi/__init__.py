"""rwkv7mi — MI355X (gfx950) native RWKV-7 inference hot path.

Drop-in operators and quantized modules with the names and signatures of the
reference adapter (rwkv-rs/hf-adapter 0.8.1), each backed by a hand-written
HIP kernel in librwkv7mi.so (C ABI: include/rwkv7mi.h).  GPU tensors only.
"""
from __future__ import annotations

from . import _lib
from .fused_recurrent_update import (
    fused_recurrent_output_prepare,
    fused_recurrent_output_prepare_raw,
    fused_recurrent_scan,
    fused_recurrent_scan_clampw,
    fused_recurrent_scan_output_prepare,
    fused_recurrent_scan_state_prep,
    fused_recurrent_update,
)
from .self_chunk_rwkv7 import dplr_chunk_scan, self_chunk_rwkv7
from .native_quant_mm8 import MM8Linear, mm8_matmul, mm8_matmul_triton, quantize_mm8, quantize_model_mm8
from .native_quant_mm4 import (
    MM4Linear,
    dequantize_mm4,
    mm4_matmul,
    mm4_matmul_triton,
    quantize_mm4,
    quantize_model_mm4,
)
from .sm70_quant import quantize_w4_groupwise, w4_groupwise_linear
from .native_wkv_fp16 import (
    native_fp16_recurrent_available,
    native_fp16_recurrent_build_error,
    native_fp16_recurrent_output_prepare_raw,
    native_fp16_recurrent_should_use,
    native_fp16_sequence,
)
from .sampling import argmax_rows
from . import ops as _ops

_ops.register()  # torch.ops.rwkv7mi.*

__all__ = [
    "fused_recurrent_update",
    "fused_recurrent_output_prepare",
    "fused_recurrent_output_prepare_raw",
    "fused_recurrent_scan",
    "fused_recurrent_scan_clampw",
    "fused_recurrent_scan_state_prep",
    "fused_recurrent_scan_output_prepare",
    "self_chunk_rwkv7",
    "dplr_chunk_scan",
    "quantize_mm8",
    "mm8_matmul",
    "mm8_matmul_triton",
    "MM8Linear",
    "quantize_model_mm8",
    "quantize_mm4",
    "dequantize_mm4",
    "mm4_matmul",
    "mm4_matmul_triton",
    "MM4Linear",
    "quantize_model_mm4",
    "quantize_w4_groupwise",
    "w4_groupwise_linear",
    "argmax_rows",
    "native_fp16_recurrent_should_use",
    "native_fp16_recurrent_available",
    "native_fp16_recurrent_build_error",
    "native_fp16_recurrent_output_prepare_raw",
    "native_fp16_sequence",
]
