"""C-ABI library checks that need no GPU: it loads, exports every symbol the
header declares, and the Python wrappers reject CPU tensors and bad shapes
before any device call."""
from __future__ import annotations

import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "rwkv7mi.h"


def test_library_exports_every_declared_symbol():
    from rwkv7mi import _lib

    lib = _lib.load()
    names = _lib.declared_symbols(HEADER)
    assert len(names) >= 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.rwkv7mi_abi_version() == 100


def test_python_signatures_cover_header():
    from rwkv7mi import _lib

    names = set(_lib.declared_symbols(HEADER))
    assert names <= set(_lib.SIGNATURES), sorted(names - set(_lib.SIGNATURES))


def test_header_has_no_torch_types():
    text = HEADER.read_text()
    assert not re.search(r"\b(at::|torch::|Tensor)\b", text)


def test_cpu_tensors_raise_instead_of_falling_back():
    from rwkv7mi import fused_recurrent_update

    B, H, N = 1, 2, 64
    vec = [torch.zeros(B, H, N) for _ in range(6)]
    state = torch.zeros(B, H, N, N)
    with pytest.raises(RuntimeError, match="GPU only"):
        fused_recurrent_update(*vec, state)


def test_shape_errors_are_value_errors():
    from rwkv7mi import fused_recurrent_update, fused_recurrent_scan

    state = torch.zeros(1, 2, 64, 64)
    with pytest.raises(ValueError):
        fused_recurrent_update(*[torch.zeros(1, 3, 64) for _ in range(6)], state)
    with pytest.raises(ValueError):
        fused_recurrent_update(*[torch.zeros(1, 2, 64) for _ in range(6)], torch.zeros(1, 2, 64, 32))
    with pytest.raises(ValueError):
        fused_recurrent_scan(*[torch.zeros(1, 4, 2, 32) for _ in range(6)], torch.zeros(1, 2, 32, 32))


def test_policy_matches_reference_aliases():
    from rwkv7mi.native_quant_policy import normalize_native_mm_policy, should_quantize_linear

    assert normalize_native_mm_policy("lm-head-only") == "speed"
    assert normalize_native_mm_policy(None) == "memory"
    with pytest.raises(ValueError):
        normalize_native_mm_policy("bogus")
    assert should_quantize_linear("model.layers.0.ffn.key", 16_000_000, min_params=8_000_000)
    assert not should_quantize_linear("model.layers.0.ffn.key", 16_000_000, min_params=8_000_000, policy="speed")
    assert should_quantize_linear("lm_head", 16_000_000, min_params=8_000_000, policy="speed")
    assert not should_quantize_linear("lm_head", 100, min_params=8_000_000, policy="speed")
