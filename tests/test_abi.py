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


def _up256(v):
    return (v + 255) & ~255


@pytest.mark.parametrize("nprob", [1, 3, 4])
def test_mm8g_workspace_covers_every_buffer_the_kernels_index(nprob):
    """The many-row MM8 GEMM indexes its workspace as x' hi and lo halves
    [nprob][rows][ceil(I/128)*128] fp16, row sums [nprob][rows][3] fp32 and,
    with S > 1 K splits, partials [S][nprob][rows][O] fp32 (rows unpadded: the
    tile kernels mask rows beyond the last).  The size function must cover all
    of it for every split count a launch can take: explicit S, and the automatic
    one (the fewest, a power of two, that keeps a split within 8 blocks of
    128 inputs), over odd rows (rows % 64 in 1..32 and 33..63) and ragged I / O."""
    from rwkv7mi import _lib

    lib = _lib.load()
    size = lib.rwkv7mi_mm8t_gemm_workspace_bytes
    for rows in (17, 33, 64, 65, 96, 100, 127, 200, 256):
        for I, O in ((4096, 4096), (16384, 4096), (4096, 16384), (1040, 272), (2048, 65536)):
            KB = -(-I // 128)
            auto = 1
            while auto < KB and -(-KB // auto) > 8:
                auto *= 2
            for S in sorted({1, 2, auto, min(KB, 2 * auto), KB}):
                need = (2 * _up256(nprob * rows * KB * 128 * 2) + _up256(nprob * rows * 3 * 4)
                        + (_up256(S * nprob * rows * O * 4) if S > 1 else 0))
                got = size(nprob, rows, I, O, S)
                assert got >= need, (nprob, rows, I, O, S, got, need)
            need_auto = (2 * _up256(nprob * rows * KB * 128 * 2) + _up256(nprob * rows * 3 * 4)
                         + (_up256(auto * nprob * rows * O * 4) if auto > 1 else 0))
            assert size(nprob, rows, I, O, 0) >= need_auto, (nprob, rows, I, O)
    assert size(0, 64, 4096, 4096, 0) == 0 and size(5, 64, 4096, 4096, 0) == 0


def test_split_workspaces_grow_with_rows_and_outputs():
    """Every workspace-size function is monotone in rows and outputs, so a
    slot reserved for the largest call of a model covers its smaller ones."""
    import ctypes

    from rwkv7mi import _lib

    lib = _lib.load()
    t = lib.rwkv7mi_mm8t_matmul_workspace_bytes
    g = lib.rwkv7mi_mm8t_gemm_workspace_bytes
    ranks = (ctypes.c_int64 * 4)(64, 64, 128, 32)
    for I in (4096, 16384):
        prev = 0
        for rows in range(1, 17):
            cur = t(1, rows, I, 4096)
            assert cur >= prev, (I, rows)
            prev = cur
        assert t(1, 16, I, 4096) <= t(1, 16, I, 8192)
        prev = 0
        for rows in range(17, 257, 7):
            cur = g(3, rows, I, 4096, 0)
            assert cur >= prev and cur <= g(3, rows, I, 8192, 0), (I, rows)
            prev = cur
    prev = 0
    for rows in (1, 2, 8, 16, 33, 64, 65, 200):
        cur = lib.rwkv7mi_lora_workspace_bytes(4, ranks, rows, 4096)
        assert cur >= prev and cur >= 4 * min(rows, 64) * (64 + 64 + 128 + 32), rows
        prev = cur
