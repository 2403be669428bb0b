"""The allocation-free many-row MM8 GEMM (rwkv7mi_mm8t_gemm_multi_noalloc)
against the workspace entry point (rwkv7mi_mm8t_gemm_multi), both called
through the C ABI: bit-identical outputs on two calls in a row, the second one
smaller, so leftovers of the first call in the shared scratch cannot leak into
the second; a call beyond the fixed scratch is refused with RWKV7MI_ESIZE
before anything runs.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _mods(nprob, I, O, seed):
    from rwkv7mi import MM8Linear

    torch.manual_seed(seed)
    return [MM8Linear(torch.nn.Linear(I, O, bias=False).cuda().half()) for _ in range(nprob)]


def _args(xs, mods, outs, epis, residuals):
    from rwkv7mi import _lib

    arr = _lib.ptr_array
    k = len(mods)
    return (k, arr(xs), arr([m.w_blk for m in mods]), arr([m.mx for m in mods]), arr([m.rx for m in mods]),
            arr([m.my.reshape(-1) for m in mods]), arr([m.ry.reshape(-1) for m in mods]), arr([None] * k),
            arr(residuals), arr(outs), (ctypes.c_int * k)(*epis))


def _run_pair(nprob, rows, I, O, seed, epis):
    from rwkv7mi import _lib

    mods = _mods(nprob, I, O, seed)
    g = torch.Generator(device="cuda").manual_seed(seed)
    xs = [torch.randn(rows, I, device="cuda", dtype=torch.float16, generator=g) for _ in range(nprob)]
    res = [torch.randn(rows, O, device="cuda", dtype=torch.float16, generator=g) if e == _lib.EPI_RESIDUAL else None
           for e in epis]
    ref = [torch.empty(rows, O, device="cuda", dtype=torch.float16) for _ in range(nprob)]
    got = [torch.full((rows, O), float("nan"), device="cuda", dtype=torch.float16) for _ in range(nprob)]
    need = int(_lib.load().rwkv7mi_mm8t_gemm_workspace_bytes(nprob, rows, I, O, 0))
    ws = torch.empty(need + 256, device="cuda", dtype=torch.uint8)
    off = (-ws.data_ptr()) % 256
    stream = _lib.stream_of(xs[0])
    _lib.call("rwkv7mi_mm8t_gemm_multi", *_args(xs, mods, ref, epis, res), rows, I, O, _lib.F16, _lib.F16, 0,
              ctypes.c_void_p(ws.data_ptr() + off), need, stream)
    _lib.call("rwkv7mi_mm8t_gemm_multi_noalloc", *_args(xs, mods, got, epis, res), rows, I, O, _lib.F16, _lib.F16,
              0, stream)
    torch.cuda.synchronize()
    for a, b in zip(got, ref):
        assert torch.isfinite(b).all()
        assert torch.equal(a, b)


def test_noalloc_gemm_equals_workspace_gemm_two_calls():
    from rwkv7mi import _lib

    print("no-alloc GEMM: call 1 (3 x [64, 4096] @ 4096x4096)", flush=True)
    _run_pair(3, 64, 4096, 4096, 1, [_lib.EPI_NONE, _lib.EPI_RELU2, _lib.EPI_RESIDUAL])
    print("no-alloc GEMM: call 2, smaller (1 x [24, 2048] @ 2048x1024)", flush=True)
    _run_pair(1, 24, 2048, 1024, 2, [_lib.EPI_RESIDUAL])


def test_noalloc_gemm_split_k_shape():
    """16384 inputs: sixteen K splits, the partials in the scratch."""
    from rwkv7mi import _lib

    print("no-alloc GEMM: [40, 16384] @ 16384x2048", flush=True)
    _run_pair(1, 40, 16384, 2048, 3, [_lib.EPI_NONE])


def test_noalloc_gemm_rejects_oversize():
    from rwkv7mi import _lib

    need = int(_lib.load().rwkv7mi_mm8t_gemm_workspace_bytes(1, 256, 4096, 65536, 0))
    assert need > (80 << 20)
    dummy = [torch.empty(16, device="cuda", dtype=torch.float16)]
    arr = _lib.ptr_array
    rc = _lib.load().rwkv7mi_mm8t_gemm_multi_noalloc(
        1, arr(dummy), arr(dummy), arr(dummy), arr(dummy), arr(dummy), arr(dummy), arr([None]), arr([None]),
        arr(dummy), (ctypes.c_int * 1)(0), 256, 4096, 65536, _lib.F16, _lib.F16, 0, _lib.stream_of(dummy[0]))
    assert rc == -3
    assert b"scratch" in _lib.load().rwkv7mi_last_error()
