"""GPU parity of the many-row MM8 tile GEMM (17..256 rows over blocked
weights): against the fp64 oracle on the dequantised weights for ragged and
model shapes, every split count (including uneven ones), grouped launches,
bias / relu^2 / aliased-residual epilogues, all activation and metadata
dtypes, repeat determinism, the workspace contract, and a 64-row decode-size
R/K/V group at the 7.2B shapes."""
from __future__ import annotations

import types

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _cuda(x, dtype):
    return torch.tensor(np.asarray(x), dtype=dtype, device="cuda")


def _np(t):
    return t.detach().cpu().numpy()


def _rel_err(got, ref):
    return np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)


def _packed(rng, I, O, dtype=torch.float16, bias=False):
    from rwkv7mi.native_quant_mm8 import quantize_mm8_blocked

    Wl = _cuda(rng.standard_normal((O, I)) * 0.02, dtype)
    w_blk, mx, rx, my, ry = quantize_mm8_blocked(Wl)
    b = _cuda(rng.standard_normal(O) * 0.1, dtype) if bias else None
    return types.SimpleNamespace(w_blk=w_blk, mx=mx, rx=rx, my=my.reshape(-1), ry=ry.reshape(-1), bias=b,
                                 in_features=I, out_features=O)


def _ref(oracle, x, mod):
    from rwkv7mi.native_quant_mm8 import mm8_unblock

    w_u8 = mm8_unblock(mod.w_blk, mod.in_features, mod.out_features)
    meta = [_np(t.float()) for t in (mod.mx, mod.rx, mod.my, mod.ry)]
    y = oracle.mm8_matmul(_np(x.float()).astype(np.float64), _np(w_u8), *meta)
    if mod.bias is not None:
        y = y + _np(mod.bias.float()).astype(np.float64)
    return y


@pytest.mark.parametrize("IO", [(4096, 4096), (16384, 512), (144, 40), (1024, 65), (2064, 200), (16, 16)])
@pytest.mark.parametrize("rows", [17, 33, 64, 100, 256])
def test_mm8g_matches_oracle(oracle, IO, rows):
    from rwkv7mi.native_quant_mm8 import mm8_matmul

    I, O = IO
    rng = np.random.default_rng(I + 7 * O + rows)
    mod = _packed(rng, I, O)
    x = _cuda(rng.standard_normal((rows, I)), torch.float16)
    args = (mod.w_blk, mod.mx, mod.rx, mod.my, mod.ry)
    y = mm8_matmul(x, *args)
    y2 = mm8_matmul(x, *args)
    torch.cuda.synchronize()
    err = _rel_err(_np(y).astype(np.float64), _ref(oracle, x, mod))
    assert err <= 2e-3, (IO, rows, err)
    assert torch.equal(y, y2), "repeated calls must be bit-identical"


@pytest.mark.parametrize("splits", [1, 2, 3, 5, 8, 0])
def test_mm8g_split_counts(oracle, splits):
    """Every split count, uneven ones included (21 K blocks over 5 or 8 splits),
    agrees with the oracle; the same count repeats bit for bit.  A split holds
    at most 8 K blocks, so one or two splits take narrower inputs."""
    from rwkv7mi.native_quant_mm8 import mm8_gemm_multi_into

    O, rows = 384, 64
    I = {1: 1024, 2: 2048}.get(splits, 2688)
    rng = np.random.default_rng(100 + splits)
    mod = _packed(rng, I, O)
    x = _cuda(rng.standard_normal((rows, I)), torch.float16)
    y = torch.empty(rows, O, device="cuda", dtype=torch.float16)
    y2 = torch.empty_like(y)
    mm8_gemm_multi_into([x], [mod], [y], splits=splits)
    mm8_gemm_multi_into([x], [mod], [y2], splits=splits)
    torch.cuda.synchronize()
    assert _rel_err(_np(y).astype(np.float64), _ref(oracle, x, mod)) <= 2e-3
    assert torch.equal(y, y2)


@pytest.mark.parametrize("rows", [20, 64])
def test_mm8g_multi_equals_single(oracle, rows):
    from rwkv7mi.native_quant_mm8 import mm8_gemm_multi_into

    rng = np.random.default_rng(rows + 1)
    I, O = 1024, 640
    mods = [_packed(rng, I, O, bias=(p == 1)) for p in range(3)]
    xs = [_cuda(rng.standard_normal((rows, I)), torch.float16) for _ in range(3)]
    outs = [torch.empty(rows, O, device="cuda", dtype=torch.float16) for _ in range(3)]
    mm8_gemm_multi_into(xs, mods, outs, splits=4)
    single = []
    for m, x in zip(mods, xs):
        o = torch.empty(rows, O, device="cuda", dtype=torch.float16)
        mm8_gemm_multi_into([x], [m], [o], splits=4)
        single.append(o)
    torch.cuda.synchronize()
    for a, b, m, x in zip(outs, single, mods, xs):
        assert torch.equal(a, b)
        assert _rel_err(_np(a).astype(np.float64), _ref(oracle, x, m)) <= 2e-3


@pytest.mark.parametrize("splits", [1, 4])
def test_mm8g_epilogues(oracle, splits):
    """bias, relu^2 and a residual add whose output aliases the residual."""
    from rwkv7mi import _lib
    from rwkv7mi.native_quant_mm8 import mm8_gemm_multi_into

    rng = np.random.default_rng(9 + splits)
    I, O, rows = 1024, 4096, 48
    mod = _packed(rng, I, O, bias=True)
    x = _cuda(rng.standard_normal((rows, I)), torch.float16)
    res = _cuda(rng.standard_normal((rows, O)), torch.float16)
    base = _ref(oracle, x, mod)
    y = torch.empty(rows, O, device="cuda", dtype=torch.float16)
    r2 = torch.empty_like(y)
    acc = res.clone()
    mm8_gemm_multi_into([x], [mod], [y], splits=splits)
    mm8_gemm_multi_into([x], [mod], [r2], epilogues=[_lib.EPI_RELU2], splits=splits)
    mm8_gemm_multi_into([x], [mod], [acc], residuals=[acc], epilogues=[_lib.EPI_RESIDUAL], splits=splits)
    torch.cuda.synchronize()
    assert np.abs(_np(y) - base).max() <= 2e-3 * np.abs(base).max()
    rr = np.maximum(base, 0) ** 2
    assert np.abs(_np(r2) - rr).max() <= 4e-3 * np.abs(rr).max()
    add = base + _np(res).astype(np.float64)
    assert np.abs(_np(acc) - add).max() <= 2e-3 * np.abs(add).max()


@pytest.mark.parametrize("act", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("meta", [torch.float16, torch.float32, torch.bfloat16])
def test_mm8g_dtypes(oracle, act, meta):
    from rwkv7mi.native_quant_mm8 import mm8_gemm_multi_into

    I, O, rows = 2048, 768, 40
    rng = np.random.default_rng(11)
    mod = _packed(rng, I, O, dtype=meta)
    x = _cuda(rng.standard_normal((rows, I)), act)
    y = torch.empty(rows, O, device="cuda", dtype=act)
    mm8_gemm_multi_into([x], [mod], [y])
    torch.cuda.synchronize()
    # fp32 activations stage x' as fp16 hi + lo (as the <= 16-row GEMV does):
    # ~1e-6 typical, up to a few 1e-5 on rows whose lo parts sit just below
    # the fp16 normal range (measured); fp16-rounded x' alone would be ~2e-4
    tol = {torch.float16: 2e-3, torch.float32: 1e-4, torch.bfloat16: 8e-3}[act]
    err = _rel_err(_np(y.float()).astype(np.float64), _ref(oracle, x, mod))
    assert err <= tol, (act, meta, err)


def test_mm8g_rkv_7p2b_bsz64(oracle):
    """The bsz-64 decode R/K/V launch at the 7.2B shapes (4096 x 4096, three
    problems, the automatic split count)."""
    from rwkv7mi.native_quant_mm8 import mm8_gemm_multi_into

    rng = np.random.default_rng(64)
    I = O = 4096
    rows = 64
    mods = [_packed(rng, I, O) for _ in range(3)]
    xs = [_cuda(rng.standard_normal((rows, I)), torch.float16) for _ in range(3)]
    outs = [torch.empty(rows, O, device="cuda", dtype=torch.float16) for _ in range(3)]
    mm8_gemm_multi_into(xs, mods, outs)
    torch.cuda.synchronize()
    for o, m, x in zip(outs, mods, xs):
        assert _rel_err(_np(o).astype(np.float64), _ref(oracle, x, m)) <= 2e-3


def test_mm8g_workspace_contract():
    from rwkv7mi import _lib
    from rwkv7mi.native_quant_mm8 import mm8_gemm_workspace_bytes

    rng = np.random.default_rng(3)
    I, O, rows = 2048, 256, 32
    mod = _packed(rng, I, O)
    need = mm8_gemm_workspace_bytes(1, rows, I, O, 4)
    assert need >= 4 * rows * O * 4 + 2 * rows * I * 2  # partials and x' (hi and lo halves)
    one = mm8_gemm_workspace_bytes(1, rows, 1024, O, 1)  # x' and row sums only
    assert 2 * rows * 1024 * 2 < one <= 2 * rows * 1024 * 2 + 1024
    x = _cuda(rng.standard_normal((rows, I)), torch.float16)
    y = torch.empty(rows, O, device="cuda", dtype=torch.float16)
    ws = torch.empty(need - 256, device="cuda", dtype=torch.uint8)
    arr = _lib.ptr_array
    args = [1, arr([x]), arr([mod.w_blk]), arr([mod.mx]), arr([mod.rx]), arr([mod.my]), arr([mod.ry]), None, None,
            arr([y]), (__import__("ctypes").c_int * 1)(0), rows, I, O, _lib.F16, _lib.F16, 4]
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.call("rwkv7mi_mm8t_gemm_multi", *args, _lib.ptr(ws), int(ws.numel()), _lib.stream_of(x))
    with pytest.raises(ValueError, match="1024 inputs"):
        _lib.call("rwkv7mi_mm8t_gemm_multi", *args[:-1], 1, None, 0, _lib.stream_of(x))
    torch.cuda.synchronize()
