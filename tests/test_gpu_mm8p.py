"""GPU parity of the prefill MM8 GEMMs (more than 256 rows over blocked
weights): the route that materialises the fp16 dequantised weight in MFMA
operand order (its workspace bit-equal to rwkv7mi_mm8_dequant) and the
in-register dequantising entry, against the fp64 oracle on the dequantised
weights for ragged rows / columns and in_features that end mid-tile, grouped
launches, bias / relu^2 / residual epilogues, the non-fp16 chunked route, and
the module routes that take it."""
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


# fp16 output rounding (2^-11) plus the fp16 rounding of (w - 128) ry in the
# B operand (the same rounding the reference's materialised fp16 weight has)
TOL = 3e-3


@pytest.mark.parametrize("IO,rows", [(io, r) for io in [(4096, 4096), (1024, 300), (144, 40), (2064, 520),
                                                        (16384, 256), (80, 16)] for r in (257, 600, 1024)]
                         + [((4096, 16384), 300), ((16384, 4096), 300), ((4096, 16384), 1100)])
def test_mm8p_matches_oracle(oracle, IO, rows):
    from rwkv7mi.native_quant_mm8 import mm8_gemm_prefill_multi_into

    I, O = IO
    rng = np.random.default_rng(I + O + rows)
    mod = _packed(rng, I, O)
    x = _cuda(rng.standard_normal((rows, I)), torch.float16)
    y = torch.full((rows, O), float("nan"), device="cuda", dtype=torch.float16)
    print(f"mm8p: I={I} O={O} rows={rows}", flush=True)
    mm8_gemm_prefill_multi_into([x], [mod], [y])
    torch.cuda.synchronize()
    err = _rel_err(_np(y).astype(np.float64), _ref(oracle, x, mod))
    assert err <= TOL, (IO, rows, err)


def test_mm8p_multi_and_epilogues(oracle):
    from rwkv7mi import _lib
    from rwkv7mi.native_quant_mm8 import mm8_gemm_prefill_multi_into

    I, O, rows = 1024, 784, 700
    rng = np.random.default_rng(7)
    mods = [_packed(rng, I, O, bias=True) for _ in range(3)]
    xs = [_cuda(rng.standard_normal((rows, I)), torch.float16) for _ in range(3)]
    outs = [torch.empty(rows, O, device="cuda", dtype=torch.float16) for _ in range(3)]
    res = _cuda(rng.standard_normal((rows, O)), torch.float16)
    want_res = _np(res).astype(np.float64)
    print("mm8p: three problems, none / relu^2 / residual in place", flush=True)
    mm8_gemm_prefill_multi_into(xs, mods, [outs[0], outs[1], res], residuals=[None, None, res],
                                epilogues=[_lib.EPI_NONE, _lib.EPI_RELU2, _lib.EPI_RESIDUAL])
    torch.cuda.synchronize()
    base = [_ref(oracle, x, m) for x, m in zip(xs, mods)]
    assert _rel_err(_np(outs[0]).astype(np.float64), base[0]) <= TOL
    rr = np.maximum(base[1], 0) ** 2
    assert np.abs(_np(outs[1]) - rr).max() <= 2 * TOL * np.abs(rr).max()
    add = base[2] + want_res
    assert np.abs(_np(res) - add).max() <= TOL * np.abs(add).max()


@pytest.mark.parametrize("act", [torch.float32, torch.bfloat16])
def test_mm8p_other_dtypes_take_tile_chunks(oracle, act):
    """bf16 activations take the dequantise-then-GEMM route (the weight
    materialised in bf16); fp32 runs the 64-row tile GEMM over 256-row chunks."""
    from rwkv7mi.native_quant_mm8 import mm8_gemm_prefill_multi_into

    I, O, rows = 1024, 256, 600
    rng = np.random.default_rng(9)
    mod = _packed(rng, I, O, dtype=act)
    x = _cuda(rng.standard_normal((rows, I)), act)
    y = torch.empty(rows, O, device="cuda", dtype=act)
    mm8_gemm_prefill_multi_into([x], [mod], [y])
    torch.cuda.synchronize()
    tol = 1e-4 if act == torch.float32 else 8e-3
    assert _rel_err(_np(y.float()).astype(np.float64), _ref(oracle, x, mod)) <= tol


def test_mm8p_module_routes(oracle):
    """MM8Linear.forward / the functional mm8_matmul and the model's
    QuantLinear take the prefill GEMM above 256 rows, identical results."""
    from rwkv7mi.model import QuantLinear
    from rwkv7mi.native_quant_mm8 import MM8Linear

    torch.manual_seed(0)
    lin = torch.nn.Linear(512, 384, bias=True).cuda().half()
    m = MM8Linear(lin)
    x = torch.randn(3, 200, 512, device="cuda", dtype=torch.float16)
    y = m(x)
    q = QuantLinear(m)
    y2 = torch.empty(600, 384, device="cuda", dtype=torch.float16)
    q.apply(x.reshape(600, 512), y2)
    torch.cuda.synchronize()
    assert torch.equal(y.reshape(600, 384), y2)
    mod = types.SimpleNamespace(w_blk=m.w_blk, mx=m.mx, rx=m.rx, my=m.my.reshape(-1), ry=m.ry.reshape(-1),
                                bias=m.bias, in_features=512, out_features=384)
    err = _rel_err(_np(y.reshape(600, 384)).astype(np.float64), _ref(oracle, x.reshape(600, 512), mod))
    assert err <= TOL


@pytest.mark.parametrize("IO", [(4096, 4096), (144, 40), (2064, 520), (80, 16)])
def test_mm8p_workspace_is_the_dequantised_weight(IO):
    """The workspace the prefill GEMM reads holds rwkv7mi_mm8_dequant's fp16
    weight bit for bit: record (group g, step sb, sub-step h, lane n + 16 kg,
    j) is W_hat[64 sb + 16 kg + 8 h + j, 32 (g // 2) + 8 (n // 4) + 4 (g % 2)
    + n % 4], zero past I or O."""
    from rwkv7mi import _lib
    from rwkv7mi import workspace as _ws
    from rwkv7mi.native_quant_mm8 import dequantize_mm8, mm8_gemm_prefill_multi_into, mm8_unblock

    I, O = IO
    rng = np.random.default_rng(7 * I + O)
    mod = _packed(rng, I, O)
    x = _cuda(rng.standard_normal((300, I)), torch.float16)
    y = torch.empty((300, O), device="cuda", dtype=torch.float16)
    print(f"mm8p workspace: I={I} O={O}", flush=True)
    mm8_gemm_prefill_multi_into([x], [mod], [y])
    need = int(_lib.load().rwkv7mi_mm8t_gemm_prefill_ws_bytes(1, I, O))
    G, SB = 2 * ((O + 31) // 32), (I + 63) // 64
    assert need == G * SB * 2048
    ws = _ws.reserve(x.device, need, "mm8p")
    torch.cuda.synchronize()
    # g = 2 p + b, n = 4 a + c: column 32 p + 8 a + 4 b + c
    got = _np(ws[:need].view(torch.float16)).reshape(G // 2, 2, SB, 2, 4, 4, 4, 8)  # p, b, sb, h, kg, a, c, j
    got = got.transpose(2, 4, 3, 7, 0, 5, 1, 6).reshape(SB * 64, G * 16)          # (sb, kg, h, j) x (p, a, b, c)
    w_u8 = mm8_unblock(mod.w_blk, I, O)
    want = _np(dequantize_mm8(w_u8, mod.mx, mod.rx, mod.my.reshape(-1, 1), mod.ry.reshape(-1, 1),
                              out_dtype=torch.float16))
    assert np.array_equal(got[:I, :O].view(np.uint16), want.view(np.uint16))
    assert not got[I:].any() and not got[:, O:].any()


@pytest.mark.parametrize("IO,rows", [((4096, 4096), 600), ((2064, 520), 257), ((144, 40), 1024)])
def test_mm8p_in_register_entry_matches_oracle(oracle, IO, rows):
    """rwkv7mi_mm8t_gemm_prefill (the weight dequantised in registers, no
    workspace) stays available beside the workspace route."""
    import ctypes

    from rwkv7mi import _lib

    I, O = IO
    rng = np.random.default_rng(3 * I + O + rows)
    mod = _packed(rng, I, O, bias=True)
    x = _cuda(rng.standard_normal((rows, I)), torch.float16)
    y = torch.full((rows, O), float("nan"), device="cuda", dtype=torch.float16)
    print(f"mm8p in-register: I={I} O={O} rows={rows}", flush=True)
    arr = lambda ts: _lib.ptr_array(ts)
    _lib.call("rwkv7mi_mm8t_gemm_prefill", 1, arr([x]), arr([mod.w_blk]), arr([mod.mx]), arr([mod.rx]),
              arr([mod.my]), arr([mod.ry]), arr([mod.bias]), arr([None]), arr([y]), (ctypes.c_int * 1)(0),
              rows, I, O, _lib.F16, _lib.F16, _lib.stream_of(x))
    torch.cuda.synchronize()
    err = _rel_err(_np(y).astype(np.float64), _ref(oracle, x, mod))
    assert err <= TOL, (IO, rows, err)


@pytest.mark.parametrize("IO,rows,epi,dt", [((768, 768), 600, 0, "f16"), ((768, 3072), 300, 1, "f16"),
                                            ((3072, 768), 513, 2, "f16"), ((144, 80), 257, 0, "f16"),
                                            ((4096, 4096), 1024, 2, "f16"), ((768, 3072), 300, 1, "bf16"),
                                            ((3072, 768), 513, 2, "bf16")])
def test_dense_prefill_gemm_matches_fp64(IO, rows, epi, dt):
    """rwkv7mi_dense_gemm_prefill_ws (fp16 nn.Linear weight, copied into
    operand order, then the prefill MFMA GEMM) against fp64 x @ W^T + b with
    the relu^2 / residual epilogues; and DenseLinear routes above 256 rows."""
    import ctypes

    from rwkv7mi import _lib
    from rwkv7mi import workspace as _ws
    from rwkv7mi.model import DenseLinear
    from rwkv7mi.native_quant_mm8 import mm8_prefill_workspace_bytes

    I, O = IO
    tdt = torch.float16 if dt == "f16" else torch.bfloat16
    rng = np.random.default_rng(I * 7 + O + rows + epi)
    x = _cuda(rng.standard_normal((rows, I)), tdt)
    W = _cuda(rng.standard_normal((O, I)) * 0.05, tdt)
    b = _cuda(rng.standard_normal(O) * 0.1, tdt)
    res = _cuda(rng.standard_normal((rows, O)), tdt) if epi == 2 else None
    y = torch.full((rows, O), float("nan"), device="cuda", dtype=tdt)
    print(f"dense prefill: I={I} O={O} rows={rows} epi={epi} {dt}", flush=True)
    need = mm8_prefill_workspace_bytes(1, I, O)
    ws = _ws.reserve(x.device, need, "mm8p")
    arr = _lib.ptr_array
    _lib.call("rwkv7mi_dense_gemm_prefill_ws", 1, arr([x]), arr([W]), arr([b]), arr([res]), arr([y]),
              (ctypes.c_int * 1)(epi), rows, I, O, _lib.dtype_code(x), _lib.ptr(ws), need, _lib.stream_of(x))
    torch.cuda.synchronize()
    f64 = lambda t: _np(t.float()).astype(np.float64)
    ref = f64(x) @ f64(W).T + f64(b)
    if epi == 1:
        ref = np.maximum(ref, 0.0) ** 2
    elif epi == 2:
        ref = ref + f64(res)
    tol = TOL if dt == "f16" else 1.6e-2  # bf16 output rounding 2^-8
    assert _rel_err(f64(y), ref) <= tol, (IO, rows, epi, dt)
    # the model's DenseLinear takes the same entry above 256 rows
    lin = DenseLinear(W, b)
    y2 = torch.empty_like(y)
    lin.apply(x, y2, act=3 if epi == 1 else 0, residual=res)
    torch.cuda.synchronize()
    assert torch.equal(y2, y)


def test_mm8p_rejects():
    from rwkv7mi import _lib

    with pytest.raises(ValueError):
        _lib.call("rwkv7mi_mm8t_gemm_prefill", 0, None, None, None, None, None, None, None, None, None, None,
                  300, 128, 16, _lib.F16, _lib.F16, None)
    with pytest.raises(ValueError):
        _lib.call("rwkv7mi_mm8t_gemm_prefill_ws", 1, None, None, None, None, None, None, None, None, None, None,
                  300, 128, 16, _lib.F16, _lib.F16, None, 0, None)
