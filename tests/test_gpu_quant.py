"""GPU parity: MM8 / W4-group packers (bit-exact) and fused dequant GEMV/GEMM
(fp64 oracle, relative tolerance) including epilogues and ragged batches."""
from __future__ import annotations

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


@pytest.mark.parametrize("shape", [(256, 128), (128, 256), (512, 512), (3, 8), (9, 16)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_mm8_pack_bit_exact(oracle, shape, dtype):
    from rwkv7mi import quantize_mm8

    rng = np.random.default_rng(sum(shape))
    W = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    Wt = _cuda(W, dtype)
    w_u8, mx, rx, my, ry = quantize_mm8(Wt)
    torch.cuda.synchronize()
    npdt = np.float16 if dtype == torch.float16 else np.float32
    q, omx, orx, omy, ory = oracle.mm8_pack(_np(Wt.float()), out_dtype=npdt)
    np.testing.assert_array_equal(_np(w_u8), q)
    for got, ref in ((mx, omx), (rx, orx), (my, omy), (ry, ory)):
        np.testing.assert_array_equal(_np(got).view(np.uint16 if npdt == np.float16 else np.uint32),
                                      np.asarray(ref).view(np.uint16 if npdt == np.float16 else np.uint32))
    assert my.shape == (shape[0], 1) and ry.shape == (shape[0], 1)


SHAPES_MM8 = [(2048, 2048), (2048, 8192), (8192, 2048), (1000, 1032), (128, 64)]


@pytest.mark.parametrize("IO", SHAPES_MM8)
@pytest.mark.parametrize("rows", [1, 8, 32, 64, 65, 3])
def test_mm8_matmul(oracle, IO, rows):
    from rwkv7mi.native_quant_mm8 import mm8_matmul, quantize_mm8

    I, O = IO
    rng = np.random.default_rng(I + O + rows)
    W = (rng.standard_normal((I, O)) * 0.02).astype(np.float16)
    x = rng.standard_normal((rows, I)).astype(np.float16)
    packed = quantize_mm8(_cuda(W, torch.float16))
    xt = _cuda(x, torch.float16)
    y = mm8_matmul(xt, *packed)
    y2 = mm8_matmul(xt, *packed)  # second call exercises the counter reset
    torch.cuda.synchronize()
    ref = oracle.mm8_matmul(x.astype(np.float64), *(_np(p) for p in packed))
    err = _rel_err(_np(y).astype(np.float64), ref)
    assert err <= 2e-3, err
    assert torch.equal(y, y2), "repeated calls must be bit-identical"


def test_mm8_epilogues_and_module(oracle):
    from rwkv7mi import MM8Linear

    rng = np.random.default_rng(5)
    I, O, rows = 1024, 4096, 4
    lin = torch.nn.Linear(I, O, bias=True).to(device="cuda", dtype=torch.float16)
    with torch.no_grad():
        lin.weight.copy_(_cuda(rng.standard_normal((O, I)) * 0.02, torch.float16))
        lin.bias.copy_(_cuda(rng.standard_normal(O) * 0.1, torch.float16))
    mod = MM8Linear(lin)
    assert mod.w_u8.shape == (I, O) and mod.my.shape == (I, 1)
    x = _cuda(rng.standard_normal((rows, I)), torch.float16)
    res = _cuda(rng.standard_normal((rows, O)), torch.float16)
    packed = [_np(b) for b in (mod.w_u8, mod.mx, mod.rx, mod.my, mod.ry)]
    base = oracle.mm8_matmul(_np(x).astype(np.float64), *packed) + _np(lin.bias).astype(np.float64)
    y = mod(x)
    out = torch.empty_like(y)
    mod.rwkv7_forward_into(x, out)
    y_relu2 = mod.rwkv7_forward_relu2(x)
    y_add = mod.rwkv7_forward_add(x, res)
    y3 = mod(x.reshape(2, 2, I))
    torch.cuda.synchronize()
    scale = np.abs(base).max()
    assert np.abs(_np(y) - base).max() <= 2e-3 * scale
    assert torch.equal(out, y)
    assert torch.equal(y3.reshape(rows, O), y)
    relu2 = np.maximum(base, 0) ** 2
    assert np.abs(_np(y_relu2) - relu2).max() <= 4e-3 * np.abs(relu2).max()
    add = base + _np(res).astype(np.float64)
    assert np.abs(_np(y_add) - add).max() <= 2e-3 * np.abs(add).max()


@pytest.mark.parametrize("group", [128, 256])
@pytest.mark.parametrize("shape", [(24, 256), (4096, 4096), (64, 1024)])
def test_w4g_pack_bit_exact(oracle, group, shape):
    from rwkv7mi import quantize_w4_groupwise

    rng = np.random.default_rng(shape[0] + group)
    W = (rng.standard_normal(shape) * 0.02).astype(np.float16)
    packed, scales, k = quantize_w4_groupwise(_cuda(W, torch.float16), group_size=group)
    torch.cuda.synchronize()
    op, osc, ok = oracle.w4g_pack(W.astype(np.float32), group)
    assert k == ok
    np.testing.assert_array_equal(_np(packed), op)
    np.testing.assert_array_equal(_np(scales).view(np.uint16), osc.view(np.uint16))


@pytest.mark.parametrize("OI", [(4096, 4096), (16384, 4096), (4096, 16384), (256, 512)])
@pytest.mark.parametrize("rows", [1, 4, 16, 40])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_w4g_linear(oracle, OI, rows, dtype):
    from rwkv7mi import quantize_w4_groupwise, w4_groupwise_linear

    O, I = OI
    rng = np.random.default_rng(O + I + rows)
    W = (rng.standard_normal((O, I)) * 0.02).astype(np.float16)
    packed, scales, k = quantize_w4_groupwise(_cuda(W, torch.float16))
    x = _cuda(rng.standard_normal((rows, I)), dtype)
    y = w4_groupwise_linear(x, packed, scales.to(dtype), O, I)
    torch.cuda.synchronize()
    ref = oracle.w4g_linear(_np(x).astype(np.float64), _np(packed), _np(scales.to(dtype)).astype(np.float64))
    assert _rel_err(_np(y).astype(np.float64), ref) <= 2e-3


@pytest.mark.parametrize("group", [128, 256])
@pytest.mark.parametrize("shape", [(6, 512), (4096, 4096)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_w4a_pack_bit_exact(oracle, group, shape, dtype):
    """Asymmetric (min/max affine) group W4: packed nibbles, scales and biases
    bit-identical to the oracle's fp32 restatement."""
    from rwkv7mi.sm70_quant import quantize_w4_affine_groupwise

    rng = np.random.default_rng(shape[0] + group)
    Wt = _cuda(rng.standard_normal(shape) * 0.02, dtype)
    packed, scales, biases, k = quantize_w4_affine_groupwise(Wt, group_size=group)
    torch.cuda.synchronize()
    op, osc, obi = oracle.w4a_pack(_np(Wt.float()), group, out_dtype=np.float32)
    assert k == shape[1]
    np.testing.assert_array_equal(_np(packed), op)
    cast = lambda a: _np(torch.tensor(a).to(dtype).float())
    np.testing.assert_array_equal(_np(scales.float()), cast(osc))
    np.testing.assert_array_equal(_np(biases.float()), cast(obi))


@pytest.mark.parametrize("OI", [(4096, 4096), (16384, 4096), (4096, 16384), (256, 512)])
@pytest.mark.parametrize("rows", [1, 4, 16, 40])
def test_w4a_linear(oracle, OI, rows):
    from rwkv7mi.sm70_quant import quantize_w4_affine_groupwise, w4_affine_groupwise_linear

    O, I = OI
    rng = np.random.default_rng(O + 3 * I + rows)
    W = _cuda(rng.standard_normal((O, I)) * 0.02, torch.float16)
    packed, scales, biases, _ = quantize_w4_affine_groupwise(W)
    x = _cuda(rng.standard_normal((rows, I)), torch.float16)
    y = w4_affine_groupwise_linear(x, packed, scales, biases, O, I)
    torch.cuda.synchronize()
    ref = oracle.w4a_linear(_np(x).astype(np.float64), _np(packed), _np(scales), _np(biases))
    assert _rel_err(_np(y).astype(np.float64), ref) <= 2e-3


@pytest.mark.parametrize("rows", [1, 4, 16])
def test_w4_head_shape_c4(oracle, rows):
    """BASELINE configs[3]'s vocabulary head, 4096 x 65536, through the
    symmetric group-128 W4 and the asymmetric (affine) form, at its batch
    sizes 1 / 4 / 16."""
    from rwkv7mi import quantize_w4_groupwise, w4_groupwise_linear
    from rwkv7mi.sm70_quant import quantize_w4_affine_groupwise, w4_affine_groupwise_linear

    O, I = 65536, 4096
    rng = np.random.default_rng(65536 + rows)
    W = torch.randn(O, I, device="cuda", dtype=torch.float16, generator=torch.Generator("cuda").manual_seed(rows))
    W *= 0.02
    x = _cuda(rng.standard_normal((rows, I)), torch.float16)
    packed, scales, _ = quantize_w4_groupwise(W)
    y = w4_groupwise_linear(x, packed, scales, O, I)
    torch.cuda.synchronize()
    ref = oracle.w4g_linear(_np(x).astype(np.float64), _np(packed), _np(scales))
    assert _rel_err(_np(y).astype(np.float64), ref) <= 2e-3
    pa, sa, ba, _ = quantize_w4_affine_groupwise(W)
    ya = w4_affine_groupwise_linear(x, pa, sa, ba, O, I)
    torch.cuda.synchronize()
    refa = oracle.w4a_linear(_np(x).astype(np.float64), _np(pa), _np(sa), _np(ba))
    assert _rel_err(_np(ya).astype(np.float64), refa) <= 2e-3


@pytest.mark.parametrize("case", [
    # (O, I, group, rows, act dtype, affine)
    (200, 384, 128, 1, torch.float16, False),     # ragged columns, I not a multiple of 256
    (200, 384, 128, 7, torch.float16, True),
    (1040, 2048, 256, 2, torch.float16, False),   # group 256
    (1040, 2048, 256, 16, torch.bfloat16, True),  # bf16 activations (hi + lo staging)
    (520, 1536, 128, 5, torch.float32, True),     # fp32 activations
    (4096, 16384, 128, 16, torch.float16, True),  # x re-staged per chunk (too big for LDS at once)
    (48, 16384, 256, 3, torch.bfloat16, False),   # three column groups, bf16 x in four chunks
])
def test_w4_stream_gemv_edges(oracle, case):
    """The streaming <= 16-row W4 GEMV on its edge shapes: ragged column
    groups, a half step at the end of K, group 256, every activation dtype,
    the chunked x staging, both the symmetric and the affine form."""
    from rwkv7mi import quantize_w4_groupwise, w4_groupwise_linear
    from rwkv7mi.sm70_quant import quantize_w4_affine_groupwise, w4_affine_groupwise_linear

    O, I, group, rows, act, aff = case
    rng = np.random.default_rng(O + I + rows + group)
    W = _cuda(rng.standard_normal((O, I)) * 0.02, torch.float16)
    x = _cuda(rng.standard_normal((rows, I)), act)
    if aff:
        q, s, b, _ = quantize_w4_affine_groupwise(W, group_size=group)
        y = w4_affine_groupwise_linear(x, q, s, b, O, I, group_size=group)
        ref = oracle.w4a_linear(_np(x.float()).astype(np.float64), _np(q), _np(s), _np(b), group)
    else:
        q, s, _ = quantize_w4_groupwise(W, group_size=group)
        y = w4_groupwise_linear(x, q, s, O, I, group_size=group)
        ref = oracle.w4g_linear(_np(x.float()).astype(np.float64), _np(q), _np(s), group)
    torch.cuda.synchronize()
    # fp16 / fp32: exact products, fp32 sums (the tolerance is the output
    # rounding); bf16 outputs round to 8 bits
    tol = {torch.float16: 2e-3, torch.float32: 1e-4, torch.bfloat16: 8e-3}[act]
    err = _rel_err(_np(y.float()).astype(np.float64), ref)
    assert err <= tol, (case, err)


@pytest.mark.parametrize("rows", [1, 6])
def test_w4_stream_gemv_epilogues(oracle, rows):
    """Bias, residual (in place: out aliases the residual) and relu^2 epilogues
    of the symmetric W4 GEMV against the oracle."""
    from rwkv7mi import _lib
    from rwkv7mi import quantize_w4_groupwise
    from rwkv7mi.sm70_quant import w4_groupwise_linear_into

    O, I = 784, 1024
    rng = np.random.default_rng(rows)
    W = _cuda(rng.standard_normal((O, I)) * 0.02, torch.float16)
    q, s, _ = quantize_w4_groupwise(W)
    x = _cuda(rng.standard_normal((rows, I)), torch.float16)
    bias = _cuda(rng.standard_normal(O) * 0.1, torch.float16)
    base = oracle.w4g_linear(_np(x).astype(np.float64), _np(q), _np(s)) + _np(bias).astype(np.float64)
    y = torch.empty(rows, O, device="cuda", dtype=torch.float16)
    w4_groupwise_linear_into(x, q, s, y, bias=bias)
    r2 = torch.empty_like(y)
    w4_groupwise_linear_into(x, q, s, r2, bias=bias, epilogue=_lib.EPI_RELU2)
    res = _cuda(rng.standard_normal((rows, O)), torch.float16)
    want_res = base + _np(res).astype(np.float64)
    w4_groupwise_linear_into(x, q, s, res, bias=bias, residual=res, epilogue=_lib.EPI_RESIDUAL)
    torch.cuda.synchronize()
    assert np.abs(_np(y) - base).max() <= 2e-3 * np.abs(base).max()
    rr = np.maximum(base, 0) ** 2
    assert np.abs(_np(r2) - rr).max() <= 4e-3 * np.abs(rr).max()
    assert np.abs(_np(res) - want_res).max() <= 2e-3 * np.abs(want_res).max()


# ---------------------------------------------------------------- reference bytes
# The device packers against the reference packers' own outputs
# (tests/golden/quant_packers.npz, written by tests/golden/make_quant_golden.py
# from rwkv7_hf/native_quant_mm8.py:62-97, native_quant_mm4.py:77-105 and
# sm70_quant.py:502-519): every byte and every scale bit.
import quant_golden as qg  # noqa: E402


def _dt(W):
    return torch.float16 if W.dtype == np.float16 else torch.float32


def _assert_bits(got, ref, what):
    got = _np(got)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    np.testing.assert_array_equal(qg.bits(got), qg.bits(ref), err_msg=what)


@pytest.mark.parametrize("name", qg.cases("mm8"))
def test_mm8_device_packers_match_reference_bytes(name):
    from rwkv7mi.native_quant_mm8 import MM8Linear, quantize_mm8

    c = qg.case("mm8", name)
    W = _cuda(c["W"], _dt(c["W"]))
    for got, key in zip(quantize_mm8(W), ("w_u8", "mx", "rx", "my", "ry")):
        _assert_bits(got, c[key], f"{name} {key}")
    # the module's blocked packer (nn.Linear.weight = W^T) materialises the same reference tensors
    lin = torch.nn.Linear(W.shape[0], W.shape[1], bias=False, device="cuda", dtype=W.dtype)
    with torch.no_grad():
        lin.weight.copy_(W.t())
    mod = MM8Linear(lin)
    for key in ("w_u8", "mx", "rx", "my", "ry"):
        _assert_bits(getattr(mod, key), c[key], f"{name} MM8Linear {key}")


@pytest.mark.parametrize("name", qg.cases("mm4"))
def test_mm4_device_packers_match_reference_bytes(name):
    from rwkv7mi.native_quant_mm4 import outmajor_to_reference, quantize_mm4, quantize_mm4_outmajor

    c = qg.case("mm4", name)
    W = _cuda(c["W"], _dt(c["W"]))
    packed, mx, rx, my, ry, m_orig, m_pad = quantize_mm4(W)
    assert [m_orig, m_pad] == c["m"].tolist()
    for got, key in ((packed, "packed"), (mx, "mx"), (rx, "rx"), (my, "my"), (ry, "ry")):
        _assert_bits(got, c[key], f"{name} {key}")
    if W.shape[0] % 2 == 0:  # the module's out-major packer needs an even in_features
        pt, mx2, rx2, my2, ry2, _, _ = quantize_mm4_outmajor(W.t().contiguous())
        _assert_bits(outmajor_to_reference(pt, W.shape[0]), c["packed"], f"{name} out-major packed")
        for got, key in ((mx2, "mx"), (rx2, "rx"), (my2, "my"), (ry2, "ry")):
            _assert_bits(got, c[key], f"{name} out-major {key}")


@pytest.mark.parametrize("name", qg.cases("w4g"))
def test_w4g_device_packer_matches_reference_bytes(name):
    from rwkv7mi import quantize_w4_groupwise

    c = qg.case("w4g", name)
    group, k = c["group"].tolist()
    packed, scales, kk = quantize_w4_groupwise(_cuda(c["W"], _dt(c["W"])), group_size=group)
    assert kk == k
    _assert_bits(packed, c["packed"], f"{name} packed")
    _assert_bits(scales, c["scales"], f"{name} scales")
