"""GPU parity of the MM4 path: the affine packer (reference layout) is
bit-identical to the oracle, the inputs-paired packer holds the same nibbles
and metadata, the fused GEMV/GEMM matches the fp64 oracle, MM4Linear's group
and affine routes (with epilogues) match, and its state dict carries the
reference's layout."""
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


def _nibbles_rows_pairs(p):
    """[R, C] bytes -> [R, 2C] nibbles (low first)."""
    p = np.asarray(p)
    u = np.empty((p.shape[0], p.shape[1] * 2), np.uint8)
    u[:, 0::2] = p & 15
    u[:, 1::2] = p >> 4
    return u


@pytest.mark.parametrize("IO", [(256, 128), (128, 256), (64, 37), (96, 1), (512, 1024)])
def test_mm4_pack_reference_layout_bit_exact(oracle, IO):
    from rwkv7mi import quantize_mm4

    I, O = IO
    rng = np.random.default_rng(I + 3 * O)
    W = (rng.standard_normal((I, O)) * 0.02).astype(np.float32)
    packed, mx, rx, my, ry, m_orig, m_pad = quantize_mm4(_cuda(W, torch.float32))
    torch.cuda.synchronize()
    q, omx, orx, omy, ory, om, omp = oracle.mm4_pack(W, out_dtype=np.float32)
    assert (m_orig, m_pad) == (om, omp) == (O, O + (O & 1))
    np.testing.assert_array_equal(_np(packed), q)
    for got, ref in ((mx, omx), (rx, orx), (my, omy), (ry, ory)):
        np.testing.assert_array_equal(_np(got).reshape(-1).view(np.uint32), np.asarray(ref).reshape(-1).view(np.uint32))


@pytest.mark.parametrize("OI", [(128, 256), (37, 64), (4096, 4096)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_mm4_pack_outmajor_same_nibbles(OI, dtype):
    from rwkv7mi.native_quant_mm4 import outmajor_to_reference, quantize_mm4, quantize_mm4_outmajor

    O, I = OI
    rng = np.random.default_rng(O + I)
    Wl = _cuda(rng.standard_normal((O, I)) * 0.02, dtype)
    a = quantize_mm4(Wl.t().contiguous())
    b = quantize_mm4_outmajor(Wl)
    torch.cuda.synchronize()
    ua = _nibbles_rows_pairs(_np(a[0]))            # [I, Mp]
    ub = _nibbles_rows_pairs(_np(b[0])).T          # [I, Mp]
    np.testing.assert_array_equal(ua, ub)
    for x, y in zip(a[1:5], b[1:5]):
        assert torch.equal(x, y)
    assert a[5:] == b[5:]
    assert torch.equal(outmajor_to_reference(b[0], I), a[0])


@pytest.mark.parametrize("IO", [(4096, 4096), (1024, 4097), (16384, 512), (96, 40)])
@pytest.mark.parametrize("rows", [1, 5, 16, 33])
def test_mm4t_matmul_matches_oracle(oracle, IO, rows):
    from rwkv7mi.native_quant_mm4 import mm4t_matmul_into, quantize_mm4, quantize_mm4_outmajor

    I, O = IO
    rng = np.random.default_rng(I + O + rows)
    Wl = _cuda(rng.standard_normal((O, I)) * 0.02, torch.float16)
    pt, mx, rx, my, ry, m_orig, _ = quantize_mm4_outmajor(Wl)
    ref_layout = quantize_mm4(Wl.t().contiguous())
    x = rng.standard_normal((rows, I)).astype(np.float16)
    out = torch.empty(rows, O, device="cuda", dtype=torch.float16)
    mm4t_matmul_into(_cuda(x, torch.float16), pt, mx, rx, my.reshape(-1), ry.reshape(-1), out)
    torch.cuda.synchronize()
    deq = oracle.mm4_dequant(*(_np(t) for t in ref_layout[:5]), m_orig)
    ref = x.astype(np.float64) @ deq
    assert _rel_err(_np(out).astype(np.float64), ref) <= 2e-3


def test_dequantize_mm4_matches_oracle(oracle):
    from rwkv7mi import dequantize_mm4, mm4_matmul, quantize_mm4

    rng = np.random.default_rng(8)
    W = _cuda(rng.standard_normal((256, 77)) * 0.02, torch.float16)
    q = quantize_mm4(W)
    deq = dequantize_mm4(*q[:5], q[5], out_dtype=torch.float32)
    x = _cuda(rng.standard_normal((3, 256)), torch.float32)
    y = mm4_matmul(x, *q[:5], q[5])
    torch.cuda.synchronize()
    ref = oracle.mm4_dequant(*(_np(t) for t in q[:5]), q[5])
    assert deq.shape == (256, 77)
    assert np.abs(_np(deq) - ref).max() <= 1e-6 * np.abs(ref).max()
    assert _rel_err(_np(y), _np(x).astype(np.float64) @ ref) <= 1e-5


@pytest.mark.parametrize("group_size", [0, 128])
def test_mm4linear_routes_epilogues_and_state_dict(oracle, group_size):
    from rwkv7mi import MM4Linear

    rng = np.random.default_rng(11 + group_size)
    I, O, rows = 1024, 2048, 3
    lin = torch.nn.Linear(I, O, bias=True).to(device="cuda", dtype=torch.float16)
    with torch.no_grad():
        lin.weight.copy_(_cuda(rng.standard_normal((O, I)) * 0.02, torch.float16))
        lin.bias.copy_(_cuda(rng.standard_normal(O) * 0.1, torch.float16))
    mod = MM4Linear(lin, group_size=group_size)
    assert mod.groupwise == (group_size == 128)
    x = _cuda(rng.standard_normal((rows, I)), torch.float16)
    res = _cuda(rng.standard_normal((rows, O)), torch.float16)
    if group_size:
        deq = oracle.w4g_dequant(_np(mod.packed_group), _np(mod.group_scales).astype(np.float64), group_size).T
    else:
        deq = oracle.mm4_dequant(_np(mod.packed), *(_np(t) for t in (mod.mx, mod.rx_s, mod.my, mod.ry_s)), O)
    base = _np(x).astype(np.float64) @ deq + _np(lin.bias).astype(np.float64)
    y = mod(x)
    out = torch.empty_like(y)
    mod.rwkv7_forward_into(x, out)
    r2 = mod.rwkv7_forward_relu2(x)
    add = mod.rwkv7_forward_add(x, res)
    torch.cuda.synchronize()
    scale = np.abs(base).max()
    assert np.abs(_np(y) - base).max() <= 2e-3 * scale
    assert torch.equal(out, y)
    relu2 = np.maximum(base, 0) ** 2
    assert np.abs(_np(r2) - relu2).max() <= 4e-3 * np.abs(relu2).max()
    ref_add = base + _np(res).astype(np.float64)
    assert np.abs(_np(add) - ref_add).max() <= 2e-3 * np.abs(ref_add).max()
    sd = mod.state_dict()
    if not group_size:
        assert "packed" in sd and "packed_t" not in sd and tuple(sd["packed"].shape) == (I, O // 2)
        mod2 = MM4Linear(lin, group_size=0)
        with torch.no_grad():
            mod2.packed_t.zero_()
        mod2.load_state_dict(sd)
        assert torch.equal(mod2.packed_t, mod.packed_t)


def test_quantize_model_mm4_group_policy():
    from rwkv7mi.native_quant_mm4 import MM4Linear, native_mm4_group_size_for_module, quantize_model_mm4

    assert native_mm4_group_size_for_module("model.layers.0.ffn.key", 128, "ffn_key") == 128
    assert native_mm4_group_size_for_module("model.layers.0.attn.r_proj", 128, "ffn_key") == 0
    assert native_mm4_group_size_for_module("lm_head", 128, "lm_head_and_value") == 128
    net = torch.nn.Sequential(torch.nn.Linear(512, 512), torch.nn.Linear(512, 256)).to("cuda", torch.float16)
    n = quantize_model_mm4(net, min_params=0, group_size=128)
    assert n == 2 and all(isinstance(m, MM4Linear) and m.groupwise for m in net)
    y = net(torch.randn(2, 512, device="cuda", dtype=torch.float16))
    torch.cuda.synchronize()
    assert y.shape == (2, 256) and torch.isfinite(y).all()


@pytest.mark.parametrize("rows", [1, 4, 16])
def test_mm4_head_shape_c4(oracle, rows):
    """BASELINE configs[3]'s head shape, 4096 x 65536, on the MM4 affine GEMV."""
    from rwkv7mi.native_quant_mm4 import mm4t_matmul_into, quantize_mm4, quantize_mm4_outmajor

    I, O = 4096, 65536
    rng = np.random.default_rng(7 + rows)
    Wl = torch.randn(O, I, device="cuda", dtype=torch.float16, generator=torch.Generator("cuda").manual_seed(rows))
    Wl *= 0.02
    pt, mx, rx, my, ry, m_orig, _ = quantize_mm4_outmajor(Wl)
    ref_layout = quantize_mm4(Wl.t().contiguous())
    x = rng.standard_normal((rows, I)).astype(np.float16)
    out = torch.empty(rows, O, device="cuda", dtype=torch.float16)
    mm4t_matmul_into(_cuda(x, torch.float16), pt, mx, rx, my.reshape(-1), ry.reshape(-1), out)
    torch.cuda.synchronize()
    deq = oracle.mm4_dequant(*(_np(t) for t in ref_layout[:5]), m_orig)
    ref = x.astype(np.float64) @ deq
    assert _rel_err(_np(out).astype(np.float64), ref) <= 2e-3
