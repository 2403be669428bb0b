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


# ---------------------------------------------------- reference-layout fused kernel
# Tolerances (relative to max|y|), about twice the largest error measured on an
# MI355X over the cases below (fp32 9e-7, fp16 4e-4, bf16 2.5e-3): x*ry_s enters
# the MFMA as fp16 hi + lo (~2^-22 per product) with fp32 sums, so the fp16 /
# bf16 figures are their one output rounding.
_TOL = {torch.float32: 2e-6, torch.float16: 1e-3, torch.bfloat16: 5e-3}


def _fused_case(oracle, I, O, rows, dtype, seed):
    from rwkv7mi import quantize_mm4

    rng = np.random.default_rng(seed)
    W = _cuda(rng.standard_normal((I, O)) * 0.02, dtype)
    q = quantize_mm4(W)
    x = rng.standard_normal((rows, I)).astype(np.float32)
    xd = _cuda(x, dtype)
    deq = oracle.mm4_dequant(_np(q[0]), *(_np(t.float()) for t in q[1:5]), q[5])
    return q, xd, _np(xd.float()).astype(np.float64) @ deq


@pytest.mark.parametrize("IO", [(4096, 4096), (1024, 4097), (16384, 512), (96, 40), (300, 24), (5, 3)])
@pytest.mark.parametrize("rows", [1, 5, 16, 33, 64])
def test_mm4_reference_layout_fused_matches_oracle(oracle, IO, rows):
    """mm4_matmul_triton over packed [I, Mp/2]: aligned rows (Mp % 16 == 0),
    bytewise rows (odd O, narrow O), ragged K ranges and 16-row tiles."""
    from rwkv7mi import mm4_matmul_triton

    I, O = IO
    q, xd, ref = _fused_case(oracle, I, O, rows, torch.float16, I + 7 * O + rows)
    y = mm4_matmul_triton(xd, *q[:5], q[5])
    torch.cuda.synchronize()
    assert y.shape == (rows, O) and y.dtype == torch.float16
    err = _rel_err(_np(y).astype(np.float64), ref)
    print(f"PARITY mm4 reference layout I={I} O={O} rows={rows} f16: rel {err:.2e}", flush=True)
    assert err <= _TOL[torch.float16]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("IO", [(2048, 1536), (640, 77)])
def test_mm4_reference_layout_fused_dtypes(oracle, IO, dtype):
    from rwkv7mi.native_quant_mm4 import mm4_batched_gemv_triton, mm4_gemv_triton

    I, O = IO
    q, xd, ref = _fused_case(oracle, I, O, 7, dtype, I + O)
    y = mm4_batched_gemv_triton(xd, *q[:5], q[5])
    y1 = mm4_gemv_triton(xd[3], *q[:5], q[5])
    torch.cuda.synchronize()
    assert y1.shape == (O,)
    assert torch.equal(y1, y[3])  # a row's result does not depend on the other rows of its tile
    err = _rel_err(_np(y.float()).astype(np.float64), ref)
    print(f"PARITY mm4 reference layout I={I} O={O} rows=7 {dtype}: rel {err:.2e}", flush=True)
    assert err <= _TOL[dtype]


def test_mm4_reference_layout_epilogues(oracle):
    from rwkv7mi._lib import EPI_RELU2, EPI_RESIDUAL
    from rwkv7mi.native_quant_mm4 import mm4_matmul_into

    I, O, rows = 1024, 1000, 9
    q, xd, ref = _fused_case(oracle, I, O, rows, torch.float16, 11)
    rng = np.random.default_rng(12)
    bias = _cuda(rng.standard_normal(O) * 0.1, torch.float16)
    res = _cuda(rng.standard_normal((rows, O)), torch.float16)
    ref_b = ref + _np(bias.float()).astype(np.float64)
    out = torch.empty(rows, O, device="cuda", dtype=torch.float16)
    mm4_matmul_into(xd, *q[:5], out, bias=bias, epilogue=EPI_RELU2)
    torch.cuda.synchronize()
    r2 = np.maximum(ref_b, 0) ** 2
    assert _rel_err(_np(out).astype(np.float64), r2) <= _TOL[torch.float16]
    out2 = res.clone()  # y aliases the residual
    mm4_matmul_into(xd, *q[:5], out2, bias=bias, residual=out2, epilogue=EPI_RESIDUAL)
    torch.cuda.synchronize()
    ra = ref_b + _np(res.float()).astype(np.float64)
    assert _rel_err(_np(out2).astype(np.float64), ra) <= _TOL[torch.float16]


@pytest.mark.parametrize("name", ["f16_24x41", "f16_41x23", "f16_7x5", "f32_33x33", "f32_256x128"])
def test_mm4_reference_layout_on_reference_packed_bytes(oracle, name):
    """The fused kernel over the bytes and scales the reference packer wrote
    (committed fixture), against the fp64 dequantisation of those bytes."""
    from quant_golden import case, cases
    from rwkv7mi import mm4_matmul_triton

    if name not in cases("mm4"):
        pytest.skip(f"fixture has no case {name}")
    c = case("mm4", name)
    dtype = torch.float16 if name.startswith("f16") else torch.float32
    m, m_pad = (int(v) for v in c["m"])
    I = int(c["packed"].shape[0])
    assert int(c["packed"].shape[1]) * 2 == m_pad
    rng = np.random.default_rng(I * 31 + m)
    x = _cuda(rng.standard_normal((3, I)), dtype)
    meta = [_cuda(c[k], dtype) for k in ("mx", "rx", "my", "ry")]
    y = mm4_matmul_triton(x, _cuda(c["packed"], torch.uint8), *meta, m)
    torch.cuda.synchronize()
    ref = _np(x.float()).astype(np.float64) @ oracle.mm4_dequant(c["packed"], c["mx"], c["rx"], c["my"], c["ry"], m)
    assert _rel_err(_np(y.float()).astype(np.float64), ref) <= _TOL[dtype]


def test_mm4_reference_layout_routing(oracle):
    from rwkv7mi import mm4_matmul, mm4_matmul_triton
    from rwkv7mi.native_quant_mm4 import MM4_FUSED_MAX_ROWS, mm4_batched_dot_triton

    I, O = 512, 96
    q, xd, ref = _fused_case(oracle, I, O, MM4_FUSED_MAX_ROWS + 3, torch.float16, 21)
    big = mm4_matmul_triton(xd, *q[:5], q[5])  # above the fused row limit: dequantise + GEMM
    assert torch.equal(big, mm4_matmul(xd, *q[:5], q[5]))
    capped = mm4_matmul_triton(xd[:8], *q[:5], q[5], max_gemv_rows=4)
    assert torch.equal(capped, mm4_matmul(xd[:8], *q[:5], q[5]))
    fused = mm4_matmul_triton(xd[:8], *q[:5], q[5])
    x3 = xd[:8].reshape(2, 4, I)
    y3 = mm4_matmul_triton(x3, *q[:5], q[5])
    torch.cuda.synchronize()
    assert y3.shape == (2, 4, O)
    for y in (big, fused):
        assert _rel_err(_np(y).astype(np.float64), ref[: y.shape[0]]) <= _TOL[torch.float16]
    with pytest.raises(TypeError):
        mm4_batched_dot_triton(xd.float(), *q[:5], q[5])
    with pytest.raises(RuntimeError):
        mm4_batched_dot_triton(xd[0], *q[:5], q[5])
    with pytest.raises(ValueError):
        mm4_matmul_triton(xd[:8, :-2], *q[:5], q[5])
