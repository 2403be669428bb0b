"""GPU parity of the blocked MM8 decode path: the packer from Linear.weight is
bit-identical to the row-major packer (and so to the oracle), the blocked byte
layout matches its numpy restatement and round-trips to the reference w_u8,
the fused GEMV / small-batch GEMM matches the fp64 oracle, the grouped launch
equals single launches bit for bit, and the blocked dequantisation equals the
row-major one."""
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


@pytest.mark.parametrize("OI", [(256, 128), (128, 256), (1024, 4096), (40, 48), (3, 16)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
def test_pack_outmajor_equals_rowmajor(oracle, OI, dtype):
    from rwkv7mi.native_quant_mm8 import is_out_major, quantize_mm8, quantize_mm8_outmajor

    O, I = OI
    rng = np.random.default_rng(O * 7 + I)
    Wl = _cuda(rng.standard_normal((O, I)) * 0.02, dtype)  # Linear.weight [out, in]
    a = quantize_mm8(Wl.t().contiguous())
    b = quantize_mm8_outmajor(Wl)
    torch.cuda.synchronize()
    assert is_out_major(b[0]) and b[0].shape == (I, O)
    for x, y in zip(a, b):
        assert x.shape == y.shape
        assert torch.equal(x, y)
    if dtype == torch.float32:
        q, *_ = oracle.mm8_pack(_np(Wl.t().contiguous()), out_dtype=np.float32)
        np.testing.assert_array_equal(_np(b[0]), q)


def _block_np(w_u8):
    """numpy restatement of the blocked decode layout of w_u8 [I, O]."""
    I, O = w_u8.shape
    G, KB = (O + 15) // 16, (I + 127) // 128
    P = np.zeros((G * 16, KB * 128), np.uint8)
    P[:O, :I] = w_u8.T
    # tile (g, b), byte 1024 h + 16 (16 q + c) + e  <-  output 16 g + c, input 128 b + 64 h + 16 q + e
    return P.reshape(G, 16, KB, 2, 4, 16).transpose(0, 2, 3, 4, 1, 5).reshape(G, KB, 2048)


@pytest.mark.parametrize("OI", [(256, 128), (128, 256), (1024, 4096), (40, 48), (3, 16), (200, 1040)])
def test_block_layout_round_trip(OI):
    from rwkv7mi.native_quant_mm8 import is_blocked, mm8_block, mm8_unblock, quantize_mm8_blocked, quantize_mm8_outmajor

    O, I = OI
    rng = np.random.default_rng(O + 3 * I)
    Wl = _cuda(rng.standard_normal((O, I)) * 0.02, torch.float16)
    w_om, *meta = quantize_mm8_outmajor(Wl)
    w_blk, *meta2 = quantize_mm8_blocked(Wl)
    torch.cuda.synchronize()
    assert is_blocked(w_blk)
    for a, b in zip(meta, meta2):
        assert torch.equal(a, b)
    ref = _block_np(_np(w_om))
    np.testing.assert_array_equal(_np(w_blk), ref)
    # from the reference's row-major [I, O] and back
    np.testing.assert_array_equal(_np(mm8_block(w_om.contiguous())), ref)
    np.testing.assert_array_equal(_np(mm8_unblock(w_blk, I, O)), _np(w_om))


SHAPES = [(4096, 4096), (4096, 1024), (16384, 512), (144, 40), (1024, 65), (16, 16)]
# the RWKV-7 1.5B projection and head shapes at batch 1, 8, 32
C3 = [(2048, 2048), (2048, 8192), (8192, 2048), (2048, 65536)]


@pytest.mark.parametrize("IO", SHAPES)
@pytest.mark.parametrize("rows", [1, 2, 5, 8, 16, 17, 40, 64])
def test_mm8t_matmul_matches_oracle(oracle, IO, rows):
    from rwkv7mi.native_quant_mm8 import mm8_matmul, mm8_unblock, quantize_mm8_blocked

    I, O = IO
    rng = np.random.default_rng(I * 3 + O + rows)
    Wl = _cuda(rng.standard_normal((O, I)) * 0.02, torch.float16)
    packed = quantize_mm8_blocked(Wl)
    x = rng.standard_normal((rows, I)).astype(np.float16)
    xt = _cuda(x, torch.float16)
    y = mm8_matmul(xt, *packed)
    y2 = mm8_matmul(xt, *packed)
    torch.cuda.synchronize()
    w_u8 = mm8_unblock(packed[0], I, O)
    ref = oracle.mm8_matmul(x.astype(np.float64), *(_np(p) for p in (w_u8, *packed[1:])))
    err = _rel_err(_np(y).astype(np.float64), ref)
    assert err <= 2e-3, err
    assert torch.equal(y, y2), "repeated calls must be bit-identical"


@pytest.mark.parametrize("IO", C3)
@pytest.mark.parametrize("rows", [1, 8, 32])
def test_mm8t_c3_shapes(oracle, IO, rows):
    test_mm8t_matmul_matches_oracle(oracle, IO, rows)


@pytest.mark.parametrize("act", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("meta", [torch.float32, torch.float16])
def test_mm8t_dtypes(oracle, act, meta):
    from rwkv7mi.native_quant_mm8 import mm8_matmul, quantize_mm8_outmajor

    I, O, rows = 2048, 768, 6
    rng = np.random.default_rng(11)
    Wl = _cuda(rng.standard_normal((O, I)) * 0.02, meta)
    packed = quantize_mm8_outmajor(Wl)
    x = _cuda(rng.standard_normal((rows, I)), act)
    y = mm8_matmul(x, *packed)
    torch.cuda.synchronize()
    ref = oracle.mm8_matmul(_np(x.float()).astype(np.float64), *(_np(p.float()) if p.is_floating_point() else _np(p)
                                                                   for p in packed))
    tol = 1e-4 if act == torch.float32 else 8e-3  # x' staged as fp16 hi + lo (fp16 alone: ~2e-4)
    err = _rel_err(_np(y.float()).astype(np.float64), ref)
    assert err <= tol, (act, meta, err)


def test_mm8t_epilogues_in_place_and_module(oracle):
    from rwkv7mi import MM8Linear
    from rwkv7mi.native_quant_mm8 import is_blocked

    rng = np.random.default_rng(5)
    I, O, rows = 1024, 4096, 3
    lin = torch.nn.Linear(I, O, bias=True).to(device="cuda", dtype=torch.float16)
    with torch.no_grad():
        lin.weight.copy_(_cuda(rng.standard_normal((O, I)) * 0.02, torch.float16))
        lin.bias.copy_(_cuda(rng.standard_normal(O) * 0.1, torch.float16))
    mod = MM8Linear(lin)
    assert is_blocked(mod.w_blk) and mod.rwkv7_workspace_bytes(rows) == 0
    assert tuple(mod.w_u8.shape) == (I, O) and mod.w_u8.is_contiguous()
    x = _cuda(rng.standard_normal((rows, I)), torch.float16)
    res = _cuda(rng.standard_normal((rows, O)), torch.float16)
    packed = [_np(b) for b in (mod.w_u8, mod.mx, mod.rx, mod.my, mod.ry)]
    base = oracle.mm8_matmul(_np(x).astype(np.float64), *packed) + _np(lin.bias).astype(np.float64)
    y = mod(x)
    relu2 = mod.rwkv7_forward_relu2(x)
    acc = res.clone()
    mod._run(x, out=acc, residual=acc, epilogue=2)  # y aliases the residual
    torch.cuda.synchronize()
    scale = np.abs(base).max()
    assert np.abs(_np(y) - base).max() <= 2e-3 * scale
    r2 = np.maximum(base, 0) ** 2
    assert np.abs(_np(relu2) - r2).max() <= 4e-3 * np.abs(r2).max()
    add = base + _np(res).astype(np.float64)
    assert np.abs(_np(acc) - add).max() <= 2e-3 * np.abs(add).max()
    # the state dict holds the reference's keys and layout, and loads back
    sd = {k: v.clone() for k, v in mod.state_dict().items()}
    assert set(sd) == {"w_u8", "mx", "rx", "my", "ry", "bias"}
    assert tuple(sd["w_u8"].shape) == (I, O) and torch.equal(sd["w_u8"], mod.w_u8)
    mod2 = MM8Linear(lin)
    with torch.no_grad():
        mod2.w_blk.zero_()
    mod2.load_state_dict(sd)
    assert torch.equal(mod2.w_blk, mod.w_blk)
    with pytest.raises(RuntimeError):
        mod2.load_state_dict({k: v for k, v in sd.items() if k != "w_u8"})


@pytest.mark.parametrize("rows", [1, 8, 20])
def test_mm8t_multi_equals_single(rows):
    from rwkv7mi import MM8Linear
    from rwkv7mi.native_quant_mm8 import mm8_matmul_multi_into

    rng = np.random.default_rng(rows)
    I, O = 512, 384
    mods, xs = [], []
    for p in range(3):
        lin = torch.nn.Linear(I, O, bias=(p == 1)).to(device="cuda", dtype=torch.float16)
        with torch.no_grad():
            lin.weight.copy_(_cuda(rng.standard_normal((O, I)) * 0.02, torch.float16))
        mods.append(MM8Linear(lin))
        xs.append(_cuda(rng.standard_normal((rows, I)), torch.float16))
    outs = [torch.empty(rows, O, device="cuda", dtype=torch.float16) for _ in range(3)]
    mm8_matmul_multi_into(xs, mods, outs)
    single = []  # one-problem launches of the same kernel (the module routes > 16 rows elsewhere)
    for m, x in zip(mods, xs):
        o = torch.empty(rows, O, device="cuda", dtype=torch.float16)
        mm8_matmul_multi_into([x], [m], [o])
        single.append(o)
    torch.cuda.synchronize()
    for a, b in zip(outs, single):
        assert torch.equal(a, b)


_LORA_TAIL_CASES = [(8, 4096, 4096, (64, 64, 128, 32), 4), (2, 512, 384, (64, 64, 128), 4),
                    (16, 1024, 256, (16, 8, 256, 24), 3), (3, 4096, 1024, (64,), 1),
                    (64, 4096, 4096, (64, 64, 128, 32), 8), (24, 1024, 512, (64, 64, 128), 4),
                    (41, 2048, 384, (16, 8, 256, 24), 3)]


# fp16 at every shape; bf16 and fp32 at one GEMV (8 rows) and one tile-GEMM (24 rows) shape
@pytest.mark.parametrize("rows,I,O,ranks,splits,dt",
                         [c + (torch.float16,) for c in _LORA_TAIL_CASES]
                         + [c + (dt,) for c in _LORA_TAIL_CASES if c[0] in (8, 24)
                            for dt in (torch.bfloat16, torch.float32)])
def test_mm8t_multi_lora_tail(rows, I, O, ranks, splits, dt):
    """The grouped GEMV (up to 16 rows) or tile GEMM (17..64) with the LoRA down
    projections as tail workgroups: the products equal the plain grouped launch bit for bit, and the down partials
    summed over the K ranges match an fp32 torch product (the reference's
    ``x @ W_down^T``, rwkv7_hf/fused_lora.py:795-803) on the same operands
    (fp32 and bf16 ones split into fp16 hi + lo, ~2^-22 relative)."""
    from rwkv7mi import MM8Linear
    from rwkv7mi.native_quant_mm8 import mm8_gemm_multi_into, mm8_matmul_multi_into, mm8_matmul_multi_lora_into

    rng = np.random.default_rng(rows * 131 + I + len(ranks))
    mods, xs = [], []
    for p in range(3):
        lin = torch.nn.Linear(I, O, bias=(p == 1)).to(device="cuda", dtype=dt)
        with torch.no_grad():
            lin.weight.copy_(_cuda(rng.standard_normal((O, I)) * 0.02, dt))
        mods.append(MM8Linear(lin))
        xs.append(_cuda(rng.standard_normal((rows, I)), dt))
    lxs = [_cuda(rng.standard_normal((rows, I)), dt) for _ in ranks]
    lws = [_cuda(rng.standard_normal((r, I)) * 0.05, dt) for r in ranks]
    part = torch.full((splits * rows * sum(ranks) + 7,), float("nan"), device="cuda", dtype=torch.float32)
    outs = [torch.empty(rows, O, device="cuda", dtype=dt) for _ in range(3)]
    plain = [torch.empty(rows, O, device="cuda", dtype=dt) for _ in range(3)]
    mm8_matmul_multi_lora_into(xs, mods, outs, lxs, lws, part, splits=splits)
    (mm8_matmul_multi_into if rows <= 16 else mm8_gemm_multi_into)(xs, mods, plain)
    torch.cuda.synchronize()
    for a, b in zip(outs, plain):
        assert torch.equal(a, b)
    off = 0
    for lx, lw, r in zip(lxs, lws, ranks):
        got = part[off:off + splits * rows * r].view(splits, rows, r).sum(0)
        ref = lx.float() @ lw.float().t()
        err = (got - ref).abs().max().item() / ref.abs().max().item()
        assert err < 1e-5, (r, err)
        off += splits * rows * r
    assert torch.isnan(part[off:]).all()  # nothing past the partials


def test_mm8t_multi_lora_rejects():
    from rwkv7mi import MM8Linear
    from rwkv7mi.native_quant_mm8 import mm8_matmul_multi_lora_into

    I, O = 256, 128
    lin = torch.nn.Linear(I, O, bias=False).to(device="cuda", dtype=torch.float16)
    m = MM8Linear(lin)
    x = torch.randn(2, I, device="cuda", dtype=torch.float16)
    out = torch.empty(2, O, device="cuda", dtype=torch.float16)
    lw = torch.randn(64, I, device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError):  # partial buffer too small
        mm8_matmul_multi_lora_into([x], [m], [out], [x], [lw], torch.empty(10, device="cuda"), splits=4)
    with pytest.raises(ValueError):  # rank not a multiple of 8
        mm8_matmul_multi_lora_into([x], [m], [out], [x], [lw[:60].contiguous()],
                                   torch.empty(4096, device="cuda"), splits=4)
    x65 = torch.randn(65, I, device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError):  # more than 64 rows
        mm8_matmul_multi_lora_into([x65], [m], [torch.empty(65, O, device="cuda", dtype=torch.float16)], [x65], [lw],
                                   torch.empty(65536, device="cuda"), splits=4)


@pytest.mark.parametrize("IO", [(256, 512), (4096, 1024)])
def test_mm8t_dequant_equals_rowmajor(IO):
    from rwkv7mi import _lib
    from rwkv7mi.native_quant_mm8 import mm8_block, quantize_mm8_outmajor

    I, O = IO
    rng = np.random.default_rng(I)
    Wl = _cuda(rng.standard_normal((O, I)) * 0.02, torch.float16)
    w_om, mx, rx, my, ry = quantize_mm8_outmajor(Wl)
    w = mm8_block(w_om)
    a = torch.empty(O, I, device="cuda", dtype=torch.float16)
    b = torch.empty(I, O, device="cuda", dtype=torch.float16)
    s = _lib.stream_of(a)
    _lib.call("rwkv7mi_mm8t_dequant", _lib.ptr(w), _lib.ptr(mx), _lib.ptr(rx), _lib.ptr(my), _lib.ptr(ry),
              _lib.ptr(a), I, O, _lib.F16, _lib.F16, s)
    wc = w_om.contiguous()
    _lib.call("rwkv7mi_mm8_dequant", _lib.ptr(wc), _lib.ptr(mx), _lib.ptr(rx), _lib.ptr(my), _lib.ptr(ry),
              _lib.ptr(b), I, O, _lib.F16, _lib.F16, s)
    torch.cuda.synchronize()
    assert torch.equal(a.t(), b)


def test_mm8t_rejects_bad_shapes():
    from rwkv7mi import _lib

    x = torch.zeros(1, 24, device="cuda", dtype=torch.float16)
    w = torch.zeros(8, 24, device="cuda", dtype=torch.uint8)
    m8 = torch.zeros(8, device="cuda", dtype=torch.float16)
    m24 = torch.zeros(24, device="cuda", dtype=torch.float16)
    y = torch.zeros(1, 8, device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError, match="multiple of 16"):
        _lib.call("rwkv7mi_mm8t_matmul", _lib.ptr(x), _lib.ptr(w), _lib.ptr(m8), _lib.ptr(m8), _lib.ptr(m24),
                  _lib.ptr(m24), None, None, _lib.ptr(y), 1, 24, 8, 0, _lib.F16, _lib.F16, _lib.stream_of(x))


def _round(a, dtype):
    return _np(torch.tensor(a, dtype=torch.float64).to(dtype).to(torch.float64))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", [
    # (rows, I, O, nprob, naux, epilogue): the 7.2B R/K/V and FFN-key shapes,
    # the 1.5B ones, a ragged width
    (1, 4096, 4096, 3, 4, 0), (2, 4096, 4096, 3, 3, 0), (1, 4096, 16384, 1, 0, 1), (2, 4096, 16384, 1, 0, 1),
    (1, 2048, 2048, 3, 4, 0), (2, 2048, 8192, 1, 0, 1), (4, 2048, 2048, 2, 2, 0), (3, 1024, 200, 2, 1, 0),
])
def test_mm8t_lnmix_matches_oracle_and_unfused(oracle, dtype, case):
    """LN + token-shift mix inside the GEMV (the decode form of
    fused_decode_norm_mix.py:161 / :296 feeding MM8Linear) against the fp64
    oracle (LN, h rounded, mix rounded, dequant product) and against the
    unfused mix kernel + grouped GEMV."""
    from rwkv7mi import MM8Linear, _lib
    from rwkv7mi.fused_decode_norm_mix import fused_attn_norm_mix6_decode
    from rwkv7mi.native_quant_mm8 import mm8_lnmix_multi_into, mm8_matmul_multi_into

    rows, I, O, k, na, epi = case
    rng = np.random.default_rng(rows * 131 + I + O + k)
    # a residual stream with an offset and a few large channels
    xr = rng.standard_normal((rows, I)) * 2.0 + 3.0
    xr[:, :: max(I // 7, 1)] *= 20.0
    x = _cuda(xr, dtype)
    prev = _cuda(rng.standard_normal((rows, I)), dtype)
    lnw = _cuda(1.0 + 0.2 * rng.standard_normal(I), dtype)
    lnb = _cuda(0.1 * rng.standard_normal(I), dtype)
    mixes = [_cuda(rng.uniform(0, 1, I), dtype) for _ in range(k + na)]
    mods = []
    for _ in range(k):
        lin = torch.nn.Linear(I, O, bias=False).to(device="cuda", dtype=dtype)
        with torch.no_grad():
            lin.weight.copy_(_cuda(rng.standard_normal((O, I)) * 0.02, dtype))
        mods.append(MM8Linear(lin))
    outs = [torch.full((rows, O), float("nan"), device="cuda", dtype=dtype) for _ in range(k)]
    h_out = torch.full((rows, I), float("nan"), device="cuda", dtype=dtype)
    aux = [torch.full((rows, I), float("nan"), device="cuda", dtype=dtype) for _ in range(na)]
    prev0 = prev.clone()
    epis = [_lib.EPI_RELU2 if epi else _lib.EPI_NONE] * k
    # the decode LoRA's down projections of the extra mixes (rows <= 2)
    ranks = [64, 64, 128, 32][:na] if rows <= 2 else []
    downs = [_cuda(rng.standard_normal((rr, I)) * 0.05, dtype) for rr in ranks]
    lora_out = torch.full((rows * sum(ranks) + 7,), float("nan"), device="cuda", dtype=torch.float32)
    mm8_lnmix_multi_into(x, prev, lnw, lnb, 1e-5, mixes[:k], mods, outs, epilogues=epis, h_out=h_out,
                         aux_mixes=mixes[k:], aux_outs=aux, lora_downs=downs if ranks else None,
                         lora_out=lora_out if ranks else None)
    again = [torch.empty_like(o) for o in outs]
    mm8_lnmix_multi_into(x, prev, lnw, lnb, 1e-5, mixes[:k], mods, again, epilogues=epis)
    torch.cuda.synchronize()
    assert torch.equal(prev, prev0), "prev is only read"
    for a, b in zip(outs, again):
        assert torch.equal(a, b), "repeated calls must be bit-identical"

    # fp64 oracle
    f = lambda t: _np(t.double())
    outs_ref, h_ref = oracle.attn_norm_mix6(f(x), f(prev), f(lnw), f(lnb), [f(m) for m in mixes])
    h_r = _round(h_ref, dtype)
    mixed = [_round(h_r + (f(prev) - h_r) * f(m), dtype) for m in mixes]
    tol_h = 1e-2 if dtype == torch.float16 else 4e-2
    assert np.abs(f(h_out) - h_r).max() <= tol_h * max(np.abs(h_r).max(), 1.0)
    for a in range(na):
        assert np.abs(f(aux[a]) - mixed[k + a]).max() <= tol_h * max(np.abs(mixed[k + a]).max(), 1.0)
    # LoRA down sums: [problem][row][j], fp32 over the mixes as written (rounded)
    off = 0
    for a, rr in enumerate(ranks):
        got = _np(lora_out[off:off + rows * rr]).reshape(rows, rr).astype(np.float64)
        ref = f(aux[a]) @ f(downs[a]).T
        assert np.abs(got - ref).max() <= 1e-4 * max(np.abs(ref).max(), 1.0), (a, np.abs(got - ref).max())
        off += rows * rr
    if ranks:
        assert torch.isnan(lora_out[off:]).all(), "nothing past the sums is written"
    for p in range(k):
        packed = [_np(b.float()) if b.is_floating_point() else _np(b)
                  for b in (mods[p].w_u8, mods[p].mx, mods[p].rx, mods[p].my, mods[p].ry)]
        ref = oracle.mm8_matmul(mixed[p], *packed)
        if epi:
            ref = np.maximum(ref, 0) ** 2
        tol = (2e-3 if dtype == torch.float16 else 8e-3) * (2 if epi else 1)
        assert _rel_err(f(outs[p]), ref) <= tol, p

    # the unfused route: mix kernel (six slots), then the grouped GEMV
    slots = torch.empty(6, rows, I, device="cuda", dtype=dtype)
    pv = prev.clone()
    six = (mixes + [mixes[0]] * 6)[:6]
    fused_attn_norm_mix6_decode(x, pv, lnw, lnb, *six, eps=1e-5, out=slots)
    ref_outs = [torch.empty_like(o) for o in outs]
    mm8_matmul_multi_into([slots[p] for p in range(k)], mods, ref_outs, epilogues=epis)
    torch.cuda.synchronize()
    # the statistics are summed in another order: h may differ by one unit
    # in the last place in a few elements, and the products by as little
    assert (h_out != pv).float().mean().item() < 0.02
    hd = (h_out.double() - pv.double()).abs().max().item()
    assert hd <= tol_h * max(pv.double().abs().max().item(), 1.0)
    for p in range(k):
        d = (outs[p].double() - ref_outs[p].double()).abs().max().item()
        assert d <= 4e-3 * max(ref_outs[p].double().abs().max().item(), 1.0), (p, d)


def test_mm8t_lnmix_rejects_unsupported():
    from rwkv7mi import MM8Linear, _lib
    from rwkv7mi.native_quant_mm8 import mm8_lnmix_multi_into

    I, O = 4096, 256
    lin = torch.nn.Linear(I, O, bias=False).to(device="cuda", dtype=torch.float16)
    mod = MM8Linear(lin)
    v = torch.ones(I, device="cuda", dtype=torch.float16)
    for rows in (4, 9, 16):  # the rows no longer fit one staging batch
        x = torch.zeros(rows, I, device="cuda", dtype=torch.float16)
        out = torch.empty(rows, O, device="cuda", dtype=torch.float16)
        with pytest.raises(ValueError, match="staging batch"):
            mm8_lnmix_multi_into(x, x.clone(), v, v, 1e-5, [v], [mod], [out])
    x = torch.zeros(2, I, device="cuda", dtype=torch.float16)
    out = torch.empty(2, O, device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError, match="residual"):
        mm8_lnmix_multi_into(x, x.clone(), v, v, 1e-5, [v], [mod], [out], epilogues=[_lib.EPI_RESIDUAL])
    with pytest.raises(ValueError):
        mm8_lnmix_multi_into(x, x, v, v, 1e-5, [v], [mod], [out], h_out=x)


@pytest.mark.parametrize("IO,rows", [((16384, 1024), 8), ((4096, 2048), 16), ((16384, 4096), 3)])
def test_mm8t_split_k_epilogues(oracle, IO, rows):
    """Rows whose x' exceeds one LDS chunk take split K (ranges of one chunk,
    fp32 partials added in order by a second launch): bias, relu^2 and residual
    epilogues against the fp64 oracle, and repeated calls bit-identical."""
    from rwkv7mi import MM8Linear
    from rwkv7mi.native_quant_mm8 import mm8t_workspace_bytes

    I, O = IO
    assert mm8t_workspace_bytes(1, rows, I, O) > 0, "this shape must take the split-K route"
    rng = np.random.default_rng(I + O + rows)
    lin = torch.nn.Linear(I, O, bias=True).to(device="cuda", dtype=torch.float16)
    with torch.no_grad():
        lin.weight.copy_(_cuda(rng.standard_normal((O, I)) * 0.02, torch.float16))
        lin.bias.copy_(_cuda(rng.standard_normal(O) * 0.1, torch.float16))
    m = MM8Linear(lin)
    x = _cuda(rng.standard_normal((rows, I)), torch.float16)
    res = _cuda(rng.standard_normal((rows, O)), torch.float16)
    y = m(x)
    y2 = m(x)
    r2 = m.rwkv7_forward_relu2(x)
    ad = m.rwkv7_forward_add(x, res)
    torch.cuda.synchronize()
    wd = oracle.mm8_dequant(*(_np(t) for t in (m.w_u8, m.mx, m.rx, m.my, m.ry)))
    ref = _np(x).astype(np.float64) @ wd + _np(m.bias).astype(np.float64)
    assert _rel_err(_np(y).astype(np.float64), ref) <= 2e-3
    assert torch.equal(y, y2)
    assert _rel_err(_np(r2).astype(np.float64), np.maximum(ref, 0) ** 2) <= 4e-3
    assert _rel_err(_np(ad).astype(np.float64), ref + _np(res).astype(np.float64)) <= 2e-3
