"""GPU parity: the opt-in fp16-state recurrence (csrc/wkv7_f16.hip) vs the fp16 oracle.

The state math is packed fp16 FMAs in a fixed order, so with inputs whose
fp32-computed operands (decay delta, kk, k) round to fp16 away from rounding
midpoints (oracle.wkv7_fp16_oracle.safe_w / safe_decode_inputs) the new state
and the sequence readout must equal the oracle to the bit.  With unrestricted
inputs a few operands may round the other way in the last fp16 place; there
the bar is the build's fp16-output tolerance (max-abs <= 1e-2) on outputs and
the state.  The decode output (fp32 GroupNorm over the fp16 readout, summed in
a different order) is held to max-abs <= 1e-2 throughout.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import wkv7_fp16_oracle as o

pytestmark = pytest.mark.gpu

OUT_ABS = 1e-2
F16 = np.float16


def _t(x, dtype=torch.float16):
    return torch.tensor(np.asarray(x), dtype=dtype, device="cuda")


def _np(t):
    return t.detach().cpu().numpy()


def _decode_case(rng, B, H, safe, N=64):
    if safe:
        k_raw, a, k_k, k_a = o.safe_decode_inputs(rng, B, H)
    else:
        k_k = (1.0 + 0.1 * rng.standard_normal(H * N)).astype(F16)
        k_a = rng.uniform(0.0, 1.0, H * N).astype(F16)
        k_raw = rng.standard_normal((B, H, N)).astype(F16)
        a = rng.uniform(0.0, 1.0, (B, H, N)).astype(F16)
    elapsed = rng.integers(0, 5000, B).astype(np.int32)
    ph = o.phases(elapsed, H, N)
    w_raw = o.safe_w(rng, (B, H, N), ph) if safe else rng.standard_normal((B, H, N)).astype(F16)
    r, v, g = (rng.standard_normal((B, H, N)).astype(F16) for _ in range(3))
    r_k = (rng.standard_normal(H * N) * 0.5).astype(F16)
    gn_w = (1.0 + 0.1 * rng.standard_normal(H * N)).astype(F16)
    gn_b = (0.1 * rng.standard_normal(H * N)).astype(F16)
    state = (rng.standard_normal((B, H, N, N)) * 0.5).astype(F16)
    return dict(r=r, w_raw=w_raw, k_raw=k_raw, v=v, a=a, state=state, g=g, k_k=k_k, k_a=k_a, r_k=r_k,
                gn_w=gn_w, gn_b=gn_b, elapsed=elapsed)


def _run_decode(c, advance, eps=1e-5):
    from rwkv7mi import native_fp16_recurrent_output_prepare_raw

    st = _t(c["state"])
    el = _t(c["elapsed"], torch.int32)
    out = native_fp16_recurrent_output_prepare_raw(
        _t(c["r"]), _t(c["w_raw"]), _t(c["k_raw"]), _t(c["v"]), _t(c["a"]), st, _t(c["g"]), _t(c["k_k"]),
        _t(c["k_a"]), _t(c["r_k"]), _t(c["gn_w"]), _t(c["gn_b"]), el, advance_elapsed=advance, eps=eps)
    torch.cuda.synchronize()
    return _np(out), _np(st), _np(el)


def _oracle_decode(c, eps=1e-5):
    return o.decode_output_prepare_raw(c["r"], c["w_raw"], c["k_raw"], c["v"], c["a"], c["state"], c["g"],
                                       c["k_k"], c["k_a"], c["r_k"], c["gn_w"], c["gn_b"], c["elapsed"], eps)


@pytest.mark.parametrize("B,H", [(1, 4), (3, 5), (8, 64)])
def test_fp16_decode_state_is_bit_exact(B, H):
    rng = np.random.default_rng(900 + B * H)
    c = _decode_case(rng, B, H, safe=True)
    out, st, el = _run_decode(c, advance=False)
    ref_out, ref_st = _oracle_decode(c)
    print(f"PARITY fp16 decode B={B} H={H}: state bits equal {np.mean(st == ref_st):.6f}, "
          f"out max-abs {np.abs(out.astype(np.float64) - ref_out).max():.3g}", flush=True)
    np.testing.assert_array_equal(st, ref_st)
    assert np.abs(out.astype(np.float64) - ref_out.astype(np.float64)).max() <= OUT_ABS
    np.testing.assert_array_equal(el, c["elapsed"])  # not advanced


@pytest.mark.parametrize("B,H", [(2, 3), (16, 32)])
def test_fp16_decode_unrestricted_inputs(B, H):
    rng = np.random.default_rng(950 + B * H)
    c = _decode_case(rng, B, H, safe=False)
    out, st, _ = _run_decode(c, advance=False)
    ref_out, ref_st = _oracle_decode(c)
    same = np.mean(st == ref_st)
    err = np.abs(st.astype(np.float64) - ref_st.astype(np.float64)).max()
    print(f"PARITY fp16 decode unrestricted B={B} H={H}: state bits equal {same:.6f}, max-abs {err:.3g}",
          flush=True)
    assert same >= 0.98
    assert err <= OUT_ABS
    assert np.abs(out.astype(np.float64) - ref_out.astype(np.float64)).max() <= OUT_ABS


def test_fp16_decode_advances_elapsed_after_every_head_read_it():
    rng = np.random.default_rng(977)
    B, H = 4, 48  # many heads per batch row
    c = _decode_case(rng, B, H, safe=True)
    out, st, el = _run_decode(c, advance=True)
    ref_out, ref_st = _oracle_decode(c)
    np.testing.assert_array_equal(el, c["elapsed"] + 1)
    np.testing.assert_array_equal(st, ref_st)  # every head used the pre-advance phase
    # a second step continues from the moved phase
    c2 = dict(c, state=st, elapsed=el)
    c2["w_raw"] = o.safe_w(rng, (B, H, 64), o.phases(el, H))
    _, st2, el2 = _run_decode(c2, advance=True)
    _, ref_st2 = _oracle_decode(c2)
    np.testing.assert_array_equal(st2, ref_st2)
    np.testing.assert_array_equal(el2, c["elapsed"] + 2)


def _seq_case(rng, B, T, H, w0=False, N=64):
    elapsed = rng.integers(0, 3000, B).astype(np.int32)
    ph = o.phases(elapsed, H, N)[:, None] + np.arange(T).reshape(1, T, 1, 1)
    w0v = (rng.standard_normal(H * N) * 0.5).astype(F16) if w0 else None
    w = o.safe_w(rng, (B, T, H, N), ph, None if w0v is None else w0v.astype(np.float32).reshape(1, 1, H, N))
    r, v = (rng.standard_normal((B, T, H, N)).astype(F16) for _ in range(2))
    k = (rng.standard_normal((B, T, H, N)) * 0.3).astype(F16)
    kk = rng.standard_normal((B, T, H, N))
    kk = kk / np.linalg.norm(kk, axis=-1, keepdims=True)
    a = rng.uniform(0.0, 1.0, (B, T, H, N))
    state = (rng.standard_normal((B, H, N, N)) * 0.5).astype(F16)
    return dict(r=r, w=w, k=k, v=v, neg_kk=(-kk).astype(F16), kka=(kk * a).astype(F16), state=state,
                elapsed=elapsed, w0=w0v)


def _run_seq(c):
    from rwkv7mi import native_fp16_sequence

    st = _t(c["state"])
    el = _t(c["elapsed"], torch.int32)
    y = native_fp16_sequence(_t(c["r"]), _t(c["w"]), _t(c["k"]), _t(c["v"]), _t(c["neg_kk"]), _t(c["kka"]), st,
                             el, w0=None if c["w0"] is None else _t(c["w0"]))
    torch.cuda.synchronize()
    return _np(y), _np(st), _np(el)


@pytest.mark.parametrize("B,T,H,w0", [(1, 1, 2, False), (2, 37, 3, False), (2, 37, 3, True), (3, 64, 4, True),
                                      (1, 9, 64, False)])
def test_fp16_sequence_is_bit_exact(B, T, H, w0):
    rng = np.random.default_rng(1000 + B * T * H + int(w0))
    c = _seq_case(rng, B, T, H, w0=w0)
    y, st, el = _run_seq(c)
    ref_y, ref_st = o.sequence(c["r"], c["w"], c["k"], c["v"], c["neg_kk"], c["kka"], c["state"], c["elapsed"],
                               w0=c["w0"])
    print(f"PARITY fp16 sequence B={B} T={T} H={H} w0={w0}: y bits equal {np.mean(y == ref_y):.6f}, "
          f"state bits equal {np.mean(st == ref_st):.6f}", flush=True)
    np.testing.assert_array_equal(st, ref_st)
    np.testing.assert_array_equal(y, ref_y)
    np.testing.assert_array_equal(el, c["elapsed"])  # the sequence reads elapsed only


def test_fp16_sequence_split_equals_one_call_at_full_size():
    """B=8, T=4096, H=64 (the scan benchmark's shape): one call equals two calls
    split at a slab-misaligned token with elapsed moved on, to the bit."""
    from rwkv7mi import native_fp16_sequence

    B, T, H, N = 8, 4096, 64, 64
    g = torch.Generator(device="cuda").manual_seed(5)
    rn = lambda s=1.0: (torch.randn(B, T, H, N, device="cuda", generator=g) * s).half()
    r, w, k, v = rn(), rn(), rn(0.3), rn()
    kk = torch.nn.functional.normalize(torch.randn(B, T, H, N, device="cuda", generator=g), dim=-1)
    a = torch.rand(B, T, H, N, device="cuda", generator=g)
    nkk, kka = (-kk).half().contiguous(), (kk * a).half().contiguous()
    s0 = (torch.randn(B, H, N, N, device="cuda", generator=g) * 0.5).half()
    el = torch.randint(0, 1000, (B,), device="cuda", dtype=torch.int32)
    st_a = s0.clone()
    y_a = native_fp16_sequence(r, w, k, v, nkk, kka, st_a, el)
    t1 = 1237
    st_b = s0.clone()
    part = lambda x, lo, hi: x[:, lo:hi].contiguous()
    y1 = native_fp16_sequence(*(part(x, 0, t1) for x in (r, w, k, v, nkk, kka)), st_b, el)
    y2 = native_fp16_sequence(*(part(x, t1, T) for x in (r, w, k, v, nkk, kka)), st_b, el + t1)
    torch.cuda.synchronize()
    assert torch.isfinite(y_a).all() and torch.isfinite(st_a).all()
    assert torch.equal(st_a, st_b)
    assert torch.equal(y_a, torch.cat([y1, y2], 1))


def test_fp16_sequence_one_token_matches_decode_state():
    """The decode kernel's state update equals the sequence kernel's on the
    same fp16 operands (k, -kk, kk*a formed as the decode kernel forms them)."""
    from rwkv7mi import native_fp16_sequence

    rng = np.random.default_rng(31)
    B, H = 3, 6
    c = _decode_case(rng, B, H, safe=True)
    _, st_dec, _ = _run_decode(c, advance=False)
    kh, nkk, b = o.decode_prep(c["k_raw"], c["a"], c["k_k"], c["k_a"])
    st = _t(c["state"])
    one = lambda x: _t(np.asarray(x)[:, None])
    native_fp16_sequence(one(c["r"]), one(c["w_raw"]), one(kh), one(c["v"]), one(nkk), one(b), st,
                         _t(c["elapsed"], torch.int32))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_np(st), st_dec)


def test_fp16_decode_v_interpolation_in_kernel_equals_torch_form():
    """v_mode 2 forms v + (v_first - v) * v_gate in-kernel with the roundings of
    the reference's fp16 torch ops; v_mode 1 stores v as v_first."""
    from rwkv7mi import native_fp16_recurrent_output_prepare_raw as op

    rng = np.random.default_rng(41)
    B, H = 3, 8
    c = _decode_case(rng, B, H, safe=False)
    vf = _t(rng.standard_normal((B, H, 64)))
    gate = _t(rng.uniform(0, 1, (B, H, 64)))
    args = lambda st, v: (_t(c["r"]), _t(c["w_raw"]), _t(c["k_raw"]), v, _t(c["a"]), st, _t(c["g"]), _t(c["k_k"]),
                          _t(c["k_a"]), _t(c["r_k"]), _t(c["gn_w"]), _t(c["gn_b"]), _t(c["elapsed"], torch.int32))
    v = _t(c["v"])
    st_a, st_b = _t(c["state"]), _t(c["state"])
    mixed = v + (vf - v) * gate  # fp16 torch ops, one rounding each
    out_a = op(*args(st_a, mixed.contiguous()), advance_elapsed=False, eps=1e-5)
    out_b = op(*args(st_b, v.clone()), advance_elapsed=False, eps=1e-5, v_first=vf, v_gate=gate, v_mode=2)
    vf1 = torch.zeros_like(v)
    st_c = _t(c["state"])
    op(*args(st_c, v), advance_elapsed=False, eps=1e-5, v_first=vf1, v_mode=1)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b) and torch.equal(st_a, st_b)
    assert torch.equal(vf1, v)
