"""Pins of the fp16-state oracle (oracle/wkv7_fp16_oracle.py), CPU only.

* fma16 / add16  vs exact rational arithmetic rounded to fp16 by hand
                 (round-half-even, subnormals); a planted unfused
                 multiply-then-add fails the same comparison
* dither         vs known answers of the 32-bit golden-ratio hash and its bound
* decay_delta    vs the fp64 closed form exp(-e^-1/2 sigmoid(w)) - 1 + dither
* row_step       from a zero state equals fp16(k_j v_i) to the bit; a full
                 decode step and a 16-token sequence agree with the fp64 DPLR
                 oracle (oracle.py) fed the same fp16 operands, with a planted
                 sign error in the low-rank term failing that comparison
* sequence       split at any token (elapsed moved on) equals one call to the
                 bit; w0 added in fp32 equals a pre-added w when the sum is exact
Also the product-side validation of rwkv7mi.native_wkv_fp16 that runs without
a GPU (the reference's tests/test_native_wkv_fp16.py:14-34, :83-101).
"""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import wkv7_fp16_oracle as o

F16 = np.float16


def _round16_exact(x: Fraction) -> float:
    """Round a rational to fp16, half to even, with subnormals (finite range only)."""
    if x == 0:
        return 0.0
    sign = -1 if x < 0 else 1
    ax = abs(x)
    e = ax.numerator.bit_length() - ax.denominator.bit_length()
    if Fraction(2) ** e > ax:
        e -= 1
    e = max(e, -14)                      # subnormal quantum 2^-24
    q = Fraction(2) ** (e - 10)
    m = ax / q
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * float(n * q)


def _random_f16(rng, n, lo_exp=-24, hi_exp=7):
    """Finite fp16 values spread over exponents, including subnormals."""
    mant = rng.integers(0, 1024, n)
    exp = rng.integers(lo_exp, hi_exp, n)
    sign = rng.choice([-1.0, 1.0], n)
    vals = sign * (1.0 + mant / 1024.0) * np.exp2(exp.astype(np.float64))
    sub = rng.random(n) < 0.05
    vals[sub] = sign[sub] * mant[sub] * 2.0 ** -24
    return vals.astype(F16)


def test_fma16_equals_exact_rational_rounding():
    rng = np.random.default_rng(11)
    n = 6000
    a, b = _random_f16(rng, n), _random_f16(rng, n)
    c = _random_f16(rng, n, -24, 12)
    # near-cancellation and near-midpoint cases: c close to -a*b
    k = n // 3
    c[:k] = (-(a[:k].astype(np.float64) * b[:k].astype(np.float64))).astype(F16)
    got = o.fma16(a, b, c)
    exact = np.array([_round16_exact(Fraction(float(x)) * Fraction(float(y)) + Fraction(float(z)))
                      for x, y, z in zip(a, b, c)])
    fin = np.isfinite(exact) & (np.abs(exact) <= 65504)
    assert fin.sum() > n * 0.9
    np.testing.assert_array_equal(got[fin].astype(np.float64), exact[fin])
    # a planted unfused form (product rounded to fp16 first) differs somewhere
    unfused = ((a.astype(np.float64) * b.astype(np.float64)).astype(F16).astype(np.float64)
               + c.astype(np.float64)).astype(F16)
    assert (unfused[fin].astype(np.float64) != exact[fin]).any()


def test_add16_equals_exact_rational_rounding():
    rng = np.random.default_rng(12)
    x, y = _random_f16(rng, 3000, -24, 14), _random_f16(rng, 3000, -24, 14)
    exact = np.array([_round16_exact(Fraction(float(p)) + Fraction(float(q))) for p, q in zip(x, y)])
    np.testing.assert_array_equal(o.add16(x, y).astype(np.float64), exact)


def test_dither_known_answers_and_bound():
    # int32(0x9E3779B9 * phase) rounded to fp32, times 2^-41
    known = {0: 0, 1: -1640531584, 2: 1013904256, 3: -626627264, 64: -1914802688,
             4095: -647752128, 2**31 - 1: -506952128, 12345678: -1646121088}
    for ph, val in known.items():
        assert float(o.dither(ph)) == val * 2.0 ** -41, ph
    assert float(o.dither(-1)) == 1640531584 * 2.0 ** -41  # phase wraps mod 2^32
    ph = np.random.default_rng(3).integers(0, 2**31, 100000)
    d = o.dither(ph)
    assert np.abs(d).max() <= 2.0 ** -10
    assert abs(float(d.astype(np.float64).mean())) < 2.0 ** -15  # centred


def test_decay_delta_closed_form():
    w = np.linspace(-8, 8, 4001).astype(F16).astype(np.float32)
    for phase in (np.zeros(w.shape, np.int64), np.arange(w.size, dtype=np.int64) * 977 + 5):
        got = o.decay_delta(w, phase).astype(np.float64)
        exact = (np.exp(-math.exp(-0.5) / (1.0 + np.exp(-w.astype(np.float64)))) - 1.0
                 + o.dither(phase).astype(np.float64))
        ulp = np.abs(np.spacing(exact.astype(F16))).astype(np.float64)
        assert np.all(np.abs(got - exact) <= 0.5 * ulp + 1e-6)
    # the delta falls from 0 toward exp(-e^-1/2) - 1 as w grows
    d0 = o.decay_delta(w, np.zeros(w.shape, np.int64)).astype(np.float64)
    assert np.all(np.diff(d0) <= 0) and d0[0] <= 0 and d0[-1] >= math.exp(-math.exp(-0.5)) - 1.0 - 1e-3


def test_row_step_from_zero_state_is_k_outer_v():
    rng = np.random.default_rng(5)
    B, H, N = 2, 3, 64
    vec = lambda s=1.0: (rng.standard_normal((B, H, N)) * s).astype(F16)
    r, wd, k, nkk, b, v = vec(), vec(0.1), vec(), vec(0.2), vec(0.2), vec()
    S2, y = o.row_step(np.zeros((B, H, N, N), F16), r, wd, k, nkk, b, v)
    kv = (v.astype(np.float64)[..., :, None] * k.astype(np.float64)[..., None, :]).astype(F16)
    np.testing.assert_array_equal(S2, kv)  # S[i, j] = fp16(v_i k_j): value rows, key columns
    ref = v.astype(np.float64) * (k.astype(np.float64) * r.astype(np.float64)).sum(-1, keepdims=True)
    assert np.abs(y.astype(np.float64) - ref).max() <= 2e-2 * max(1.0, np.abs(ref).max())


def _dplr64(oracle, S16, r, wd, k, nkk, b, v):
    """The fp64 DPLR step of oracle.py on the same fp16 operands: w = 1 + wd,
    kk = -nkk, a = b / kk (so that kk * a = b)."""
    kk = -nkk.astype(np.float64)
    bb = b.astype(np.float64)
    a = np.divide(bb, kk, out=np.zeros_like(bb), where=kk != 0)
    return oracle.wkv7_update(r.astype(np.float64), 1.0 + wd.astype(np.float64), k.astype(np.float64),
                              v.astype(np.float64), kk, a, S16.astype(np.float64))


def test_decode_step_agrees_with_fp64_dplr(oracle):
    rng = np.random.default_rng(6)
    B, H, N = 3, 4, 64
    S = rng.standard_normal((B, H, N, N)).astype(F16)
    k_raw, a, k_k, k_a = o.safe_decode_inputs(rng, B, H)
    a = rng.uniform(0.5, 1.0, (B, H, N)).astype(F16)
    r, v, g = (rng.standard_normal((B, H, N)).astype(F16) for _ in range(3))
    w_raw = rng.standard_normal((B, H, N)).astype(F16)
    r_k = (rng.standard_normal(H * N) * 0.5).astype(F16)
    gn_w = (1.0 + 0.1 * rng.standard_normal(H * N)).astype(F16)
    gn_b = (0.1 * rng.standard_normal(H * N)).astype(F16)
    elapsed = np.array([0, 7, 1000])
    out, S2 = o.decode_output_prepare_raw(r, w_raw, k_raw, v, a, S, g, k_k, k_a, r_k, gn_w, gn_b, elapsed, 1e-5)

    kh, nkk, b = o.decode_prep(k_raw, a, k_k, k_a)
    wd = o.decay_delta(w_raw.astype(np.float32), o.phases(elapsed, H))
    y64, S64 = _dplr64(oracle, S, r, wd, kh, nkk, b, v)
    scale = max(1.0, np.abs(S64).max())
    err = np.abs(S2.astype(np.float64) - S64).max()
    assert err <= 2e-3 * scale, err  # fp16 roundings: about 3.5e-4 of the scale here
    # the same comparison catches a sign error in the low-rank term
    _, S_bad = _dplr64(oracle, S, r, wd, kh, nkk, -b, v)
    assert np.abs(S_bad - S64).max() > 10 * 2e-3 * scale
    # output prep: GroupNorm + bonus + gate of the fp16 readout, against fp64 on the fp64 readout
    ref = oracle.output_prepare(y64.reshape(B, H * N), r.reshape(B, -1).astype(np.float64),
                                kh.reshape(B, -1).astype(np.float64), v.reshape(B, -1).astype(np.float64),
                                g.reshape(B, -1).astype(np.float64), r_k, gn_w, gn_b, H, 1e-5).reshape(B, H, N)
    assert np.abs(out.astype(np.float64) - ref).max() <= 5e-2 * max(1.0, np.abs(ref).max())


def _seq_inputs(rng, B, T, H, N=64, elapsed=None, w0=None):
    ph = o.phases(np.zeros(B) if elapsed is None else elapsed, H, N)[:, None] + np.arange(T).reshape(1, T, 1, 1)
    w = o.safe_w(rng, (B, T, H, N), ph, None if w0 is None else w0.astype(np.float32).reshape(1, 1, H, N))
    r, v = (rng.standard_normal((B, T, H, N)).astype(F16) for _ in range(2))
    k = (rng.standard_normal((B, T, H, N)) * 0.3).astype(F16)
    kk = rng.standard_normal((B, T, H, N))
    kk = kk / np.linalg.norm(kk, axis=-1, keepdims=True)
    a = rng.uniform(0.2, 1.0, (B, T, H, N))
    return r, w, k, v, (-kk).astype(F16), (kk * a).astype(F16)


def test_sequence_agrees_with_fp64_scan(oracle):
    rng = np.random.default_rng(7)
    B, T, H, N = 2, 16, 2, 64
    elapsed = np.array([3, 500])
    r, w, k, v, nkk, kka = _seq_inputs(rng, B, T, H, elapsed=elapsed)
    S = (rng.standard_normal((B, H, N, N)) * 0.5).astype(F16)
    y, S2 = o.sequence(r, w, k, v, nkk, kka, S, elapsed)
    ph = o.phases(elapsed, H)[:, None] + np.arange(T).reshape(1, T, 1, 1)
    wd = o.decay_delta(w.astype(np.float32), ph).astype(np.float64)
    kk = -nkk.astype(np.float64)
    a = np.divide(kka.astype(np.float64), kk, out=np.zeros(kk.shape), where=kk != 0)
    y64, S64 = oracle.wkv7_scan(r.astype(np.float64), 1.0 + wd, k.astype(np.float64), v.astype(np.float64),
                                kk, a, S.astype(np.float64))
    assert np.abs(S2.astype(np.float64) - S64).max() <= 2e-3 * max(1.0, np.abs(S64).max())
    assert np.abs(y.astype(np.float64) - y64).max() <= 5e-3 * max(1.0, np.abs(y64).max())


def test_sequence_split_and_w0_are_exact():
    rng = np.random.default_rng(8)
    B, T, H, N = 2, 11, 2, 64
    elapsed = np.array([0, 41])
    r, w, k, v, nkk, kka = _seq_inputs(rng, B, T, H, elapsed=elapsed)
    S = (rng.standard_normal((B, H, N, N)) * 0.5).astype(F16)
    y, S_full = o.sequence(r, w, k, v, nkk, kka, S, elapsed)
    t1 = 4
    y1, S_mid = o.sequence(r[:, :t1], w[:, :t1], k[:, :t1], v[:, :t1], nkk[:, :t1], kka[:, :t1], S, elapsed)
    y2, S_end = o.sequence(r[:, t1:], w[:, t1:], k[:, t1:], v[:, t1:], nkk[:, t1:], kka[:, t1:], S_mid,
                           elapsed + t1)
    np.testing.assert_array_equal(S_end, S_full)
    np.testing.assert_array_equal(np.concatenate([y1, y2], 1), y)
    # w0 joins w in fp32: with both on a 2^-6 grid in [-2, 2] the sum is exact in fp16
    wq = (np.round(rng.uniform(-2, 2, (B, T, H, N)) * 64) / 64).astype(F16)
    w0 = (np.round(rng.uniform(-2, 2, H * N) * 64) / 64).astype(F16)
    ya, Sa = o.sequence(r, wq, k, v, nkk, kka, S, elapsed, w0=w0)
    yb, Sb = o.sequence(r, (wq.astype(np.float64) + w0.reshape(1, 1, H, N)).astype(F16), k, v, nkk, kka, S,
                        elapsed)
    np.testing.assert_array_equal(Sa, Sb)
    np.testing.assert_array_equal(ya, yb)


# ------------------------------------------- product-side validation (CPU)
def test_fp16_recurrent_policy_is_narrow():
    from rwkv7mi.native_wkv_fp16 import native_fp16_recurrent_should_use as use

    assert use(state_dtype=torch.float16, input_dtype=torch.float16, head_dim=64)
    assert not use(state_dtype=torch.float32, input_dtype=torch.float16, head_dim=64)
    assert not use(state_dtype=torch.float16, input_dtype=torch.bfloat16, head_dim=64)
    assert not use(state_dtype=torch.float16, input_dtype=torch.float16, head_dim=32)


def test_fp16_sequence_rejects_non_rank_four_inputs_before_build():
    from rwkv7mi.native_wkv_fp16 import native_fp16_sequence

    t = torch.zeros(1, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="rank four"):
        native_fp16_sequence(t, t, t, t, t, t, t, torch.zeros(1, dtype=torch.int32))


def test_fp16_operators_reject_host_tensors():
    from rwkv7mi.native_wkv_fp16 import native_fp16_recurrent_output_prepare_raw, native_fp16_sequence

    x = torch.zeros(1, 2, 3, 64, dtype=torch.float16)
    st = torch.zeros(1, 3, 64, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="CUDA fp16"):
        native_fp16_sequence(x, x, x, x, x, x, st, torch.zeros(1, dtype=torch.int32))
    v = torch.zeros(1, 3, 64, dtype=torch.float16)
    p = torch.zeros(3 * 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="CUDA fp16"):
        native_fp16_recurrent_output_prepare_raw(v, v, v, v, v, st, v, p, p, p, p, p,
                                                 torch.zeros(1, dtype=torch.int32), advance_elapsed=True, eps=1e-5)
    with pytest.raises(ValueError, match="unsupported dtype or shape"):
        native_fp16_recurrent_output_prepare_raw(v, v, v, v, v, st.float(), v, p, p, p, p, p,
                                                 torch.zeros(1, dtype=torch.int32), advance_elapsed=True, eps=1e-5)


def test_state_dtype_switches_follow_the_reference(monkeypatch):
    """RWKV7_NATIVE_GRAPH_STATE_DTYPE / RWKV7_NATIVE_GRAPH_FP16_RECURRENT as the
    reference reads them (rwkv7_hf/native_graph_runtime.py:119-147, :312-316)."""
    from rwkv7mi.model import native_graph_state_dtype

    monkeypatch.delenv("RWKV7_NATIVE_GRAPH_STATE_DTYPE", raising=False)
    monkeypatch.delenv("RWKV7_NATIVE_GRAPH_FP16_RECURRENT", raising=False)
    assert native_graph_state_dtype(torch.float16) == torch.float32
    monkeypatch.setenv("RWKV7_NATIVE_GRAPH_STATE_DTYPE", "fp16")
    with pytest.raises(RuntimeError, match="RWKV7_NATIVE_GRAPH_FP16_RECURRENT"):
        native_graph_state_dtype(torch.float16)
    assert native_graph_state_dtype(torch.float32) == torch.float32  # fp16 state only for fp16 models
    monkeypatch.setenv("RWKV7_NATIVE_GRAPH_FP16_RECURRENT", "1")
    assert native_graph_state_dtype(torch.float16) == torch.float16
    monkeypatch.setenv("RWKV7_NATIVE_GRAPH_STATE_DTYPE", "bf16")
    with pytest.raises(ValueError):
        native_graph_state_dtype(torch.float16)


def test_fp16_state_cache_carries_elapsed_through_batch_edits():
    from rwkv7mi.model import NativeRWKV7Cache, NativeRWKV7Config

    cfg = NativeRWKV7Config(vocab_size=64, hidden_size=128, num_hidden_layers=2, intermediate_size=256)
    c = NativeRWKV7Cache.zeros(cfg, 3, "cpu", torch.float16, state_dtype=torch.float16)
    assert c.state_dtype == torch.float16 and c.fp16_elapsed.dtype == torch.int32
    c.fp16_elapsed.copy_(torch.tensor([5, 6, 7], dtype=torch.int32))
    c.select_batch([2, 0])
    assert c.fp16_elapsed.tolist() == [7, 5]
    c.batch_repeat_interleave(2)
    assert c.fp16_elapsed.tolist() == [7, 7, 5, 5]
    d = c.clone()
    d.fp16_elapsed.add_(1)
    assert c.fp16_elapsed.tolist() == [7, 7, 5, 5]
    c.zero_()
    assert c.fp16_elapsed.tolist() == [0, 0, 0, 0]
    assert NativeRWKV7Cache.zeros(cfg, 2, "cpu", torch.float16).fp16_elapsed is None
    with pytest.raises(ValueError, match="fp16 activations"):
        NativeRWKV7Cache.zeros(cfg, 2, "cpu", torch.float32, state_dtype=torch.float16)
