"""Pins of the numpy restatements of the elementwise / small-GEMM ops around
the scan (oracle/oracle.py) against torch's own CPU library routines — the
arithmetic the reference's torch forms call — and against closed forms:

* layer_norm                  vs torch.nn.functional.layer_norm (fp64)
* group_norm_heads            vs torch.nn.functional.group_norm (fp64)
* attn_norm_mix6 / seq_norm_mix: mix = 0 gives h, mix = 1 gives prev; a
  one-token sequence equals the decode form; the carried row is h[:, -1]
* wavg_lora                   vs torch.nn.functional.linear + tanh / sigmoid
* decode_raw_prep / state_prep vs torch.nn.functional.normalize, sigmoid, exp
* output_prepare              vs group_norm + per-head bonus, and the wkv7
                              output prep (fp64 C scan) composed the same way
Planted mistakes (biased vs unbiased variance, wrong eps, missing bias) are
caught by the same comparisons.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

T = lambda a: torch.tensor(np.asarray(a), dtype=torch.float64)


def _rng(seed):
    return np.random.default_rng(seed)


def test_layer_norm_matches_torch(oracle):
    rng = _rng(1)
    x, w, b = rng.standard_normal((5, 96)), 1 + 0.1 * rng.standard_normal(96), 0.1 * rng.standard_normal(96)
    ref = F.layer_norm(T(x), (96,), T(w), T(b), eps=1e-5).numpy()
    np.testing.assert_allclose(oracle.layer_norm(x, w, b), ref, rtol=1e-12, atol=1e-12)
    # planted: unbiased variance would differ
    unb = (x - x.mean(-1, keepdims=True)) / np.sqrt(x.var(-1, ddof=1, keepdims=True) + 1e-5) * w + b
    assert np.abs(unb - ref).max() > 1e-4


def test_group_norm_heads_matches_torch(oracle):
    rng = _rng(2)
    H, N = 4, 64
    x = rng.standard_normal((3, H * N))
    w, b = 1 + 0.1 * rng.standard_normal(H * N), 0.1 * rng.standard_normal(H * N)
    eps = N * 1e-5
    ref = F.group_norm(T(x), H, T(w), T(b), eps=eps).numpy()
    np.testing.assert_allclose(oracle.group_norm_heads(x, w, b, H, eps), ref, rtol=1e-12, atol=1e-12)
    assert np.abs(oracle.group_norm_heads(x, w, b, H, 1e-5) - ref).max() > 1e-6  # eps matters


def test_mix_closed_forms_and_sequence_equivalence(oracle):
    rng = _rng(3)
    B, D = 2, 64
    x, prev = rng.standard_normal((B, D)), rng.standard_normal((B, D))
    w, b = 1 + 0.1 * rng.standard_normal(D), 0.1 * rng.standard_normal(D)
    (o0, o1, oh), h = oracle.attn_norm_mix6(x, prev, w, b, [np.zeros(D), np.ones(D), np.full(D, 0.5)])
    np.testing.assert_allclose(h, oracle.layer_norm(x, w, b), rtol=0, atol=0)
    np.testing.assert_allclose(o0, h, atol=1e-15)
    np.testing.assert_allclose(o1, prev, atol=1e-15)
    np.testing.assert_allclose(oh, 0.5 * (h + prev), atol=1e-15)
    mixes = [rng.random(D) for _ in range(6)]
    dec, _ = oracle.attn_norm_mix6(x, prev, w, b, mixes)
    seq, last = oracle.seq_norm_mix(x[:, None], prev, w, b, mixes)
    for a, s in zip(dec, seq):
        np.testing.assert_allclose(s[:, 0], a, atol=1e-15)
    xs = rng.standard_normal((B, 5, D))
    seq, last = oracle.seq_norm_mix(xs, prev, w, b, [np.ones(D)])
    h = oracle.layer_norm(xs, w, b)
    np.testing.assert_allclose(last, h[:, -1], atol=1e-15)
    np.testing.assert_allclose(seq[0][:, 1:], h[:, :-1], atol=1e-15)  # mix 1 = previous token's h
    np.testing.assert_allclose(seq[0][:, 0], prev, atol=1e-15)


def test_wavg_lora_matches_torch(oracle):
    rng = _rng(4)
    rows, D, A = 3, 48, 40
    xs = [rng.standard_normal((rows, D)) for _ in range(4)]
    ranks = (8, 8, 16, 8)
    downs = [0.2 * rng.standard_normal((r, D)) for r in ranks]
    ups = [0.2 * rng.standard_normal((A, r)) for r in ranks]
    biases = [0.1 * rng.standard_normal(A), 0.1 * rng.standard_normal(A), None, 0.1 * rng.standard_normal(A)]
    got = oracle.wavg_lora(*xs, *downs, *ups, *biases)
    tb = lambda i: None if biases[i] is None else T(biases[i])
    ref = [
        F.linear(torch.tanh(F.linear(T(xs[0]), T(downs[0]))), T(ups[0]), tb(0)),
        F.linear(F.linear(T(xs[1]), T(downs[1])), T(ups[1]), tb(1)),
        F.linear(torch.sigmoid(F.linear(T(xs[2]), T(downs[2]))), T(ups[2])),
        torch.sigmoid(F.linear(F.linear(T(xs[3]), T(downs[3])), T(ups[3]), tb(3))),
    ]
    for g, r in zip(got, ref):
        np.testing.assert_allclose(g, r.numpy(), rtol=1e-12, atol=1e-12)


def test_prep_functions_match_torch(oracle):
    rng = _rng(5)
    B, H, N = 2, 3, 64
    k_raw, w_raw, a = rng.standard_normal((B, H, N)), rng.standard_normal((B, H, N)), rng.random((B, H, N))
    k_k, k_a = 0.85 + 0.1 * rng.standard_normal(H * N), 1 + 0.1 * rng.standard_normal(H * N)
    kk, k, w = oracle.decode_raw_prep(k_raw, w_raw, a, k_k, k_a)
    kk_ref = F.normalize(T(k_raw) * T(k_k).view(1, H, N), dim=-1, p=2.0, eps=1e-12).numpy()
    np.testing.assert_allclose(kk, kk_ref, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(k, (T(k_raw) * (1 + (T(a) - 1) * T(k_a).view(1, H, N))).numpy(), rtol=1e-14)
    np.testing.assert_allclose(w, torch.exp(-0.606531 * torch.sigmoid(T(w_raw))).numpy(), rtol=1e-14)
    # the prefill form gives the same kk / k and log(w)
    v, vf, vg = rng.standard_normal((B, H * N)), rng.standard_normal((B, H * N)), rng.random((B, H * N))
    kk2, k2, v2, logw = oracle.state_prep(k_raw.reshape(B, -1), a.reshape(B, -1), w_raw.reshape(B, -1), v, vf, vg,
                                          k_k, k_a, H)
    np.testing.assert_allclose(kk2, kk.reshape(B, -1), rtol=1e-14, atol=1e-15)
    np.testing.assert_allclose(k2, k.reshape(B, -1), rtol=1e-14)
    np.testing.assert_allclose(np.exp(logw), w.reshape(B, -1), rtol=1e-14)
    np.testing.assert_allclose(v2, (T(v) + (T(vf) - T(v)) * T(vg)).numpy(), rtol=1e-14)


def test_output_prepare_matches_group_norm_and_decode_form(oracle):
    rng = _rng(6)
    B, H, N = 2, 3, 64
    r, w, k, v = (rng.standard_normal((B, H, N)) for _ in range(4))
    w = np.exp(-np.exp(rng.normal(-0.5, 0.5, (B, H, N))))
    kk = rng.standard_normal((B, H, N))
    kk /= np.linalg.norm(kk, axis=-1, keepdims=True)
    a = rng.random((B, H, N))
    state = rng.standard_normal((B, H, N, N))
    g = rng.standard_normal((B, H, N))
    r_k, gn_w, gn_b = 0.1 * rng.standard_normal((H, N)), 1 + 0.1 * rng.standard_normal(H * N), 0.1 * rng.standard_normal(H * N)
    eps = N * 1e-5
    out, st = oracle.wkv7_output_prepare(r, w, k, v, kk, a, state, g, r_k, gn_w, gn_b, eps)
    y, st2 = oracle.wkv7_update(r, w, k, v, kk, a, state)
    np.testing.assert_allclose(st, st2, atol=0)
    normed = F.group_norm(T(y.reshape(B, -1)), H, T(gn_w), T(gn_b), eps=eps).numpy().reshape(B, H, N)
    bonus = (r * k * r_k[None]).sum(-1, keepdims=True) * v
    np.testing.assert_allclose(out, (normed + bonus) * g, rtol=1e-10, atol=1e-12)
    flat = oracle.output_prepare(y.reshape(B, -1), r.reshape(B, -1), k.reshape(B, -1), v.reshape(B, -1),
                                 g.reshape(B, -1), r_k, gn_w, gn_b, H, eps)
    np.testing.assert_allclose(flat, out.reshape(B, -1), rtol=1e-10, atol=1e-12)


def test_seq_shift_mix_closed_forms(oracle):
    """The reference-convention sequence mix (x already normalised): mix = 0
    gives x, mix = 1 gives the one-token shift with the carried row first, and
    it equals seq_norm_mix of an identity-normalised input (a planted
    off-by-one shift would fail the mix = 1 case)."""
    rng = _rng(31)
    B, Tn, D = 2, 5, 16
    x = rng.standard_normal((B, Tn, D))
    prev0 = rng.standard_normal((B, D))
    (o0, o1), last = oracle.seq_shift_mix(x, prev0, [np.zeros(D), np.ones(D)])
    np.testing.assert_array_equal(o0, x)
    np.testing.assert_allclose(o1[:, 0], prev0, rtol=0, atol=1e-14)
    np.testing.assert_allclose(o1[:, 1:], x[:, :-1], rtol=0, atol=1e-14)
    np.testing.assert_array_equal(last, x[:, -1])
    # rows that are already LayerNorm outputs with unit affine: LN leaves them (almost) as they are
    xn = oracle.layer_norm(x, np.ones(D), np.zeros(D), eps=0.0)
    mixes = [rng.random(D) for _ in range(3)]
    outs_a, _ = oracle.seq_shift_mix(xn, oracle.layer_norm(prev0, np.ones(D), np.zeros(D), eps=0.0), mixes)
    outs_b, _ = oracle.seq_norm_mix(xn, oracle.layer_norm(prev0, np.ones(D), np.zeros(D), eps=0.0), np.ones(D),
                                    np.zeros(D), mixes, eps=0.0)
    for a, b in zip(outs_a, outs_b):
        np.testing.assert_allclose(a[:, 1:], b[:, 1:], rtol=1e-9, atol=1e-9)
