"""Pins of the CPU wkv7 oracle against forms the mathematics fixes (CPU only).

The oracle (oracle/wkv7_oracle.c) iterates the reference's rank-1 update
(rwkv7_hf/fused_recurrent_update.py:757-783).  Each test below computes the
expected result a different way, so a dropped term, a sign error or a
transposed state would fail at least one of them.
"""
from __future__ import annotations

import numpy as np
import pytest


def _inputs(rng, B, T, H, N, *, scale=0.2):
    r = rng.standard_normal((B, T, H, N)) * scale
    w = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H, N))))
    k = rng.standard_normal((B, T, H, N)) * scale
    v = rng.standard_normal((B, T, H, N)) * scale
    kk = rng.standard_normal((B, T, H, N))
    kk /= np.linalg.norm(kk, axis=-1, keepdims=True)
    a = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H, N))))
    state = rng.standard_normal((B, H, N, N)) * scale
    return r, w, k, v, kk, a, state


def _matrix_form(r, w, k, v, kk, a, state):
    """S_t = S_{t-1} (diag(w_t) + alpha_t beta_t^T) + v_t k_t^T with an explicit
    N x N transition matrix (alpha = -kk, beta = kk * a); y_t = S_t r_t."""
    B, T, H, N = r.shape
    S = state.copy()
    y = np.zeros_like(r)
    for t in range(T):
        for b in range(B):
            for h in range(H):
                P = np.diag(w[b, t, h]) + np.outer(-kk[b, t, h], kk[b, t, h] * a[b, t, h])
                S[b, h] = S[b, h] @ P + np.outer(v[b, t, h], k[b, t, h])
                y[b, t, h] = S[b, h] @ r[b, t, h]
    return y, S


def test_matches_explicit_transition_matrix(oracle):
    # shapes and scales of the reference's own differential test
    # (tests/test_dplr_prefill_scan.py:36-46: seed 7007, B=2, T=7, H=2, N=4)
    rng = np.random.default_rng(7007)
    args = _inputs(rng, 2, 7, 2, 4)
    y, S = oracle.wkv7_scan(*args)
    y2, S2 = _matrix_form(*args)
    np.testing.assert_allclose(y, y2, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(S, S2, rtol=1e-12, atol=1e-12)


def test_head64_matches_transition_matrix(oracle):
    rng = np.random.default_rng(11)
    args = _inputs(rng, 1, 5, 2, 64)
    y, S = oracle.wkv7_scan(*args)
    y2, S2 = _matrix_form(*args)
    np.testing.assert_allclose(y, y2, rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(S, S2, rtol=1e-11, atol=1e-11)


def test_a_zero_is_decayed_linear_attention(oracle):
    """a = 0 removes the DPLR term: y_t = S0 (prod w) r_t + sum_s v_s (k_s * prod_{u in (s,t]} w_u) . r_t."""
    rng = np.random.default_rng(3)
    r, w, k, v, kk, a, state = _inputs(rng, 1, 9, 1, 8)
    a[:] = 0.0
    y, S = oracle.wkv7_scan(r, w, k, v, kk, a, state)
    T = r.shape[1]
    for t in range(T):
        decay0 = np.prod(w[0, : t + 1, 0], axis=0)
        expect = state[0, 0] @ (decay0 * r[0, t, 0])
        for s in range(t + 1):
            d = np.prod(w[0, s + 1 : t + 1, 0], axis=0) if s < t else np.ones(8)
            expect = expect + v[0, s, 0] * np.dot(k[0, s, 0] * d, r[0, t, 0])
        np.testing.assert_allclose(y[0, t, 0], expect, rtol=1e-12, atol=1e-12)


def test_no_decay_no_dplr_is_plain_linear_attention(oracle):
    rng = np.random.default_rng(4)
    r, w, k, v, kk, a, state = _inputs(rng, 2, 6, 2, 4)
    w[:] = 1.0
    a[:] = 0.0
    state[:] = 0.0
    y, _ = oracle.wkv7_scan(r, w, k, v, kk, a, state)
    # y_t = sum_{s<=t} v_s (k_s . r_t)
    scores = np.einsum("bshn,bthn->bhts", k, r)
    mask = np.tril(np.ones((6, 6)))
    expect = np.einsum("bhts,bshn->bthn", scores * mask, v)
    np.testing.assert_allclose(y, expect, rtol=1e-12, atol=1e-12)


def test_single_token_from_zero_state(oracle):
    rng = np.random.default_rng(5)
    r, w, k, v, kk, a, state = _inputs(rng, 3, 1, 2, 64)
    state[:] = 0.0
    y, S = oracle.wkv7_scan(r, w, k, v, kk, a, state)
    expect = v[:, 0] * np.sum(k[:, 0] * r[:, 0], axis=-1, keepdims=True)
    np.testing.assert_allclose(y[:, 0], expect, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(S, np.einsum("bhi,bhj->bhij", v[:, 0], k[:, 0]), rtol=1e-12, atol=1e-12)


def test_unit_kk_projects_out_one_key_column(oracle):
    """kk = e_j, a = 1, w = 1: the transition I - e_j e_j^T zeroes key column j."""
    rng = np.random.default_rng(6)
    N = 8
    r, w, k, v, kk, a, state = _inputs(rng, 1, 1, 1, N)
    w[:] = 1.0
    a[:] = 1.0
    kk[:] = 0.0
    kk[0, 0, 0, 3] = 1.0
    _, S = oracle.wkv7_scan(r, w, k, v, kk, a, state)
    expect = state[0, 0].copy()
    expect[:, 3] = 0.0
    expect += np.outer(v[0, 0, 0], k[0, 0, 0])
    np.testing.assert_allclose(S[0, 0], expect, rtol=1e-12, atol=1e-12)


def test_empty_sequence_keeps_state(oracle):
    rng = np.random.default_rng(8)
    args = list(_inputs(rng, 2, 0, 2, 4))
    y, S = oracle.wkv7_scan(*args)
    assert y.shape == (2, 0, 2, 4)
    np.testing.assert_array_equal(S, args[-1])


def test_f32_scan_close_to_f64(oracle):
    rng = np.random.default_rng(9)
    args = _inputs(rng, 2, 33, 2, 64)
    y, S = oracle.wkv7_scan(*args)
    y32, S32 = oracle.wkv7_scan_f32(*args)
    np.testing.assert_allclose(y32, y, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(S32, S, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("bad", ["drop_vk", "sign", "transpose"])
def test_planted_mistakes_are_caught(oracle, bad):
    """The matrix-form check rejects typical restatement mistakes (planted in a
    CPU copy of the recurrence, never in the product)."""
    rng = np.random.default_rng(10)
    r, w, k, v, kk, a, state = _inputs(rng, 1, 4, 1, 6)
    S = state[0, 0].copy()
    ys = []
    for t in range(4):
        dot = S @ kk[0, t, 0]
        if bad == "sign":
            S = S * w[0, t, 0] + np.outer(dot, kk[0, t, 0] * a[0, t, 0]) + np.outer(v[0, t, 0], k[0, t, 0])
        elif bad == "drop_vk":
            S = S * w[0, t, 0] - np.outer(dot, kk[0, t, 0] * a[0, t, 0])
        else:
            S = (S * w[0, t, 0] - np.outer(dot, kk[0, t, 0] * a[0, t, 0]) + np.outer(v[0, t, 0], k[0, t, 0])).T
        ys.append(S @ r[0, t, 0])
    y2, _ = _matrix_form(r, w, k, v, kk, a, state)
    assert not np.allclose(np.array(ys), y2[0, :, 0], atol=1e-6)
