"""CPU oracle of the opt-in fp16-state recurrence — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module, and only as the checker (or the timed CPU
baseline).  The product (``hf-adapter_amd/``) never imports it.

Restates rwkv7_hf/native_wkv_fp16.py (rwkv-rs/hf-adapter 0.8.1) in numpy:
the fp16 state arithmetic is emulated to the bit (``fma16``: one correctly
rounded fp16 rounding per fused multiply-add, in the kernel's order), and the
fp32 parts (decay delta, kk normalisation, GroupNorm epilogue) follow the
reference's fp32 steps.  Pinned by tests/test_oracle_fp16.py against exact
rational arithmetic (``fma16``), closed forms (the dither, the decay delta,
one step from a zero state) and the fp64 DPLR oracle (the full step).
"""
from __future__ import annotations

import math

import numpy as np

F16 = np.float16
F32 = np.float32
LOG2E = math.log2(math.e)
DECAY_LOG2 = math.exp(-0.5) * LOG2E  # e^-1/2 log2(e): exp(-e^-1/2 s) = 2^(-DECAY_LOG2 s)
GOLDEN32 = 0x9E3779B9


def fma16(a, b, c):
    """fp16 a*b + c with a single round-to-nearest-even (IEEE fusedMultiplyAdd).

    Evaluated as RN16(RN64(a*b + c)), which equals the single rounding for every
    finite fp16 result: a*b of two fp16 values is exact in fp64 (22 significant
    bits); both addends are multiples of 2^-48, so the fp64 sum is inexact only
    when the exact sum needs more than 53 bits, i.e. when |a*b| < 2^-31 |c|
    (a finite result bounds |a*b| below 2^17); then |a*b| is far below half an
    fp16 ulp of c and both roundings return c.
    """
    a64 = np.asarray(a, F16).astype(np.float64)
    b64 = np.asarray(b, F16).astype(np.float64)
    c64 = np.asarray(c, F16).astype(np.float64)
    return (a64 * b64 + c64).astype(F16)


def add16(x, y):
    """fp16 x + y (the exact sum fits fp64: one rounding)."""
    return (np.asarray(x, F16).astype(np.float64) + np.asarray(y, F16).astype(np.float64)).astype(F16)


def dither(phase):
    """rotator1 (rwkv7_hf/native_wkv_fp16.py:117-120): 2^-41 * float(int32(0x9E3779B9 * phase))."""
    ph = np.asarray(phase, np.int64) & 0xFFFFFFFF
    prod = (ph.astype(np.uint64) * np.uint64(GOLDEN32)) & np.uint64(0xFFFFFFFF)
    signed = prod.astype(np.int64) - (prod >= np.uint64(1 << 31)).astype(np.int64) * (1 << 32)
    return F32(2.0 ** -41) * signed.astype(F32)


def decay_delta(wv, phase):
    """w_delta (rwkv7_hf/native_wkv_fp16.py:122-138) in fp32 steps, rounded to fp16:
    exp(-e^-1/2 sigmoid(w)) - 1 + dither(phase) = 2^(-DECAY_LOG2 / (1 + 2^(-log2(e) w))) - 1 + dither."""
    wv = np.asarray(wv, F32)
    t = np.exp2(F32(-LOG2E) * wv)
    d = np.exp2(F32(-DECAY_LOG2) / (F32(1.0) + t)) - F32(1.0) + dither(phase)
    return d.astype(F16)


def row_step(S, r, wd, k, nkk, b, v):
    """One token on fp16 state rows (rwkv7_hf/native_wkv_fp16.py:279-300, :390-410).

    S [..., 64 (value i), 64 (key j)] fp16; r, wd, k, nkk (= -kk), b (= kk*a), v
    [..., 64] fp16.  Returns (S', y): sa = pairwise-chained sum of nkk*S over
    key pairs (even and odd columns in two chains, then added),
    S' = fma(S, wd, fma(k, v_i, fma(sa, b, S))), y = the same pairwise chain of S'*r.
    """
    S = np.asarray(S, F16)
    N = S.shape[-1]
    lo = np.zeros(S.shape[:-1], F16)
    hi = np.zeros(S.shape[:-1], F16)
    n = np.asarray(nkk, F16)[..., None, :]
    for jp in range(N // 2):
        lo = fma16(n[..., 2 * jp], S[..., 2 * jp], lo)
        hi = fma16(n[..., 2 * jp + 1], S[..., 2 * jp + 1], hi)
    sa = add16(lo, hi)[..., None]
    vi = np.asarray(v, F16)[..., :, None]
    kj = np.asarray(k, F16)[..., None, :]
    S2 = fma16(S, np.asarray(wd, F16)[..., None, :], fma16(kj, vi, fma16(sa, np.asarray(b, F16)[..., None, :], S)))
    rj = np.asarray(r, F16)[..., None, :]
    lo = np.zeros(S.shape[:-1], F16)
    hi = np.zeros(S.shape[:-1], F16)
    for jp in range(N // 2):
        lo = fma16(S2[..., 2 * jp], rj[..., 2 * jp], lo)
        hi = fma16(S2[..., 2 * jp + 1], rj[..., 2 * jp + 1], hi)
    return S2, add16(lo, hi)


def phases(elapsed, H, N=64):
    """phase[b, h, i] = elapsed[b] + h*N + i."""
    e = np.asarray(elapsed, np.int64).reshape(-1, 1, 1)
    return e + (np.arange(H, dtype=np.int64) * N).reshape(1, H, 1) + np.arange(N, dtype=np.int64).reshape(1, 1, N)


def decode_prep(k_raw, a, k_k, k_a):
    """Raw-input prep of the fp16 decode kernel (rwkv7_hf/native_wkv_fp16.py:251-267), fp32:
    kk = fp16(k_raw k_k / max(|k_raw k_k|, 1e-12)), k = fp16(k_raw (a k_a + 1 - k_a)),
    b = fp16(kk a).  Returns (k, -kk, b) fp16 [B,H,N]."""
    f = lambda x: np.asarray(x, F16).astype(F32)
    kr, af = f(k_raw), f(a)
    H, N = kr.shape[1], kr.shape[2]
    kku = kr * f(k_k).reshape(1, H, N)
    nrm = np.sqrt((kku.astype(np.float64) ** 2).sum(-1, keepdims=True)).astype(F32)
    kkh = (kku / np.maximum(nrm, F32(1e-12))).astype(F16)
    kaw = f(k_a).reshape(1, H, N)
    kh = (kr * (af * kaw + (F32(1.0) - kaw))).astype(F16)
    b = (kkh.astype(F32) * af).astype(F16)
    return kh, (-kkh).astype(F16), b


def decode_output_prepare_raw(r, w_raw, k_raw, v, a, state, g, k_k, k_a, r_k, gn_w, gn_b, elapsed, eps):
    """rwkv7_native_fp16_recurrent_output_raw (rwkv7_hf/native_wkv_fp16.py:200-336).

    Vectors [B,H,64] fp16, state [B,H,64,64] fp16, per-channel params [H*64]
    fp16, elapsed int [B].  Returns (out [B,H,64] fp16, new state fp16).
    """
    r16 = np.asarray(r, F16)
    B, H, N = r16.shape
    kh, nkk, b = decode_prep(k_raw, a, k_k, k_a)
    wd = decay_delta(np.asarray(w_raw, F16).astype(F32), phases(elapsed, H, N))
    S2, y = row_step(state, r16, wd, kh, nkk, b, v)
    f = lambda x: np.asarray(x, F16).astype(np.float64)
    yf = y.astype(np.float64)
    mean = yf.mean(-1, keepdims=True)
    cen = yf - mean
    var = (cen ** 2).mean(-1, keepdims=True)
    corr = (f(r16) * f(kh) * f(r_k).reshape(1, H, N)).sum(-1, keepdims=True)
    out = (cen / np.sqrt(var + eps) * f(gn_w).reshape(1, H, N) + f(gn_b).reshape(1, H, N) + corr * f(v)) * f(g)
    return out.astype(F16), S2


def sequence(r, w, k, v, neg_kk, kka, state, elapsed, w0=None):
    """rwkv7_native_fp16_sequence (rwkv7_hf/native_wkv_fp16.py:338-436).

    Inputs [B,T,H,64] fp16 (w raw; w0 [H*64] added in fp32 when given), state
    [B,H,64,64] fp16, elapsed int [B] (token t uses phase elapsed + 64 h + i + t).
    Returns (y [B,T,H,64] fp16, new state fp16).
    """
    r = np.asarray(r, F16)
    B, T, H, N = r.shape
    S = np.array(state, F16, copy=True)
    y = np.zeros((B, T, H, N), F16)
    w32 = np.asarray(w, F16).astype(F32)
    if w0 is not None:
        w32 = w32 + np.asarray(w0, F16).astype(F32).reshape(1, 1, H, N)
    ph = phases(elapsed, H, N)
    for t in range(T):
        wd = decay_delta(w32[:, t], ph + t)
        S, y[:, t] = row_step(S, r[:, t], wd, np.asarray(k, F16)[:, t], np.asarray(neg_kk, F16)[:, t],
                              np.asarray(kka, F16)[:, t], np.asarray(v, F16)[:, t])
    return y, S


# ------------------------------------------------------------ test inputs
def _safe16(x64, rel=2.0 ** -18, absolute=0.0):
    """True where the fp64 value x64 is further than max(rel |x64|, absolute)
    from the nearest fp16 rounding midpoint, so that any fp32 evaluation of it
    within that error rounds to the same fp16 value."""
    x64 = np.asarray(x64, np.float64)
    h = x64.astype(F16)
    up = np.nextafter(h, F16(np.inf)).astype(np.float64)
    dn = np.nextafter(h, F16(-np.inf)).astype(np.float64)
    hd = h.astype(np.float64)
    m_up = (hd + up) * 0.5
    m_dn = (hd + dn) * 0.5
    dist = np.minimum(np.abs(x64 - m_up), np.abs(x64 - m_dn))
    return dist > np.maximum(rel * np.abs(x64), max(absolute, 2.0 ** -40))


def exact_decay_delta(wv, phase):
    """The decay delta in fp64 (test-input selection only)."""
    wv = np.asarray(wv, np.float64)
    return np.exp(-math.exp(-0.5) / (1.0 + np.exp(-wv))) - 1.0 + dither(phase).astype(np.float64)


def safe_w(rng, shape, phase, w0_32=None, scale=1.0):
    """fp16 raw-w values whose decay delta (at `phase`, plus w0 when given) sits
    away from fp16 rounding midpoints, so that any faithful fp32 evaluation
    rounds to the same fp16 delta.  The fp32 evaluation ends in 2^x - 1 with
    2^x near 1, so its error is absolute (a few 2^-24): the margin is 2^-19."""
    w = (rng.standard_normal(shape) * scale).astype(F16)
    for _ in range(64):
        wv = w.astype(F32) + (0 if w0_32 is None else w0_32)
        bad = ~_safe16(exact_decay_delta(wv, phase), absolute=2.0 ** -19)
        if not bad.any():
            return w
        w = np.where(bad, (rng.standard_normal(shape) * scale).astype(F16), w)
    raise RuntimeError("could not draw safe w values")


def safe_decode_inputs(rng, B, H, N=64):
    """k_raw, a, k_k, k_a (fp16) whose kk, k and kk*a round to fp16 away from
    midpoints; redraws whole heads until every channel is safe."""
    k_k = (1.0 + 0.1 * rng.standard_normal(H * N)).astype(F16)
    k_a = rng.uniform(0.0, 1.0, H * N).astype(F16)
    k_raw = rng.standard_normal((B, H, N)).astype(F16)
    a = rng.uniform(0.0, 1.0, (B, H, N)).astype(F16)
    for _ in range(256):
        kr, af = k_raw.astype(np.float64), a.astype(np.float64)
        kku = kr * k_k.astype(np.float64).reshape(1, H, N)
        kk = kku / np.maximum(np.sqrt((kku ** 2).sum(-1, keepdims=True)), 1e-12)
        ka = k_a.astype(np.float64).reshape(1, H, N)
        kval = kr * (af * ka + 1.0 - ka)
        ok = _safe16(kk) & _safe16(kval)
        head_bad = ~ok.all(-1, keepdims=True)
        if not head_bad.any():
            return k_raw, a, k_k, k_a
        k_raw = np.where(head_bad, rng.standard_normal((B, H, N)).astype(F16), k_raw)
        a = np.where(head_bad, rng.uniform(0.0, 1.0, (B, H, N)).astype(F16), a)
    raise RuntimeError("could not draw safe decode inputs")
