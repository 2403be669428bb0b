"""CPU oracle of the rwkv7mi hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module, and only as the checker (or the timed CPU
baseline).  The product (``hf-adapter_amd/``) never imports it.

Each function cites the reference (rwkv-rs/hf-adapter 0.8.1) it restates.
The C part (``wkv7_oracle.c``, built by ``make -C oracle``) holds the fp64
DPLR scan and the bit-exact fp32 packers; numpy holds the rest in fp64.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------ wkv7
def wkv7_scan(r, w, k, v, kk, a, state):
    """fp64 sequential DPLR scan; inputs [B,T,H,N], state [B,H,N,N].

    rwkv7_hf/fused_recurrent_update.py:757-783 (one token) iterated as in
    torch_recurrent_scan (:800-844).  Returns (y [B,T,H,N] f64, final state f64).
    """
    arrs = [np.ascontiguousarray(x, dtype=np.float64) for x in (r, w, k, v, kk, a)]
    B, T, H, N = arrs[0].shape
    st = np.array(state, dtype=np.float64, copy=True, order="C")
    y = np.zeros((B, T, H, N), dtype=np.float64)
    f = lib().wkv7_ref_scan_f64
    f.argtypes = [ctypes.c_int64] * 4 + [ctypes.c_void_p] * 8
    f(B, T, H, N, *map(_p, arrs), _p(st), _p(y))
    return y, st


def wkv7_scan_f32(r, w, k, v, kk, a, state):
    """Same recurrence in fp32 (OpenMP over heads) — the CPU baseline kernel."""
    arrs = [np.ascontiguousarray(x, dtype=np.float32) for x in (r, w, k, v, kk, a)]
    B, T, H, N = arrs[0].shape
    st = np.array(state, dtype=np.float32, copy=True, order="C")
    y = np.zeros((B, T, H, N), dtype=np.float32)
    f = lib().wkv7_ref_scan_f32
    f.argtypes = [ctypes.c_int64] * 4 + [ctypes.c_void_p] * 8
    f(B, T, H, N, *map(_p, arrs), _p(st), _p(y))
    return y, st


def num_threads() -> int:
    f = lib().oracle_num_threads
    f.restype = ctypes.c_int
    return int(f())


def wkv7_update(r, w, k, v, kk, a, state):
    """One decode step, [B,H,N] vectors: rwkv7_hf/fused_recurrent_update.py:757-783."""
    y, st = wkv7_scan(*(np.asarray(x)[:, None] for x in (r, w, k, v, kk, a)), state)
    return y[:, 0], st


def group_norm_heads(x, weight, bias, H, eps):
    """F.group_norm over H groups of a [B, H*N] tensor (biased variance)."""
    x = np.asarray(x, dtype=np.float64)
    B = x.shape[0]
    g = x.reshape(B, H, -1)
    mean = g.mean(-1, keepdims=True)
    var = ((g - mean) ** 2).mean(-1, keepdims=True)
    out = ((g - mean) / np.sqrt(var + eps)).reshape(B, -1)
    return out * np.asarray(weight, np.float64).reshape(1, -1) + np.asarray(bias, np.float64).reshape(1, -1)


def wkv7_output_prepare(r, w, k, v, kk, a, state, g, r_k, gn_w, gn_b, eps):
    """rwkv7_hf/fused_recurrent_update.py:846-915 in fp64; returns ([B,H,N], state)."""
    r, k, v, g = (np.asarray(x, np.float64) for x in (r, k, v, g))
    B, H, N = r.shape
    y, st = wkv7_update(r, w, k, v, kk, a, state)
    normed = group_norm_heads(y.reshape(B, H * N), gn_w, gn_b, H, eps).reshape(B, H, N)
    corr = (r * k * np.asarray(r_k, np.float64).reshape(1, H, N)).sum(-1, keepdims=True) * v
    return (normed + corr) * g, st


def decode_raw_prep(k_raw, w_raw, a, k_k, k_a):
    """Raw-input prep of rwkv7_hf/fused_recurrent_update.py:1150-1153 (fp64):
    kk = normalize(k_raw * k_k), k = k_raw (1 + (a - 1) k_a), w = exp(-0.606531 sigmoid(w_raw))."""
    k_raw, w_raw, a = (np.asarray(x, np.float64) for x in (k_raw, w_raw, a))
    B, H, N = k_raw.shape
    kk_u = k_raw * np.asarray(k_k, np.float64).reshape(1, H, N)
    nrm = np.sqrt((kk_u ** 2).sum(-1, keepdims=True))
    kk = kk_u / np.maximum(nrm, 1e-12)
    k = k_raw * (1.0 + (a - 1.0) * np.asarray(k_a, np.float64).reshape(1, H, N))
    w = np.exp(-0.606531 * (1.0 / (1.0 + np.exp(-w_raw))))
    return kk, k, w


# ------------------------------------------------------------------- MM8
def mm8_pack(W: np.ndarray, out_dtype=np.float16):
    """quantize_mm8 (rwkv7_hf/native_quant_mm8.py:62-97) for W [N_in, M_out].

    Returns (w_u8, mx, rx, my [N,1], ry [N,1]) with metadata cast to out_dtype.
    """
    W = np.ascontiguousarray(W, dtype=np.float32)
    n, m = W.shape
    q = np.zeros((n, m), np.uint8)
    mx = np.zeros(m, np.float32)
    rx = np.zeros(m, np.float32)
    my = np.zeros(n, np.float32)
    ry = np.zeros(n, np.float32)
    f = lib().mm8_ref_pack
    f.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64] + [ctypes.c_void_p] * 5
    f(_p(W), n, m, _p(q), _p(mx), _p(rx), _p(my), _p(ry))
    return (q, mx.astype(out_dtype), rx.astype(out_dtype), my.astype(out_dtype).reshape(n, 1),
            ry.astype(out_dtype).reshape(n, 1))


def mm8_dequant(w_u8, mx, rx, my, ry):
    """fp64 W_hat = (w + 0.5) ry rx + my + mx (rwkv7_hf/native_quant_mm8.py:100-108)."""
    q = np.asarray(w_u8, np.float64)
    return ((q + 0.5) * np.asarray(ry, np.float64).reshape(-1, 1) * np.asarray(rx, np.float64).reshape(1, -1)
            + np.asarray(my, np.float64).reshape(-1, 1) + np.asarray(mx, np.float64).reshape(1, -1))


def mm8_matmul(x, w_u8, mx, rx, my, ry):
    """fp64 x @ W_hat (rwkv7_hf/native_quant_mm8.py:111-119)."""
    return np.asarray(x, np.float64) @ mm8_dequant(w_u8, mx, rx, my, ry)


def mm8_matmul_split(x, w_u8, mx, rx, my, ry):
    """The algebraic split of rwkv7_hf/native_quant_mm8.py:246-251, fp64:
    rx * ((x ry) @ (w + 0.5)) + sum(x my) + mx sum(x).  Independent of mm8_matmul."""
    x = np.asarray(x, np.float64)
    ryv = np.asarray(ry, np.float64).reshape(-1)
    myv = np.asarray(my, np.float64).reshape(-1)
    big = (x * ryv) @ (np.asarray(w_u8, np.float64) + 0.5)
    return (big * np.asarray(rx, np.float64).reshape(1, -1) + (x @ myv)[:, None]
            + x.sum(1, keepdims=True) * np.asarray(mx, np.float64).reshape(1, -1))


# ------------------------------------------------------------- W4 group
def w4g_pack(W: np.ndarray, group: int = 128, out_dtype=np.float16):
    """quantize_w4_groupwise (rwkv7_hf/sm70_quant.py:502-519) for W [O, I]."""
    W = np.ascontiguousarray(W, dtype=np.float32)
    o, i = W.shape
    packed = np.zeros((o, i // 2), np.uint8)
    scales = np.zeros((o, i // group), np.float32)
    f = lib().w4g_ref_pack
    f.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    f(_p(W), o, i, group, _p(packed), _p(scales))
    return packed, scales.astype(out_dtype), i


def w4g_dequant(packed, scales, group: int = 128):
    """fp64 W[o,i] = (nib - 8) * scales[o, i // group] (rwkv7_hf/sm70_quant.py:598-610)."""
    p = np.asarray(packed)
    q = np.empty((p.shape[0], p.shape[1] * 2), np.float64)
    q[:, 0::2] = (p & 15).astype(np.float64) - 8
    q[:, 1::2] = (p >> 4).astype(np.float64) - 8
    return q * np.repeat(np.asarray(scales, np.float64), group, axis=1)


def w4g_linear(x, packed, scales, group: int = 128):
    return np.asarray(x, np.float64) @ w4g_dequant(packed, scales, group).T


# ----------------------------------------------- W4 group, asymmetric (affine)
def w4a_pack(W: np.ndarray, group: int = 128, out_dtype=np.float16):
    """Min/max affine group W4 for W [O, I], in fp32 numpy arithmetic (IEEE
    correctly rounded, round half to even): per (o, group) s = max((max - min)
    / 15, 1e-8), b = min, q = clamp(rint((w - b) / s), 0, 15); returns
    (packed [O, I/2] (low nibble = even input), scales, biases [O, I/group]).
    This build's own asymmetric format: it follows the form of MLX's affine
    mode (rwkv7_hf/mlx_quant.py:258-290, whose arithmetic lives in MLX, not in
    the reference) — parity with MLX is unpinned."""
    W = np.ascontiguousarray(W, dtype=np.float32)
    o, i = W.shape
    g = W.reshape(o, i // group, group)
    mn = g.min(-1)
    mx = g.max(-1)
    s = np.maximum((mx - mn) / np.float32(15.0), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.rint((g - mn[..., None]) / s[..., None]), 0, 15).astype(np.uint8).reshape(o, i)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return packed, s.astype(out_dtype), mn.astype(out_dtype)


def w4a_dequant(packed, scales, biases, group: int = 128):
    """fp64 W[o, i] = q[o, i] * scales[o, i // group] + biases[o, i // group]."""
    p = np.asarray(packed)
    q = np.empty((p.shape[0], p.shape[1] * 2), np.float64)
    q[:, 0::2] = (p & 15).astype(np.float64)
    q[:, 1::2] = (p >> 4).astype(np.float64)
    rep = lambda t: np.repeat(np.asarray(t, np.float64), group, axis=1)
    return q * rep(scales) + rep(biases)


def w4a_linear(x, packed, scales, biases, group: int = 128):
    return np.asarray(x, np.float64) @ w4a_dequant(packed, scales, biases, group).T


# ------------------------------------------------------------ MM4 affine
def mm4_pack(W: np.ndarray, out_dtype=np.float16):
    """quantize_mm4 (rwkv7_hf/native_quant_mm4.py:77-105) for W [N_in, M_out]."""
    W = np.ascontiguousarray(W, dtype=np.float32)
    n, m_orig = W.shape
    if m_orig % 2:
        W = np.concatenate([W, np.zeros((n, 1), np.float32)], axis=1)
    m = W.shape[1]
    packed = np.zeros((n, m // 2), np.uint8)
    mx = np.zeros(m, np.float32)
    rx = np.zeros(m, np.float32)
    my = np.zeros(n, np.float32)
    ry = np.zeros(n, np.float32)
    f = lib().mm4_ref_pack
    f.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64] + [ctypes.c_void_p] * 5
    f(_p(W), n, m, _p(packed), _p(mx), _p(rx), _p(my), _p(ry))
    return (packed, mx.astype(out_dtype), rx.astype(out_dtype), my.astype(out_dtype).reshape(n, 1),
            ry.astype(out_dtype).reshape(n, 1), m_orig, m)


def mm4_dequant(packed, mx, rx, my, ry, m_orig):
    """fp64 (u4 + 0.5) ry rx + my + mx (rwkv7_hf/native_quant_mm4.py:108-122)."""
    p = np.asarray(packed)
    u = np.empty((p.shape[0], p.shape[1] * 2), np.float64)
    u[:, 0::2] = p & 15
    u[:, 1::2] = p >> 4
    deq = ((u + 0.5) * np.asarray(ry, np.float64).reshape(-1, 1) * np.asarray(rx, np.float64).reshape(1, -1)
           + np.asarray(my, np.float64).reshape(-1, 1) + np.asarray(mx, np.float64).reshape(1, -1))
    return deq[:, :m_orig]


# ------------------------------------------------- elementwise / small ops
def layer_norm(x, w, b, eps=1e-5):
    """F.layer_norm over the last dim, fp64."""
    x = np.asarray(x, np.float64)
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * np.asarray(w, np.float64) + np.asarray(b, np.float64)


def attn_norm_mix6(x, prev, w, b, mixes, eps=1e-5):
    """rwkv7_hf/fused_decode_norm_mix.py:203-241: h = LN(x); out_i = h + (prev - h) mix_i; returns (outs, h)."""
    h = layer_norm(x, w, b, eps)
    return [h + (np.asarray(prev, np.float64) - h) * np.asarray(m, np.float64) for m in mixes], h


def seq_norm_mix(x, prev0, w, b, mixes, eps=1e-5):
    """rwkv7_hf/native_jit_prefill.py:533-540: shift of LN(x) over T with carried prev0; returns (outs, h[:, -1])."""
    h = layer_norm(x, w, b, eps)
    prev = np.concatenate([np.asarray(prev0, np.float64)[:, None], h[:, :-1]], 1)
    return [h + (prev - h) * np.asarray(m, np.float64) for m in mixes], h[:, -1]


def seq_shift_mix(x, prev0, mixes):
    """rwkv7_hf/fused_time_mix.py:424-427, 480-483 (the sequence mixes' torch form,
    fp64): x is already normalised; prev = [prev0, x[:, :-1]];
    out_i = x + (prev - x) mix_i; returns (outs, x[:, -1])."""
    x = np.asarray(x, np.float64)
    prev = np.concatenate([np.asarray(prev0, np.float64)[:, None], x[:, :-1]], 1)
    return [x + (prev - x) * np.asarray(m, np.float64) for m in mixes], x[:, -1]


def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def wavg_lora(xw, xa, xg, xv, W1, A1, G1, V1, W2, A2, G2, V2, w0, a0, g0, v0):
    """rwkv7_hf/fused_lora.py:795-803 (fp64): returns (w, a_pre, g, v_gate)."""
    f = lambda t: np.asarray(t, np.float64)
    bias = lambda t: 0.0 if t is None else f(t)
    w = np.tanh(f(xw) @ f(W1).T) @ f(W2).T + bias(w0)
    a = (f(xa) @ f(A1).T) @ f(A2).T + bias(a0)
    g = _sig(f(xg) @ f(G1).T) @ f(G2).T + bias(g0)
    v = _sig((f(xv) @ f(V1).T) @ f(V2).T + bias(v0))
    return w, a, g, v


def output_prepare(y, r, k, v, g, r_k, gn_w, gn_b, H, eps):
    """rwkv7_hf/fused_output.py:39-84 (fp64) over rows of H*N."""
    f = lambda t: np.asarray(t, np.float64)
    y, r, k, v, g = map(f, (y, r, k, v, g))
    rows = y.shape[0]
    N = y.shape[1] // H
    n = group_norm_heads(y, gn_w, gn_b, H, eps)
    corr = (r.reshape(rows, H, N) * k.reshape(rows, H, N) * f(r_k).reshape(1, H, N)).sum(-1, keepdims=True)
    return (n + (corr * v.reshape(rows, H, N)).reshape(rows, H * N)) * g


def state_prep(k_raw, a, w_raw, v, v_first, v_gate, k_k, k_a, H):
    """rwkv7_hf/native_jit_prefill.py:779-790 (fp64): returns (kk, k, v, log_w)."""
    f = lambda t: np.asarray(t, np.float64)
    k_raw, a, w_raw, v = map(f, (k_raw, a, w_raw, v))
    rows = k_raw.shape[0]
    N = k_raw.shape[1] // H
    kk = (k_raw * f(k_k).reshape(1, -1)).reshape(rows, H, N)
    kk = (kk / np.maximum(np.linalg.norm(kk, axis=-1, keepdims=True), 1e-12)).reshape(rows, H * N)
    k = k_raw * (1 + (a - 1) * f(k_a).reshape(1, -1))
    if v_gate is not None:
        v = v + (f(v_first) - v) * f(v_gate)
    logw = -0.606531 * _sig(w_raw)
    return kk, k, v, logw
