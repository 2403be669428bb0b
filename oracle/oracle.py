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
