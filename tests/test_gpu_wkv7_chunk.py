"""GPU parity: chunked DPLR prefill vs the fp64 sequential oracle.

Inputs follow BASELINE.json configs[1]: r,k,v ~ N(0,1) fp16, k L2-normalised,
kk = k, a = sigmoid(N(0,1)), w = exp(-exp(x)), x ~ N(-0.5, 0.5) in fp32.
Tolerance: y max-abs <= 1e-2 for fp16/fp32 outputs (for bf16 outputs, whose
rounding step is 2^-8 relative, max-abs <= max(1e-2, 2^-8 max|y|)); fp32 state
max-abs error <= 1e-4 x max|state|.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(rng, B, T, H, N=64, dtype=torch.float16, state_scale=0.0, real_decay=False):
    r, k, v = (rng.standard_normal((B, T, H, N)) for _ in range(3))
    k /= np.maximum(np.linalg.norm(k, axis=-1, keepdims=True), 1e-12)
    a = 1 / (1 + np.exp(-rng.standard_normal((B, T, H, N))))
    if real_decay:  # model form: exp(-0.606531 * sigmoid(x))
        w = np.exp(-0.606531 / (1 + np.exp(-rng.standard_normal((B, T, H, N)))))
    else:
        w = np.exp(-np.exp(rng.normal(-0.5, 0.5, (B, T, H, N))))
    st = rng.standard_normal((B, H, N, N)) * state_scale
    d = lambda x: torch.tensor(x, dtype=dtype, device="cuda")
    args = [d(r), torch.tensor(w, dtype=torch.float32, device="cuda"), d(k), d(v), d(k), d(a)]
    return args, torch.tensor(st, dtype=torch.float32, device="cuda"), st


def _check(oracle, args, state_np, y, s):
    torch.cuda.synchronize()
    ref_y, ref_s = oracle.wkv7_scan(*(x.double().cpu().numpy() for x in args), state_np)
    ey = np.abs(y.double().cpu().numpy() - ref_y).max() if ref_y.size else 0.0
    es = np.abs(s.double().cpu().numpy() - ref_s).max() / max(np.abs(ref_s).max(), 1e-30)
    tol_y = 1e-2
    if y.dtype == torch.bfloat16 and ref_y.size:
        tol_y = max(tol_y, 2.0 ** -8 * np.abs(ref_y).max())
    assert ey <= tol_y, (ey, tol_y)
    assert es <= 1e-4, es
    return ey, es


@pytest.mark.parametrize("B,T,H", [(1, 16, 1), (2, 64, 4), (1, 37, 2), (2, 1, 3), (1, 0, 2), (3, 300, 5)])
def test_chunk_matches_oracle(oracle, B, T, H):
    from rwkv7mi import dplr_chunk_scan

    rng = np.random.default_rng(9 + T)
    args, st, st_np = _inputs(rng, B, T, H, state_scale=0.1)
    y, s = dplr_chunk_scan(*args, st)
    assert y.shape == (B, T, H, 64)
    _check(oracle, args, st_np, y, s)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_chunk_dtypes(oracle, dtype):
    from rwkv7mi import dplr_chunk_scan

    rng = np.random.default_rng(21)
    args, st, st_np = _inputs(rng, 2, 96, 3, dtype=dtype, state_scale=0.1)
    y, s = dplr_chunk_scan(*args, st)
    _check(oracle, args, st_np, y, s)


def test_chunk_real_model_decay_long(oracle):
    from rwkv7mi import self_chunk_rwkv7

    rng = np.random.default_rng(22)
    args, st, st_np = _inputs(rng, 1, 1024, 2, real_decay=True)
    y, s = self_chunk_rwkv7(*args, st, chunk_size=16)
    _check(oracle, args, st_np, y, s)


def test_chunk_strong_decay_mixed_tiles(oracle):
    """Channels 32-63 decay hard (about -7 log2 per token, chunk totals -110 to
    -180, where the centring of the gated rows matters) and channels 0-31
    weakly, in one chunk; then every channel decays hard.  Totals stay inside
    the span the centred form keeps exact (-240)."""
    from rwkv7mi import dplr_chunk_scan

    rng = np.random.default_rng(27)
    B, T, H, N = 2, 80, 3, 64
    args, st, st_np = _inputs(rng, B, T, H, state_scale=0.1)
    x = rng.normal(-0.5, 0.5, (B, T, H, N))
    x[..., 32:] = rng.normal(1.6, 0.15, (B, T, H, N - 32))
    args[1] = torch.tensor(np.exp(-np.exp(x)), dtype=torch.float32, device="cuda")
    y, s = dplr_chunk_scan(*args, st)
    _check(oracle, args, st_np, y, s)
    args[1] = torch.tensor(np.exp(-np.exp(rng.normal(1.6, 0.15, (B, T, H, N)))), dtype=torch.float32,
                           device="cuda")
    y, s = dplr_chunk_scan(*args, st)
    _check(oracle, args, st_np, y, s)


def test_chunk_log_decay_input(oracle):
    from rwkv7mi import self_chunk_rwkv7

    rng = np.random.default_rng(23)
    args, st, st_np = _inputs(rng, 2, 64, 2, state_scale=0.1)
    logw = torch.log(args[1])
    y, s = self_chunk_rwkv7(args[0], logw, *args[2:], st, chunk_size=32, w_is_log=True)
    _check(oracle, args, st_np, y, s)


def test_chunk_equals_sequential_kernel():
    """Two independent device algorithms (WY chunk vs on-chip sequential scan)."""
    from rwkv7mi import dplr_chunk_scan, fused_recurrent_scan

    rng = np.random.default_rng(24)
    args, st, _ = _inputs(rng, 2, 512, 4, state_scale=0.1)
    y1, s1 = dplr_chunk_scan(*args, st)
    y2, s2 = fused_recurrent_scan(*args, st)
    torch.cuda.synchronize()
    assert (y1.float() - y2.float()).abs().max().item() <= 1e-2
    assert ((s1 - s2).abs().max() / s2.abs().max()).item() <= 2e-4


def test_chunk_split_sequence_continues_state(oracle):
    """Prefill in two calls with the carried state == one call (cache continuation)."""
    from rwkv7mi import dplr_chunk_scan

    rng = np.random.default_rng(25)
    args, st, _ = _inputs(rng, 1, 160, 2)
    y_full, s_full = dplr_chunk_scan(*args, st)
    first = [x[:, :64] for x in args]
    second = [x[:, 64:] for x in args]
    y1, s_mid = dplr_chunk_scan(*first, st)
    y2, s_end = dplr_chunk_scan(*second, s_mid)
    torch.cuda.synchronize()
    assert (torch.cat([y1, y2], 1).float() - y_full.float()).abs().max().item() <= 1e-2
    assert ((s_end - s_full).abs().max() / s_full.abs().max()).item() <= 1e-4


def test_self_chunk_rejects_ragged_like_reference():
    from rwkv7mi import self_chunk_rwkv7

    rng = np.random.default_rng(26)
    args, st, _ = _inputs(rng, 1, 20, 1)
    with pytest.raises(ValueError):
        self_chunk_rwkv7(*args, st, chunk_size=16)
    with pytest.raises(ValueError):
        self_chunk_rwkv7(*[x[:, :16] for x in args], st, chunk_size=8)


@pytest.mark.parametrize("H", [32, 64])
def test_chunk_full_size_properties(H):
    """BASELINE configs[1] size (B=8, T=4096): finite, sequential-kernel agreement."""
    from rwkv7mi import fused_recurrent_scan, self_chunk_rwkv7

    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    B, T, N = 8, 4096, 64
    r = torch.randn(B, T, H, N, generator=g, device="cuda").half()
    k = torch.randn(B, T, H, N, generator=g, device="cuda")
    k = (k / k.norm(dim=-1, keepdim=True)).half()
    v = torch.randn(B, T, H, N, generator=g, device="cuda").half()
    a = torch.sigmoid(torch.randn(B, T, H, N, generator=g, device="cuda")).half()
    w = torch.exp(-torch.exp(torch.randn(B, T, H, N, generator=g, device="cuda") * 0.5 - 0.5))
    st = torch.zeros(B, H, N, N, device="cuda")
    y1, s1 = self_chunk_rwkv7(r, w, k, v, k, a, st)
    y2, s2 = fused_recurrent_scan(r, w, k, v, k, a, st)
    torch.cuda.synchronize()
    assert torch.isfinite(y1).all() and torch.isfinite(s1).all()
    assert (y1.float() - y2.float()).abs().max().item() <= 1e-2
    assert ((s1 - s2).abs().max() / s2.abs().max()).item() <= 2e-4
