"""GPU parity: wkv7 decode-step and sequential-scan kernels vs the fp64 oracle.

Tolerances (stated by the build's target): activation outputs (fp16/bf16)
max-abs <= 1e-2; fp32 state max-abs error <= 1e-4 x max|state|.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

STATE_REL = 1e-4
OUT_ABS = 1e-2


def _vec(rng, shape, scale=0.2):
    return rng.standard_normal(shape) * scale


def _decode_inputs(rng, B, H, N=64):
    r, k, v = (_vec(rng, (B, H, N)) for _ in range(3))
    w = np.exp(-np.exp(rng.normal(-0.5, 0.5, (B, H, N))))
    kk = rng.standard_normal((B, H, N))
    kk /= np.linalg.norm(kk, axis=-1, keepdims=True)
    a = 1 / (1 + np.exp(-rng.standard_normal((B, H, N))))
    state = rng.standard_normal((B, H, N, N)) * 0.1
    return r, w, k, v, kk, a, state


def _t(x, dtype):
    return torch.tensor(np.asarray(x), dtype=dtype, device="cuda")


def _f64(t):
    return t.detach().double().cpu().numpy()


def _state_ok(got, ref):
    err = np.abs(_f64(got) - ref).max()
    assert err <= STATE_REL * np.abs(ref).max(), (err, np.abs(ref).max())


@pytest.mark.parametrize("B,H", [(1, 4), (2, 32), (8, 64), (3, 5)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_decode_update(oracle, B, H, dtype):
    from rwkv7mi import fused_recurrent_update

    rng = np.random.default_rng(100 + B * H)
    r, w, k, v, kk, a, state = _decode_inputs(rng, B, H)
    # the kernel sees the activation-dtype-rounded inputs; so does the oracle
    args = [_t(x, dtype) for x in (r, w, k, v, kk, a)]
    args[1] = _t(w, torch.float32)  # decay in fp32 as the reference computes it
    st = _t(state, torch.float32)
    y, new_state = fused_recurrent_update(*args, st)
    torch.cuda.synchronize()
    ref_y, ref_s = oracle.wkv7_update(*(_f64(x) for x in args), state)
    _state_ok(new_state, ref_s)
    assert np.abs(_f64(y) - ref_y).max() <= OUT_ABS
    assert torch.equal(st, _t(state, torch.float32)), "input state must not be modified"


def test_decode_update_in_place_and_flat(oracle):
    from rwkv7mi import fused_recurrent_update

    rng = np.random.default_rng(7)
    B, H, N = 4, 8, 64
    r, w, k, v, kk, a, state = _decode_inputs(rng, B, H)
    args = [_t(x, torch.float16).reshape(B, H * N) for x in (r, k, v, kk, a)]
    wt = _t(w, torch.float32).reshape(B, H * N)
    st = _t(state, torch.float32)
    y, new_state = fused_recurrent_update(args[0], wt, args[1], args[2], args[3], args[4], st, state_out=st)
    torch.cuda.synchronize()
    assert new_state.data_ptr() == st.data_ptr()
    assert y.shape == (B, H * N)
    ref_y, ref_s = oracle.wkv7_update(_f64(args[0]).reshape(B, H, N), _f64(wt).reshape(B, H, N),
                                      *(_f64(x).reshape(B, H, N) for x in args[1:]), state)
    _state_ok(st, ref_s)
    assert np.abs(_f64(y).reshape(B, H, N) - ref_y).max() <= OUT_ABS


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_decode_output_prepare(oracle, dtype):
    from rwkv7mi import fused_recurrent_output_prepare

    rng = np.random.default_rng(11)
    B, H, N = 3, 16, 64
    r, w, k, v, kk, a, state = _decode_inputs(rng, B, H)
    g = _vec(rng, (B, H, N))
    r_k = rng.standard_normal((H, N)) * 0.1
    gn_w = rng.standard_normal(H * N)
    gn_b = rng.standard_normal(H * N)
    eps = N * 1e-5
    t = lambda x: _t(x, dtype)
    args = [t(r), _t(w, torch.float32), t(k), t(v), t(kk), t(a)]
    out, new_state = fused_recurrent_output_prepare(*args, _t(state, torch.float32), t(g), t(r_k), t(gn_w),
                                                    t(gn_b), eps=eps)
    torch.cuda.synchronize()
    ref, ref_s = oracle.wkv7_output_prepare(*(_f64(x) for x in args), state, _f64(t(g)), _f64(t(r_k)),
                                            _f64(t(gn_w)), _f64(t(gn_b)), eps)
    _state_ok(new_state, ref_s)
    assert np.abs(_f64(out) - ref).max() <= OUT_ABS * max(1.0, np.abs(ref).max() / 4)


@pytest.mark.parametrize("v_mode", [0, 1, 2])
def test_decode_output_prepare_raw(oracle, v_mode):
    from rwkv7mi import fused_recurrent_output_prepare_raw

    rng = np.random.default_rng(707)  # reference raw test seed (tests/test_fused_recurrent_output_raw.py)
    B, H, N = 2, 4, 64
    dt = torch.float16
    r, w_raw, k_raw, v, g = (_vec(rng, (B, H, N)) for _ in range(5))
    a = 1 / (1 + np.exp(-rng.standard_normal((B, H, N))))
    state = rng.standard_normal((B, H, N, N)) * 0.1
    k_k = rng.standard_normal((H, N))
    k_a = rng.standard_normal((H, N)) * 0.1
    r_k = rng.standard_normal((H, N)) * 0.1
    gn_w, gn_b = rng.standard_normal(H * N), rng.standard_normal(H * N)
    v_first0 = _vec(rng, (B, H * N))
    v_gate = 1 / (1 + np.exp(-rng.standard_normal((B, H * N))))
    eps = N * 1e-5
    T = [_t(x, dt) for x in (r, w_raw, k_raw, v, a, g, k_k, k_a, r_k, gn_w, gn_b)]
    vf = _t(v_first0, dt)
    vg = _t(v_gate, dt)
    out, new_state = fused_recurrent_output_prepare_raw(
        *T[:5], _t(state, torch.float32), *T[5:], eps=eps, v_first=vf if v_mode else None,
        v_gate=vg if v_mode == 2 else None, v_mode=v_mode)
    torch.cuda.synchronize()
    F = [_f64(x) for x in T]
    kk, k, w = oracle.decode_raw_prep(F[2], F[1], F[4], F[6], F[7])
    vv = F[3]
    if v_mode == 2:
        vfirst = _f64(_t(v_first0, dt)).reshape(B, H, N)
        vv = vv + (vfirst - vv) * _f64(vg).reshape(B, H, N)
    ref, ref_s = oracle.wkv7_output_prepare(F[0], w, k, vv, kk, F[4], state, F[5], F[8], F[9], F[10], eps)
    _state_ok(new_state, ref_s)
    assert np.abs(_f64(out) - ref).max() <= OUT_ABS * max(1.0, np.abs(ref).max() / 4)
    if v_mode == 1:
        assert torch.equal(vf.reshape(B, H, N), T[3])


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,v_mode,nl", [(1, 2, 4), (3, 2, 4), (8, 1, 3), (32, 2, 4), (64, 2, 4), (2, 0, 3)])
@pytest.mark.parametrize("ranks", [(64, 64, 128, 32), (24, 128, 8, 96)])
def test_decode_fused_lora(oracle, dt, B, v_mode, nl, ranks):
    """LoRA up projections fused into the decode kernel == the fp64 oracle composition
    (LoRA, then the raw decode prep) with the reference's roundings of the mid and
    output tensors to the activation dtype, and == the unfused kernels."""
    from rwkv7mi import fused_recurrent_output_prepare_raw
    from rwkv7mi.fused_lora import fused_wavg_lora_output_prepare_raw, lora_multi

    rng = np.random.default_rng(B * 11 + v_mode + nl)
    H, N, D = 4, 64, 512
    A = H * N
    ranks = ranks[:nl]
    xs = [_t(_vec(rng, (B, D), 1.0), dt) for _ in range(nl)]
    downs = [_t(rng.standard_normal((r, D)) * 0.05, dt) for r in ranks]
    ups = [_t(rng.standard_normal((A, r)) * 0.1, dt) for r in ranks]
    biases = [_t(rng.standard_normal(A) * 0.1, dt), _t(rng.standard_normal(A) * 0.1, dt), None,
              _t(rng.standard_normal(A) * 0.1, dt)][:nl]
    r, k_raw, v = (_t(_vec(rng, (B, A)), dt) for _ in range(3))
    state = rng.standard_normal((B, H, N, N)) * 0.1
    k_k = _t(rng.standard_normal((H, N)), dt)
    k_a = _t(rng.standard_normal((H, N)) * 0.1, dt)
    r_k = _t(rng.standard_normal((H, N)) * 0.1, dt)
    gn_w, gn_b = _t(rng.standard_normal(A), dt), _t(rng.standard_normal(A), dt)
    v_first0 = _vec(rng, (B, A))
    eps = N * 1e-5
    vf = _t(v_first0, dt)
    out = torch.empty(B, A, device="cuda", dtype=dt)
    st = _t(state, torch.float32)
    fused_wavg_lora_output_prepare_raw(r, k_raw, v, xs, downs, ups, biases, st, k_k, k_a, r_k, gn_w, gn_b,
                                       eps=eps, out=out, v_first=vf if v_mode else None, v_mode=v_mode)
    # unfused kernels on the same inputs
    lo = [torch.empty(B, A, device="cuda", dtype=dt) for _ in range(nl)]
    acts_d, acts_u = [1, 0, 2, 0][:nl], [0, 2, 0, 2][:nl]
    lora_multi(xs, downs, ups, biases, lo, acts_d, acts_u)
    vf2 = _t(v_first0, dt)
    out2, st2 = fused_recurrent_output_prepare_raw(
        r.view(B, H, N), lo[0].view(B, H, N), k_raw.view(B, H, N), v.view(B, H, N), lo[1].view(B, H, N),
        _t(state, torch.float32), lo[2].view(B, H, N), k_k, k_a, r_k, gn_w, gn_b, eps=eps,
        v_first=vf2 if v_mode else None, v_gate=lo[3] if v_mode == 2 else None, v_mode=v_mode)
    torch.cuda.synchronize()
    # oracle: fp64 LoRA with the mid / output tensors rounded to dt, then the decode prep
    rnd = lambda a: _f64(torch.tensor(a, dtype=dt))
    sig = lambda z: 1 / (1 + np.exp(-z))
    act = {0: lambda z: z, 1: np.tanh, 2: sig}
    ys = []
    for q in range(nl):
        mid = rnd(act[acts_d[q]](_f64(xs[q]) @ _f64(downs[q]).T))
        y = mid @ _f64(ups[q]).T + (0 if biases[q] is None else _f64(biases[q]))
        ys.append(rnd(act[acts_u[q]](y)))
    kk, k, w = oracle.decode_raw_prep(_f64(k_raw).reshape(B, H, N), ys[0].reshape(B, H, N),
                                      ys[1].reshape(B, H, N), _f64(k_k), _f64(k_a))
    vv = _f64(v).reshape(B, H, N)
    if v_mode == 2:
        vv = vv + (_f64(_t(v_first0, dt)).reshape(B, H, N) - vv) * ys[3].reshape(B, H, N)
    ref, ref_s = oracle.wkv7_output_prepare(_f64(r).reshape(B, H, N), w, k, vv, kk, ys[1].reshape(B, H, N), state,
                                            ys[2].reshape(B, H, N), _f64(r_k), _f64(gn_w), _f64(gn_b), eps)
    # a one-ulp difference of a rounded LoRA output moves the state by ~2^-11 of a term
    ssc = np.abs(ref_s).max()
    assert np.abs(_f64(st) - ref_s).max() <= 1e-3 * ssc
    tol = OUT_ABS if dt == torch.float16 else 4 * OUT_ABS
    assert np.abs(_f64(out).reshape(B, H, N) - ref).max() <= tol * max(1.0, np.abs(ref).max() / 4)
    assert np.abs(_f64(st) - _f64(st2)).max() <= 1e-3 * ssc
    assert np.abs(_f64(out) - _f64(out2).reshape(B, A)).max() <= tol * max(1.0, np.abs(ref).max() / 4)
    if v_mode == 1:
        assert torch.equal(vf, v)
    # whole-K down sums handed in (the layout the LN-mix GEMV prologue writes)
    sums = torch.cat([(xs[q].double() @ downs[q].double().T).float().reshape(-1) for q in range(nl)])
    out3 = torch.empty_like(out)
    st3 = _t(state, torch.float32)
    vf3 = _t(v_first0, dt)
    fused_wavg_lora_output_prepare_raw(r, k_raw, v, xs, downs, ups, biases, st3, k_k, k_a, r_k, gn_w, gn_b,
                                       eps=eps, out=out3, v_first=vf3 if v_mode else None, v_mode=v_mode,
                                       down_sums=sums.contiguous())
    torch.cuda.synchronize()
    assert np.abs(_f64(st3) - ref_s).max() <= 1e-3 * ssc
    assert np.abs(_f64(out3).reshape(B, H, N) - ref).max() <= tol * max(1.0, np.abs(ref).max() / 4)


def test_decode_fused_lora_rejects_unsupported():
    from rwkv7mi.fused_lora import fused_lora_decode_supported

    assert fused_lora_decode_supported((64, 64, 128, 32), 8)
    assert fused_lora_decode_supported((64, 64, 128, 32), 64)
    assert not fused_lora_decode_supported((64, 64, 128, 32), 65)
    assert fused_lora_decode_supported((64, 64, 120, 40), 1)
    assert not fused_lora_decode_supported((64, 64, 124, 32), 1)
    assert not fused_lora_decode_supported((64, 64, 256, 32), 1)


@pytest.mark.parametrize("B,T,H", [(1, 1, 2), (2, 37, 4), (1, 256, 8), (2, 0, 2)])
def test_sequential_scan(oracle, B, T, H):
    from rwkv7mi import fused_recurrent_scan

    rng = np.random.default_rng(1000 + T)
    N = 64
    r, k, v = (_vec(rng, (B, T, H, N), 1.0) for _ in range(3))
    k /= np.maximum(np.linalg.norm(k, axis=-1, keepdims=True), 1e-12)
    kk = k.copy()
    a = -kk
    w = np.exp(-np.exp(rng.normal(-0.5, 0.5, (B, T, H, N))))
    state = rng.standard_normal((B, H, N, N)) * 0.1
    dt = torch.float16
    # the scan takes (kk, a) of the native form: a_vec = -kk, b_vec = kk * a
    gate = 1 / (1 + np.exp(-rng.standard_normal((B, T, H, N))))
    args = [_t(r, dt), _t(w, torch.float32), _t(k, dt), _t(v, dt), _t(kk, dt), _t(gate, dt)]
    y, final = fused_recurrent_scan(*args, _t(state, torch.float32))
    torch.cuda.synchronize()
    ref_y, ref_s = oracle.wkv7_scan(*(_f64(x) for x in args), state)
    _state_ok(final, ref_s)
    if T:
        assert np.abs(_f64(y) - ref_y).max() <= OUT_ABS
    assert y.shape == (B, T, H, N)
