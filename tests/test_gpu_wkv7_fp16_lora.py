"""GPU parity: the fp16-state decode with the W/A/G/V LoRA up projections inside
the kernel (rwkv7mi_wkv7_fp16_decode_lora_output_prepare, reached through
fused_wavg_lora_output_prepare_raw with an fp16 state).

* With down-projection sums handed in whose activated, fp16-rounded mids are
  multiples of 2^-12 and fp16-rounding-safe, and coarse up weights and biases,
  every up-projection sum is exact in fp32 in any order; the fp16 LoRA outputs
  are then known on the host, and the fused kernel must equal the unfused
  fp16-state kernel fed with them to the bit (output, state, v_first, elapsed),
  for one K split and for several.
* From activations (the down launch inside the call) the result tracks the fp64
  LoRA composition with the reference's fp16 roundings of the mid and output
  tensors followed by the fp16 oracle decode: state max-abs <= 1e-2 and output
  max-abs <= 1e-2 x max(1, max|out| / 4), the fp32-state fused kernel's bar.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import wkv7_fp16_oracle as o

pytestmark = pytest.mark.gpu

OUT_ABS = 1e-2
F16 = np.float16
ACT_D = [1, 0, 2, 0]  # tanh, none, sigmoid, none (W, A, G, V down)
ACT_U = [0, 2, 0, 2]  # none, sigmoid, none, sigmoid (up)


def _t(x, dtype=torch.float16):
    return torch.tensor(np.asarray(x), dtype=dtype, device="cuda")


def _np(t):
    return t.detach().cpu().numpy()


def _sig(z):
    return 1.0 / (1.0 + np.exp(-z))


_ACT = {0: lambda z: z, 1: np.tanh, 2: _sig}


def _draw_sums(rng, act, shape):
    """Down sums (multiples of 2^-12) whose activated value rounds to an fp16
    multiple of 2^-12 away from rounding midpoints."""
    if act == 0:
        return rng.integers(-4096, 4097, shape) / 4096.0
    lo, hi = (0.3, 3.0) if act == 1 else (-1.0, 3.0)
    s = np.zeros(shape)
    bad = np.ones(shape, bool)
    for _ in range(64):
        cand = rng.integers(int(lo * 4096), int(hi * 4096) + 1, shape) / 4096.0
        if act == 1:
            cand = cand * rng.choice([-1.0, 1.0], shape)
        s = np.where(bad, cand, s)
        bad = ~o._safe16(_ACT[act](s))
        if not bad.any():
            return s
    raise RuntimeError("could not draw safe LoRA sums")


def _exact_case(rng, B, H, nl, ranks, splits):
    A = H * 64
    sums, mids, parts = [], [], []
    for q in range(nl):
        R = ranks[q]
        s = _draw_sums(rng, ACT_D[q], (B, R))
        mids.append(_ACT[ACT_D[q]](s).astype(F16).astype(np.float64))
        # split partials: small multiples of 2^-12, the last one closing the sum
        p = rng.integers(-64, 65, (splits, B, R)) / 4096.0
        p[-1] = s - p[:-1].sum(0)
        parts.append(p.reshape(-1))
        sums.append(s)
    ups = [rng.integers(-8, 9, (A, R)) / 32.0 for R in ranks[:nl]]
    ys = [mids[q] @ ups[q].T for q in range(nl)]
    biases = [rng.integers(-1024, 1025, A) / 1024.0, None, None, None][:nl]
    for q in (1, 3):
        if q >= nl:
            continue
        # a per-channel bias under which every row's sigmoid rounds safely
        bq = np.zeros(A)
        for c in range(A):
            for _ in range(400):
                cand = rng.integers(-1024, 1025) / 1024.0
                if o._safe16(_sig(ys[q][:, c] + cand)).all():
                    bq[c] = cand
                    break
            else:
                raise RuntimeError("could not draw a safe bias")
        biases[q] = bq
    outs = []
    for q in range(nl):
        y = ys[q] + (0 if biases[q] is None else biases[q])
        outs.append(_ACT[ACT_U[q]](y).astype(F16))
    return np.concatenate(parts).astype(np.float32), ups, biases, outs


def _decode_inputs(rng, B, H):
    N = 64
    return dict(r=rng.standard_normal((B, H, N)).astype(F16), k_raw=rng.standard_normal((B, H, N)).astype(F16),
                v=rng.standard_normal((B, H, N)).astype(F16),
                k_k=(1.0 + 0.1 * rng.standard_normal(H * N)).astype(F16),
                k_a=rng.uniform(0.0, 1.0, H * N).astype(F16), r_k=(rng.standard_normal(H * N) * 0.5).astype(F16),
                gn_w=(1.0 + 0.1 * rng.standard_normal(H * N)).astype(F16),
                gn_b=(0.1 * rng.standard_normal(H * N)).astype(F16),
                state=(rng.standard_normal((B, H, N, N)) * 0.5).astype(F16),
                elapsed=rng.integers(0, 5000, B).astype(np.int32), v_first=rng.standard_normal((B, H, N)).astype(F16))


@pytest.mark.parametrize("B,H,v_mode,nl,ranks,splits", [
    (1, 4, 2, 4, (64, 64, 128, 32), 1),
    (5, 3, 1, 3, (24, 128, 8), 3),
    (8, 2, 0, 3, (64, 64, 128), 1),
    (3, 4, 2, 4, (24, 128, 8, 96), 20),
    (64, 2, 2, 4, (64, 32, 128, 32), 1),
])
def test_fp16_fused_lora_equals_unfused_kernel_to_the_bit(B, H, v_mode, nl, ranks, splits):
    from rwkv7mi import native_fp16_recurrent_output_prepare_raw
    from rwkv7mi.fused_lora import fused_wavg_lora_output_prepare_raw

    rng = np.random.default_rng(7000 + B * 13 + nl * 5 + splits)
    ranks = ranks[:nl]
    A = H * 64
    part, ups, biases, lo = _exact_case(rng, B, H, nl, ranks, splits)
    c = _decode_inputs(rng, B, H)
    D = 64  # the activations are not read when the down sums are handed in
    xs = [torch.zeros(B, D, device="cuda", dtype=torch.float16) for _ in range(nl)]
    downs = [torch.zeros(R, D, device="cuda", dtype=torch.float16) for R in ranks]
    st_f, el_f = _t(c["state"]), _t(c["elapsed"], torch.int32)
    vf_f = _t(c["v_first"])
    out_f = torch.empty(B, A, device="cuda", dtype=torch.float16)
    fused_wavg_lora_output_prepare_raw(
        _t(c["r"]).view(B, A), _t(c["k_raw"]).view(B, A), _t(c["v"]).view(B, A), xs, downs, [_t(u) for u in ups],
        [None if b is None else _t(b) for b in biases], st_f, _t(c["k_k"]), _t(c["k_a"]), _t(c["r_k"]),
        _t(c["gn_w"]), _t(c["gn_b"]), eps=64e-5, out=out_f, v_first=vf_f if v_mode else None, v_mode=v_mode,
        down_sums=_t(part, torch.float32), down_splits=splits, elapsed=el_f, advance_elapsed=True)
    st_u, el_u = _t(c["state"]), _t(c["elapsed"], torch.int32)
    vf_u = _t(c["v_first"])
    bhn = lambda x: _t(x).view(B, H, 64)
    out_u = native_fp16_recurrent_output_prepare_raw(
        bhn(c["r"]), bhn(lo[0]), bhn(c["k_raw"]), bhn(c["v"]), bhn(lo[1]), st_u, bhn(lo[2]), _t(c["k_k"]),
        _t(c["k_a"]), _t(c["r_k"]), _t(c["gn_w"]), _t(c["gn_b"]), el_u, advance_elapsed=True, eps=64e-5,
        v_first=vf_u if v_mode else None, v_gate=bhn(lo[3]) if v_mode == 2 else None, v_mode=v_mode)
    torch.cuda.synchronize()
    print(f"PARITY fp16 fused LoRA B={B} H={H} v_mode={v_mode} splits={splits}: out bits equal "
          f"{torch.eq(out_f.view(-1), out_u.view(-1)).float().mean().item():.6f}, state bits equal "
          f"{torch.eq(st_f, st_u).float().mean().item():.6f}", flush=True)
    assert torch.equal(out_f.view(-1), out_u.view(-1))
    assert torch.equal(st_f, st_u)
    assert torch.equal(vf_f, vf_u)
    if v_mode == 1:
        assert torch.equal(vf_f.view(-1), _t(c["v"]).view(-1))
    assert _np(el_f).tolist() == (c["elapsed"] + 1).tolist() == _np(el_u).tolist()


@pytest.mark.parametrize("B,v_mode,nl", [(1, 2, 4), (6, 1, 3), (32, 2, 4)])
def test_fp16_fused_lora_from_activations_tracks_oracle(B, v_mode, nl):
    from rwkv7mi.fused_lora import fused_wavg_lora_output_prepare_raw

    rng = np.random.default_rng(7100 + B + nl)
    H, N, D = 4, 64, 512
    A = H * N
    ranks = (64, 64, 128, 32)[:nl]
    xs = [rng.standard_normal((B, D)).astype(F16) for _ in range(nl)]
    downs = [(rng.standard_normal((R, D)) * 0.05).astype(F16) for R in ranks]
    ups = [(rng.standard_normal((A, R)) * 0.1).astype(F16) for R in ranks]
    biases = [(rng.standard_normal(A) * 0.1).astype(F16), (rng.standard_normal(A) * 0.1).astype(F16), None,
              (rng.standard_normal(A) * 0.1).astype(F16)][:nl]
    c = _decode_inputs(rng, B, H)
    st, el = _t(c["state"]), _t(c["elapsed"], torch.int32)
    vf = _t(c["v_first"])
    out = torch.empty(B, A, device="cuda", dtype=torch.float16)
    fused_wavg_lora_output_prepare_raw(
        _t(c["r"]).view(B, A), _t(c["k_raw"]).view(B, A), _t(c["v"]).view(B, A), [_t(x) for x in xs],
        [_t(d) for d in downs], [_t(u) for u in ups], [None if b is None else _t(b) for b in biases], st,
        _t(c["k_k"]), _t(c["k_a"]), _t(c["r_k"]), _t(c["gn_w"]), _t(c["gn_b"]), eps=64e-5, out=out,
        v_first=vf if v_mode else None, v_mode=v_mode, elapsed=el, advance_elapsed=False)
    torch.cuda.synchronize()
    # fp64 LoRA with the mid and output tensors rounded to fp16, then the fp16 oracle
    f64 = lambda x: np.asarray(x, np.float64)
    lo = []
    for q in range(nl):
        mid = _ACT[ACT_D[q]](f64(xs[q]) @ f64(downs[q]).T).astype(F16)
        y = f64(mid) @ f64(ups[q]).T + (0 if biases[q] is None else f64(biases[q]))
        lo.append(_ACT[ACT_U[q]](y).astype(F16).reshape(B, H, N))
    v = c["v"]
    if v_mode == 2:
        d = (f64(c["v_first"]) - f64(v)).astype(F16)
        m = (f64(d) * f64(lo[3])).astype(F16)
        v = (f64(v) + f64(m)).astype(F16)
    ref_out, ref_st = o.decode_output_prepare_raw(c["r"], lo[0], c["k_raw"], v, lo[1], c["state"], lo[2],
                                                  c["k_k"], c["k_a"], c["r_k"], c["gn_w"], c["gn_b"], c["elapsed"],
                                                  64e-5)
    got_out, got_st = f64(_np(out)).reshape(B, H, N), f64(_np(st))
    e_st = np.abs(got_st - f64(ref_st)).max()
    e_out = np.abs(got_out - f64(ref_out)).max()
    print(f"PARITY fp16 fused LoRA from activations B={B} v_mode={v_mode}: state max-abs {e_st:.3g}, "
          f"out max-abs {e_out:.3g}", flush=True)
    assert e_st <= OUT_ABS
    assert e_out <= OUT_ABS * max(1.0, np.abs(f64(ref_out)).max() / 4)
    if v_mode == 1:
        assert torch.equal(vf.view(-1), _t(c["v"]).view(-1))
    assert _np(el).tolist() == c["elapsed"].tolist()


def test_fp16_fused_lora_rejects_bad_calls():
    from rwkv7mi.fused_lora import fused_wavg_lora_output_prepare_raw

    B, H, D, A = 2, 2, 64, 128
    z = lambda *s, dt=torch.float16: torch.zeros(*s, device="cuda", dtype=dt)
    xs = [z(B, D) for _ in range(3)]
    downs = [z(16, D) for _ in range(3)]
    ups = [z(A, 16) for _ in range(3)]
    st = z(B, H, 64, 64)
    args = (z(B, A), z(B, A), z(B, A), xs, downs, ups, [None] * 3, st, z(A), z(A), z(A), z(A), z(A))
    with pytest.raises(ValueError, match="elapsed"):
        fused_wavg_lora_output_prepare_raw(*args, eps=1e-5, out=z(B, A))
    with pytest.raises(ValueError, match="in place"):
        fused_wavg_lora_output_prepare_raw(*args, eps=1e-5, out=z(B, A), state_out=st.clone(),
                                           elapsed=z(B, dt=torch.int32))
    with pytest.raises(ValueError, match="fp16 activations"):
        fused_wavg_lora_output_prepare_raw(z(B, A, dt=torch.bfloat16), *args[1:], eps=1e-5, out=z(B, A),
                                           elapsed=z(B, dt=torch.int32))
