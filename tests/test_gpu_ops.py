"""GPU parity of the elementwise / small-GEMM kernels around the scan
(LN + token-shift mixes, W/A/G/V LoRA, output prep, state prep) against the
fp64 oracle.  Tolerance: max-abs <= 1e-2 x max(1, max|ref|) for fp16 outputs."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _t(x, dt=torch.float16):
    return torch.tensor(np.asarray(x), dtype=dt, device="cuda")


def _f(t):
    return t.detach().double().cpu().numpy()


def _ok(got, ref, tol=1e-2):
    ref = np.asarray(ref, np.float64)
    err = np.abs(_f(got) - ref).max()
    assert err <= tol * max(1.0, np.abs(ref).max()), (err, np.abs(ref).max())


@pytest.mark.parametrize("rows,D,pre", [(1, 4096, False), (8, 768, True), (3, 2560, False)])
def test_attn_norm_mix6(oracle, rows, D, pre):
    from rwkv7mi.fused_decode_norm_mix import fused_attn_norm_mix6_decode

    rng = np.random.default_rng(D + rows)
    x = _t(rng.standard_normal((rows, D)))
    prev = _t(rng.standard_normal((rows, D)))
    w, b = _t(1 + 0.1 * rng.standard_normal(D)), _t(0.1 * rng.standard_normal(D))
    mixes = [_t(rng.random(D)) for _ in range(6)]
    pw, pb = (_t(1 + 0.1 * rng.standard_normal(D)), _t(0.1 * rng.standard_normal(D))) if pre else (None, None)
    x_np, prev_np = _f(x), _f(prev)
    outs = fused_attn_norm_mix6_decode(x, prev, w, b, *mixes, pre_norm_weight=pw, pre_norm_bias=pb)
    torch.cuda.synchronize()
    if pre:
        x_np = oracle.layer_norm(x_np, _f(pw), _f(pb))
        _ok(x, x_np)
    ref, h = oracle.attn_norm_mix6(x_np, prev_np, _f(w), _f(b), [_f(m) for m in mixes])
    for got, r in zip(outs, ref):
        _ok(got, r)
    _ok(prev, h)


@pytest.mark.parametrize("rows,D,pre,dt", [(3, 4096, False, torch.float16), (8, 1024, False, torch.float16),
                                         (5, 768, True, torch.float16), (8, 2560, False, torch.bfloat16),
                                         (2, 4096, True, torch.bfloat16), (1, 128, False, torch.float16)])
def test_attn_mix_lora(oracle, rows, D, pre, dt):
    """The fused decode attention-side launch against its parts: the pre-norm,
    LN + r/k/v mixes (the fp64 oracle, as test_attn_norm_mix6) and the LoRA
    down projections of the rounded w/a/g/v mixes per K-chunk (fp32 torch on
    the kernel's own h; bound 2e-3 of the row's |m| . |W| sum)."""
    from rwkv7mi.fused_decode_norm_mix import attn_mix_lora_chunks, attn_mix_lora_decode

    rng = np.random.default_rng(D + rows)
    x = _t(rng.standard_normal((rows, D)), dt)
    prev = _t(rng.standard_normal((rows, D)), dt)
    w, b = _t(1 + 0.1 * rng.standard_normal(D), dt), _t(0.1 * rng.standard_normal(D), dt)
    mixes = [_t(rng.random(D), dt) for _ in range(6)]
    pw, pb = (_t(1 + 0.1 * rng.standard_normal(D), dt), _t(0.1 * rng.standard_normal(D), dt)) if pre else (None, None)
    ranks = [64, 64, 128, 32] if D >= 2048 else [16, 40, 48, 8]
    downs = [_t(rng.standard_normal((r, D)) / np.sqrt(D), dt) for r in ranks]
    lmix = [1, 4, 5, 3]
    x0 = x.clone()
    outs = [torch.full((rows, D), float("nan"), device="cuda", dtype=dt) for _ in range(3)]
    h_out = torch.empty_like(x)
    x_out = torch.empty_like(x) if pre else None
    C = attn_mix_lora_chunks(D)
    assert C >= 1
    part = torch.full((C * rows * sum(ranks) + 5,), float("nan"), device="cuda", dtype=torch.float32)
    got_c = attn_mix_lora_decode(x, prev, w, b, mixes, outs, downs, lmix, part, h_out=h_out, x_out=x_out,
                                 pre_norm_weight=pw, pre_norm_bias=pb)
    torch.cuda.synchronize()
    assert got_c == C
    assert torch.equal(x, x0), "x is read only"
    x_np = _f(x)
    if pre:
        x_np = oracle.layer_norm(x_np, _f(pw), _f(pb))
        _ok(x_out, x_np)
        x_np = _f(x_out)
    ref, h = oracle.attn_norm_mix6(x_np, _f(prev), _f(w), _f(b), [_f(m) for m in mixes])
    for got, r in zip(outs, (ref[0], ref[2], ref[3])):
        _ok(got, r)
    _ok(h_out, h)
    # LoRA down of the kernel's own rounded h: mixes from h_out, rounded to dt
    hf, pf = h_out.float(), prev.float()
    kc = D // C
    off = 0
    for q, (r, W) in enumerate(zip(ranks, downs)):
        mk = (hf + (pf - hf) * mixes[lmix[q]].float()).to(dt).float()
        got = part[off:off + C * rows * r].view(C, rows, r)
        for c in range(C):
            sl = slice(c * kc, (c + 1) * kc)
            want = mk[:, sl] @ W.float()[:, sl].t()
            bound = (mk[:, sl].abs() @ W.float()[:, sl].abs().t()) * 2e-3 + 1e-6
            assert ((got[c] - want).abs() <= bound).all(), (q, c, (got[c] - want).abs().max().item())
        off += C * rows * r
    assert torch.isnan(part[off:]).all(), "nothing past the sums is written"


def test_ffn_add_norm_mix(oracle):
    from rwkv7mi.fused_decode_norm_mix import fused_ffn_add_norm_mix_decode

    rng = np.random.default_rng(3)
    rows, D = 4, 4096
    res, att, prev = (_t(rng.standard_normal((rows, D))) for _ in range(3))
    w, b, m = _t(1 + 0.1 * rng.standard_normal(D)), _t(0.1 * rng.standard_normal(D)), _t(rng.random(D))
    prev_np = _f(prev)
    x, mixed = fused_ffn_add_norm_mix_decode(res, att, prev, w, b, m)
    torch.cuda.synchronize()
    xs = _f(res) + _f(att)
    _ok(x, xs)
    (ref,), h = oracle.attn_norm_mix6(_f(x), prev_np, _f(w), _f(b), [_f(m)])
    _ok(mixed, ref)
    _ok(prev, h)


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 17])
def test_dense_multi_matches_fp64(rows, dt):
    """Grouped dense products (rwkv7mi_dense_multi): the GEMV form at 1..4 rows
    (one wave per feature, fp32 FMAs) and the MFMA form above, with bias and
    every activation, K not a multiple of a pass and N not a multiple of the
    tiles, against fp64.  Bound: 1e-5 of the row's sum |x||W| in fp32 (the
    MFMA form splits fp32 into fp16 hi + lo), else one output rounding."""
    from rwkv7mi.fused_lora import dense_multi

    rng = np.random.default_rng(rows * 7 + {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[dt])
    shapes = [(768, 768, 0), (3070, 776, 3), (37, 4096, 1), (130, 3072, 2)]  # (N, K, act)
    probs, refs = [], []
    for N, K, act in shapes:
        x = _t(rng.standard_normal((rows, K)), dt)
        W = _t(rng.standard_normal((N, K)) / np.sqrt(K), dt)
        b = _t(rng.standard_normal(N) * 0.1, dt) if act != 2 else None
        y = torch.full((rows, N), float("nan"), device="cuda", dtype=dt)
        probs.append((x, W, b, y, act))
        z = _f(x) @ _f(W).T + (0 if b is None else _f(b))
        mag = np.abs(_f(x)) @ np.abs(_f(W)).T
        ref = {0: z, 1: np.tanh(z), 2: 1 / (1 + np.exp(-z)), 3: np.maximum(z, 0) ** 2}[act]
        refs.append((ref, mag, act, z))
    dense_multi(probs, rows)
    torch.cuda.synchronize()
    for (x, W, b, y, act), (ref, mag, a, z) in zip(probs, refs):
        got = _f(y)
        assert np.isfinite(got).all()
        err = np.abs(got - ref)
        # the pre-activation error bound, carried through the activation's slope
        slope = {0: 1.0, 1: 1.0, 2: 0.25, 3: 2 * np.abs(z) + 1e-3}[a]
        pre = 1e-5 * mag if dt == torch.float32 else 0.0
        out_round = (2.0 ** -8 if dt == torch.bfloat16 else 2.0 ** -11) * np.abs(ref) if dt != torch.float32 else 0.0
        assert (err <= pre * slope + out_round + 1e-6).all(), (rows, a, err.max())


@pytest.mark.parametrize("B,T,D", [(2, 33, 768), (1, 1, 4096), (3, 5, 256)])
def test_sequence_shift_mix(oracle, B, T, D):
    from rwkv7mi.fused_time_mix import fused_attn_sequence_shift_mix, fused_ffn_sequence_shift_mix

    rng = np.random.default_rng(B * T)
    x = _t(rng.standard_normal((B, T, D)))
    prev = _t(rng.standard_normal((B, D)))
    w, b = _t(1 + 0.1 * rng.standard_normal(D)), _t(0.1 * rng.standard_normal(D))
    mixes = [_t(rng.random(D)) for _ in range(6)]
    *outs, last = fused_attn_sequence_shift_mix(x, prev, *mixes, norm_weight=w, norm_bias=b)
    fk, last_f = fused_ffn_sequence_shift_mix(x, prev, mixes[0], norm_weight=w, norm_bias=b)
    torch.cuda.synchronize()
    ref, ref_last = oracle.seq_norm_mix(_f(x), _f(prev), _f(w), _f(b), [_f(m) for m in mixes])
    for got, r in zip(outs, ref):
        _ok(got, r)
    _ok(last, ref_last)
    _ok(fk, ref[0])
    _ok(last_f, ref_last)


@pytest.mark.parametrize("D,dt,norm", [(768, torch.float16, True), (4096, torch.float16, True),
                                       (4096, torch.bfloat16, False), (5000, torch.float32, True),
                                       (8192, torch.float16, True)])
def test_sequence_shift_mix_runs_equal_one_token_calls(D, dt, norm):
    """A sequence call runs several tokens per workgroup (8 here: B*T/1024),
    each token normalised once and carried to the next as its shift input; the
    same tokens fed one per call (one token per workgroup, the shift state
    threaded between the calls) give the same bits, for six mixes and one."""
    from rwkv7mi.fused_time_mix import fused_attn_sequence_shift_mix, fused_ffn_sequence_shift_mix

    rng = np.random.default_rng(D + int(norm))
    B, T = 100, 83
    x = torch.tensor(rng.standard_normal((B, T, D)), dtype=dt, device="cuda")
    prev = torch.tensor(rng.standard_normal((B, D)), dtype=dt, device="cuda")
    w = torch.tensor(1 + 0.1 * rng.standard_normal(D), dtype=dt, device="cuda") if norm else None
    b = torch.tensor(0.1 * rng.standard_normal(D), dtype=dt, device="cuda") if norm else None
    mixes = [torch.tensor(rng.random(D), dtype=dt, device="cuda") for _ in range(6)]
    *whole, last = fused_attn_sequence_shift_mix(x, prev, *mixes, norm_weight=w, norm_bias=b)
    fk, last_f = fused_ffn_sequence_shift_mix(x, prev, mixes[0], norm_weight=w, norm_bias=b)
    parts, pk, p6, p1 = [], [], prev, prev
    for t in range(T):
        xc = x[:, t:t + 1].contiguous()
        *o, p6 = fused_attn_sequence_shift_mix(xc, p6, *mixes, norm_weight=w, norm_bias=b)
        k, p1 = fused_ffn_sequence_shift_mix(xc, p1, mixes[0], norm_weight=w, norm_bias=b)
        parts.append(o)
        pk.append(k)
    torch.cuda.synchronize()
    for i in range(6):
        assert torch.equal(whole[i], torch.cat([p[i] for p in parts], 1)), i
    assert torch.equal(fk, torch.cat(pk, 1))
    assert torch.equal(last, p6) and torch.equal(last_f, p1)


# rows above 256 take the fused many-row kernel (prefills)
@pytest.mark.parametrize("rows,D,ranks", [(1, 4096, (64, 64, 128, 32)), (8, 2048, (64, 64, 128, 32)),
                                          (40, 768, (64, 64, 128, 32)), (64, 4096, (64, 64, 128, 32)),
                                          (100, 2048, (64, 64, 128, 32)), (300, 256, (64, 64, 128, 32)),
                                          (257, 512, (64, 64, 128, 32)), (1000, 4096, (64, 64, 128, 32)),
                                          (513, 768, (96, 32, 64, 128)), (700, 320, (64, 48, 128, 32))])
def test_wavg_lora(oracle, rows, D, ranks):
    """fp16 W/A/G/V LoRA against the fp64 oracle: decode sizes (split-K down,
    up kernel), and above 256 rows the many-row kernels (ranks that are
    multiples of 32 with D a multiple of 64: the LDS-shared form; the last case
    the per-row-tile form)."""
    from rwkv7mi.fused_lora import fused_wavg_lora

    rng = np.random.default_rng(rows + D)
    A = D
    xs = [_t(rng.standard_normal((rows, D))) for _ in range(4)]
    downs = [_t(rng.standard_normal((r, D)) * 0.02) for r in ranks]
    ups = [_t(rng.standard_normal((A, r)) * 0.1) for r in ranks]
    biases = [_t(rng.standard_normal(A) * 0.01), _t(rng.standard_normal(A) * 0.01), None,
              _t(rng.standard_normal(A) * 0.01)]
    got = fused_wavg_lora(*xs, *downs, *ups, *biases)
    torch.cuda.synchronize()
    ref = oracle.wavg_lora(*map(_f, xs), *map(_f, downs), *map(_f, ups),
                           *[None if b is None else _f(b) for b in biases])
    for g, r in zip(got, ref):
        _ok(g, r)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,D", [(2, 1024), (33, 200), (64, 200), (300, 200)])
def test_wag_lora_dtypes(oracle, dt, rows, D):
    from rwkv7mi.fused_lora import fused_wag_lora

    rng = np.random.default_rng(rows * 7 + D)
    A = 512
    xs = [_t(rng.standard_normal((rows, D)), dt) for _ in range(3)]
    ranks = (32, 48, 96)
    downs = [_t(rng.standard_normal((r, D)) * 0.02, dt) for r in ranks]
    ups = [_t(rng.standard_normal((A, r)) * 0.1, dt) for r in ranks]
    biases = [_t(rng.standard_normal(A) * 0.01, dt), None, _t(rng.standard_normal(A) * 0.01, dt)]
    got = fused_wag_lora(*xs, *downs, *ups, *biases)
    torch.cuda.synchronize()
    # the intermediate is rounded to the activation dtype, as the reference's tensor is
    rnd = (lambda a: _f(torch.tensor(a, dtype=dt))) if dt != torch.float32 else (lambda a: a)
    acts = (np.tanh, lambda v: v, lambda v: 1 / (1 + np.exp(-v)))
    for q in range(3):
        mid = rnd(acts[q](_f(xs[q]) @ _f(downs[q]).T))
        ref = mid @ _f(ups[q]).T + (0 if biases[q] is None else _f(biases[q]))
        _ok(got[q], ref, tol=1e-2 if dt == torch.bfloat16 else 1e-4)


@pytest.mark.parametrize("rows", [20, 70])
def test_lora_rank_above_128(oracle, rows):
    """Ranks above 128 take 32-row launch pairs (64-row pairs hold ranks up to 128)."""
    from rwkv7mi.fused_lora import fused_wag_lora

    rng = np.random.default_rng(rows)
    D, A = 512, 256
    xs = [_t(rng.standard_normal((rows, D))) for _ in range(3)]
    ranks = (32, 160, 256)
    downs = [_t(rng.standard_normal((r, D)) * 0.02) for r in ranks]
    ups = [_t(rng.standard_normal((A, r)) * 0.1) for r in ranks]
    biases = [None, _t(rng.standard_normal(A) * 0.01), None]
    got = fused_wag_lora(*xs, *downs, *ups, *biases)
    torch.cuda.synchronize()
    rnd = lambda a: _f(torch.tensor(a, dtype=torch.float16))
    acts = (np.tanh, lambda v: v, lambda v: 1 / (1 + np.exp(-v)))
    for q in range(3):
        mid = rnd(acts[q](_f(xs[q]) @ _f(downs[q]).T))
        ref = mid @ _f(ups[q]).T + (0 if biases[q] is None else _f(biases[q]))
        _ok(got[q], ref)


def test_output_prepare_and_state_prep(oracle):
    from rwkv7mi.fused_output import fused_attn_output_prepare
    from rwkv7mi.fused_prefill import fused_prefill_state_prep

    rng = np.random.default_rng(5)
    rows, H, N = 70, 12, 64
    A = H * N
    y, r, k, v, g = (_t(rng.standard_normal((rows, A))) for _ in range(5))
    r_k, gw, gb = _t(0.1 * rng.standard_normal((H, N))), _t(1 + rng.standard_normal(A) * 0.1), _t(rng.standard_normal(A) * 0.1)
    out = fused_attn_output_prepare(y, r, k, v, g, r_k, gw, gb, num_heads=H, head_dim=N, head_v_dim=N, eps=N * 1e-5)
    torch.cuda.synchronize()
    _ok(out, oracle.output_prepare(_f(y), _f(r), _f(k), _f(v), _f(g), _f(r_k), _f(gw), _f(gb), H, N * 1e-5))
    k_raw, w_raw, vv = (_t(rng.standard_normal((rows, A))) for _ in range(3))
    a = _t(1 / (1 + np.exp(-rng.standard_normal((rows, A)))))
    k_k, k_a = _t(0.85 + 0.1 * rng.standard_normal(A)), _t(1 + 0.1 * rng.standard_normal(A))
    vfirst = _t(rng.standard_normal((rows, A)))
    vgate = _t(1 / (1 + np.exp(-rng.standard_normal((rows, A)))))
    w_log, k_out, v_out, kk = fused_prefill_state_prep(w_raw, k_raw, vv, a, k_k, k_a, v_first=vfirst, v_gate=vgate,
                                                       num_heads=H, head_dim=N, w_transform="log")
    w_dec, *_ = fused_prefill_state_prep(w_raw, k_raw, vv, a, k_k, k_a, num_heads=H, head_dim=N)
    torch.cuda.synchronize()
    rkk, rk, rv, rlog = oracle.state_prep(_f(k_raw), _f(a), _f(w_raw), _f(vv), _f(vfirst), _f(vgate), _f(k_k),
                                          _f(k_a), H)
    _ok(kk, rkk)
    _ok(k_out, rk)
    _ok(v_out, rv)
    _ok(w_log, rlog, 1e-5)
    _ok(w_dec, np.exp(rlog), 1e-5)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,n", [(1, 65536), (8, 65536), (64, 65536), (3, 1000), (2, 8)])
def test_argmax_rows_matches_torch(dtype, rows, n):
    """rwkv7mi_argmax_rows against torch.argmax: random rows, rows with
    planted ties (the first index must win), a row whose maximum is the last
    element, and rows holding NaN (the first NaN wins, as in torch)."""
    from rwkv7mi import argmax_rows

    g = torch.Generator(device="cuda").manual_seed(rows * 7 + n)
    x = torch.randn(rows, n, device="cuda", generator=g).to(dtype)
    if rows >= 3:
        x[0, n // 3] = x[0, 2 * n // 3] = 50.0  # a tie
        x[1, -1] = 60.0  # the last element
        x[2, n // 4] = float("nan")
        x[2, n // 2] = float("nan")
    if rows >= 8:
        x[3] = float("-inf")  # every entry equal: index 0
        x[4, 4095] = x[4, 4096] = 70.0  # a tie across two slices of the many-workgroup form
    got = argmax_rows(x)
    out2 = torch.full((rows,), -1, device="cuda", dtype=torch.int64)
    got2 = argmax_rows(x, out2=out2)
    # the single-workgroup entry point gives the same indices
    from rwkv7mi import _lib
    one = torch.full((rows,), -1, device="cuda", dtype=torch.int64)
    _lib.call("rwkv7mi_argmax_rows", _lib.ptr(x), rows, n, int(x.stride(0)), _lib.dtype_code(x), _lib.ptr(one),
              None, _lib.stream_of(x))
    torch.cuda.synchronize()
    ref = x.argmax(-1)
    assert torch.equal(got, ref)
    assert torch.equal(got2, ref) and torch.equal(out2, ref)
    assert torch.equal(one, ref)
    if rows >= 3:
        assert int(got[0]) == n // 3 and int(got[1]) == n - 1 and int(got[2]) == n // 4
