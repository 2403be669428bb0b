"""GPU tests of the drop-in seams: the reference's fused scan variants
(rwkv7_hf/fused_recurrent_update.py:1420, 1541, 1710), the sequence shift
mixes in the reference's calling convention (fused_time_mix.py:413-515), the
chunk kernel's status word, workspace growth under captured graphs, the
``forward`` contract (native_model.py:618-853), the quantized-module hooks
(``rwkv7_forward_ffn``, workspace sizing) and ``quantize_model_mm8``'s cache
invalidation (native_quant_mm8.py:631-684).

Tolerances: scan outputs max-abs <= 1e-2 (fp16), fp32 state <= 1e-4 relative,
as the north star states; elementwise ops max-abs <= 1e-2 x max(1, |ref|);
MM8 products relative <= 2e-3 of the fp64 product on the dequantised weights.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _t(a, dtype=torch.float16):
    return torch.tensor(np.asarray(a), dtype=dtype, device="cuda")


def _f(t):
    return t.double().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t, np.float64)


def _ok(got, ref, tol=1e-2):
    got = _f(got)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref).max() if ref.size else 0.0
    assert err <= tol * max(1.0, np.abs(ref).max() if ref.size else 1.0), err


def _scan_inputs(rng, B, T, H, N=64):
    r, k, v = (rng.standard_normal((B, T, H, N)) for _ in range(3))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    a = 1 / (1 + np.exp(-rng.standard_normal((B, T, H, N))))
    return r, k, v, a


def _check_scan(oracle, r, w, k, v, kk, a, st, y, s):
    torch.cuda.synchronize()
    ref_y, ref_s = oracle.wkv7_scan(*(_f(x) for x in (r, w, k, v, kk, a)), st)
    _ok(y, ref_y)
    assert np.abs(_f(s) - ref_s).max() <= 1e-4 * max(np.abs(ref_s).max(), 1e-30)


@pytest.mark.parametrize("T", [48, 37])
def test_scan_clampw_matches_oracle(oracle, T):
    """w_raw -> exp(-0.606531 sigmoid(w_raw)) inside the chunk kernel."""
    from rwkv7mi import fused_recurrent_scan_clampw

    rng = np.random.default_rng(40 + T)
    B, H, N = 2, 3, 64
    r, k, v, a = _scan_inputs(rng, B, T, H)
    w_raw = rng.standard_normal((B, T, H, N)) * 2
    st = 0.1 * rng.standard_normal((B, H, N, N))
    args = [_t(x) for x in (r, w_raw, k, v, k, a)]
    y, s = fused_recurrent_scan_clampw(*args, _t(st, torch.float32))
    # the decay the reference computes from the fp16 w_raw
    w = np.exp(-0.606531 / (1 + np.exp(-_f(args[1]))))
    _check_scan(oracle, args[0], w, *args[2:], st, y, s)
    # flat [B, T, H*N] inputs come back flat
    yf, _ = fused_recurrent_scan_clampw(*[x.reshape(B, T, H * N) for x in args], _t(st, torch.float32))
    assert yf.shape == (B, T, H * N)
    assert torch.equal(yf.reshape(B, T, H, N), y)


@pytest.mark.parametrize("vgate", [False, True])
def test_scan_state_prep_matches_oracle(oracle, vgate):
    from rwkv7mi import fused_recurrent_scan_state_prep

    rng = np.random.default_rng(50 + vgate)
    B, T, H, N = 2, 40, 2, 64
    A = H * N
    r, k_raw, v_raw, a = (rng.standard_normal((B, T, H, N)) for _ in range(4))
    a = 1 / (1 + np.exp(-a))
    w_raw = rng.standard_normal((B, T, H, N))
    k_k, k_a = 0.85 + 0.1 * rng.standard_normal(A), 1 + 0.1 * rng.standard_normal(A)
    vf = rng.standard_normal((B, T, H, N))
    vg = 1 / (1 + np.exp(-rng.standard_normal((B, T, H, N))))
    st = 0.1 * rng.standard_normal((B, H, N, N))
    tr, tw, tk, tv, ta = (_t(x) for x in (r, w_raw, k_raw, v_raw, a))
    kw = dict(v_first=_t(vf), v_gate=_t(vg)) if vgate else {}
    y, s, k_adj, v_adj = fused_recurrent_scan_state_prep(tr, tw, tk, tv, ta, _t(st, torch.float32), _t(k_k),
                                                         _t(k_a), **kw)
    torch.cuda.synchronize()
    flat = lambda t: _f(t).reshape(B * T, A)
    kk, k_ref, v_ref, logw = oracle.state_prep(flat(tk), flat(ta), flat(tw), flat(tv),
                                               flat(kw["v_first"]) if vgate else None,
                                               flat(kw["v_gate"]) if vgate else None, _f(_t(k_k)), _f(_t(k_a)), H)
    _ok(k_adj.reshape(B * T, A), k_ref)
    _ok(v_adj.reshape(B * T, A), v_ref)
    shp = (B, T, H, N)
    # the scan consumed the kernel's own rounded k / v and kk: the oracle runs on those
    ref_y, ref_s = oracle.wkv7_scan(_f(tr), np.exp(logw).reshape(shp), _f(k_adj), _f(v_adj), kk.reshape(shp),
                                    _f(ta), st)
    _ok(y, ref_y)
    assert np.abs(_f(s) - ref_s).max() <= 1e-4 * np.abs(ref_s).max()


def test_scan_output_prepare_matches_oracle(oracle):
    from rwkv7mi import fused_recurrent_scan_output_prepare

    rng = np.random.default_rng(60)
    B, T, H, N = 2, 33, 3, 64
    A = H * N
    r, k, v, a = _scan_inputs(rng, B, T, H)
    w = np.exp(-np.exp(rng.normal(-0.5, 0.5, (B, T, H, N))))
    g = rng.standard_normal((B, T, H, N))
    r_k = 0.1 * rng.standard_normal((H, N))
    gw, gb = 1 + 0.1 * rng.standard_normal(A), 0.1 * rng.standard_normal(A)
    st = 0.1 * rng.standard_normal((B, H, N, N))
    args = [_t(r), _t(w, torch.float32), _t(k), _t(v), _t(k), _t(a)]
    prep, s = fused_recurrent_scan_output_prepare(*args, _t(st, torch.float32), _t(g), _t(r_k), _t(gw), _t(gb),
                                                  eps=N * 1e-5)
    torch.cuda.synchronize()
    ref_y, ref_s = oracle.wkv7_scan(*(_f(x) for x in args), st)
    assert np.abs(_f(s) - ref_s).max() <= 1e-4 * np.abs(ref_s).max()
    # the kernel hands the output prep its y rounded to fp16, as the reference's tensor is
    y16 = _f(_t(ref_y)).reshape(B * T, A)
    ref = oracle.output_prepare(y16, _f(args[0]).reshape(B * T, A), _f(args[2]).reshape(B * T, A),
                                _f(args[3]).reshape(B * T, A), _f(_t(g)).reshape(B * T, A), _f(_t(r_k)),
                                _f(_t(gw)), _f(_t(gb)), H, N * 1e-5)
    _ok(prep.reshape(B * T, A), ref, tol=2e-2)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_sequence_shift_mix_reference_convention(oracle, dtype):
    """x already normalised, no norm arguments: (xr, xw, xk, xv, xa, xg, x[:, -1]);
    a workspace is filled in the reference's physical order r, k, v, w, a, g."""
    from rwkv7mi.fused_time_mix import fused_attn_sequence_shift_mix, fused_ffn_sequence_shift_mix

    rng = np.random.default_rng(70)
    B, T, D = 2, 9, 256
    x = _t(rng.standard_normal((B, T, D)), dtype)
    prev = _t(rng.standard_normal((B, D)), dtype)
    mixes = [_t(rng.random(D), dtype) for _ in range(6)]
    ws = torch.empty(6, B, T, D, device="cuda", dtype=dtype)
    *outs, last = fused_attn_sequence_shift_mix(x, prev, *mixes, block_size=256, workspace=ws)
    torch.cuda.synchronize()
    ref, ref_last = oracle.seq_shift_mix(_f(x), _f(prev), [_f(m) for m in mixes])
    for o, rr in zip(outs, ref):
        _ok(o, rr)
    assert torch.equal(last, x[:, -1])
    for logical, slot in enumerate((0, 3, 1, 2, 4, 5)):
        assert outs[logical].data_ptr() == ws[slot].data_ptr()
    fk, lastf = fused_ffn_sequence_shift_mix(x, prev, mixes[2])
    torch.cuda.synchronize()
    _ok(fk, ref[2])
    assert torch.equal(lastf, x[:, -1])


def test_chunk_status_word(oracle):
    """Ordinary calls leave the status clear; a chunk whose log2-decay span is
    far beyond 252 reports the clamp (no timeout either way)."""
    from rwkv7mi import dplr_chunk_scan
    from rwkv7mi.self_chunk_rwkv7 import CHUNK_STATUS_CLAMPED, CHUNK_STATUS_TIMEOUT, wkv7_chunk_status

    wkv7_chunk_status(clear=True)
    rng = np.random.default_rng(80)
    B, T, H, N = 1, 32, 2, 64
    r, k, v, a = _scan_inputs(rng, B, T, H)
    w = np.exp(-np.exp(rng.normal(-0.5, 0.5, (B, T, H, N))))
    args = [_t(r), _t(w, torch.float32), _t(k), _t(v), _t(k), _t(a)]
    dplr_chunk_scan(*args, torch.zeros(B, H, N, N, device="cuda"))
    assert wkv7_chunk_status(clear=True) == 0
    # about -26 log2 per token: chunk totals near -420
    args[1] = _t(np.exp(-np.exp(rng.normal(2.9, 0.05, (B, T, H, N)))), torch.float32)
    dplr_chunk_scan(*args, torch.zeros(B, H, N, N, device="cuda"))
    st = wkv7_chunk_status(clear=True)
    assert st & CHUNK_STATUS_CLAMPED and not st & CHUNK_STATUS_TIMEOUT
    assert wkv7_chunk_status(clear=True) == 0


def _tiny_mm8_model(hidden=256, layers=2, vocab=1024, ffn=512):
    from rwkv7mi.model import NativeRWKV7Config, NativeRWKV7ForCausalLM, random_weights

    cfg = NativeRWKV7Config(vocab_size=vocab, hidden_size=hidden, num_hidden_layers=layers, intermediate_size=ffn,
                            decay_low_rank_dim=32, a_low_rank_dim=32, gate_low_rank_dim=64, v_low_rank_dim=32,
                            use_native_mm8=True, native_mm8_min_params=0)
    w = random_weights(cfg, seed=3, device="cpu", dtype=torch.float16)
    return cfg, NativeRWKV7ForCausalLM(cfg, w, device="cuda", dtype=torch.float16)


def test_workspace_growth_keeps_captured_graphs_valid():
    """Capture a 20-row runner (many-row GEMM, "mm8g" slot), then grow every
    slot far beyond its size; replays of the older graph must still equal the
    eager step bit for bit, and the replaced buffers stay allocated."""
    from rwkv7mi import workspace as ws

    cfg, model = _tiny_mm8_model()
    B = 20
    rng = np.random.default_rng(90)
    ids = torch.tensor(rng.integers(0, cfg.vocab_size, (B, 6)), device="cuda")
    c1 = model(ids).past_key_values
    c2 = c1.clone()
    runner = model.graph_runner(B)
    before = ws.retired_bytes(torch.device("cuda", 0))
    for slot in ("mm8", "mm8g", "lora"):
        cur = ws.reserve(torch.device("cuda", 0), 0, slot=slot)
        ws.reserve(torch.device("cuda", 0), 4 * int(cur.numel()), slot=slot)
    assert ws.retired_bytes(torch.device("cuda", 0)) > before
    model.graph_runner(64)  # a second runner captured against the grown slots
    for step in range(3):
        tok = torch.tensor(rng.integers(0, cfg.vocab_size, (B,)), device="cuda")
        eager = model(tok[:, None], past_key_values=c1, use_graph=False).logits[:, -1]
        got = runner.replay(tok, c2).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, eager), step


def test_forward_contract():
    """labels -> shifted cross-entropy over all tokens; logits_to_keep; inputs_embeds
    == input_ids; tuple form; all-ones masks accepted, token-dropping masks refused."""
    cfg, model = _tiny_mm8_model(layers=1)
    rng = np.random.default_rng(91)
    B, T = 2, 12
    ids = torch.tensor(rng.integers(0, cfg.vocab_size, (B, T)), device="cuda")
    full = model(ids, logits_to_keep=0).logits
    assert full.shape == (B, T, cfg.vocab_size)
    last = model(ids).logits
    assert last.shape == (B, 1, cfg.vocab_size)
    # (2 head rows run the GEMV, 24 rows the tile GEMM: equal up to summation order)
    near = lambda a, b: (a.float() - b.float()).abs().max().item() <= 2e-3 * b.float().abs().max().item()
    assert near(last[:, 0], full[:, -1])
    three = model(ids, logits_to_keep=3).logits
    assert three.shape == (B, 3, cfg.vocab_size) and near(three, full[:, -3:])
    labels = ids.clone()
    labels[0, 5] = -100
    out = model(ids, labels=labels)
    ref = torch.nn.functional.cross_entropy(full[:, :-1].float().reshape(-1, cfg.vocab_size),
                                            labels[:, 1:].reshape(-1), ignore_index=-100)
    assert abs(out.loss.item() - ref.item()) <= 1e-4 * max(1.0, abs(ref.item()))
    emb = model.emb[ids]
    by_embeds = model(inputs_embeds=emb, logits_to_keep=0).logits
    assert torch.equal(by_embeds, full)
    tup = model(ids, return_dict=False)
    assert isinstance(tup, tuple) and torch.equal(tup[0], last)
    ok = model(ids, attention_mask=torch.ones(B, T, device="cuda", dtype=torch.long))
    assert torch.equal(ok.logits, last)
    mask = torch.ones(B, T, device="cuda", dtype=torch.long)
    mask[1, 0] = 0
    with pytest.raises(ValueError):
        model(ids, attention_mask=mask)
    with pytest.raises(ValueError):
        model(ids, inputs_embeds=emb)
    legacy = model(ids, return_legacy_cache=True).past_key_values
    assert isinstance(legacy, tuple) and len(legacy) == 4 and legacy.get_seq_length() == T
    # a legacy tuple continues like the cache object it came from
    cache = model(ids).past_key_values
    tok = ids[:, -1:]
    a = model(tok, past_key_values=legacy, use_graph=False).logits
    b = model(tok, past_key_values=cache, use_graph=False).logits
    assert torch.equal(a, b)


def test_cache_bound_reorder_is_in_place():
    """select_batch on a cache bound to a graph runner permutes the runner's
    buffers in place and keeps the binding."""
    cfg, model = _tiny_mm8_model(layers=1)
    rng = np.random.default_rng(92)
    B = 3
    ids = torch.tensor(rng.integers(0, cfg.vocab_size, (B, 5)), device="cuda")
    cache = model(ids).past_key_values
    ref = cache.clone()
    tok = torch.tensor(rng.integers(0, cfg.vocab_size, (B,)), device="cuda")
    runner = model.graph_runner(B)
    runner.replay(tok, cache)
    model(tok[:, None], past_key_values=ref, use_graph=False)
    idx = torch.tensor([2, 0, 1], device="cuda")
    cache.select_batch(idx)
    ref.select_batch(idx)
    assert cache._native_graph_bound_to(runner)
    assert cache.rwkv7_cache_metrics()["native_graph_bound_selects"] == 1
    for s1, s2 in zip(cache._state, ref._state):
        assert torch.equal(s1, s2)
    assert torch.equal(runner.replay(tok, cache),
                       model(tok[:, None], past_key_values=ref, use_graph=False).logits[:, -1])


def test_mm8_forward_ffn_and_workspace_hook(oracle):
    from rwkv7mi import MM8Linear
    from rwkv7mi.native_quant_mm8 import GEMM_ROWS, GEMV_ROWS

    torch.manual_seed(5)
    key = MM8Linear(torch.nn.Linear(256, 512, bias=False).cuda().half())
    value = MM8Linear(torch.nn.Linear(512, 256, bias=False).cuda().half())
    for rows in (1, 8, 40):
        x = torch.randn(rows, 256, device="cuda", dtype=torch.float16)
        res = torch.randn(rows, 256, device="cuda", dtype=torch.float16)
        got = key.rwkv7_forward_ffn(x, value, res)
        h = key.rwkv7_forward_relu2(x)
        ref = value.rwkv7_forward_add(h, res)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), rows
        assert got.data_ptr() != res.data_ptr()
    assert key.rwkv7_forward_ffn(x, torch.nn.Linear(512, 256), res) is None
    assert key.rwkv7_workspace_bytes(GEMV_ROWS) == 0
    assert key.rwkv7_workspace_bytes(GEMV_ROWS + 1) > 0
    assert key.rwkv7_workspace_bytes(GEMM_ROWS + 1) == 0


def test_quantize_model_mm8_swaps_and_invalidates(oracle):
    """quantize_model_mm8 on a plain module tree: the policy's targets become
    MM8Linear with the reference packer's bytes, outputs match the fp64 product
    on the dequantised weights, and the model's pack / graph-runner caches are
    dropped."""
    from rwkv7mi import MM8Linear, quantize_model_mm8

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.key = torch.nn.Linear(256, 1024, bias=False)
            self.value = torch.nn.Linear(1024, 256, bias=False)
            self.small = torch.nn.Linear(32, 32)

    class Toy(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.ffn = Block()
            self.lm_head = torch.nn.Linear(256, 2048, bias=False)

    torch.manual_seed(6)
    toy = Toy().cuda().half()
    w_key = toy.ffn.key.weight.detach().float().cpu().numpy()
    toy._rwkv7_native_graph_runner_cache = {"stale": 1}
    toy._rwkv7_native_jit_pack_cache = [1]
    n = quantize_model_mm8(toy, min_params=200_000)
    assert n == 3
    assert isinstance(toy.ffn.key, MM8Linear) and isinstance(toy.lm_head, MM8Linear)
    assert isinstance(toy.ffn.small, torch.nn.Linear)
    assert not hasattr(toy, "_rwkv7_native_graph_runner_cache") and not hasattr(toy, "_rwkv7_native_jit_pack_cache")
    assert toy._rwkv7_native_mm_quantization == "mm8" and toy._rwkv7_native_mm_replaced_modules == 3
    packed = oracle.mm8_pack(w_key.T.astype(np.float16).astype(np.float32))
    m = toy.ffn.key
    np.testing.assert_array_equal(m.w_u8.cpu().numpy(), packed[0])
    x = torch.randn(3, 256, device="cuda", dtype=torch.float16)
    y = m(x)
    torch.cuda.synchronize()
    wd = oracle.mm8_dequant(*(t.cpu().numpy() for t in (m.w_u8, m.mx, m.rx, m.my, m.ry)))
    ref = _f(x) @ wd
    assert np.abs(_f(y) - ref).max() <= 2e-3 * np.abs(ref).max()
    assert quantize_model_mm8(torch.nn.Sequential(torch.nn.Linear(8, 8)).cuda(), policy="speed") == 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_mm8_dequant_matches_oracle(oracle, dtype):
    from rwkv7mi import MM8Linear

    """The dequantised weight in the activation dtype (rwkv7_hf/native_quant_mm8.py:100-108)."""
    from rwkv7mi.native_quant_mm8 import dequantize_mm8, quantize_mm8

    rng = np.random.default_rng(93)
    W = rng.standard_normal((300, 200)) * 0.02
    w_u8, mx, rx, my, ry = quantize_mm8(_t(W))
    got = dequantize_mm8(w_u8, mx, rx, my, ry, out_dtype=dtype)
    blk = MM8Linear(torch.nn.Linear(300, 200, bias=False).cuda().half())
    with torch.no_grad():
        blk.load_state_dict({"w_u8": w_u8, "mx": mx, "rx": rx, "my": my, "ry": ry})
    got_blk = dequantize_mm8(blk.w_blk, blk.mx, blk.rx, blk.my, blk.ry, out_dtype=dtype)
    torch.cuda.synchronize()
    assert got.shape == got_blk.shape == (300, 200) and torch.equal(got, got_blk)
    ref = oracle.mm8_dequant(*(t.cpu().numpy() for t in (w_u8, mx, rx, my, ry)))
    tol = 2.0 ** -10 if dtype == torch.float16 else 1e-6
    assert np.abs(_f(got) - ref).max() <= tol * np.abs(ref).max()


def test_torch_ops_match_python_functions():
    """torch.ops.rwkv7mi.* run the same kernels as the Python operators, and the
    in-place forms update their marked arguments (also inside a captured graph)."""
    import rwkv7mi
    from rwkv7mi import dplr_chunk_scan, fused_recurrent_update, mm8_matmul, quantize_mm8

    rng = np.random.default_rng(95)
    B, T, H, N = 2, 32, 2, 64
    r, k, v, a = _scan_inputs(rng, B, T, H)
    w = np.exp(-np.exp(rng.normal(-0.5, 0.5, (B, T, H, N))))
    args = [_t(r), _t(w, torch.float32), _t(k), _t(v), _t(k), _t(a)]
    st = _t(0.1 * rng.standard_normal((B, H, N, N)), torch.float32)
    y1, s1 = dplr_chunk_scan(*args, st)
    y2, s2 = torch.ops.rwkv7mi.chunk_scan(*args, st, 0)
    assert torch.equal(y1, y2) and torch.equal(s1, s2)
    st_in = st.clone()
    y3 = torch.empty_like(args[0])
    torch.ops.rwkv7mi.chunk_scan_(*args, st_in, 0, y3)
    assert torch.equal(y3, y1) and torch.equal(st_in, s1)
    # captured: replays from the same start state give the same result each time
    st_g, y_g = st.clone(), torch.empty_like(args[0])
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        torch.ops.rwkv7mi.chunk_scan_(*args, st_g, 0, y_g)
    for _ in range(3):
        st_g.copy_(st)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_g, y1) and torch.equal(st_g, s1)
    # one-token update, out of place and in place
    one = [x[:, 0] for x in args]
    o1, n1 = fused_recurrent_update(*one, st)
    o2, n2 = torch.ops.rwkv7mi.fused_recurrent_update(*one, st)
    assert torch.equal(o1, o2) and torch.equal(n1, n2)
    st2, o3 = st.clone(), torch.empty_like(o1)
    torch.ops.rwkv7mi.fused_recurrent_update_(*one, st2, o3)
    assert torch.equal(o3, o1) and torch.equal(st2, n1)
    # MM8
    W = _t(rng.standard_normal((256, 128)) * 0.02)
    q = quantize_mm8(W)
    q2 = torch.ops.rwkv7mi.quantize_mm8(W)
    assert all(torch.equal(u, v2) for u, v2 in zip(q, q2))
    x = _t(rng.standard_normal((3, 256)))
    ym = mm8_matmul(x, *q)
    assert torch.equal(torch.ops.rwkv7mi.mm8_matmul(x, *q), ym)
    out = torch.empty_like(ym)
    torch.ops.rwkv7mi.mm8_matmul_out(x, *q, out)
    assert torch.equal(out, ym)
    # sequence shift mix
    xs = _t(rng.standard_normal((B, 5, 64)))
    prev = _t(rng.standard_normal((B, 64)))
    mixes = [_t(rng.random(64)) for _ in range(2)]
    got = torch.ops.rwkv7mi.seq_shift_mix(xs, prev, mixes)
    ref = rwkv7mi.fused_time_mix.fused_ffn_sequence_shift_mix(xs, prev, mixes[1])
    assert len(got) == 3 and torch.equal(got[1], ref[0]) and torch.equal(got[2], ref[1])


def test_graph_packs_round_trip():
    """extract_graph_packs gives the reference's 41-entry tuples (quantized
    projections as MM8Linear callables, layer 0's placeholders); a model built
    from them decodes bit for bit like the original."""
    from rwkv7mi import MM8Linear
    from rwkv7mi.model import NativeRWKV7ForCausalLM

    cfg, model = _tiny_mm8_model(layers=2)
    packs, H, N, eps = model.extract_graph_packs()
    assert len(packs) == 2 and all(len(p) == 41 for p in packs)
    assert (H, N, eps) == (cfg.num_heads, 64, 64 * 1e-5)
    p0, p1 = packs
    assert p0[4] == 1 and p1[4] == 0 and float(p1[5].abs().sum()) == 0
    assert isinstance(p0[20], MM8Linear) and isinstance(p0[38], MM8Linear) and p0[40].numel() == 0
    assert tuple(p0[30].shape) == (1, cfg.hidden_size) and float(p0[31].abs().sum()) == 0  # no V LoRA on layer 0
    assert tuple(p1[30].shape) == (cfg.v_low_rank_dim, cfg.hidden_size)
    twin = NativeRWKV7ForCausalLM.from_graph_packs(cfg, packs, embeddings=model.emb, norm_weight=model.norm[0],
                                                   norm_bias=model.norm[1], lm_head=model.lm_head.m)
    assert twin._rwkv7_native_mm_replaced_modules == model._rwkv7_native_mm_replaced_modules
    ids = torch.tensor(np.random.default_rng(96).integers(0, cfg.vocab_size, (2, 7)), device="cuda")
    a = model(ids).logits
    b = twin(ids).logits
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    with pytest.raises(ValueError):
        NativeRWKV7ForCausalLM.from_graph_packs(cfg, packs[:1], embeddings=model.emb, norm_weight=model.norm[0],
                                               norm_bias=model.norm[1], lm_head=model.lm_head.m)
