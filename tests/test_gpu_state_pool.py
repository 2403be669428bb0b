"""The serving state-slot pool on the GPU: the HIP slot-copy kernel against
torch indexing (bit-exact: byte moves), the allocator's generation checks,
clone / reset / snapshot / restore, and graph-bucketed decode over arbitrary
slot sets equal, row for row, to the dense cache decode of the same rows at
the same bucket size; a continuous-batching sequence (requests joining and
leaving) against isolated single-request runs."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _cfg():
    from rwkv7mi.model import NativeRWKV7Config

    return NativeRWKV7Config(vocab_size=512, hidden_size=256, num_hidden_layers=2, intermediate_size=1024,
                             decay_low_rank_dim=16, a_low_rank_dim=16, gate_low_rank_dim=32, v_low_rank_dim=16)


@pytest.fixture(scope="module")
def model():
    from rwkv7mi.model import NativeRWKV7ForCausalLM

    return NativeRWKV7ForCausalLM.from_random(_cfg(), seed=0, device="cuda", dtype=torch.float16)


def test_slot_copy_matches_indexing():
    from rwkv7mi.state_pool import _slot_copy
    from rwkv7mi import _lib

    g = torch.Generator("cuda").manual_seed(0)
    src = torch.randn(3, 10, 48, device="cuda", generator=g)  # [layers, rows, 48 floats = 192 bytes]
    dst = torch.randn(3, 6, 48, device="cuda", generator=g)
    keep = dst.clone()
    sidx = torch.tensor([7, 0, 3, 9], device="cuda")
    didx = torch.tensor([5, 1, 0, 4], device="cuda")
    act = torch.tensor([1, 0, 1, 1], dtype=torch.uint8, device="cuda")
    st = _lib.stream_of(src)
    _slot_copy(src.data_ptr(), src[0].numel() * 4, 192, sidx, dst.data_ptr(), dst[0].numel() * 4, 192, didx, act,
               4, 192, 3, st)
    want = keep.clone()
    for r in range(4):
        if act[r]:
            want[:, didx[r]] = src[:, sidx[r]]
    torch.cuda.synchronize()
    assert torch.equal(dst, want)
    # zero fill, identity source rows
    _slot_copy(None, 0, 0, None, dst.data_ptr(), dst[0].numel() * 4, 192, didx[:2], None, 2, 192, 3, st)
    want[:, didx[:2]] = 0
    torch.cuda.synchronize()
    assert torch.equal(dst, want)
    with pytest.raises(ValueError):
        _slot_copy(src.data_ptr(), 0, 4, None, dst.data_ptr(), 0, 4, None, None, 1, 12, 1, st)


def test_allocator_generations_and_copies():
    from rwkv7mi.state_pool import RWKV7StatePool

    pool = RWKV7StatePool(_cfg(), 4, device="cuda")
    handles = pool.allocate(["a", "b", "c"])
    slots = [s for s, _ in handles]
    gens = [g for _, g in handles]
    assert slots == [0, 1, 2] and pool.free_slots() == 1
    pool.state[:, 0].normal_()
    pool.xpa[:, 0].normal_()
    pool.v_first[0].normal_()
    pool.seen_tokens[0] = 11
    pool.clone([0], [2])
    torch.cuda.synchronize()
    assert torch.equal(pool.state[:, 2], pool.state[:, 0]) and torch.equal(pool.xpa[:, 2], pool.xpa[:, 0])
    assert torch.equal(pool.v_first[2], pool.v_first[0]) and pool.seen_tokens[2] == 11
    snap = pool.snapshot(0)
    pool.reset([0])
    torch.cuda.synchronize()
    assert not pool.state[:, 0].any() and pool.seen_tokens[0] == 0
    pool.restore(snap, 0)
    assert torch.equal(pool.state[:, 0], pool.state[:, 2])
    bad = dict(snap, checksum="0" * 64)
    with pytest.raises(ValueError):
        pool.restore(bad, 1)
    pool.free([1], [gens[1]])
    with pytest.raises(ValueError):  # stale handle
        pool.free([1], [gens[1]])
    (s2, g2), = pool.allocate(["d"])
    assert s2 == 1 and g2 == gens[1] + 1
    with pytest.raises(ValueError):
        pool.check([1], [gens[1]])
    with pytest.raises(ValueError):
        pool.check([0, 0])
    with pytest.raises(RuntimeError):
        pool.allocate(["e", "f"])


def test_pooled_decode_equals_dense_rows(model):
    from rwkv7mi.state_pool import PooledDecoder, RWKV7StatePool

    cfg = model.config
    pool = RWKV7StatePool(cfg, 6, device="cuda")
    dec = PooledDecoder(model, pool)
    handles = pool.allocate(list("abcde"))
    rng = np.random.default_rng(0)
    # prefill each request alone (mixed prompt lengths)
    for (s, g), T in zip(handles, (5, 3, 7, 2, 4)):
        ids = torch.tensor(rng.integers(0, cfg.vocab_size, (1, T)), device="cuda")
        dec.prefill([s], [g], ids)
    order = [handles[3], handles[0], handles[4]]  # any slot order
    slots = [s for s, _ in order]
    gens = [g for _, g in order]
    tok = torch.tensor(rng.integers(0, cfg.vocab_size, (3,)), device="cuda")
    # dense reference at the same bucket (4): rows gathered by hand, the pad row zeros
    ref_cache = pool.gather_cache(slots + [pool.scratch_slot], allow_scratch=True)
    ref_cache2 = ref_cache.clone()
    runner = model.graph_runner(4)
    ref_logits = runner.replay(torch.cat([tok, tok[:1]]), ref_cache2).clone()
    # (the runner's buffers are reused by the pooled step: keep copies)
    ref_state = [t.clone() for t in ref_cache2._state]
    ref_xpa = [t.clone() for t in ref_cache2._xpa]
    got = dec.step(slots, gens, tok)
    torch.cuda.synchronize()
    assert torch.equal(got, ref_logits[:3])
    for i, s in enumerate(slots):
        for l in range(cfg.num_hidden_layers):
            assert torch.equal(pool.state[l, s], ref_state[l][i])
            assert torch.equal(pool.xpa[l, s], ref_xpa[l][i])
    assert pool.seen_tokens[slots[0]] == 2 + 1


def test_continuous_batching_matches_isolated_runs(model):
    from rwkv7mi.state_pool import PooledDecoder, RWKV7StatePool

    cfg = model.config
    pool = RWKV7StatePool(cfg, 8, device="cuda")
    dec = PooledDecoder(model, pool)
    rng = np.random.default_rng(1)
    prompts = {r: torch.tensor(rng.integers(0, cfg.vocab_size, (1, 4)), device="cuda") for r in "ABCDE"}
    toks = {r: rng.integers(0, cfg.vocab_size, (3,)) for r in "ABCDE"}
    live = {}
    for r in "ABCD":
        (s, g), = pool.allocate([r])
        live[r] = (s, g)
        dec.prefill([s], [g], prompts[r])
    got = {r: [] for r in "ABCDE"}
    schedule = [list("ABCD"), list("ACDE"), list("EAC")]
    for t, names in enumerate(schedule):
        if "B" in live and "B" not in names:  # B finishes
            pool.free([live["B"][0]], [live["B"][1]])
            del live["B"]
        if "E" in names and "E" not in live:  # E joins into B's old slot
            (s, g), = pool.allocate(["E"])
            live["E"] = (s, g)
            dec.prefill([s], [g], prompts["E"])
        step_tokens = [int(toks[r][sum(r in sc for sc in schedule[:t])]) for r in names]
        logits = dec.step([live[r][0] for r in names], [live[r][1] for r in names], step_tokens)
        for r, lg in zip(names, logits):
            got[r].append(lg.float())
    # isolated single-request runs (eager, batch 1) of the same token streams
    for r in "ABCDE":
        out = model(prompts[r], use_graph=False)
        cache = out.past_key_values
        n = sum(r in sc for sc in schedule)
        for j in range(n):
            lg = model(torch.tensor([[int(toks[r][j])]], device="cuda"), past_key_values=cache,
                       use_graph=False).logits[0, -1].float()
            ref = got[r][j]
            assert (lg - ref).abs().max().item() <= 2e-2 * max(1.0, lg.abs().max().item()), (r, j)


def test_two_bound_caches_alternate_and_pool_step_between(model):
    """Two bsz-1 caches alternating through the bsz-1 decode graph each keep
    their own state: rebinding the runner gives the previously bound cache a
    copy of the runner's buffers (rwkv7_hf/native_graph_runtime.py:618-630).
    A pooled step on the same bucket in between leaves a bound cache's state
    alone, and its returned logits survive the bucket's next replay."""
    from rwkv7mi.state_pool import PooledDecoder, RWKV7StatePool

    cfg = model.config
    rng = np.random.default_rng(5)
    prompts = [torch.tensor(rng.integers(0, cfg.vocab_size, (1, T)), device="cuda") for T in (6, 4)]
    toks = rng.integers(0, cfg.vocab_size, (2, 4))
    graph_caches = [model(p).past_key_values for p in prompts]
    eager_caches = [model(p).past_key_values for p in prompts]
    pool = RWKV7StatePool(cfg, 2, device="cuda")
    dec = PooledDecoder(model, pool)
    (slot, gen), = pool.allocate(["x"])
    dec.prefill([slot], [gen], prompts[1])
    kept = None
    for j in range(4):
        for i in (0, 1):
            t = torch.tensor([[int(toks[i, j])]], device="cuda")
            got = model(t, past_key_values=graph_caches[i], use_graph=True).logits
            ref = model(t, past_key_values=eager_caches[i], use_graph=False).logits
            assert torch.equal(got, ref), (i, j)
        if j == 1:  # a pooled step on the bsz-1 bucket while cache 1 is bound to it
            kept = dec.step([slot], [gen], [int(toks[1, 0])])
            kept_copy = kept.clone()
    torch.cuda.synchronize()
    assert torch.equal(kept, kept_copy)  # not overwritten by later replays of the bucket
    for gc, ec in zip(graph_caches, eager_caches):
        for l in range(cfg.num_hidden_layers):
            assert torch.equal(gc._state[l], ec._state[l]) and torch.equal(gc._xpa[l], ec._xpa[l])
