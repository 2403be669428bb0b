"""Host-side contract of NativeRWKV7Cache (rwkv7_hf/model_cache.py:48-466) on
CPU tensors: the cache is bookkeeping over tensors, so its edits run without
a GPU.  Covers the tuple / legacy conversions, sizes, batch edits, device
moves, detach, crop, the graph-binding version protocol and the metrics, and
the forward-argument helpers (logits_to_keep, attention masks, cache coercion).
"""
from __future__ import annotations

import pytest
import torch


def _cache(B=3, L=2, H=2, N=4, D=8, seen=5):
    from rwkv7mi.model import NativeRWKV7Cache

    g = torch.Generator().manual_seed(0)
    st = [torch.randn(B, H, N, N, generator=g) for _ in range(L)]
    xa = [torch.randn(B, D, generator=g) for _ in range(L)]
    xf = [torch.randn(B, D, generator=g) for _ in range(L)]
    vf = torch.randn(B, H * N, generator=g)
    return NativeRWKV7Cache(st, xa, xf, vf, seen_tokens=seen)


def test_tuple_view_and_legacy_round_trip():
    from rwkv7mi.model import NativeRWKV7Cache

    c = _cache()
    state, xpa, xpf, v_first = c
    assert len(c) == 4 and state is c._state and v_first is c._v_first
    legacy = c.to_legacy_cache()
    assert isinstance(legacy, tuple) and legacy.get_seq_length() == 5 and legacy.seen_tokens == 5
    assert legacy.get_seq_length(layer_idx=7) == 0 and legacy.get_seq_length(layer_idx=-1) == 0
    back = NativeRWKV7Cache.from_legacy_cache(legacy)
    assert back.seen_tokens == 5 and back._state is state
    assert NativeRWKV7Cache.from_legacy_cache(c) is c
    assert NativeRWKV7Cache.from_legacy_cache(None).get_batch_size() is None
    assert NativeRWKV7Cache.from_legacy_cache(()).seen_tokens == 0
    with pytest.raises(TypeError):
        NativeRWKV7Cache.from_legacy_cache((1, 2, 3))
    assert c[0] is state and c[3] is v_first


def test_sizes_and_flags():
    c = _cache()
    assert c.get_batch_size() == 3 and c.max_batch_size == 3 and c.max_cache_len == -1
    assert c.get_seq_length() == 5 and c.get_seq_length(1) == 5 and c.get_seq_length(2) == 0
    assert c.get_mask_sizes(torch.arange(4)) == (9, 0) and c.get_mask_sizes(2) == (7, 0)
    assert c.get_mask_sizes(None) == (5, 0)
    assert c.is_initialized and c.has_previous_state() and c.has_previous_state(1) and not c.has_previous_state(2)
    assert not c.is_sliding and c.get_max_cache_shape() == -1
    assert len(c.states) == 2 and c.states[1]["recurrent_state"] is c._state[1]
    assert "seen_tokens=5" in repr(c)


def test_select_repeat_compact_reorder():
    c = _cache()
    ref = c.clone()
    c.select_batch(torch.tensor([2, 0]))
    assert c.get_batch_size() == 2
    assert torch.equal(c._state[1][0], ref._state[1][2]) and torch.equal(c._v_first[1], ref._v_first[0])
    d = ref.clone()
    out = d.batch_select([1], inplace=False)
    assert out is not d and out.get_batch_size() == 1 and d.get_batch_size() == 3
    d.compact(torch.tensor([0, 1]))
    assert d.get_batch_size() == 2
    d.batch_select_indices(torch.tensor([1]))
    assert d.get_batch_size() == 1 and torch.equal(d._xpa[0][0], ref._xpa[0][1])
    e = ref.clone()
    e.reorder_cache(torch.tensor([2, 1, 0]))
    assert torch.equal(e._xpf[1][0], ref._xpf[1][2])
    e.batch_repeat_interleave(2)
    assert e.get_batch_size() == 6 and torch.equal(e._state[0][1], e._state[0][0])
    with pytest.raises(ValueError):
        e.batch_repeat_interleave(0)
    m = e.rwkv7_cache_metrics()
    assert m["reorder_calls"] == 1 and m["batch_repeat_interleave_calls"] == 1 and m["batch_size"] == 6


def test_to_detach_crop_reset():
    c = _cache()
    c2 = c.to(dtype=torch.float64, inplace=False)
    assert c2._xpa[0].dtype == torch.float64 and c2._state[0].dtype == torch.float32  # state stays fp32
    assert c._xpa[0].dtype == torch.float32
    c3 = c.clone().to(copy=True)
    assert c3._state[0].data_ptr() != c._state[0].data_ptr()
    d = c.clone().detach()
    assert d.rwkv7_cache_metrics()["detaches"] == 1
    assert c.crop(10) is c and c.seen_tokens == 5
    with pytest.raises(NotImplementedError):
        c.crop(3)
    c.crop(-5)
    assert c.seen_tokens == 0 and c._state is None and not c.is_initialized
    z = _cache()
    z.zero_()
    assert all(float(t.abs().sum()) == 0 for t in (*z._state, *z._xpa, *z._xpf, z._v_first))
    for name in ("update", "update_recurrent_state", "update_conv_state", "offload", "prefetch",
                 "early_initialization", "update_indexer"):
        with pytest.raises(NotImplementedError):
            getattr(z, name)()


def test_graph_binding_version_protocol():
    class Runner:
        def __init__(self):
            self.calls = []

        def reorder_batch_inplace(self, idx):
            self.calls.append(idx)
            return True

    c = _cache()
    r = Runner()
    c._bind_native_graph_runner(r)
    assert c._native_graph_bound_to(r) and c._native_graph_bound_runner() is r
    state0 = c._state
    c.select_batch(torch.tensor([1, 2, 0]))  # same size: the runner permutes in place
    assert r.calls and c._state is state0 and c._native_graph_bound_to(r)
    c.select_batch(torch.tensor([0]))  # a different size drops the binding
    assert not c._native_graph_bound_to(r) and c.get_batch_size() == 1
    c2 = _cache()
    c2._bind_native_graph_runner(r)
    c2.batch_repeat_interleave(2)
    assert c2._native_graph_bound_runner() is None


def test_forward_helpers():
    from rwkv7mi.model import (NativeRWKV7Cache, _as_native_cache, _check_attention_mask, _resolve_logits_to_keep,
                               _slice_logits)

    assert _resolve_logits_to_keep(None, None) is None
    assert _resolve_logits_to_keep(3, None) == 3 and _resolve_logits_to_keep(None, 2) == 2
    with pytest.raises(ValueError):
        _resolve_logits_to_keep(3, 2)
    lg = torch.randn(2, 6, 5)
    assert torch.equal(_slice_logits(lg, 0), lg) and torch.equal(_slice_logits(lg, 2), lg[:, -2:])
    assert torch.equal(_slice_logits(lg, 99), lg)
    _check_attention_mask(None, 2, 3, allow_trailing=False)
    _check_attention_mask(torch.ones(2, 3), 2, 3, allow_trailing=False)
    _check_attention_mask(torch.ones(2, 7), 2, 3, allow_trailing=True)
    with pytest.raises(ValueError):
        _check_attention_mask(torch.ones(2, 7), 2, 3, allow_trailing=False)
    with pytest.raises(ValueError):
        _check_attention_mask(torch.tensor([[1, 0, 1], [1, 1, 1]]), 2, 3, allow_trailing=False)
    with pytest.raises(TypeError):
        _check_attention_mask([[1, 1, 1]], 1, 3, allow_trailing=False)
    c = _cache()
    assert _as_native_cache(c) is c
    assert _as_native_cache(None) is None and _as_native_cache(NativeRWKV7Cache()) is None
    via_tuple = _as_native_cache(tuple(c))
    assert isinstance(via_tuple, NativeRWKV7Cache) and via_tuple._state is c._state
    assert _as_native_cache(object()) is None  # an empty foreign cache is no cache (model_cache.py:480-504)

    class Foreign(tuple):
        def get_seq_length(self):
            return 3

    with pytest.raises(TypeError):
        _as_native_cache(Foreign((1, 2)))
