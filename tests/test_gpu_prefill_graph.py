"""The hipGraph prefill runner: replays equal the eager prefill bit for bit
(logits and every cache tensor), for fresh prompts (state from zeros) and
for cache continuation (carry_state), replay after replay, at a short shape
(rows through the 64-row tile GEMM) and a long one (rows through the
prefill GEMM); the returned cache continues into graph decode like the
eager one."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    from rwkv7mi.model import NativeRWKV7Config, NativeRWKV7ForCausalLM

    cfg = NativeRWKV7Config(vocab_size=512, hidden_size=256, num_hidden_layers=2, intermediate_size=1024,
                            decay_low_rank_dim=16, a_low_rank_dim=16, gate_low_rank_dim=32, v_low_rank_dim=16,
                            use_native_mm8=True, native_mm8_min_params=1)
    return NativeRWKV7ForCausalLM.from_random(cfg, seed=0, device="cuda", dtype=torch.float16)


def _eq_cache(a, b):
    for x, y in zip((*a._state, *a._xpa, *a._xpf, a._v_first), (*b._state, *b._xpa, *b._xpf, b._v_first)):
        assert torch.equal(x, y)


@pytest.mark.parametrize("B,T", [(2, 24), (2, 320)])
def test_prefill_graph_equals_eager(model, B, T):
    V = model.config.vocab_size
    r = model.prefill_graph_runner(B, T, logits_to_keep=1)
    for rep in range(3):
        ids = torch.randint(0, V, (B, T), device="cuda", generator=torch.Generator("cuda").manual_seed(rep))
        c_e = model.new_cache(B)
        le = model.prefill_(ids, c_e, logits_to_keep=1)
        lg, c_g = r.replay(ids)
        torch.cuda.synchronize()
        assert torch.equal(lg, le), rep
        _eq_cache(c_e, c_g)
        assert c_g.seen_tokens == T


def test_prefill_graph_carry_state_and_decode(model):
    V = model.config.vocab_size
    B, T = 3, 16
    g = torch.Generator("cuda").manual_seed(7)
    first = torch.randint(0, V, (B, T), device="cuda", generator=g)
    second = torch.randint(0, V, (B, T), device="cuda", generator=g)
    c_e = model.new_cache(B)
    model.prefill_(first, c_e)
    le = model.prefill_(second, c_e)
    fresh = model.prefill_graph_runner(B, T)
    cont = model.prefill_graph_runner(B, T, carry_state=True)
    _, c1 = fresh.replay(first)
    lg, c2 = cont.replay(second, c1)
    torch.cuda.synchronize()
    assert torch.equal(lg, le)
    _eq_cache(c_e, c2)
    assert c2.seen_tokens == 2 * T
    with pytest.raises(ValueError):
        fresh.replay(second, c1)
    tok = torch.randint(0, V, (B, 1), device="cuda", generator=g)
    a = model(tok, past_key_values=c_e).logits
    b = model(tok, past_key_values=c2).logits
    torch.cuda.synchronize()
    assert torch.equal(a, b)
