"""BASELINE configs[4] on the GPU: the RWKV-7 7.2B architecture (D = 4096,
H = 64, F = 16384, V = 65536, LoRA 64/64/128/32) with MM8 weights under the
"memory" policy, fp16 activations, fp32 state.

* A width-true two-layer slice against the fp64 per-token oracle (with the
  MM8 weights dequantised into it), through prefill and graph-replayed decode
  at bsz 1 (the fused LN-mix GEMV route) and bsz 3.
* The full 32-layer model: hipGraph decode equals eager decode bit for bit at
  bsz 1, 8 and 64, with finite logits.
* The B = 8 x T = 4096 prefill once, and its cache against a prompt split into
  two prefills of 2048 tokens (the cache-continuation contract).

Tolerances: logits max-abs <= 2e-2 x max|logit| with ids equal wherever the
oracle's top-2 margin exceeds twice that; recurrent state relative <= 2e-2.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

LOGIT_REL = 2e-2


def _cfg(layers):
    from rwkv7mi.model import NativeRWKV7Config

    return NativeRWKV7Config(vocab_size=65536, hidden_size=4096, num_hidden_layers=layers, intermediate_size=16384,
                             decay_low_rank_dim=64, a_low_rank_dim=64, gate_low_rank_dim=128, v_low_rank_dim=32,
                             use_native_mm8=True, native_mm8_min_params=8_000_000, native_mm8_policy="memory")


def _close(got, ref):
    got = got.float().cpu().numpy().astype(np.float64)
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= LOGIT_REL * scale, (np.abs(got - ref).max(), scale)
    top2 = np.sort(ref, -1)[:, -2:]
    sure = top2[:, 1] - top2[:, 0] > 2 * LOGIT_REL * scale
    np.testing.assert_array_equal(got.argmax(-1)[sure], ref.argmax(-1)[sure])


def test_7p2b_two_layer_slice_matches_oracle():
    from oracle.model_oracle import ModelOracle
    from rwkv7mi.model import NativeRWKV7ForCausalLM, QuantLinear, random_weights
    from rwkv7mi.native_quant_mm8 import dequantize_mm8

    cfg = _cfg(2)
    print("7.2B slice: building (2 layers, MM8 memory policy)", flush=True)
    w = random_weights(cfg, seed=0, device="cuda", dtype=torch.float16)
    model = NativeRWKV7ForCausalLM(cfg, w, device="cuda", dtype=torch.float16)
    named = {"lm_head": model.lm_head}
    for L in model.layers:
        p = f"model.layers.{L.idx}."
        named.update({p + "attn.r_proj": L.r_proj, p + "attn.k_proj": L.k_proj, p + "attn.v_proj": L.v_proj,
                      p + "attn.o_proj": L.o_proj, p + "ffn.key": L.key, p + "ffn.value": L.value})
    override = {}
    for name, lin in named.items():
        assert isinstance(lin, QuantLinear), name  # every projection of the 7.2B shapes has >= 8M weights
        m = lin.m
        override[name] = dequantize_mm8(m.w_blk, m.mx, m.rx, m.my, m.ry, out_dtype=torch.float32).cpu().numpy()
    ref_w = {k: v.float().cpu().numpy() for k, v in w.items() if k[: -len(".weight")] not in override}
    del w
    ora = ModelOracle(cfg, ref_w, override)
    del ref_w, override
    rng = np.random.default_rng(4)
    for B in (1, 3):
        print(f"7.2B slice: B={B} prefill 12 tokens + 3 graph decode steps", flush=True)
        ids = rng.integers(0, cfg.vocab_size, (B, 12))
        ref_logits, st = ora.run(ids)
        out = model(torch.tensor(ids, device="cuda"))
        torch.cuda.synchronize()
        _close(out.logits[:, -1], ref_logits[:, -1])
        cache = out.past_key_values
        for i in range(cfg.num_hidden_layers):
            s = cache._state[i].double().cpu().numpy()
            assert np.abs(s - st["state"][i]).max() <= 2e-2 * np.abs(st["state"][i]).max()
        for _ in range(3):
            nxt = rng.integers(0, cfg.vocab_size, (B,))
            r = ora.step(nxt, st)
            lg = model(torch.tensor(nxt[:, None], device="cuda"), past_key_values=cache).logits
            torch.cuda.synchronize()
            _close(lg[:, -1], r)


@pytest.fixture(scope="module")
def full_model():
    from rwkv7mi.model import NativeRWKV7ForCausalLM

    print("7.2B: building the 32-layer MM8 model", flush=True)
    model = NativeRWKV7ForCausalLM.from_random(_cfg(32), seed=0, device="cuda", dtype=torch.float16)
    assert model._rwkv7_native_mm_replaced_modules == 193
    yield model
    model._graph_runners.clear()


@pytest.mark.parametrize("B", [1, 8, 64])
def test_7p2b_graph_decode_equals_eager(full_model, B):
    model = full_model
    rng = np.random.default_rng(5 + B)
    print(f"7.2B: graph vs eager decode, B={B}", flush=True)
    ids = torch.tensor(rng.integers(0, 65536, (B, 4)), device="cuda")
    c1 = model(ids).past_key_values
    c2 = c1.clone()
    runner = model.graph_runner(B)
    for step in range(3):
        tok = torch.tensor(rng.integers(0, 65536, (B,)), device="cuda")
        eager = model(tok[:, None], past_key_values=c1, use_graph=False).logits[:, -1]
        got = runner.replay(tok, c2).clone()
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, eager), step
    for a, b in zip(c1._state, c2._state):
        assert torch.equal(a, b)
    del model._graph_runners[B]


def test_7p2b_prefill_b8_t4096_split_continuation(full_model):
    """One B=8 x T=4096 prefill vs two prefills of 2048 tokens continuing the
    cache: the same recurrent state, shift rows and next logits (the chunk
    boundaries coincide; only library-GEMM tiling may differ)."""
    model = full_model
    g = torch.Generator(device="cuda").manual_seed(0)
    ids = torch.randint(0, 65536, (8, 4096), device="cuda", generator=g)
    print("7.2B: prefill B=8 x T=4096", flush=True)
    one = model(ids)
    torch.cuda.synchronize()
    print("7.2B: prefill 2 x 2048 with the cache carried", flush=True)
    half = model(ids[:, :2048])
    two = model(ids[:, 2048:], past_key_values=half.past_key_values)
    torch.cuda.synchronize()
    assert one.past_key_values.seen_tokens == two.past_key_values.seen_tokens == 4096
    a, b = one.logits.float(), two.logits.float()
    assert torch.isfinite(a).all()
    assert (a - b).abs().max().item() <= LOGIT_REL * a.abs().max().item()
    ca, cb = one.past_key_values, two.past_key_values
    for i in range(32):
        sa, sb = ca._state[i], cb._state[i]
        assert torch.isfinite(sa).all()
        assert ((sa - sb).abs().max() / sa.abs().max()).item() <= 2e-2, i
        for xa_, xb_ in ((ca._xpa[i], cb._xpa[i]), (ca._xpf[i], cb._xpf[i])):
            assert (xa_.float() - xb_.float()).abs().max().item() <= 2e-2 * max(1.0, xa_.float().abs().max().item())
    tok = ids[:, -1:]
    la = model(tok, past_key_values=ca, use_graph=False).logits.float()
    lb = model(tok, past_key_values=cb, use_graph=False).logits.float()
    assert (la - lb).abs().max().item() <= LOGIT_REL * la.abs().max().item()
