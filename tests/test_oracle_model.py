"""The fp64 model oracle (oracle/model_oracle.py) against the reference's own
model: golden logits and greedy ids written by tests/golden/make_model_golden.py
from rwkv7_hf.native_model.NativeRWKV7ForCausalLM (fp32, CPU) for this build's
name-keyed random weights.  Tolerance: logits max-abs <= 1e-5 x max|logit|
(fp32 reference vs fp64 oracle); greedy ids bit-exact."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"

CFGS = {
    "tiny": dict(vocab_size=512, hidden_size=128, num_hidden_layers=2, intermediate_size=256,
                 decay_low_rank_dim=32, a_low_rank_dim=32, gate_low_rank_dim=64, v_low_rank_dim=32),
    "c1": dict(vocab_size=65536, hidden_size=768, num_hidden_layers=12, intermediate_size=3072,
               decay_low_rank_dim=64, a_low_rank_dim=64, gate_low_rank_dim=128, v_low_rank_dim=32),
}


def golden_case(name):
    from rwkv7mi.model import NativeRWKV7Config, random_weights

    g = np.load(GOLDEN / f"model_{name}.npz")
    cfg = NativeRWKV7Config(**CFGS[name])
    w = random_weights(cfg, seed=0, device="cpu", dtype=torch.float32)
    return cfg, w, g


@pytest.mark.parametrize("name", ["tiny", "c1"])
def test_model_oracle_matches_reference_golden(name):
    from oracle.model_oracle import ModelOracle

    cfg, w, g = golden_case(name)
    ora = ModelOracle(cfg, {k: v.numpy() for k, v in w.items()})
    del w
    lg, st = ora.run(g["ids"])
    ref = g["logits"].astype(np.float64)
    assert np.abs(lg[0, -1] - ref).max() <= 1e-5 * np.abs(ref).max()
    nxt, seq = int(lg[0, -1].argmax()), []
    for _ in range(len(g["greedy"])):
        seq.append(nxt)
        nxt = int(ora.step(np.array([nxt]), st)[0].argmax())
    np.testing.assert_array_equal(seq, g["greedy"])


def test_sequence_oracle_equals_per_token_oracle():
    """run_seq (token-parallel products, per-token recurrence) is the same
    model as the per-token step: logits and every cache tensor agree to fp64
    rounding, from zero state and continuing a cache."""
    from oracle.model_oracle import ModelOracle

    cfg, w, _ = golden_case("tiny")
    ora = ModelOracle(cfg, {k: v.numpy() for k, v in w.items()})
    ids = np.random.default_rng(2).integers(0, cfg.vocab_size, (2, 11))
    lg, st = ora.run(ids[:, :7])
    lg2, st2 = ora.run_seq(ids[:, :7], keep=7)
    np.testing.assert_allclose(lg2, lg, rtol=0, atol=1e-10 * np.abs(lg).max())
    lg, st = ora.run(ids[:, 7:], st)
    lg2, st2 = ora.run_seq(ids[:, 7:], st2, keep=1)
    np.testing.assert_allclose(lg2[:, -1], lg[:, -1], rtol=0, atol=1e-10 * np.abs(lg).max())
    for key in ("state", "xpa", "xpf"):
        for a, b in zip(st[key], st2[key]):
            np.testing.assert_allclose(b, a, rtol=0, atol=1e-10 * max(1.0, np.abs(a).max()))
    np.testing.assert_allclose(st2["v_first"], st["v_first"], rtol=0, atol=1e-10)
