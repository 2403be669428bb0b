"""Prepacked MM8 checkpoints on the GPU: a model saved with
``save_prepacked`` and loaded with ``load_prepacked`` (no quantisation at
load) gives bit-identical logits to the model that was saved; the manifest
is checked before any buffer is built (tampered entries raise); a converted
directory loads through ``load_pretrained`` to the same logits as the
model built from the same state dict."""
from __future__ import annotations

import json

import pytest
import torch

pytestmark = pytest.mark.gpu


def _cfg():
    from rwkv7mi.model import NativeRWKV7Config

    return NativeRWKV7Config(vocab_size=512, hidden_size=256, num_hidden_layers=2, intermediate_size=1024,
                             decay_low_rank_dim=16, a_low_rank_dim=16, gate_low_rank_dim=32, v_low_rank_dim=16,
                             use_native_mm8=True, native_mm8_min_params=1, native_mm8_policy="all")


def test_prepacked_round_trip(tmp_path):
    from rwkv7mi import converter as conv
    from rwkv7mi.model import NativeRWKV7ForCausalLM, random_weights

    cfg = _cfg()
    w = random_weights(cfg, seed=1, dtype=torch.float16)
    model = NativeRWKV7ForCausalLM(cfg, w, device="cuda", dtype=torch.float16)
    assert model._rwkv7_native_mm_replaced_modules > 0
    man = conv.save_prepacked(model, tmp_path, source_state=w)
    assert len(man["modules"]) == model._rwkv7_native_mm_replaced_modules
    assert all(len(e["source_weight_sha256"]) == 64 for e in man["modules"])
    loaded = conv.load_prepacked(tmp_path, device="cuda", dtype=torch.float16)
    assert loaded._rwkv7_native_mm_replaced_modules == model._rwkv7_native_mm_replaced_modules
    ids = torch.randint(0, cfg.vocab_size, (2, 9), device="cuda", generator=torch.Generator("cuda").manual_seed(0))
    a = model(ids, use_graph=False)
    b = loaded(ids, use_graph=False)
    torch.cuda.synchronize()
    assert torch.equal(a.logits, b.logits)
    for s1, s2 in zip(a.past_key_values._state, b.past_key_values._state):
        assert torch.equal(s1, s2)
    # decode continues identically
    tok = torch.randint(0, cfg.vocab_size, (2, 1), device="cuda")
    assert torch.equal(model(tok, past_key_values=a.past_key_values, use_graph=False).logits,
                       loaded(tok, past_key_values=b.past_key_values, use_graph=False).logits)
    # load_pretrained picks the prepacked route from the manifest
    again = conv.load_pretrained(tmp_path, device="cuda", dtype=torch.float16)
    assert torch.equal(again(ids, use_graph=False).logits, a.logits)


@pytest.mark.parametrize("field,value", [("input_features", 7), ("format", "other.v0"),
                                         ("activation_dtype", "bfloat16"), ("blocked_shape", [1, 1, 2048]),
                                         ("packer_version", "rwkv7mi-mm8-0"), ("scale_dtype", "float32")])
def test_prepacked_manifest_rejects(tmp_path, field, value):
    from rwkv7mi import converter as conv
    from rwkv7mi.model import NativeRWKV7ForCausalLM, random_weights

    cfg = _cfg()
    model = NativeRWKV7ForCausalLM(cfg, random_weights(cfg, seed=2, dtype=torch.float16), device="cuda",
                                   dtype=torch.float16)
    conv.save_prepacked(model, tmp_path)
    man = json.loads((tmp_path / "manifest.json").read_text())
    man["modules"][1][field] = value
    (tmp_path / "manifest.json").write_text(json.dumps(man))
    with pytest.raises(ValueError):
        conv.load_prepacked(tmp_path, device="cuda", dtype=torch.float16)


def test_converted_directory_loads(tmp_path):
    from rwkv7mi import converter as conv
    from rwkv7mi.model import NativeRWKV7ForCausalLM, random_weights

    cfg = _cfg()
    w = random_weights(cfg, seed=3, dtype=torch.float16)
    conv.save_hf_directory(tmp_path, cfg, w)
    m1 = conv.load_pretrained(tmp_path, device="cuda", dtype=torch.float16, use_native_mm8=True,
                              native_mm8_policy="all", native_mm8_min_params=1)
    assert m1._rwkv7_native_mm_replaced_modules > 0
    cfg.use_native_mm8 = True
    m2 = NativeRWKV7ForCausalLM(cfg, w, device="cuda", dtype=torch.float16)
    ids = torch.randint(0, cfg.vocab_size, (1, 5), device="cuda")
    assert torch.equal(m1(ids, use_graph=False).logits, m2(ids, use_graph=False).logits)


def test_prepacked_source_digest_checked(tmp_path):
    """load_prepacked(source_state=...) accepts the weights a directory was
    packed from and refuses a changed one."""
    from rwkv7mi import converter as conv
    from rwkv7mi.model import NativeRWKV7ForCausalLM, random_weights

    cfg = _cfg()
    w = random_weights(cfg, seed=4, dtype=torch.float16)
    cfg.use_native_mm8 = True
    model = NativeRWKV7ForCausalLM(cfg, w, device="cuda", dtype=torch.float16)
    man = conv.save_prepacked(model, tmp_path, source_state=w)
    conv.load_prepacked(tmp_path, device="cuda", dtype=torch.float16, source_state=w)
    name = man["modules"][0]["module"] + ".weight"
    changed = dict(w)
    changed[name] = w[name].clone()
    changed[name].view(-1)[0] += 1
    with pytest.raises(ValueError, match="digest"):
        conv.load_prepacked(tmp_path, device="cuda", dtype=torch.float16, source_state=changed)
