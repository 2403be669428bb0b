"""The Hugging Face face of the model, on the CPU (no kernel runs): the
config and model classes resolve through AutoConfig / AutoModelForCausalLM
(model_type "rwkv7_native", as rwkv7_hf/native_model.py:857-859 registers
the reference's), GenerationMixin's per-step inputs slice to the last token
once a recurrent cache exists (rwkv7_hf/model_generation.py:38-97), beam
reordering permutes the cache rows (model_generation.py:15-35), and
save_pretrained / from_pretrained round-trip a converted directory."""
from __future__ import annotations

import pytest
import torch


def _cfg(**kw):
    from rwkv7mi.model import NativeRWKV7Config

    return NativeRWKV7Config(vocab_size=64, hidden_size=128, num_hidden_layers=2, intermediate_size=256,
                             decay_low_rank_dim=16, a_low_rank_dim=16, gate_low_rank_dim=16, v_low_rank_dim=16, **kw)


def _model():
    from rwkv7mi.model import NativeRWKV7ForCausalLM, random_weights

    cfg = _cfg()
    return NativeRWKV7ForCausalLM(cfg, random_weights(cfg, seed=0, dtype=torch.float32), device="cpu",
                                  dtype=torch.float32)


def test_auto_classes_resolve():
    from transformers import AutoConfig, AutoModelForCausalLM, GenerationMixin, PreTrainedModel

    from rwkv7mi.model import NativeRWKV7Config, NativeRWKV7ForCausalLM

    assert isinstance(AutoConfig.for_model("rwkv7_native", vocab_size=64, hidden_size=128), NativeRWKV7Config)
    assert AutoModelForCausalLM._model_mapping[NativeRWKV7Config] is NativeRWKV7ForCausalLM
    assert issubclass(NativeRWKV7ForCausalLM, PreTrainedModel) and issubclass(NativeRWKV7ForCausalLM, GenerationMixin)
    m = _model()
    assert m.can_generate() and m.generation_config is not None
    assert m.device == torch.device("cpu") and m.dtype == torch.float32


def test_config_fields_and_round_trip():
    from rwkv7mi.model import NativeRWKV7Config

    cfg = _cfg()
    assert (cfg.num_heads, cfg.attention_hidden_size, cfg.num_attention_heads) == (2, 128, 2)
    assert cfg.tie_word_embeddings is False
    again = NativeRWKV7Config(**cfg.to_dict())
    assert again.to_dict() == cfg.to_dict()
    with pytest.raises(ValueError):
        NativeRWKV7Config(hidden_size=128, head_dim=32)
    with pytest.raises(ValueError):
        NativeRWKV7Config(hidden_size=128, num_heads=2, attention_hidden_size=192)


def test_generation_inputs_slice_after_the_first_step():
    m = _model()
    ids = torch.tensor([[1, 2, 3], [4, 5, 6]])
    mask = torch.ones(2, 3, dtype=torch.long)
    first = m.prepare_inputs_for_generation(ids, past_key_values=None, attention_mask=mask, logits_to_keep=1)
    assert torch.equal(first["input_ids"], ids) and first["past_key_values"] is None
    assert first["use_cache"] is True and first["logits_to_keep"] == 1
    cache = m.new_cache(2)
    cache.seen_tokens = 3
    nxt = m.prepare_inputs_for_generation(ids, past_key_values=cache, attention_mask=mask)
    assert torch.equal(nxt["input_ids"], ids[:, -1:]) and nxt["past_key_values"] is cache
    assert tuple(nxt["attention_mask"].shape) == (2, 1)
    emb = torch.randn(2, 3, 128)
    assert m.prepare_inputs_for_generation(None, inputs_embeds=emb)["inputs_embeds"] is emb


def test_reorder_cache_permutes_rows():
    from rwkv7mi.model import NativeRWKV7ForCausalLM

    m = _model()
    cache = m.new_cache(3)
    cache.seen_tokens = 4
    for l in range(2):
        cache._state[l].copy_(torch.arange(3.0).view(3, 1, 1, 1).expand_as(cache._state[l]))
    out = NativeRWKV7ForCausalLM._reorder_cache(cache, torch.tensor([2, 0, 0]))
    assert out.get_batch_size() == 3 and out.seen_tokens == 4
    assert out._state[1][:, 0, 0, 0].tolist() == [2.0, 0.0, 0.0]
    assert NativeRWKV7ForCausalLM._reorder_cache(None, torch.tensor([0])) is None


def test_save_and_from_pretrained_round_trip(tmp_path):
    from transformers import AutoModelForCausalLM

    m = _model()
    m.save_pretrained(tmp_path)
    m2 = AutoModelForCausalLM.from_pretrained(tmp_path, device="cpu", dtype="auto")
    assert type(m2) is type(m) and m2.dtype == torch.float32
    assert m2.config.to_dict()["hidden_size"] == 128
    a, b = m.dense_state_dict(), m2.dense_state_dict()
    assert a.keys() == b.keys() and all(torch.equal(a[k].cpu(), b[k].cpu()) for k in a)
