"""The official-checkpoint converter and the converted / prepacked directory
formats, on the CPU.

Pins: the reference converter test's name and config cases
(rwkv7_hf ... tests/test_convert_config.py:240-247 for ``translate_name``,
:111-133 for shape inference and the rejected transposed output
projection); a round trip through an independently written inverse of the
official layout (LoRA matrices transposed, time-mix vectors flat, layer 0's
pre-norm present or absent); ``config.json`` + safetensors save / load; the
CLI on a ``torch.save``'d official checkpoint."""
from __future__ import annotations

import json

import pytest
import torch

from rwkv7mi import converter as conv
from rwkv7mi.model import NativeRWKV7Config, parameter_shapes, random_weights


class ShapeTensor:
    def __init__(self, *shape):
        self.shape = tuple(shape)


def _shape_weights(hidden=1024, layers=3, head_dim=64, attn=None):
    attn = hidden if attn is None else attn
    heads = attn // head_dim
    w = {"emb.weight": ShapeTensor(65536, hidden), "blocks.0.att.w1": ShapeTensor(hidden, 64),
         "blocks.0.att.g1": ShapeTensor(hidden, 96), "blocks.0.att.a1": ShapeTensor(hidden, 32)}
    if layers > 1:
        w["blocks.1.att.v1"] = ShapeTensor(hidden, 16)
    for i in range(layers):
        w[f"blocks.{i}.ffn.key.weight"] = ShapeTensor(hidden * 4, hidden)
        w[f"blocks.{i}.att.r_k"] = ShapeTensor(heads, head_dim)
        for p in ("receptance", "key", "value"):
            w[f"blocks.{i}.att.{p}.weight"] = ShapeTensor(attn, hidden)
        w[f"blocks.{i}.att.output.weight"] = ShapeTensor(hidden, attn)
        w[f"blocks.{i}.att.ln_x.weight"] = ShapeTensor(attn)
        w[f"blocks.{i}.att.ln_x.bias"] = ShapeTensor(attn)
    return w


def test_translate_name_reference_cases():
    assert conv.translate_name("blocks.2.att.receptance.weight", 3) == ("model.layers.2.attn.r_proj.weight", False)
    assert conv.translate_name("blocks.2.att.w1", 3) == ("model.layers.2.attn.w_lora.lora.0.weight", True)
    assert conv.translate_name("blocks.2.att.w0", 3) == ("model.layers.2.attn.w_lora.lora.2.bias", False)
    assert conv.translate_name("blocks.0.att.v1", 3) == ("", False)
    assert conv.translate_name("blocks.1.att.g2", 3) == ("model.layers.1.attn.g_lora.lora.2.weight", True)
    assert conv.translate_name("blocks.1.att.ln_x.bias", 3) == ("model.layers.1.attn.g_norm.bias", False)
    assert conv.translate_name("blocks.0.ln0.weight", 3) == ("model.layers.0.pre_norm.weight", False)
    assert conv.translate_name("blocks.1.ffn.x_k", 3) == ("model.layers.1.ffn.x_k", False)
    assert conv.translate_name("head.weight", 3) == ("lm_head.weight", False)
    with pytest.raises(KeyError):
        conv.translate_name("blocks.3.att.key.weight", 3)
    with pytest.raises(KeyError):
        conv.translate_name("something.else", 3)


def test_infer_config_and_rejections():
    cfg = conv.infer_config(_shape_weights())
    assert (cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers) == (65536, 1024, 4096, 3)
    assert (cfg.head_dim, cfg.num_heads, cfg.attention_hidden_size) == (64, 16, 1024)
    assert (cfg.decay_low_rank_dim, cfg.gate_low_rank_dim, cfg.a_low_rank_dim, cfg.v_low_rank_dim) == (64, 96, 32, 16)
    bad = _shape_weights()
    bad["blocks.2.att.output.weight"] = ShapeTensor(1024, 960)
    with pytest.raises(ValueError, match="blocks.2.att.output.weight"):
        conv.infer_config(bad)
    gap = _shape_weights()
    gap["blocks.5.ffn.key.weight"] = ShapeTensor(4096, 1024)
    with pytest.raises(ValueError, match="contiguous"):
        conv.infer_config(gap)
    with pytest.raises(ValueError, match="attention width"):  # A != D (the reference allows it; these kernels do not)
        conv.infer_config(_shape_weights(attn=896, head_dim=64))


def _official_from_hf(hf: dict, cfg, *, with_ln0=True) -> dict:
    """Inverse of the conversion, written per key family: the official
    layout of an RWKV-7 checkpoint."""
    off = {"emb.weight": hf["model.embeddings.weight"], "ln_out.weight": hf["model.norm.weight"],
           "ln_out.bias": hf["model.norm.bias"], "head.weight": hf["lm_head.weight"]}
    proj = {"r_proj": "receptance", "k_proj": "key", "v_proj": "value", "o_proj": "output"}
    for i in range(cfg.num_hidden_layers):
        p, b = f"model.layers.{i}.", f"blocks.{i}."
        if i == 0 and with_ln0:
            off[b + "ln0.weight"], off[b + "ln0.bias"] = hf[p + "pre_norm.weight"], hf[p + "pre_norm.bias"]
        off[b + "ln1.weight"], off[b + "ln1.bias"] = hf[p + "attn_norm.weight"], hf[p + "attn_norm.bias"]
        off[b + "ln2.weight"], off[b + "ln2.bias"] = hf[p + "ffn_norm.weight"], hf[p + "ffn_norm.bias"]
        for m in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"):
            off[b + "att." + m] = hf[p + "attn." + m].reshape(-1)  # stored flat
        for m in ("k_k", "k_a"):
            off[b + "att." + m] = hf[p + "attn." + m]
        off[b + "att.r_k"] = hf[p + "attn.r_k"]
        for hn, on in proj.items():
            off[b + f"att.{on}.weight"] = hf[p + f"attn.{hn}.weight"]
        off[b + "att.ln_x.weight"], off[b + "att.ln_x.bias"] = hf[p + "attn.g_norm.weight"], hf[p + "attn.g_norm.bias"]
        for kind in ("w", "a", "g", "v"):
            q = p + f"attn.{kind}_lora.lora."
            if q + "0.weight" not in hf:
                continue
            off[b + f"att.{kind}1"] = hf[q + "0.weight"].t().contiguous()  # [D, rank]
            off[b + f"att.{kind}2"] = hf[q + "2.weight"].t().contiguous()  # [rank, A]
            if q + "2.bias" in hf:
                off[b + f"att.{kind}0"] = hf[q + "2.bias"]
        off[b + "ffn.x_k"] = hf[p + "ffn.x_k"]
        off[b + "ffn.key.weight"], off[b + "ffn.value.weight"] = hf[p + "ffn.key.weight"], hf[p + "ffn.value.weight"]
    off["blocks.0.att.v0"] = torch.zeros(cfg.hidden_size)  # unused in layer 0, dropped
    return off


CFG = NativeRWKV7Config(vocab_size=300, hidden_size=128, num_hidden_layers=3, decay_low_rank_dim=16,
                        a_low_rank_dim=16, gate_low_rank_dim=32, v_low_rank_dim=8)


@pytest.mark.parametrize("with_ln0", [True, False])
def test_round_trip_through_the_official_layout(with_ln0):
    hf = random_weights(CFG, seed=3, dtype=torch.float32)
    off = _official_from_hf(hf, CFG, with_ln0=with_ln0)
    cfg, got = conv.convert_state_dict(dict(off), torch.float16)
    assert (cfg.hidden_size, cfg.num_hidden_layers, cfg.vocab_size) == (128, 3, 300)
    assert (cfg.decay_low_rank_dim, cfg.gate_low_rank_dim, cfg.v_low_rank_dim) == (16, 32, 8)
    assert set(got) == set(parameter_shapes(CFG))
    for k, v in hf.items():
        if not with_ln0 and k.startswith("model.layers.0.pre_norm"):
            fill = 1.0 if k.endswith("weight") else 0.0
            assert torch.equal(got[k], torch.full_like(got[k], fill)), k
            continue
        assert got[k].dtype == torch.float16 and tuple(got[k].shape) == tuple(v.shape), k
        assert torch.equal(got[k], v.to(torch.float16)), k


def test_convert_rejects_shape_mismatch():
    hf = random_weights(CFG, seed=4, dtype=torch.float32)
    off = _official_from_hf(hf, CFG)
    off["blocks.1.att.w1"] = torch.zeros(128, 15)
    with pytest.raises((ValueError, KeyError)):
        conv.convert_state_dict(off)


def test_directory_save_load_and_cli(tmp_path):
    hf = random_weights(CFG, seed=5, dtype=torch.float32)
    off = _official_from_hf(hf, CFG)
    pth = tmp_path / "rwkv7.pth"
    torch.save(off, pth)
    out = tmp_path / "conv"
    assert conv.main(["--input", str(pth), "--output", str(out), "--precision", "bf16"]) == 0
    cj = json.loads((out / "config.json").read_text())
    assert cj["model_type"] == "rwkv7_native" and cj["hidden_size"] == 128 and cj["torch_dtype"] == "bfloat16"
    cfg, state = conv.load_hf_directory(out)
    assert cfg.num_hidden_layers == 3 and cfg.v_low_rank_dim == 8
    for k, v in hf.items():
        assert torch.equal(state[k], v.to(torch.bfloat16)), k
    # a reference-written config.json (extra fields) is read by name
    ref_cfg = dict(cj, attn_mode="chunk", fuse_norm=False, hidden_ratio=4.0, value_dim=[128] * 3)
    assert conv.config_from_json(ref_cfg).hidden_size == 128
