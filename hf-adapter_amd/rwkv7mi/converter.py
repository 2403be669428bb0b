"""On-disk formats: the official RWKV-7 ``.pth`` -> Hugging Face converter, and
a prepacked MM8 checkpoint with a per-module manifest.

Converter (rwkv7_hf/converter.py:152-326 config inference and shape checks,
:333-365 ``translate_name``, :475-543 the translated state dict): official
keys ``blocks.{i}.att.*`` / ``blocks.{i}.ffn.*`` / ``emb`` / ``ln_out`` /
``head`` become the HF keys this package's model reads
(``model.layers.{i}.attn.r_proj.weight`` ...).  The LoRA matrices ``{w,a,g,v}1``
and ``{w,a,g,v}2`` are stored transposed in the official checkpoint; time-mix
vectors are reshaped to the HF template's shapes; layer 0's ``pre_norm`` is
filled with ones / zeros when absent and the unused ``blocks.0.att.v0/v1/v2``
are dropped.  The output directory holds ``config.json`` and
``model.safetensors``; :func:`load_pretrained` builds the model from it (or
from a directory the reference converter wrote: the same keys, its
``config.json`` fields are read by name).

Prepacked checkpoint (the per-module loader metadata of
docs/quantization/VLLM_QUANTIZATION_PORTING.md:411-430): the MM8 modules'
bytes in the GEMV's blocked layout with their scales, ``prepacked.safetensors``,
and ``manifest.json`` with one entry per module (format, features, dtypes,
epilogue, sha256 of the source weight, packer version) validated before any
GPU buffer is allocated, so loading skips quantisation.

Checkpoints are read with ``torch.load(weights_only=True)`` (or safetensors):
nothing in a file is executed.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import re
from pathlib import Path
from typing import Dict, Sequence, Tuple

import torch

DTYPES = {
    "fp16": ("float16", torch.float16),
    "float16": ("float16", torch.float16),
    "bf16": ("bfloat16", torch.bfloat16),
    "bfloat16": ("bfloat16", torch.bfloat16),
    "fp32": ("float32", torch.float32),
    "float32": ("float32", torch.float32),
}

PREPACKED_FORMAT = "rwkv7mi.mm8_blocked.v1"
PACKER_VERSION = "rwkv7mi-mm8-1"
# the reference converter's fills for layer 0's optional pre-norm
_ALLOWED_MISSING = ("model.layers.0.pre_norm.weight", "model.layers.0.pre_norm.bias")


# ------------------------------------------------------------- inference
def tensor_shape(weights: Dict[str, torch.Tensor], name: str) -> tuple:
    """The shape of checkpoint entry ``name`` (KeyError when it is absent)."""
    t = weights.get(name)
    if t is None:
        raise KeyError(f"checkpoint lacks {name}")
    return tuple(map(int, t.shape))


_BLOCK_KEY = re.compile(r"blocks\.(\d+)\.ffn\.key\.weight")


def infer_num_layers(weights: Dict[str, torch.Tensor]) -> int:
    """Layer count: the FFN key matrices must be numbered 0 .. L-1 with no gap."""
    found = {int(m.group(1)) for m in map(_BLOCK_KEY.fullmatch, weights) if m}
    if not found:
        raise KeyError("checkpoint has no blocks.<i>.ffn.key.weight entries")
    n = max(found) + 1
    gaps = sorted(set(range(n)) - found)
    if gaps:
        raise ValueError(f"block numbering is not contiguous from 0 (absent: {gaps[:8]})")
    return n


def infer_attention_shape(weights: Dict[str, torch.Tensor]) -> tuple:
    """``(heads, head_dim, heads * head_dim)``, read from the last two
    dimensions of layer 0's ``r_k``."""
    rk = tensor_shape(weights, "blocks.0.att.r_k")
    heads, head_dim = (rk[-2], rk[-1]) if len(rk) >= 2 else (0, 0)
    if heads < 1 or head_dim < 1:
        raise ValueError(f"blocks.0.att.r_k {rk} does not end in (heads, head_dim)")
    return heads, head_dim, heads * head_dim


def _layer_expectations(i: int, hidden: int, attn: int) -> dict:
    """The exact shapes every layer's projections and group norm must have."""
    att = f"blocks.{i}.att."
    return {att + "receptance.weight": (attn, hidden), att + "key.weight": (attn, hidden),
            att + "value.weight": (attn, hidden), att + "output.weight": (hidden, attn),
            att + "ln_x.weight": (attn,), att + "ln_x.bias": (attn,)}


def validate_layer_shapes(weights, num_layers, hidden, heads, head_dim, attn):
    """Check every layer against layer 0's geometry: FFN key input width,
    ``r_k`` = [1 .., heads, head_dim], and the table of projection shapes."""
    for i in range(num_layers):
        fk = tensor_shape(weights, f"blocks.{i}.ffn.key.weight")
        if len(fk) != 2 or fk[1] != hidden:
            raise ValueError(f"blocks.{i}.ffn.key.weight {fk}: input width is not {hidden}")
        rk = tensor_shape(weights, f"blocks.{i}.att.r_k")
        if rk[-2:] != (heads, head_dim) or set(rk[:-2]) - {1}:
            raise ValueError(f"blocks.{i}.att.r_k {rk}: not [1.., {heads}, {head_dim}]")
        for name, want in _layer_expectations(i, hidden, attn).items():
            got = tensor_shape(weights, name)
            if got != want:
                raise ValueError(f"{name} {got}: this geometry needs {want}")


def infer_config(weights: Dict[str, torch.Tensor]):
    """The model config an official checkpoint implies (rwkv7_hf/converter.py:268-326)."""
    from .model import NativeRWKV7Config

    hidden = tensor_shape(weights, "blocks.0.ffn.key.weight")[1]
    ffn = tensor_shape(weights, "blocks.0.ffn.key.weight")[0]
    layers = infer_num_layers(weights)
    heads, head_dim, attn = infer_attention_shape(weights)
    for i in range(layers):
        vd = tensor_shape(weights, f"blocks.{i}.att.value.weight")[0]
        if vd != attn:
            raise ValueError(f"every value projection must output attention_hidden_size={attn}; "
                             f"blocks.{i}.att.value.weight gives {vd}")
    validate_layer_shapes(weights, layers, hidden, heads, head_dim, attn)
    if attn != hidden:
        raise ValueError(f"this build requires attention width == hidden size; got {attn} vs {hidden}")
    try:
        v_rank = tensor_shape(weights, "blocks.1.att.v1")[1]
    except KeyError:
        v_rank = 32
    return NativeRWKV7Config(
        vocab_size=tensor_shape(weights, "emb.weight")[0], hidden_size=hidden, num_hidden_layers=layers,
        head_dim=head_dim, num_heads=heads, intermediate_size=ffn,
        decay_low_rank_dim=tensor_shape(weights, "blocks.0.att.w1")[1],
        a_low_rank_dim=tensor_shape(weights, "blocks.0.att.a1")[1],
        gate_low_rank_dim=tensor_shape(weights, "blocks.0.att.g1")[1], v_low_rank_dim=v_rank)


# ------------------------------------------------------------- names
_EMB_HEAD = {"emb.weight": "model.embeddings.weight", "ln_out.weight": "model.norm.weight",
             "ln_out.bias": "model.norm.bias", "head.weight": "lm_head.weight"}
_PROJ = {"receptance": "r_proj", "key": "k_proj", "value": "v_proj", "ln_x": "g_norm", "output": "o_proj"}
_BLOCK = {"att": "attn", "ffn": "ffn", "ln0": "pre_norm", "ln1": "attn_norm", "ln2": "ffn_norm"}
_LORA = {"0": "2.bias", "1": "0.weight", "2": "2.weight"}
_UNUSED = {"blocks.0.att.v0", "blocks.0.att.v1", "blocks.0.att.v2"}


def translate_name(name: str, num_layers: int) -> Tuple[str, bool]:
    """Official key -> (HF key, transposed); ``("", False)`` for dropped keys
    (rwkv7_hf/converter.py:333-365)."""
    if name in _UNUSED:
        return "", False
    if name in _EMB_HEAD:
        return _EMB_HEAD[name], False
    parts = name.split(".")
    if len(parts) < 4 or parts[0] != "blocks":
        raise KeyError(f"Unexpected RWKV weight name: {name}")
    if int(parts[1]) not in range(num_layers):
        raise KeyError(f"Layer index out of range in {name}")
    parts[0] = "model.layers"
    parts[2] = _BLOCK[parts[2]]
    transposed = False
    if re.match(r"[wvag][012]$", parts[3]):
        kind, num = parts[3]
        parts[3] = f"{kind}_lora.lora." + _LORA[num]
        transposed = num in ("1", "2")
    elif parts[2] == "attn" and parts[3] in _PROJ:
        parts[3] = _PROJ[parts[3]]
    return ".".join(parts), transposed


# ------------------------------------------------------------- convert
def convert_state_dict(weights: Dict[str, torch.Tensor], dtype: torch.dtype = torch.float16):
    """``(config, hf_state_dict)`` from an official state dict.  Entries are
    popped from ``weights`` as they are translated (one checkpoint resident)."""
    from .model import parameter_shapes

    cfg = infer_config(weights)
    expected = parameter_shapes(cfg)
    missing = set(expected)
    out: Dict[str, torch.Tensor] = {}
    for src in list(weights):
        w = weights.pop(src)
        dst, transposed = translate_name(src, cfg.num_hidden_layers)
        if not dst:
            continue
        if dst not in expected:
            raise KeyError(f"Translated name not in the model: {src} -> {dst}")
        w = w.detach()
        if transposed:
            w = w.t()
        shape = expected[dst]
        if tuple(w.shape) != tuple(shape):
            if int(w.numel()) != int(torch.Size(shape).numel()):
                raise ValueError(f"Shape mismatch {src} -> {dst}: {tuple(w.shape)} vs {tuple(shape)}")
            w = w.reshape(shape)
        out[dst] = w.to(dtype).contiguous().clone()
        missing.discard(dst)
    left = sorted(missing - set(_ALLOWED_MISSING))
    if left:
        raise KeyError(f"Uninitialized parameters: {left[:20]} ... total={len(left)}")
    for name in sorted(missing & set(_ALLOWED_MISSING)):
        fill = torch.ones if name.endswith("weight") else torch.zeros
        out[name] = fill(expected[name], dtype=dtype)
    return cfg, out


def _config_json(cfg, dtype_name: str) -> dict:
    return {
        "model_type": "rwkv7_native", "architectures": ["NativeRWKV7ForCausalLM"], "torch_dtype": dtype_name,
        "vocab_size": cfg.vocab_size, "hidden_size": cfg.hidden_size, "num_hidden_layers": cfg.num_hidden_layers,
        "head_dim": cfg.head_dim, "num_heads": cfg.num_heads, "intermediate_size": cfg.intermediate_size,
        "attention_hidden_size": cfg.attention_hidden_size, "decay_low_rank_dim": cfg.decay_low_rank_dim,
        "a_low_rank_dim": cfg.a_low_rank_dim, "gate_low_rank_dim": cfg.gate_low_rank_dim,
        "v_low_rank_dim": cfg.v_low_rank_dim, "norm_eps": cfg.norm_eps, "pad_token_id": 0, "eos_token_id": 0,
        "bos_token_id": 1, "tie_word_embeddings": False,
    }


def config_from_json(d: dict):
    """A config from ``config.json`` (this converter's or the reference's: the
    shape fields are read by name, the rest ignored)."""
    from .model import NativeRWKV7Config

    need = ("vocab_size", "hidden_size", "num_hidden_layers")
    if any(k not in d for k in need):
        raise ValueError(f"config.json lacks {[k for k in need if k not in d]}")
    kw = {k: d[k] for k in ("vocab_size", "hidden_size", "num_hidden_layers", "head_dim", "num_heads",
                            "intermediate_size", "decay_low_rank_dim", "a_low_rank_dim", "gate_low_rank_dim",
                            "v_low_rank_dim", "norm_eps") if d.get(k) is not None}
    return NativeRWKV7Config(**kw)


def save_hf_directory(output, cfg, state: Dict[str, torch.Tensor], *, dtype_name: str = "float16") -> Path:
    """``config.json`` + ``model.safetensors`` (CPU tensors)."""
    from safetensors.torch import save_file

    out = Path(output)
    out.mkdir(parents=True, exist_ok=True)
    (out / "config.json").write_text(json.dumps(_config_json(cfg, dtype_name), indent=2) + "\n")
    save_file({k: v.detach().cpu().contiguous() for k, v in state.items()}, str(out / "model.safetensors"),
              metadata={"format": "pt"})
    return out


def load_hf_directory(path) -> tuple:
    """``(config, state_dict)`` of a converted directory (one or more
    ``*.safetensors`` files)."""
    from safetensors.torch import load_file

    p = Path(path)
    cfg = config_from_json(json.loads((p / "config.json").read_text()))
    files = sorted(p.glob("*.safetensors"))
    files = [f for f in files if f.name != "prepacked.safetensors"]
    if not files:
        raise FileNotFoundError(f"no *.safetensors in {p}")
    state: Dict[str, torch.Tensor] = {}
    for f in files:
        state.update(load_file(str(f)))
    return cfg, state


def load_pretrained(path, *, device="cuda", dtype=torch.float16, use_native_mm8: bool | None = None,
                    native_mm8_policy: str | None = None, native_mm8_min_params: int | None = None):
    """A :class:`NativeRWKV7ForCausalLM` from a converted directory; with a
    ``manifest.json`` next to it the MM8 modules come prepacked."""
    from .model import NativeRWKV7ForCausalLM

    p = Path(path)
    if (p / "manifest.json").exists():
        return load_prepacked(p, device=device, dtype=dtype)
    cfg, state = load_hf_directory(p)
    if use_native_mm8 is not None:
        cfg.use_native_mm8 = bool(use_native_mm8)
    if native_mm8_policy is not None:
        cfg.native_mm8_policy = native_mm8_policy
    if native_mm8_min_params is not None:
        cfg.native_mm8_min_params = int(native_mm8_min_params)
    return NativeRWKV7ForCausalLM(cfg, state, device=device, dtype=dtype)


# ------------------------------------------------------------- prepacked MM8
def _sha256(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


_EPILOGUE = {"ffn.key": "relu2", "ffn.value": "residual", "attn.o_proj": "residual"}


def save_prepacked(model, output, *, source_state: Dict[str, torch.Tensor] | None = None) -> dict:
    """Write ``prepacked.safetensors`` (the model's MM8 modules in the blocked
    layout: ``<module>.w_blk``, ``.mx``, ``.rx``, ``.my``, ``.ry``), the
    remaining (dense) parameters in ``model.safetensors``, ``config.json`` and
    ``manifest.json``.  ``source_state`` (the unquantised HF state dict)
    supplies each module's ``source_weight_sha256``."""
    from safetensors.torch import save_file

    from .model import QuantLinear

    out = Path(output)
    out.mkdir(parents=True, exist_ok=True)
    cfg = model.config
    packed: Dict[str, torch.Tensor] = {}
    manifest = {"format": PREPACKED_FORMAT, "packer_version": PACKER_VERSION, "modules": []}
    dense = dict(model.dense_state_dict())
    for name, lin in model.named_linears():
        if not isinstance(lin, QuantLinear):
            continue
        m = lin.m
        for field in ("w_blk", "mx", "rx", "my", "ry"):
            packed[f"{name}.{field}"] = getattr(m, field).detach().cpu().contiguous()
        entry = {
            "format": PREPACKED_FORMAT, "module": name, "input_features": int(m.in_features),
            "output_features": int(m.out_features), "activation_dtype": str(model.dtype).replace("torch.", ""),
            "scale_dtype": str(m.mx.dtype).replace("torch.", ""),
            "epilogue": next((v for k, v in _EPILOGUE.items() if name.endswith(k)), "none"),
            "blocked_shape": list(m.w_blk.shape), "packer_version": PACKER_VERSION,
        }
        if source_state is not None and name + ".weight" in source_state:
            entry["source_weight_sha256"] = _sha256(source_state[name + ".weight"])
        manifest["modules"].append(entry)
        dense.pop(name + ".weight", None)
    save_file(packed, str(out / "prepacked.safetensors"), metadata={"format": PREPACKED_FORMAT})
    save_file({k: v.detach().cpu().contiguous() for k, v in dense.items()}, str(out / "model.safetensors"),
              metadata={"format": "pt"})
    cj = _config_json(cfg, str(model.dtype).replace("torch.", ""))
    cj.update({"use_native_mm8": True, "native_mm8_policy": cfg.native_mm8_policy,
               "native_mm8_min_params": cfg.native_mm8_min_params})
    (out / "config.json").write_text(json.dumps(cj, indent=2) + "\n")
    (out / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n")
    return manifest


def validate_manifest(manifest: dict, cfg, dtype: torch.dtype) -> None:
    """Check every entry against the config before any GPU buffer exists."""
    from .native_quant_mm8 import mm8_block_shape

    if manifest.get("format") != PREPACKED_FORMAT:
        raise ValueError(f"unsupported prepacked format {manifest.get('format')!r} (expected {PREPACKED_FORMAT})")
    if manifest.get("packer_version") != PACKER_VERSION:
        raise ValueError(f"prepacked by {manifest.get('packer_version')!r}; this build reads {PACKER_VERSION!r}")
    from .model import parameter_shapes

    shapes = parameter_shapes(cfg)
    seen = set()
    for e in manifest.get("modules", []):
        name = e.get("module", "")
        if e.get("format") != PREPACKED_FORMAT:
            raise ValueError(f"{name}: format {e.get('format')!r}")
        if name + ".weight" not in shapes:
            raise ValueError(f"{name}: not a linear of this config")
        o, i = shapes[name + ".weight"]
        if (e.get("input_features"), e.get("output_features")) != (i, o):
            raise ValueError(f"{name}: features {(e.get('input_features'), e.get('output_features'))} vs ({i}, {o})")
        if list(e.get("blocked_shape", [])) != list(mm8_block_shape(i, o)):
            raise ValueError(f"{name}: blocked shape {e.get('blocked_shape')} vs {list(mm8_block_shape(i, o))}")
        dname = str(dtype).replace("torch.", "")
        if e.get("activation_dtype") != dname:
            raise ValueError(f"{name}: packed for {e.get('activation_dtype')} activations, loading {dtype}")
        if e.get("scale_dtype") != dname:  # the kernels read mx / rx / my / ry in the activation dtype
            raise ValueError(f"{name}: scales stored as {e.get('scale_dtype')}, the kernels need {dname}")
        if e.get("packer_version") != PACKER_VERSION:
            raise ValueError(f"{name}: packer {e.get('packer_version')!r}, this build reads {PACKER_VERSION!r}")
        if name in seen:
            raise ValueError(f"{name}: listed twice")
        seen.add(name)


def load_prepacked(path, *, device="cuda", dtype=torch.float16,
                   source_state: Dict[str, torch.Tensor] | None = None):
    """The model from a prepacked directory: the manifest is validated, then
    the MM8 modules are built from the stored bytes (no quantisation).  Each
    stored tensor must have the dtype the manifest declares.  With
    ``source_state`` (the unquantised HF state dict), every module's
    ``source_weight_sha256`` is checked against it."""
    from safetensors.torch import load_file

    from .model import NativeRWKV7ForCausalLM
    from .native_quant_mm8 import MM8Linear

    p = Path(path)
    cj = json.loads((p / "config.json").read_text())
    cfg = config_from_json(cj)
    cfg.use_native_mm8 = True
    cfg.native_mm8_policy = cj.get("native_mm8_policy", cfg.native_mm8_policy)
    cfg.native_mm8_min_params = int(cj.get("native_mm8_min_params", cfg.native_mm8_min_params))
    manifest = json.loads((p / "manifest.json").read_text())
    validate_manifest(manifest, cfg, dtype)
    packed = load_file(str(p / "prepacked.safetensors"))
    state = load_file(str(p / "model.safetensors"))
    prebuilt = {}
    for e in manifest["modules"]:
        n = e["module"]
        missing = [f for f in ("w_blk", "mx", "rx", "my", "ry") if f"{n}.{f}" not in packed]
        if missing:
            raise ValueError(f"{n}: prepacked.safetensors lacks {missing}")
        t = {f: packed[f"{n}.{f}"] for f in ("w_blk", "mx", "rx", "my", "ry")}
        for f in ("mx", "rx", "my", "ry"):
            if str(t[f].dtype).replace("torch.", "") != e["scale_dtype"]:
                raise ValueError(f"{n}.{f}: stored as {t[f].dtype}, manifest says {e['scale_dtype']}")
        if source_state is not None:
            want = e.get("source_weight_sha256")
            src = source_state.get(n + ".weight")
            if want is None or src is None:
                raise ValueError(f"{n}: cannot verify the source weight (no digest or no source tensor)")
            if _sha256(src) != want:
                raise ValueError(f"{n}: source weight digest differs from the one it was packed from")
        prebuilt[n] = MM8Linear.from_packed(t["w_blk"].to(device), t["mx"].to(device), t["rx"].to(device),
                                           t["my"].to(device), t["ry"].to(device), e["input_features"],
                                           e["output_features"])
    return NativeRWKV7ForCausalLM(cfg, state, device=device, dtype=dtype, prepacked=prebuilt)


# ------------------------------------------------------------- CLI
def convert(args: argparse.Namespace) -> Path:
    dtype_name, dtype = DTYPES[args.precision]
    weights = torch.load(args.input, weights_only=True, map_location="cpu", mmap=bool(args.low_memory))
    cfg, state = convert_state_dict(weights, dtype)
    out = save_hf_directory(args.output, cfg, state, dtype_name=dtype_name)
    if args.prepack_mm8:
        from .model import NativeRWKV7ForCausalLM

        cfg.use_native_mm8 = True
        model = NativeRWKV7ForCausalLM(cfg, state, device=args.device, dtype=dtype)
        save_prepacked(model, out, source_state=state)
    print(f"Saved RWKV-7 model to: {out}")
    return out


def build_parser(prog: str | None = None) -> argparse.ArgumentParser:
    ap = argparse.ArgumentParser(prog=prog, description="Convert an official RWKV-7 .pth checkpoint into a "
                                                       "model directory (config.json + model.safetensors).")
    ap.add_argument("--input", required=True, help="official RWKV-7 .pth checkpoint")
    ap.add_argument("--output", required=True, help="output directory")
    ap.add_argument("--precision", choices=sorted(DTYPES), default="fp16")
    ap.add_argument("--low-memory", action="store_true", help="memory-map the checkpoint")
    ap.add_argument("--prepack-mm8", action="store_true",
                    help="also write the MM8 modules prepacked (needs a GPU: the packer is a HIP kernel)")
    ap.add_argument("--device", default="cuda")
    return ap


def main(argv: Sequence[str] | None = None) -> int:
    convert(build_parser().parse_args(argv))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
