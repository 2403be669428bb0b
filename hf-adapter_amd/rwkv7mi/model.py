"""RWKV-7 causal LM on the rwkv7mi gfx950 kernels.

Mirrors the reference adapter's native model (rwkv-rs/hf-adapter 0.8.1):
config fields of ``NativeRWKV7Config`` (rwkv7_hf/model_config.py:54-101),
parameter names of the converted checkpoints (rwkv7_hf/model_layers.py:12-131,
model_backbone.py:123-125, native_model.py:414), the recurrent cache contract
of ``NativeRWKV7Cache`` (rwkv7_hf/model_cache.py:48-466: per-layer state
``[B,H,N,N]`` fp32, ``xpa/xpf [B,D]``, ``v_first [B,A]``, ``seen_tokens``),
the per-layer decode body of ``_block_ip_batched``
(rwkv7_hf/native_jit_decode.py:481-901), the sequence prefill engine
(rwkv7_hf/native_jit_prefill.py:223-1057) and the graph-captured decode
runner (rwkv7_hf/native_graph_runtime.py:212-711, ``torch.cuda.graph`` =
hipGraph on ROCm).  Every operator is a HIP kernel from librwkv7mi.so except
the embedding row gather and, for prefills of more than 256 rows, the plain
library GEMMs of dense (unquantised) projections (rocBLAS through torch).
"""
from __future__ import annotations

import ctypes
import os
import weakref
import zlib
from dataclasses import dataclass

import torch

from . import _lib
from . import workspace as _ws
from .fused_decode_norm_mix import (attn_mix_lora_chunks, attn_mix_lora_decode, fused_attn_norm_mix6_decode,
                                    fused_ffn_add_norm_mix_decode, layer_norm)
from .fused_lora import (ACT_NONE, ACT_SIGMOID, ACT_TANH, dense_multi, fused_lora_decode_supported,
                         fused_wavg_lora_output_prepare_raw, lora_multi, lora_workspace_bytes)
from .fused_output import fused_attn_output_prepare
from .fused_prefill import fused_prefill_state_prep
from .fused_recurrent_update import fused_recurrent_output_prepare_raw
from .native_wkv_fp16 import (native_fp16_recurrent_output_prepare_raw, native_fp16_recurrent_should_use,
                              native_fp16_sequence)
from .fused_time_mix import fused_attn_sequence_shift_mix, fused_ffn_sequence_shift_mix
from .sampling import argmax_rows, argmax_workspace_bytes
from .native_quant_mm8 import (GEMM_ROWS, GEMV_ROWS, MM8Linear, is_blocked, mm8_gemm_multi_into, mm8_gemm_prefill_multi_into,
                               mm8_gemm_workspace_bytes, mm8_prefill_workspace_bytes, mm8_lnmix_multi_into, mm8_matmul_multi_into,
                               mm8_matmul_multi_lora_into,
                               mm8_matmul_partials, mm8t_workspace_bytes)
from .native_quant_policy import should_quantize_linear
from .self_chunk_rwkv7 import _run_chunk, check_wkv7_chunk_status

EXP_HALF = 0.606531


try:
    from transformers import GenerationMixin as _GenerationMixin
    from transformers import PretrainedConfig as _PretrainedConfig
    from transformers import PreTrainedModel as _PreTrainedModel
except Exception:  # pragma: no cover - transformers absent: plain bases
    _PretrainedConfig = object

    class _PreTrainedModel(torch.nn.Module):  # type: ignore[no-redef]
        def __init__(self, config):
            super().__init__()
            self.config = config

    class _GenerationMixin:  # type: ignore[no-redef]
        pass


class NativeRWKV7Config(_PretrainedConfig):
    """The fields of the reference's ``NativeRWKV7Config`` that shape the
    inference path (rwkv7_hf/model_config.py:25-101), as a Hugging Face
    config of the same ``model_type``, so converted directories and
    ``AutoConfig`` read it.  Only head size 64 has kernels here."""

    model_type = "rwkv7_native"

    def __init__(self, vocab_size: int = 65536, hidden_size: int = 768, num_hidden_layers: int = 12,
                 head_dim: int = 64, num_heads: int | None = None, intermediate_size: int | None = None,
                 decay_low_rank_dim: int = 64, a_low_rank_dim: int = 64, gate_low_rank_dim: int = 128,
                 v_low_rank_dim: int = 32, norm_eps: float = 1e-5, use_native_mm8: bool = False,
                 native_mm8_min_params: int = 8_000_000, native_mm8_policy: str = "memory",
                 attention_hidden_size: int | None = None, extra: dict | None = None, **kwargs):
        kwargs.setdefault("tie_word_embeddings", False)  # RWKV keeps an independent output head
        kwargs.pop("num_attention_heads", None)
        if _PretrainedConfig is not object:
            super().__init__(**kwargs)
        self.vocab_size = int(vocab_size)
        self.hidden_size = int(hidden_size)
        self.num_hidden_layers = int(num_hidden_layers)
        self.head_dim = int(head_dim)
        if self.head_dim != 64:
            raise ValueError("rwkv7mi kernels require head_dim = 64")
        if num_heads is None:
            num_heads = (attention_hidden_size or self.hidden_size) // self.head_dim
        self.num_heads = int(num_heads)
        if attention_hidden_size is not None and int(attention_hidden_size) != self.num_heads * self.head_dim:
            raise ValueError("attention_hidden_size must equal num_heads * head_dim")
        self.num_attention_heads = self.num_heads
        self.intermediate_size = int(intermediate_size) if intermediate_size is not None else 4 * self.hidden_size
        self.decay_low_rank_dim = int(decay_low_rank_dim)
        self.a_low_rank_dim = int(a_low_rank_dim)
        self.gate_low_rank_dim = int(gate_low_rank_dim)
        self.v_low_rank_dim = int(v_low_rank_dim)
        self.norm_eps = float(norm_eps)
        self.use_native_mm8 = bool(use_native_mm8)
        self.native_mm8_min_params = int(native_mm8_min_params)
        self.native_mm8_policy = native_mm8_policy
        self.extra = dict(extra or {})

    @property
    def attention_hidden_size(self) -> int:
        return self.num_heads * self.head_dim

    def to_dict(self) -> dict:
        d = super().to_dict() if _PretrainedConfig is not object else dict(self.__dict__)
        d["attention_hidden_size"] = self.attention_hidden_size
        return d


# ------------------------------------------------------------------ weights
def parameter_shapes(cfg: NativeRWKV7Config) -> dict[str, tuple]:
    D, A, F, V, H, N = (cfg.hidden_size, cfg.attention_hidden_size, cfg.intermediate_size, cfg.vocab_size,
                        cfg.num_heads, cfg.head_dim)
    shapes: dict[str, tuple] = {"model.embeddings.weight": (V, D)}
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        if i == 0:
            shapes[p + "pre_norm.weight"] = (D,)
            shapes[p + "pre_norm.bias"] = (D,)
        for n in ("attn_norm", "ffn_norm"):
            shapes[p + n + ".weight"] = (D,)
            shapes[p + n + ".bias"] = (D,)
        for m in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"):
            shapes[p + "attn." + m] = (1, 1, D)
        shapes[p + "attn.k_k"] = (A,)
        shapes[p + "attn.k_a"] = (A,)
        shapes[p + "attn.r_k"] = (H, N)
        for n in ("r_proj", "k_proj", "v_proj"):
            shapes[p + f"attn.{n}.weight"] = (A, D)
        shapes[p + "attn.o_proj.weight"] = (D, A)
        loras = [("w_lora", cfg.decay_low_rank_dim, True), ("a_lora", cfg.a_low_rank_dim, True),
                 ("g_lora", cfg.gate_low_rank_dim, False)]
        if i > 0:
            loras.append(("v_lora", cfg.v_low_rank_dim, True))
        for n, rank, bias in loras:
            shapes[p + f"attn.{n}.lora.0.weight"] = (rank, D)
            shapes[p + f"attn.{n}.lora.2.weight"] = (A, rank)
            if bias:
                shapes[p + f"attn.{n}.lora.2.bias"] = (A,)
        shapes[p + "attn.g_norm.weight"] = (A,)
        shapes[p + "attn.g_norm.bias"] = (A,)
        shapes[p + "ffn.x_k"] = (D,)
        shapes[p + "ffn.key.weight"] = (F, D)
        shapes[p + "ffn.value.weight"] = (D, F)
    shapes["model.norm.weight"] = (D,)
    shapes["model.norm.bias"] = (D,)
    shapes["lm_head.weight"] = (V, D)
    return shapes


def _param_init(name: str, shape: tuple, gen: torch.Generator, device) -> torch.Tensor:
    """Non-degenerate random init (all parameters): Linear/Embedding N(0, 0.02),
    norm weight 1 / bias 0, token-shift mixes U(0, 1), k_k / k_a / r_k N(0, 0.1)
    around their typical magnitudes, LoRA biases N(0, 0.01)."""
    if name.endswith(("norm.weight",)):
        return torch.ones(shape, device=device)
    if name.endswith(("norm.bias",)):
        return torch.zeros(shape, device=device)
    leaf = name.rsplit(".", 1)[-1]
    if leaf in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"):
        return torch.rand(shape, generator=gen, device=device)
    if leaf == "k_k":
        return 0.85 + 0.1 * torch.randn(shape, generator=gen, device=device)
    if leaf == "k_a":
        return 1.0 + 0.1 * torch.randn(shape, generator=gen, device=device)
    if leaf == "r_k":
        return 0.1 * torch.randn(shape, generator=gen, device=device)
    if name.endswith("lora.2.bias"):
        return 0.01 * torch.randn(shape, generator=gen, device=device)
    return 0.02 * torch.randn(shape, generator=gen, device=device)


def random_weights(cfg: NativeRWKV7Config, *, seed: int = 0, device="cpu", dtype=torch.float16,
                   names: list[str] | None = None) -> dict[str, torch.Tensor]:
    """Seeded weights keyed by (seed, parameter name): each tensor has its own
    generator, so the values do not depend on construction order."""
    out = {}
    for name, shape in parameter_shapes(cfg).items():
        if names is not None and name not in names:
            continue
        gen = torch.Generator(device=device)
        gen.manual_seed((seed * 0x9E3779B1 + zlib.crc32(name.encode())) & 0x7FFFFFFFFFFFFFFF)
        out[name] = _param_init(name, shape, gen, device).to(dtype)
    return out


# ------------------------------------------------------------------ linears
class DenseLinear:
    """Unquantised Linear ``y = x W^T`` (projections below the MM8 size
    threshold, and every projection of an unquantised model such as the fp32
    0.1B one): the HIP dense kernel up to 256 rows; above that, for fp16 and
    bf16, the prefill MFMA GEMM (``rwkv7mi_dense_gemm_prefill_ws``: W copied
    into the ``"mm8p"`` workspace in operand order, relu^2 / residual fused),
    and for fp32 weights a plain library GEMM (hipBLASLt through torch) with
    the epilogue as torch elementwise ops."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None = None):
        self.weight = weight.contiguous()
        self.bias = None if bias is None else bias.contiguous()
        self.out_features, self.in_features = (int(s) for s in self.weight.shape)

    def apply(self, x2, out, *, act=ACT_NONE, residual=None):
        rows = int(x2.shape[0])
        if (rows > 256 and x2.dtype in (torch.float16, torch.bfloat16) and self.weight.dtype == x2.dtype
                and self.in_features % 16 == 0 and act in (0, 3) and not (act == 3 and residual is not None)
                and x2.is_contiguous() and out.is_contiguous()):
            epi = _lib.EPI_RELU2 if act == 3 else (_lib.EPI_RESIDUAL if residual is not None else _lib.EPI_NONE)
            need = mm8_prefill_workspace_bytes(1, self.in_features, self.out_features)
            ws = _ws.reserve(x2.device, need, "mm8p")
            res = None if residual is None else residual.reshape(out.shape).contiguous()
            arr = _lib.ptr_array
            _lib.call("rwkv7mi_dense_gemm_prefill_ws", 1, arr([x2]), arr([self.weight]), arr([self.bias]), arr([res]),
                      arr([out]), (ctypes.c_int * 1)(epi), rows, self.in_features, self.out_features, _lib.dtype_code(x2),
                      _lib.ptr(ws), need, _lib.stream_of(x2))
            return out
        if rows > 256:
            y = torch.nn.functional.linear(x2, self.weight, self.bias)
            if act == 3:
                y = torch.relu(y).square()
            if residual is not None:
                y = y + residual
            out.copy_(y)
            return out
        if residual is not None:
            tmp = torch.empty_like(out)
            dense_multi([(x2, self.weight, self.bias, tmp, act)], rows)
            torch.add(residual, tmp, out=out)
            return out
        dense_multi([(x2, self.weight, self.bias, out, act)], rows)
        return out


class QuantLinear:
    """MM8 Linear, all on HIP kernels: the fused blocked dequant GEMV for up to
    ``GEMV_ROWS`` rows, the 64-row MFMA tile GEMM (split K) up to ``GEMM_ROWS``
    rows, and above that the prefill GEMM over the materialised fp16
    dequantised weight (``mm8_gemm_prefill_multi_into``).  Modules whose bytes are not blocked
    take MM8Linear's own route."""

    GEMV_ROWS = GEMV_ROWS
    GEMM_ROWS = GEMM_ROWS

    def __init__(self, mm8: MM8Linear):
        self.m = mm8
        self.out_features, self.in_features = mm8.out_features, mm8.in_features

    def apply(self, x2, out, *, act=ACT_NONE, residual=None):
        rows = int(x2.shape[0])
        if self.GEMV_ROWS < rows <= self.GEMM_ROWS and is_blocked(self.m.w_blk):
            epi = _lib.EPI_RELU2 if act == 3 else (_lib.EPI_RESIDUAL if residual is not None else _lib.EPI_NONE)
            if act not in (0, 3) or (act == 3 and residual is not None):
                raise ValueError("QuantLinear: unsupported activation / residual combination")
            mm8_gemm_multi_into([x2], [self.m], [out], residuals=[residual], epilogues=[epi])
            return out
        if act not in (0, 3) or (act == 3 and residual is not None):
            raise ValueError("QuantLinear: unsupported activation / residual combination")
        epi = _lib.EPI_RELU2 if act == 3 else (_lib.EPI_RESIDUAL if residual is not None else _lib.EPI_NONE)
        if rows > self.GEMM_ROWS and is_blocked(self.m.w_blk):
            mm8_gemm_prefill_multi_into([x2], [self.m], [out], residuals=[residual], epilogues=[epi])
            return out
        return self.m._run(x2, out=out, residual=residual, epilogue=epi)

    @staticmethod
    def apply_group(lins, xs, outs):
        """The same as ``[l.apply(x, o) for ...]``; out-major MM8 modules of one
        shape run as one launch."""
        rows = int(xs[0].shape[0])
        if (all(isinstance(l, QuantLinear) for l in lins)
                and len({(l.in_features, l.out_features) for l in lins}) == 1
                and all(is_blocked(l.m.w_blk) for l in lins)):
            if rows <= QuantLinear.GEMV_ROWS:
                mm8_matmul_multi_into(list(xs), [l.m for l in lins], list(outs))
            elif rows <= QuantLinear.GEMM_ROWS:
                mm8_gemm_multi_into(list(xs), [l.m for l in lins], list(outs))
            else:
                mm8_gemm_prefill_multi_into(list(xs), [l.m for l in lins], list(outs))
            return outs
        for l, x2, o in zip(lins, xs, outs):
            l.apply(x2, o)
        return outs


# ------------------------------------------------------------------ cache
try:  # the HF Cache base lets GenerationMixin / Trainer accept the cache
    from transformers.cache_utils import Cache as _HFCache
except Exception:  # pragma: no cover - transformers absent
    class _HFCache:  # type: ignore[no-redef]
        pass


class _LegacyCache(tuple):
    """Tuple ``(state, xpa, xpf, v_first)`` that remembers the sequence length
    (the reference's legacy form, rwkv7_hf/model_cache.py:16-45)."""

    def __new__(cls, state, xpa, xpf, v_first, seen_tokens: int = 0):
        obj = super().__new__(cls, (state, xpa, xpf, v_first))
        obj._seen_tokens = int(seen_tokens)
        return obj

    def get_seq_length(self, layer_idx: int | None = 0, cache_position=None) -> int:
        n = 0 if self[0] is None else len(self[0])
        if layer_idx is not None and (int(layer_idx) < 0 or (self[0] is not None and int(layer_idx) >= n)
                                      or (self[0] is None and int(layer_idx) != 0)):
            return 0
        return self._seen_tokens

    @property
    def seen_tokens(self) -> int:
        return self._seen_tokens

    def to_legacy_cache(self):
        return self


_METRIC_KEYS = ("clones", "detaches", "device_moves", "select_batch_calls", "batch_select_calls",
                "batch_select_indices_calls", "batch_repeat_interleave_calls", "reorder_calls", "crops", "resets",
                "native_graph_bound_selects")


class NativeRWKV7Cache(_HFCache):
    """Recurrent-state cache with the reference's contract (rwkv7_hf/model_cache.py:48-466).

    Holds ``(state, xpa, xpf, v_first)``: per-layer ``state[l] [B, H, N, N]``
    fp32 (value x key), per-layer token-shift rows ``xpa[l]``, ``xpf[l]``
    ``[B, D]`` and the cross-layer ``v_first [B, A]``, plus ``seen_tokens``.
    Iterable as that 4-tuple.  An opt-in fp16 state (``zeros(...,
    state_dtype=torch.float16)``) also carries ``fp16_elapsed`` (int32 ``[B]``,
    the phase of the fp16 recurrence's decay dither), which follows the batch
    edits but is not part of the legacy tuple.  Batch edits (select / reorder / repeat), device
    moves, detach, crop-to-empty and legacy-tuple conversion follow the
    reference.  A graph runner that replays the decode step binds the cache
    (its tensors become the runner's buffers); any edit that replaces the
    tensors bumps the cache version, which unbinds it, and a batch reorder of a
    bound cache permutes the runner's buffers in place instead.
    """

    is_compileable = True

    def __init__(self, state=None, xpa=None, xpf=None, v_first=None, seen_tokens: int = 0):
        # (the HF base initialiser builds KV layer objects a recurrent cache does not use)
        self._state, self._xpa, self._xpf, self._v_first = state, xpa, xpf, v_first
        self._elapsed = None
        if state is not None and len(state) and state[0].dtype == torch.float16:
            self._elapsed = torch.zeros(int(state[0].shape[0]), device=state[0].device, dtype=torch.int32)
        self._seen_tokens = int(seen_tokens)
        self.layers = []
        self._rwkv7_cache_metrics = {k: 0 for k in _METRIC_KEYS}
        self._rwkv7_cache_version = 0
        self._bound_runner_ref = None
        self._bound_version = None

    @classmethod
    def zeros(cls, cfg: "NativeRWKV7Config", batch: int, device, dtype=torch.float16,
              state_dtype=torch.float32):
        """A zero cache whose per-layer tensors are views of layer-major
        storage ([L, B, H, N, N] state, [L, B, D] shift rows): each layer
        is contiguous and the layers are equally spaced, so one slot-copy
        launch can move a batch row of every layer.  ``state_dtype`` is fp32,
        or fp16 for the opt-in fp16-state lane (fp16 activations, head size 64)."""
        H, N, D, A, L = cfg.num_heads, cfg.head_dim, cfg.hidden_size, cfg.attention_hidden_size, cfg.num_hidden_layers
        if state_dtype not in (torch.float32, torch.float16):
            raise ValueError(f"state_dtype must be float32 or float16; got {state_dtype}")
        if state_dtype == torch.float16 and not native_fp16_recurrent_should_use(
                state_dtype=state_dtype, input_dtype=dtype, head_dim=N):
            raise ValueError("an fp16 recurrent state needs fp16 activations and head size 64")
        S = torch.zeros(L, batch, H, N, N, device=device, dtype=state_dtype)
        xa = torch.zeros(L, batch, D, device=device, dtype=dtype)
        xf = torch.zeros(L, batch, D, device=device, dtype=dtype)
        return cls(list(S.unbind(0)), list(xa.unbind(0)), list(xf.unbind(0)),
                   torch.zeros(batch, A, device=device, dtype=dtype), 0)

    # ---- graph binding / version protocol (rwkv7_hf/model_cache.py:89-114)
    def _invalidate_native_graph_binding(self) -> None:
        self._rwkv7_cache_version += 1
        self._bound_runner_ref = None
        self._bound_version = None

    _invalidate = _invalidate_native_graph_binding

    def _bind_native_graph_runner(self, runner) -> None:
        self._bound_runner_ref = weakref.ref(runner)
        self._bound_version = self._rwkv7_cache_version

    def _native_graph_bound_runner(self):
        if self._bound_version != self._rwkv7_cache_version or self._bound_runner_ref is None:
            return None
        return self._bound_runner_ref()

    def _native_graph_bound_to(self, runner) -> bool:
        return runner is not None and self._native_graph_bound_runner() is runner

    @property
    def _bound_runner(self):
        return self._native_graph_bound_runner()

    # ---- tuple view
    def __repr__(self) -> str:
        return (f"{type(self).__name__}(seen_tokens={self._seen_tokens}, batch_size={self.get_batch_size()}, "
                f"layers={0 if self._state is None else len(self._state)})")

    def __iter__(self):
        return iter((self._state, self._xpa, self._xpf, self._v_first))

    @property
    def fp16_elapsed(self) -> torch.Tensor | None:
        """int32 [B] phase of the fp16-state lane (None for an fp32 state)."""
        return self._elapsed

    @property
    def state_dtype(self) -> torch.dtype | None:
        return None if not self._state else self._state[0].dtype

    def _all_tensors(self) -> list:
        """Every tensor of the cache in a fixed order (fp16_elapsed last, when present)."""
        out = [*(self._state or ()), *(self._xpa or ()), *(self._xpf or ())]
        if self._v_first is not None:
            out.append(self._v_first)
        if self._elapsed is not None:
            out.append(self._elapsed)
        return out

    def __len__(self) -> int:
        return 4

    def __getitem__(self, idx):
        return self.to_legacy_cache()[idx]

    def to_legacy_cache(self):
        return _LegacyCache(self._state, self._xpa, self._xpf, self._v_first, seen_tokens=self._seen_tokens)

    @classmethod
    def from_legacy_cache(cls, legacy, seen_tokens: int = 0):
        """A cache from None, an empty cache, a cache of this class or a 4-tuple."""
        if legacy is None:
            return cls(seen_tokens=seen_tokens)
        if isinstance(legacy, NativeRWKV7Cache):
            return legacy
        seen = int(seen_tokens)
        if hasattr(legacy, "get_seq_length"):
            try:
                n = int(legacy.get_seq_length())
            except Exception:
                n = None
            if n == 0:
                return cls(seen_tokens=seen_tokens)
            if n is not None:
                seen = n
        if hasattr(legacy, "to_legacy_cache"):
            legacy = legacy.to_legacy_cache()
        if legacy is None or (isinstance(legacy, (list, tuple)) and len(legacy) == 0):
            return cls(seen_tokens=seen_tokens)
        if not isinstance(legacy, (list, tuple)) or len(legacy) != 4:
            raise TypeError("NativeRWKV7Cache.from_legacy_cache expects None, an empty cache, or a 4-tuple "
                            "recurrent cache")
        state, xpa, xpf, v_first = legacy
        return cls(state, xpa, xpf, v_first, seen_tokens=seen)

    # ---- sizes
    @property
    def seen_tokens(self) -> int:
        return self._seen_tokens

    @seen_tokens.setter
    def seen_tokens(self, value: int) -> None:
        self._seen_tokens = int(value)

    def _is_initialized(self, layer_idx: int | None = None) -> bool:
        if any(t is None for t in (self._state, self._xpa, self._xpf, self._v_first)):
            return False
        return layer_idx is None or 0 <= int(layer_idx) < len(self._state)

    @property
    def is_initialized(self) -> bool:
        return self._is_initialized()

    @property
    def is_sliding(self) -> bool:
        return False

    @property
    def max_batch_size(self) -> int | None:
        return self.get_batch_size()

    @property
    def max_cache_len(self) -> int:
        return -1

    @property
    def states(self) -> list[dict]:
        """Per-layer dict view (recurrent_state / attn_state / ffn_state)."""
        if self._state is None:
            return []
        return [{"recurrent_state": s, "attn_state": a, "conv_state": None, "ffn_state": f}
                for s, a, f in zip(self._state, self._xpa, self._xpf)]

    def get_seq_length(self, layer_idx: int | None = 0, cache_position=None) -> int:
        if layer_idx is not None:
            li = int(layer_idx)
            if li < 0 or (self._state is not None and li >= len(self._state)) or (self._state is None and li != 0):
                return 0
        return self._seen_tokens

    def get_max_cache_shape(self, layer_idx: int = 0) -> int:
        return -1

    def get_mask_sizes(self, cache_position, layer_idx: int = 0) -> tuple[int, int]:
        if cache_position is None:
            q = 0
        elif isinstance(cache_position, torch.Tensor):
            q = int(cache_position.numel())
        else:
            q = int(cache_position)
        return self.get_seq_length(layer_idx) + q, 0

    def get_batch_size(self) -> int | None:
        for values in (self._state, self._xpa, self._xpf):
            if values:
                return int(values[0].shape[0])
        return None if self._v_first is None else int(self._v_first.shape[0])

    def has_previous_state(self, layer_idx: int | None = None) -> bool:
        return self._is_initialized(layer_idx) and self._seen_tokens > 0

    # ---- edits
    def _map(self, fn):
        self._state = None if self._state is None else [fn(t) for t in self._state]
        self._xpa = None if self._xpa is None else [fn(t) for t in self._xpa]
        self._xpf = None if self._xpf is None else [fn(t) for t in self._xpf]
        self._v_first = None if self._v_first is None else fn(self._v_first)
        self._elapsed = None if self._elapsed is None else fn(self._elapsed)

    def clone(self) -> "NativeRWKV7Cache":
        out = type(self)(seen_tokens=self._seen_tokens)
        out._state, out._xpa, out._xpf, out._v_first = self._state, self._xpa, self._xpf, self._v_first
        out._elapsed = self._elapsed
        out._map(lambda t: t.clone())
        out._rwkv7_cache_metrics = dict(self._rwkv7_cache_metrics)
        out._rwkv7_cache_metrics["clones"] += 1
        return out

    def reset(self) -> None:
        """Drop the state (the reference's reset: the next forward starts fresh)."""
        self._invalidate_native_graph_binding()
        self._state = self._xpa = self._xpf = self._v_first = self._elapsed = None
        self._seen_tokens = 0
        self._rwkv7_cache_metrics["resets"] += 1

    def zero_(self) -> "NativeRWKV7Cache":
        """Zero the state in place, keeping the tensors (and any graph binding)."""
        for t in self._all_tensors():
            t.zero_()
        self._seen_tokens = 0
        return self

    def detach(self, *, inplace: bool = True) -> "NativeRWKV7Cache":
        target = self if inplace else self.clone()
        target._invalidate_native_graph_binding()
        target._map(lambda t: t.detach())
        target._rwkv7_cache_metrics["detaches"] += 1
        return target

    def to(self, device=None, dtype=None, *, non_blocking: bool = False, copy: bool = False,
           inplace: bool = True) -> "NativeRWKV7Cache":
        """Move the cache; ``dtype`` applies to the token-shift rows and
        ``v_first`` (the recurrent state keeps its dtype, as the kernels require)."""
        target = self if inplace else self.clone()
        target._invalidate_native_graph_binding()

        def move(t, is_state=False):
            kw = {"non_blocking": non_blocking, "copy": copy}
            if device is not None:
                kw["device"] = device
            if dtype is not None and t.is_floating_point() and not is_state:
                kw["dtype"] = dtype
            if len(kw) == 2:
                return t.clone() if copy else t
            return t.to(**kw)

        if target._state is not None:
            target._state = [move(t, True) for t in target._state]
        target._xpa = None if target._xpa is None else [move(t) for t in target._xpa]
        target._xpf = None if target._xpf is None else [move(t) for t in target._xpf]
        target._v_first = None if target._v_first is None else move(target._v_first)
        target._elapsed = None if target._elapsed is None else move(target._elapsed)
        target._rwkv7_cache_metrics["device_moves"] += 1
        return target

    def select_batch(self, indices, *, inplace: bool = True) -> "NativeRWKV7Cache":
        idx = torch.as_tensor(indices).to(dtype=torch.long)
        if inplace:
            target = self
        else:
            target = type(self)(self._state, self._xpa, self._xpf, self._v_first, seen_tokens=self._seen_tokens)
            target._elapsed = self._elapsed
            target._rwkv7_cache_metrics = dict(self._rwkv7_cache_metrics)
        runner = target._native_graph_bound_runner() if inplace else None
        if runner is not None and target.get_batch_size() == int(idx.numel()) and runner.reorder_batch_inplace(idx):
            target._rwkv7_cache_metrics["select_batch_calls"] += 1
            target._rwkv7_cache_metrics["native_graph_bound_selects"] += 1
            return target
        target._invalidate_native_graph_binding()
        target._map(lambda t: t.index_select(0, idx.to(t.device)))
        target._rwkv7_cache_metrics["select_batch_calls"] += 1
        return target

    def batch_select(self, indices, *, inplace: bool = True) -> "NativeRWKV7Cache":
        target = self.select_batch(indices, inplace=inplace)
        target._rwkv7_cache_metrics["batch_select_calls"] += 1
        return target

    def compact(self, indices, *, inplace: bool = True) -> "NativeRWKV7Cache":
        return self.batch_select(indices, inplace=inplace)

    def batch_select_indices(self, indices):
        target = self.select_batch(indices, inplace=True)
        target._rwkv7_cache_metrics["batch_select_indices_calls"] += 1
        return target

    def reorder_cache(self, beam_idx):
        target = self.select_batch(beam_idx, inplace=True)
        target._rwkv7_cache_metrics["reorder_calls"] += 1
        return target

    def batch_repeat_interleave(self, repeats: int):
        repeats = int(repeats)
        if repeats <= 0:
            raise ValueError("NativeRWKV7Cache.batch_repeat_interleave requires repeats > 0")
        self._invalidate_native_graph_binding()
        self._map(lambda t: t.repeat_interleave(repeats, dim=0))
        self._rwkv7_cache_metrics["batch_repeat_interleave_calls"] += 1
        return self

    def crop(self, max_length: int):
        """Only a no-op crop or a crop to nothing is possible for a recurrent state."""
        max_length = int(max_length)
        target = self._seen_tokens + max_length if max_length < 0 else max_length
        if target >= self._seen_tokens:
            return self
        if target <= 0:
            self._rwkv7_cache_metrics["crops"] += 1
            self.reset()
            return self
        raise NotImplementedError("NativeRWKV7Cache cannot crop recurrent state to a shorter positive prefix; "
                                  "run a fresh prefill for that prefix instead.")

    def rwkv7_cache_metrics(self) -> dict:
        m = dict(self._rwkv7_cache_metrics)
        m.update({"seen_tokens": self._seen_tokens, "batch_size": self.get_batch_size(),
                  "layers": 0 if self._state is None else len(self._state)})
        return m

    # ---- KV-cache hooks a recurrent cache does not have
    def update(self, *args, **kwargs):
        raise NotImplementedError("NativeRWKV7Cache is not a Transformer KV cache; update it through "
                                  "NativeRWKV7ForCausalLM.forward(..., past_key_values=...).")

    def update_recurrent_state(self, *args, **kwargs):
        raise NotImplementedError("NativeRWKV7Cache stores RWKV-7 state as (state, xpa, xpf, v_first); "
                                  "update it through NativeRWKV7ForCausalLM.forward(..., past_key_values=...).")

    def update_conv_state(self, *args, **kwargs):
        raise NotImplementedError("NativeRWKV7Cache does not have convolution state.")

    def update_indexer(self, *args, **kwargs):
        raise NotImplementedError("NativeRWKV7Cache does not have an indexer key cache.")

    def early_initialization(self, *args, **kwargs):
        raise NotImplementedError("NativeRWKV7Cache cannot be early-initialized as a Transformer KV cache.")

    def offload(self, *args, **kwargs):
        raise NotImplementedError("Use NativeRWKV7Cache.to(device='cpu') to offload native recurrent state.")

    def prefetch(self, *args, **kwargs):
        raise NotImplementedError("Use NativeRWKV7Cache.to(device=...) to restore native recurrent state.")



# ------------------------------------------------------------------ forward helpers
try:
    from transformers.modeling_outputs import CausalLMOutputWithPast as _CausalLMOutput
except Exception:  # pragma: no cover - transformers absent
    @dataclass
    class _CausalLMOutput:  # type: ignore[no-redef]
        loss: torch.Tensor | None = None
        logits: torch.Tensor | None = None
        past_key_values: object = None


def _as_native_cache(past_key_values) -> NativeRWKV7Cache | None:
    """The native cache behind ``past_key_values``; None for no (or an empty) cache
    (rwkv7_hf/model_cache.py:480-504)."""
    if past_key_values is None:
        return None
    if isinstance(past_key_values, NativeRWKV7Cache):
        return past_key_values if (past_key_values.is_initialized or past_key_values.seen_tokens) else None
    try:
        values = tuple(past_key_values)
    except Exception as exc:
        seen = getattr(past_key_values, "get_seq_length", lambda: 0)()
        if not seen:
            return None
        raise TypeError(f"Unsupported NativeRWKV7 cache type: {type(past_key_values)!r}") from exc
    if len(values) == 4 and all(v is not None for v in values):
        return NativeRWKV7Cache.from_legacy_cache(past_key_values)
    if not getattr(past_key_values, "get_seq_length", lambda: 0)():
        return None
    raise TypeError(f"NativeRWKV7 expects a NativeRWKV7Cache or 4-tuple recurrent cache; got "
                    f"{type(past_key_values)!r} with length {len(values)}")


def _check_attention_mask(mask, B: int, T: int, *, allow_trailing: bool) -> None:
    """All-ones masks are the same as none (rwkv7_hf/model_backbone.py:28-62);
    a mask that drops tokens has no native route here."""
    if mask is None:
        return
    if not isinstance(mask, torch.Tensor):
        raise TypeError("NativeRWKV7 attention_mask must be a torch.Tensor when provided")
    if mask.dim() == 1:
        mask = mask.view(1, -1)
    if mask.dim() != 2 or int(mask.shape[0]) != B:
        raise ValueError("NativeRWKV7 attention_mask must be shaped [batch, seq]")
    if int(mask.shape[1]) != T:
        if not allow_trailing or int(mask.shape[1]) < T:
            raise ValueError("NativeRWKV7 attention_mask must have the same [batch, seq] shape as inputs")
        mask = mask[:, -T:]
    if not bool((mask != 0).all()):
        raise ValueError("rwkv7mi: attention masks that drop tokens are not supported on the native routes "
                         "(RWKV state is order-sensitive; pass unpadded rows)")


def _resolve_logits_to_keep(logits_to_keep, num_logits_to_keep):
    if logits_to_keep is None:
        return None if num_logits_to_keep is None else int(num_logits_to_keep)
    if num_logits_to_keep is not None and int(num_logits_to_keep) != int(logits_to_keep):
        raise ValueError("logits_to_keep and num_logits_to_keep must match when both are provided")
    if isinstance(logits_to_keep, torch.Tensor) and logits_to_keep.dim() > 0:
        raise ValueError("rwkv7mi: logits_to_keep must be an integer (position lists are not supported)")
    return int(logits_to_keep)


def _slice_logits(logits: torch.Tensor, keep):
    if keep is None or int(keep) <= 0:
        return logits
    return logits[:, -min(int(keep), int(logits.shape[1])):, :]


# ------------------------------------------------------------------ model
def _env_on(name: str) -> bool:
    return os.environ.get(name, "0").strip().lower() in {"1", "true", "yes", "on"}


def native_graph_state_dtype(model_dtype: torch.dtype) -> torch.dtype:
    """Recurrent-state dtype of new caches from the reference's switches
    (rwkv7_hf/native_graph_runtime.py:119-147, :312-316):
    RWKV7_NATIVE_GRAPH_STATE_DTYPE = fp32 (default) or fp16; fp16 applies to
    fp16 models only and needs RWKV7_NATIVE_GRAPH_FP16_RECURRENT=1."""
    raw = os.environ.get("RWKV7_NATIVE_GRAPH_STATE_DTYPE", "fp32").strip().lower()
    if raw in {"fp32", "float32"}:
        return torch.float32
    if raw in {"fp16", "float16", "half"}:
        if model_dtype != torch.float16:
            return torch.float32
        if not _env_on("RWKV7_NATIVE_GRAPH_FP16_RECURRENT"):
            raise RuntimeError("FP16 native graph state requires RWKV7_NATIVE_GRAPH_FP16_RECURRENT=1")
        return torch.float16
    raise ValueError(f"RWKV7_NATIVE_GRAPH_STATE_DTYPE must be fp32 or fp16; got {raw!r}")


class _Layer:
    pass


class NativeRWKV7ForCausalLM(_PreTrainedModel, _GenerationMixin):
    """RWKV-7 causal LM (inference) over the HIP kernels; see the module docstring.

    A Hugging Face ``PreTrainedModel`` + ``GenerationMixin`` like the
    reference's (rwkv7_hf/native_model.py:371-406), registered for
    ``AutoConfig`` / ``AutoModelForCausalLM`` under ``model_type``
    ``"rwkv7_native"``: ``generate()`` drives :meth:`forward`, whose prefill is
    the chunked-scan route and whose one-token steps replay the captured
    decode graph.  The weights live in the kernels' own layouts (plain
    tensors and MM8 modules, not ``nn.Parameter`` s); ``from_pretrained`` /
    ``save_pretrained`` read and write converted directories.
    """

    config_class = NativeRWKV7Config
    base_model_prefix = "model"
    main_input_name = "input_ids"
    _tied_weights_keys: dict = {}
    _is_stateful = True  # a recurrent cache: no KV cropping or assisted decoding

    @classmethod
    def _supports_default_dynamic_cache(cls) -> bool:
        # the recurrent state is not a KV cache: GenerationMixin must not pre-build one
        return False

    @property
    def device(self) -> torch.device:
        return self._device

    @property
    def dtype(self) -> torch.dtype:
        return self._dtype

    def _init_common(self, config, device, dtype):
        _PreTrainedModel.__init__(self, config)
        self.config = config
        self._device = torch.device(device)
        self._dtype = dtype
        # run the decode LoRA projections on a second stream beside R/K/V
        self.lora_side_stream = False
        # decode: LoRA up projections inside the wkv kernel (when the shapes allow)
        self.fused_lora_decode = True
        # decode: LayerNorm + token-shift mixes inside the R/K/V and FFN-key GEMVs
        self.fused_mix_decode = True
        # decode, 2..8 rows: LN + mixes + LoRA down in one launch (off: at the
        # 7.2B widths it measured slower than the mix kernel + the LoRA-down launch)
        self.fused_mix_lora_decode = False
        # 3..16 rows: the FFN value's split-K partials are added by the next
        # layer's norm-mix kernel instead of a reduce launch of their own
        self.defer_value_reduce = True
        # up to 64 rows (without the LN-mix prologue): the LoRA down projections
        # run as tail workgroups of the R/K/V launch instead of a launch of their own
        self.rkv_lora_tail = True
        # recurrent-state dtype of the caches this model creates: fp32, or fp16
        # for the opt-in fp16-state lane (a cache's own state dtype picks the
        # route, so either kind of cache runs on either setting)
        self.state_dtype = native_graph_state_dtype(dtype)
        self._replaced = 0
        self.layers = []

    def _finish_init(self):
        self._rwkv7_native_mm_quantization = "mm8" if self._replaced else None
        self._rwkv7_native_mm_replaced_modules = self._replaced
        self._graph_runners: dict[int, "NativeGraphRunner"] = {}

    def __init__(self, config: NativeRWKV7Config, weights: dict[str, torch.Tensor] | None = None, *,
                 device="cuda", dtype=torch.float16, prepacked: dict | None = None):
        """``weights``: HF-named parameters (see :func:`parameter_shapes`);
        None gives the seeded random init (as ``cls(config)`` does for the
        reference).  ``prepacked``: module name -> :class:`MM8Linear` built
        from a prepacked checkpoint; those modules' ``.weight`` entries are not
        read."""
        if weights is None:
            weights = _LazyWeights(config, 0, device, dtype)
        self._init_common(config, device, dtype)
        cfg = config
        dev = self.device

        def get(name):
            return weights[name].to(device=dev, dtype=dtype).contiguous()

        def linear(name):
            if prepacked is not None and name in prepacked:
                self._replaced += 1
                return QuantLinear(prepacked[name])
            w = get(name + ".weight")
            if cfg.use_native_mm8 and should_quantize_linear(name, int(w.numel()),
                                                             min_params=cfg.native_mm8_min_params,
                                                             policy=cfg.native_mm8_policy):
                lin = torch.nn.Linear(int(w.shape[1]), int(w.shape[0]), bias=False, device=dev, dtype=dtype)
                with torch.no_grad():
                    lin.weight.copy_(w)
                q = QuantLinear(MM8Linear(lin))
                del lin
                self._replaced += 1
                return q
            return DenseLinear(w)

        self.emb = get("model.embeddings.weight")
        for i in range(cfg.num_hidden_layers):
            p = f"model.layers.{i}."
            L = _Layer()
            L.idx = i
            L.pre = (get(p + "pre_norm.weight"), get(p + "pre_norm.bias")) if i == 0 else None
            L.ln1 = (get(p + "attn_norm.weight"), get(p + "attn_norm.bias"))
            L.ln2 = (get(p + "ffn_norm.weight"), get(p + "ffn_norm.bias"))
            L.mix = [get(p + "attn." + m).reshape(-1) for m in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g")]
            L.k_k = get(p + "attn.k_k")
            L.k_a = get(p + "attn.k_a")
            L.r_k = get(p + "attn.r_k")
            L.r_proj, L.k_proj, L.v_proj = (linear(p + f"attn.{n}") for n in ("r_proj", "k_proj", "v_proj"))
            L.o_proj = linear(p + "attn.o_proj")
            L.lora_down = []
            L.lora_up = []
            L.lora_bias = []
            names = ["w_lora", "a_lora", "g_lora"] + (["v_lora"] if i > 0 else [])
            for n in names:
                L.lora_down.append(get(p + f"attn.{n}.lora.0.weight"))
                L.lora_up.append(get(p + f"attn.{n}.lora.2.weight"))
                bname = p + f"attn.{n}.lora.2.bias"
                L.lora_bias.append(get(bname) if bname in weights else None)
            L.gn = (get(p + "attn.g_norm.weight"), get(p + "attn.g_norm.bias"))
            L.fx_k = get(p + "ffn.x_k").reshape(-1)
            L.key = linear(p + "ffn.key")
            L.value = linear(p + "ffn.value")
            self.layers.append(L)
        self.norm = (get("model.norm.weight"), get("model.norm.bias"))
        self.lm_head = linear("lm_head")
        self._finish_init()

    # ------------------------------------------------------------- packs
    def extract_graph_packs(self):
        """The per-layer 41-entry operand tuples of the reference's graph route
        (rwkv7_hf/native_jit_packing.py:57-143), in its order:
        ``(i, H, N, eps, has_pre, pre_w, pre_b, an_w, an_b, fn_w, fn_b, x_r, x_w,
        x_k, x_v, x_a, x_g, k_k, k_a, r_k, Rw, Kw, Vw, Ow, w1, w2, w0, a1, a2, a0,
        v1, v2, v0, g1, g2, gn_w, gn_b, fx_k, fK, fV, RKVw)``.  Quantized
        projections stay callables (their ``MM8Linear`` modules), dense ones are
        ``[out, in]`` weights; layer 0's missing V LoRA and pre-norm are zeros of
        the reference's shapes, and the stacked-RKV slot is empty.  Returns
        ``(packs, H, N, eps)``; the tensors are the model's own (no copies)."""
        cfg = self.config
        H, N, D, A = cfg.num_heads, cfg.head_dim, cfg.hidden_size, cfg.attention_hidden_size
        eps = float(N * 1e-5)
        dev, dt = self.device, self.dtype
        op = lambda lin: lin.m if isinstance(lin, QuantLinear) else lin.weight
        packs = []
        for L in self.layers:
            has_pre = 1 if L.pre is not None else 0
            pre_w, pre_b = L.pre if has_pre else (torch.zeros(D, device=dev, dtype=dt),) * 2
            lo = {n: q for q, n in enumerate(("w", "a", "g", "v")[:len(L.lora_down)])}
            if "v" in lo:
                v1, v2, v0 = L.lora_down[3], L.lora_up[3], L.lora_bias[3]
            else:
                v1 = torch.zeros(1, D, device=dev, dtype=dt)
                v2 = torch.zeros(A, 1, device=dev, dtype=dt)
                v0 = torch.zeros(A, device=dev, dtype=dt)
            packs.append((
                L.idx, H, N, eps, has_pre, pre_w, pre_b, L.ln1[0], L.ln1[1], L.ln2[0], L.ln2[1],
                *L.mix, L.k_k, L.k_a, L.r_k,
                op(L.r_proj), op(L.k_proj), op(L.v_proj), op(L.o_proj),
                L.lora_down[0], L.lora_up[0], L.lora_bias[0],
                L.lora_down[1], L.lora_up[1], L.lora_bias[1],
                v1, v2, v0,
                L.lora_down[2], L.lora_up[2],
                L.gn[0], L.gn[1], L.fx_k, op(L.key), op(L.value),
                self.emb.new_empty((0,)),
            ))
        return packs, H, N, eps

    @classmethod
    def from_graph_packs(cls, config: NativeRWKV7Config, packs, *, embeddings, norm_weight, norm_bias, lm_head,
                         device="cuda", dtype=torch.float16):
        """A model over operands in the reference's 41-entry pack layout (see
        :meth:`extract_graph_packs`): the tensors are used as given (no copies
        when they already have the device and dtype); a projection is an
        ``MM8Linear`` module (fused MM8 route) or an ``[out, in]`` weight."""
        if len(packs) != config.num_hidden_layers:
            raise ValueError(f"{len(packs)} packs for {config.num_hidden_layers} layers")
        self = cls.__new__(cls)
        self._init_common(config, device, dtype)
        dev = self.device
        t = lambda x: None if x is None else x.to(device=dev, dtype=dtype).contiguous()

        def lin(x):
            if isinstance(x, MM8Linear):
                self._replaced += 1
                return QuantLinear(x)
            if isinstance(x, torch.Tensor):
                return DenseLinear(t(x))
            raise TypeError(f"pack projection must be an MM8Linear or a weight tensor, got {type(x)!r}")

        for pk in packs:
            if len(pk) != 41:
                raise ValueError(f"graph packs have 41 entries, got {len(pk)}")
            (i, H, N, eps, has_pre, pre_w, pre_b, an_w, an_b, fn_w, fn_b, x_r, x_w, x_k, x_v, x_a, x_g, k_k, k_a,
             r_k, Rw, Kw, Vw, Ow, w1, w2, w0, a1, a2, a0, v1, v2, v0, g1, g2, gn_w, gn_b, fx_k, fK, fV, _rkv) = pk
            if int(H) != config.num_heads or int(N) != config.head_dim:
                raise ValueError("pack head shape does not match the config")
            L = _Layer()
            L.idx = int(i)
            L.pre = (t(pre_w), t(pre_b)) if has_pre else None
            L.ln1, L.ln2 = (t(an_w), t(an_b)), (t(fn_w), t(fn_b))
            L.mix = [t(m).reshape(-1) for m in (x_r, x_w, x_k, x_v, x_a, x_g)]
            L.k_k, L.k_a, L.r_k = t(k_k), t(k_a), t(r_k)
            L.r_proj, L.k_proj, L.v_proj, L.o_proj = lin(Rw), lin(Kw), lin(Vw), lin(Ow)
            L.lora_down, L.lora_up, L.lora_bias = [t(w1), t(a1), t(g1)], [t(w2), t(a2), t(g2)], [t(w0), t(a0), None]
            if L.idx > 0:  # layer 0 carries zero placeholders for the V LoRA
                L.lora_down.append(t(v1))
                L.lora_up.append(t(v2))
                L.lora_bias.append(t(v0))
            L.gn = (t(gn_w), t(gn_b))
            L.fx_k = t(fx_k).reshape(-1)
            L.key, L.value = lin(fK), lin(fV)
            self.layers.append(L)
        self.emb = t(embeddings)
        self.norm = (t(norm_weight), t(norm_bias))
        self.lm_head = lin(lm_head)
        self._finish_init()
        return self

    # ------------------------------------------------------------- helpers
    @classmethod
    def from_random(cls, config: NativeRWKV7Config, *, seed: int = 0, device="cuda", dtype=torch.float16):
        """Random-init model; weights are generated one tensor at a time on ``device``."""
        return cls(config, _LazyWeights(config, seed, device, dtype), device=device, dtype=dtype)

    def new_cache(self, batch: int) -> NativeRWKV7Cache:
        return NativeRWKV7Cache.zeros(self.config, batch, self.device, self.dtype, state_dtype=self.state_dtype)

    def reserve_workspace(self, rows: int) -> None:
        """Grow the per-device scratch slots for ``rows``-row steps (before capture)."""
        if 0 < rows <= QuantLinear.GEMV_ROWS:
            tneed = 0
            for L in self.layers:
                if isinstance(L.r_proj, QuantLinear):
                    tneed = max(tneed, mm8t_workspace_bytes(3, rows, L.r_proj.in_features, L.r_proj.out_features))
            for lin in self._linears():
                if isinstance(lin, QuantLinear):
                    tneed = max(tneed, mm8t_workspace_bytes(1, rows, lin.in_features, lin.out_features))
            if tneed:
                _ws.reserve(self.device, tneed, slot="mm8t")
        if QuantLinear.GEMV_ROWS < rows <= QuantLinear.GEMM_ROWS:
            gneed = 0
            for L in self.layers:
                gneed = max(gneed, mm8_gemm_workspace_bytes(3, rows, L.r_proj.in_features, L.r_proj.out_features))
            for lin in self._linears():
                if isinstance(lin, QuantLinear):
                    gneed = max(gneed, mm8_gemm_workspace_bytes(1, rows, lin.in_features, lin.out_features))
            if gneed:
                _ws.reserve(self.device, gneed, slot="mm8g")
        if rows > QuantLinear.GEMM_ROWS:  # prefill: the fp16 dequantised weights of the widest launch
            pneed = 0
            for L in self.layers:
                if isinstance(L.r_proj, QuantLinear):
                    pneed = max(pneed, mm8_prefill_workspace_bytes(3, L.r_proj.in_features, L.r_proj.out_features))
            for lin in self._linears():
                if isinstance(lin, QuantLinear) or (isinstance(lin, DenseLinear) and lin.weight.dtype != torch.float32):
                    pneed = max(pneed, mm8_prefill_workspace_bytes(1, lin.in_features, lin.out_features))
            if pneed:
                _ws.reserve(self.device, pneed, slot="mm8p")
        cfg = self.config
        ranks = [cfg.decay_low_rank_dim, cfg.a_low_rank_dim, cfg.gate_low_rank_dim, cfg.v_low_rank_dim]
        _ws.reserve(self.device, lora_workspace_bytes(ranks, rows, cfg.hidden_size), slot="lora")

    def named_linears(self):
        """(HF module name, linear) for every projection and the head."""
        for L in self.layers:
            p = f"model.layers.{L.idx}."
            yield from ((p + "attn.r_proj", L.r_proj), (p + "attn.k_proj", L.k_proj), (p + "attn.v_proj", L.v_proj),
                        (p + "attn.o_proj", L.o_proj), (p + "ffn.key", L.key), (p + "ffn.value", L.value))
        yield "lm_head", self.lm_head

    def dense_state_dict(self) -> dict:
        """HF-named tensors of every parameter the model holds unquantised
        (the dense linears' ``.weight`` included, the MM8 modules' excluded)."""
        sd = {"model.embeddings.weight": self.emb, "model.norm.weight": self.norm[0], "model.norm.bias": self.norm[1]}
        for L in self.layers:
            p = f"model.layers.{L.idx}."
            if L.pre is not None:
                sd[p + "pre_norm.weight"], sd[p + "pre_norm.bias"] = L.pre
            sd[p + "attn_norm.weight"], sd[p + "attn_norm.bias"] = L.ln1
            sd[p + "ffn_norm.weight"], sd[p + "ffn_norm.bias"] = L.ln2
            D = self.config.hidden_size
            for m, v in zip(("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"), L.mix):
                sd[p + "attn." + m] = v.reshape(1, 1, D)
            sd[p + "attn.k_k"], sd[p + "attn.k_a"], sd[p + "attn.r_k"] = L.k_k, L.k_a, L.r_k
            names = ["w_lora", "a_lora", "g_lora", "v_lora"][:len(L.lora_down)]
            for n, d, u, b in zip(names, L.lora_down, L.lora_up, L.lora_bias):
                sd[p + f"attn.{n}.lora.0.weight"] = d
                sd[p + f"attn.{n}.lora.2.weight"] = u
                if b is not None:
                    sd[p + f"attn.{n}.lora.2.bias"] = b
            sd[p + "attn.g_norm.weight"], sd[p + "attn.g_norm.bias"] = L.gn
            sd[p + "ffn.x_k"] = L.fx_k
        for name, lin in self.named_linears():
            if isinstance(lin, DenseLinear):
                sd[name + ".weight"] = lin.weight
        return sd

    def _linears(self):
        for L in self.layers:
            yield from (L.r_proj, L.k_proj, L.v_proj, L.o_proj, L.key, L.value)
        yield self.lm_head

    def _lora(self, L, xw, xa, xg, xv, rows, outs, mids):
        """W, A (sigmoid applied), G, V-gate projections on the LoRA HIP kernels
        (split-K pair up to 256 rows, the fused many-row kernel above)."""
        n = len(L.lora_down)
        xin = [xw, xa, xg, xv][:n]
        acts_down = [ACT_TANH, ACT_NONE, ACT_SIGMOID, ACT_NONE][:n]
        acts_up = [ACT_NONE, ACT_SIGMOID, ACT_NONE, ACT_SIGMOID][:n]
        lora_multi(xin, L.lora_down, L.lora_up, L.lora_bias, outs[:n], acts_down, acts_up)

    # ------------------------------------------------------------- decode
    def _decode_buffers(self, B):
        cfg = self.config
        dev, dt = self.device, self.dtype
        D, A = cfg.hidden_size, cfg.attention_hidden_size
        ranks = [cfg.decay_low_rank_dim, cfg.a_low_rank_dim, cfg.gate_low_rank_dim, cfg.v_low_rank_dim]
        return {
            "x": torch.empty(B, D, device=dev, dtype=dt),
            "mix": torch.empty(6, B, D, device=dev, dtype=dt),
            "rkv": torch.empty(3, B, A, device=dev, dtype=dt),
            "lora": torch.empty(4, B, A, device=dev, dtype=dt),
            "mids": [torch.empty(B, r, device=dev, dtype=dt) for r in ranks],
            "prep": torch.empty(B, A, device=dev, dtype=dt),
            "fk": torch.empty(B, D, device=dev, dtype=dt),
            "kf": torch.empty(B, cfg.intermediate_size, device=dev, dtype=dt),
            "h": torch.empty(B, D, device=dev, dtype=dt),
            # this step's LayerNorm rows (the next token's shift inputs) on the fused-mix route
            "hatt": torch.empty(cfg.num_hidden_layers, B, D, device=dev, dtype=dt),
            "hffn": torch.empty(cfg.num_hidden_layers, B, D, device=dev, dtype=dt),
            # the decode LoRA's down projections summed over K (fused-mix route)
            "ldown": torch.empty(B * sum(ranks), device=dev, dtype=torch.float32),
            "ldown_tail": torch.empty(self._rkv_lora_splits(B) * B * sum(ranks), device=dev, dtype=torch.float32),
            # 2..8 rows: the fused attention-side launch's LoRA-down K-chunk sums
            "lpart": torch.empty(4 * B * sum(ranks), device=dev, dtype=torch.float32),
        }

    # K ranges of the LoRA down projections run in the R/K/V launch's tail (the
    # fused wkv kernel adds them): measured best at 8 up to 16 rows, 4 above
    RKV_LORA_SPLITS = 8
    RKV_LORA_SPLITS_MANY = 4

    def _rkv_lora_splits(self, B: int) -> int:
        return self.RKV_LORA_SPLITS if B <= GEMV_ROWS else self.RKV_LORA_SPLITS_MANY

    def _rkv_lora_fusable(self, L, B: int) -> bool:
        """Up to 64 rows: the LoRA down projections can run as tail workgroups
        of the grouped R/K/V launch (the GEMV up to 16 rows, the tile GEMM
        above; blocked MM8 of one shape, LoRA inputs in the activation dtype
        and of the model width)."""
        if not self.rkv_lora_tail or not 1 <= B <= 64:
            return False
        lins = (L.r_proj, L.k_proj, L.v_proj)
        if not all(isinstance(l, QuantLinear) and is_blocked(l.m.w_blk) for l in lins):
            return False
        if len({(l.in_features, l.out_features) for l in lins}) != 1:
            return False
        D = lins[0].in_features
        return all(d.dtype == self.dtype and d.dim() == 2 and int(d.shape[1]) == D and d.is_contiguous()
                   and int(d.shape[0]) <= 256 for d in L.lora_down)

    def _mix_fusable(self, B) -> bool:
        """True when every layer's R/K/V and FFN-key products can take the LN-mix prologue."""
        # one row: measured faster than the separate mix kernels; at two rows the
        # eight-wave prologue launch is slower than them
        if (not self.fused_mix_decode or B != 1 or self.config.hidden_size > 4096
                or self.dtype not in (torch.float16, torch.bfloat16)):
            return False
        for L in self.layers:
            for lin in (L.r_proj, L.k_proj, L.v_proj, L.key):
                if (not isinstance(lin, QuantLinear) or not is_blocked(lin.m.w_blk) or lin.m.bias is not None
                        or lin.m.mx.dtype != self.dtype):
                    return False
            if len({(l.in_features, l.out_features) for l in (L.r_proj, L.k_proj, L.v_proj)}) != 1:
                return False
        return True

    def decode_step_(self, tokens: torch.Tensor, cache: NativeRWKV7Cache, logits: torch.Tensor, bufs=None):
        """One token per row, cache updated in place; writes ``logits [B, V]``.

        No host synchronisation and no allocation when ``bufs`` is given, so the
        whole step can be captured in a hipGraph.
        """
        cfg = self.config
        B = int(tokens.shape[0])
        if bufs is None:
            bufs = self._decode_buffers(B)
        state, xpa, xpf, v_first = cache
        # an fp16 state runs the fp16-state kernels (with or without the LoRA
        # up projections inside), which also advance the dither phase
        f16 = state[0].dtype == torch.float16
        el16 = cache.fp16_elapsed if f16 else None
        last_i = len(self.layers) - 1
        if self._mix_lora_route(B):
            return self._decode_mix_lora_(tokens, cache, logits, bufs)
        x = bufs["x"]
        torch.index_select(self.emb, 0, tokens, out=x)
        H, N, eps = cfg.num_heads, cfg.head_dim, cfg.norm_eps
        mixb, rkv, lora, prep = bufs["mix"], bufs["rkv"], bufs["lora"], bufs["prep"]
        main = torch.cuda.current_stream(x.device)
        side, ev_in, ev_out = self._side(x.device) if self.lora_side_stream else (None, None, None)
        fmix = self._mix_fusable(B) and not self.lora_side_stream
        parts = None  # the previous layer's FFN value partials, not yet added to x
        for L in self.layers:
            i = L.idx
            xr, xw, xk, xv, xa, xg = (mixb[q] for q in range(6))
            n = len(L.lora_down)
            if fmix:
                # LN + the six mixes inside the R/K/V GEMV: r/k/v mixes feed the
                # products, w/a/g/v are written out for the LoRA kernels
                if L.pre is not None:
                    layer_norm(x, L.pre[0], L.pre[1], eps, out=x)
                aux = [L.mix[1], L.mix[4], L.mix[5], L.mix[3]][:n]
                flora = self.fused_lora_decode and fused_lora_decode_supported(
                    [int(d.shape[0]) for d in L.lora_down], B)
                mm8_lnmix_multi_into(x, xpa[i], L.ln1[0], L.ln1[1], eps, [L.mix[0], L.mix[2], L.mix[3]],
                                     [L.r_proj.m, L.k_proj.m, L.v_proj.m], [rkv[0], rkv[1], rkv[2]],
                                     h_out=bufs["hatt"][i], aux_mixes=aux, aux_outs=[xw, xa, xg, xv][:n],
                                     lora_downs=L.lora_down if flora else None,
                                     lora_out=bufs["ldown"] if flora else None)
            else:
                fused_attn_norm_mix6_decode(x, xpa[i], L.ln1[0], L.ln1[1], *L.mix, eps=eps, out=mixb,
                                            pre_norm_weight=L.pre[0] if L.pre else None,
                                            pre_norm_bias=L.pre[1] if L.pre else None, residual_parts=parts)
                parts = None
            if (self.fused_lora_decode and not self.lora_side_stream
                    and fused_lora_decode_supported([int(d.shape[0]) for d in L.lora_down], B)):
                # LoRA down (its own split-K launch, or tail workgroups of the
                # R/K/V launch), then the up projections inside the wkv kernel
                down_sums, down_splits = (bufs["ldown"], 1) if fmix else (None, 1)
                if not fmix:
                    if self._rkv_lora_fusable(L, B):
                        down_sums, down_splits = bufs["ldown_tail"], self._rkv_lora_splits(B)
                        mm8_matmul_multi_lora_into([xr, xk, xv], [L.r_proj.m, L.k_proj.m, L.v_proj.m],
                                                   [rkv[0], rkv[1], rkv[2]], [xw, xa, xg, xv][:n], L.lora_down,
                                                   down_sums, splits=down_splits)
                    else:
                        QuantLinear.apply_group((L.r_proj, L.k_proj, L.v_proj), (xr, xk, xv),
                                                (rkv[0], rkv[1], rkv[2]))
                fused_wavg_lora_output_prepare_raw(
                    rkv[0], rkv[1], rkv[2], [xw, xa, xg, xv][:n], L.lora_down, L.lora_up, L.lora_bias, state[i],
                    L.k_k, L.k_a, L.r_k, L.gn[0], L.gn[1], eps=N * 1e-5, out=prep, state_out=state[i],
                    v_first=v_first, v_mode=1 if i == 0 else 2, down_sums=down_sums, down_splits=down_splits,
                    elapsed=el16, advance_elapsed=f16 and i == last_i)
            else:
                if self.lora_side_stream:
                    # the LoRA projections depend only on the mixes: a second stream
                    # (a parallel branch of the captured graph) runs them beside R/K/V
                    ev_in.record(main)
                    side.wait_event(ev_in)
                    with torch.cuda.stream(side):
                        self._lora(L, xw, xa, xg, xv, B, [lora[q] for q in range(4)], bufs["mids"])
                        ev_out.record(side)
                    QuantLinear.apply_group((L.r_proj, L.k_proj, L.v_proj), (xr, xk, xv), (rkv[0], rkv[1], rkv[2]))
                    main.wait_event(ev_out)
                else:
                    if not fmix:
                        QuantLinear.apply_group((L.r_proj, L.k_proj, L.v_proj), (xr, xk, xv),
                                                (rkv[0], rkv[1], rkv[2]))
                    self._lora(L, xw, xa, xg, xv, B, [lora[q] for q in range(4)], bufs["mids"])
                if f16:
                    self._fp16_recurrence(L, rkv, lora, state[i], v_first, prep, el16, last=i == last_i)
                else:
                    fused_recurrent_output_prepare_raw(
                        rkv[0], lora[0], rkv[1], rkv[2], lora[1], state[i], lora[2], L.k_k, L.k_a, L.r_k, L.gn[0],
                        L.gn[1], eps=N * 1e-5, state_out=state[i], out=prep.view(B, H, N),
                        v_first=v_first, v_gate=lora[3] if i > 0 else None, v_mode=1 if i == 0 else 2)
            L.o_proj.apply(prep, x, residual=x)
            if fmix:
                mm8_lnmix_multi_into(x, xpf[i], L.ln2[0], L.ln2[1], eps, [L.fx_k], [L.key.m], [bufs["kf"]],
                                     epilogues=[_lib.EPI_RELU2], h_out=bufs["hffn"][i])
            else:
                fused_ffn_add_norm_mix_decode(x, None, xpf[i], L.ln2[0], L.ln2[1], L.fx_k, eps=eps,
                                              mixed=bufs["fk"])
                L.key.apply(bufs["fk"], bufs["kf"], act=3)
            if not fmix and self._value_deferrable(L, B):
                parts, _ = mm8_matmul_partials(bufs["kf"], L.value.m)
            else:
                L.value.apply(bufs["kf"], x, residual=x)
        if fmix:
            # the kernels read the shift inputs while writing this step's rows, so
            # the rows go to separate buffers and replace the cache's here
            torch._foreach_copy_(list(xpa) + list(xpf), list(bufs["hatt"].unbind(0)) + list(bufs["hffn"].unbind(0)))
        layer_norm(x, self.norm[0], self.norm[1], eps, out=bufs["h"])
        self.lm_head.apply(bufs["h"], logits)
        return logits

    def _fp16_recurrence(self, L, rkv, lora, state_l, v_first, prep, elapsed, *, last: bool) -> None:
        """One decode layer's recurrence on an fp16 state: the fp16-state kernel
        on the raw projections (rwkv7_hf/native_jit_decode.py:767-784), with the
        V interpolation v + (v_first - v) * v_gate (:762-766) formed in-kernel in
        the reference's fp16 roundings; it advances elapsed on the last layer."""
        cfg = self.config
        H, N = cfg.num_heads, cfg.head_dim
        B = int(rkv.shape[1])
        bhn = lambda t: t.view(B, H, N)
        native_fp16_recurrent_output_prepare_raw(
            bhn(rkv[0]), bhn(lora[0]), bhn(rkv[1]), bhn(rkv[2]), bhn(lora[1]), state_l, bhn(lora[2]), L.k_k,
            L.k_a, L.r_k, L.gn[0], L.gn[1], elapsed, advance_elapsed=last, eps=N * 1e-5, out=bhn(prep),
            v_first=v_first, v_gate=lora[3] if L.idx > 0 else None, v_mode=1 if L.idx == 0 else 2)

    def _value_deferrable(self, L, B) -> bool:
        """The FFN value's split reduce can move into the next layer's norm-mix
        launch: a next layer without a pre-norm, a blocked bias-free MM8 value
        that splits K at these rows into at most four ranges."""
        if not self.defer_value_reduce or L.idx + 1 >= len(self.layers) or self.layers[L.idx + 1].pre is not None:
            return False
        v = L.value
        if (not isinstance(v, QuantLinear) or not 0 < B <= QuantLinear.GEMV_ROWS or not is_blocked(v.m.w_blk)
                or v.m.bias is not None):
            return False
        need = mm8t_workspace_bytes(1, B, v.in_features, v.out_features)
        return 0 < need <= 4 * B * v.out_features * 4

    def _mix_lora_route(self, B) -> bool:
        """2..8 fp16/bf16 rows with fusable LoRA ranks: each layer's attention
        side starts with one launch (LN + r/k/v mixes + LoRA down, MFMA)."""
        cfg = self.config
        if not (2 <= B <= 8 and self.fused_lora_decode and self.fused_mix_lora_decode and not self.lora_side_stream
                and not self._mix_fusable(B) and self.dtype in (torch.float16, torch.bfloat16)
                and attn_mix_lora_chunks(cfg.hidden_size)):
            return False
        return all(fused_lora_decode_supported([int(d.shape[0]) for d in L.lora_down], B)
                   and all(d.dtype == self.dtype for d in L.lora_down) and L.mix[0].dtype == L.ln1[0].dtype
                   for L in self.layers)

    def _decode_mix_lora_(self, tokens, cache, logits, bufs):
        """decode_step_ for 2..8 rows: per layer one launch of
        attn_mix_lora_decode (LayerNorm, r/k/v mixes, the LoRA down projections
        as K-chunk sums), the R/K/V GEMV, the wkv kernel with the LoRA up
        projections, o_proj, the FFN mix, key and value."""
        cfg = self.config
        B = int(tokens.shape[0])
        N, eps = cfg.head_dim, cfg.norm_eps
        x = bufs["x"]
        torch.index_select(self.emb, 0, tokens, out=x)
        state, xpa, xpf, v_first = cache
        f16 = state[0].dtype == torch.float16
        el16 = cache.fp16_elapsed if f16 else None
        mixb, rkv, prep = bufs["mix"], bufs["rkv"], bufs["prep"]
        for L in self.layers:
            i = L.idx
            n = len(L.lora_down)
            xr, xw, xk, xv, xa, xg = (mixb[q] for q in range(6))
            if L.pre is not None:
                # the pre-normed row goes to a second buffer, then back into x
                splits = attn_mix_lora_decode(x, xpa[i], L.ln1[0], L.ln1[1], L.mix, (xr, xk, xv), L.lora_down,
                                              [1, 4, 5, 3][:n], bufs["lpart"], h_out=bufs["hatt"][i],
                                              x_out=bufs["h"], pre_norm_weight=L.pre[0], pre_norm_bias=L.pre[1],
                                              eps=eps)
                x.copy_(bufs["h"])
            else:
                splits = attn_mix_lora_decode(x, xpa[i], L.ln1[0], L.ln1[1], L.mix, (xr, xk, xv), L.lora_down,
                                              [1, 4, 5, 3][:n], bufs["lpart"], h_out=bufs["hatt"][i], eps=eps)
            QuantLinear.apply_group((L.r_proj, L.k_proj, L.v_proj), (xr, xk, xv), (rkv[0], rkv[1], rkv[2]))
            fused_wavg_lora_output_prepare_raw(
                rkv[0], rkv[1], rkv[2], [xw, xa, xg, xv][:n], L.lora_down, L.lora_up, L.lora_bias, state[i],
                L.k_k, L.k_a, L.r_k, L.gn[0], L.gn[1], eps=N * 1e-5, out=prep, state_out=state[i],
                v_first=v_first, v_mode=1 if i == 0 else 2, down_sums=bufs["lpart"], down_splits=splits,
                elapsed=el16, advance_elapsed=f16 and i == len(self.layers) - 1)
            L.o_proj.apply(prep, x, residual=x)
            fused_ffn_add_norm_mix_decode(x, None, xpf[i], L.ln2[0], L.ln2[1], L.fx_k, eps=eps, mixed=bufs["fk"])
            L.key.apply(bufs["fk"], bufs["kf"], act=3)
            L.value.apply(bufs["kf"], x, residual=x)
        # the fused launch reads the shift rows while writing this step's, so
        # they go to a separate buffer and replace the cache's here
        torch._foreach_copy_(list(xpa), list(bufs["hatt"].unbind(0)))
        layer_norm(x, self.norm[0], self.norm[1], eps, out=bufs["h"])
        self.lm_head.apply(bufs["h"], logits)
        return logits

    def _side(self, device):
        """Second stream (default priority) and its two fork/join events, per device."""
        key = torch.device(device).index
        if not hasattr(self, "_side_streams"):
            self._side_streams = {}
        if key not in self._side_streams:
            self._side_streams[key] = (torch.cuda.Stream(device=device), torch.cuda.Event(), torch.cuda.Event())
        return self._side_streams[key]

    # ------------------------------------------------------------- prefill
    def prefill_(self, input_ids: torch.Tensor | None, cache: NativeRWKV7Cache, *, logits_to_keep: int = 1,
                 inputs_embeds: torch.Tensor | None = None) -> torch.Tensor:
        """Run ``input_ids [B, T]`` (or ``inputs_embeds [B, T, D]``) through every
        layer (chunked scan), update the cache in place, and return the logits of
        the last ``logits_to_keep`` tokens ``[B, keep, V]`` (all T for
        ``logits_to_keep <= 0``), as the reference's prefill tail
        (rwkv7_hf/native_jit_prefill.py:1024-1036)."""
        cfg = self.config
        dev, dt = self.device, self.dtype
        D, A, H, N, F, eps = (cfg.hidden_size, cfg.attention_hidden_size, cfg.num_heads, cfg.head_dim,
                              cfg.intermediate_size, cfg.norm_eps)
        if inputs_embeds is not None:
            B, T = (int(s) for s in inputs_embeds.shape[:2])
            x = inputs_embeds.to(device=dev, dtype=dt).contiguous().clone()
        else:
            B, T = (int(s) for s in input_ids.shape)
            x = torch.nn.functional.embedding(input_ids.reshape(-1), self.emb).reshape(B, T, D).contiguous()
        R = B * T
        state, xpa, xpf, v_first = cache
        f16 = state[0].dtype == torch.float16
        mixb = torch.empty(6, B, T, D, device=dev, dtype=dt)
        rkv = torch.empty(3, R, A, device=dev, dtype=dt)
        lora = torch.empty(4, R, A, device=dev, dtype=dt)
        ranks = [cfg.decay_low_rank_dim, cfg.a_low_rank_dim, cfg.gate_low_rank_dim, cfg.v_low_rank_dim]
        mids = [torch.empty(R, r, device=dev, dtype=dt) for r in ranks]
        vfirst_seq = torch.empty(R, A, device=dev, dtype=dt)
        kf = torch.empty(R, F, device=dev, dtype=dt)
        for L in self.layers:
            i = L.idx
            if L.pre is not None:
                x = layer_norm(x, L.pre[0], L.pre[1], eps)
            *mixes, new_prev = fused_attn_sequence_shift_mix(x, xpa[i], *L.mix, norm_weight=L.ln1[0],
                                                             norm_bias=L.ln1[1], eps=eps, workspace=mixb)
            xpa[i].copy_(new_prev)
            xr, xw, xk, xv, xa, xg = (m.reshape(R, D) for m in mixes)
            QuantLinear.apply_group((L.r_proj, L.k_proj, L.v_proj), (xr, xk, xv), (rkv[0], rkv[1], rkv[2]))
            self._lora(L, xw, xa, xg, xv, R, [lora[q] for q in range(4)], mids)
            w_log, k_adj, v_int, kk = fused_prefill_state_prep(
                lora[0], rkv[1], rkv[2], lora[1], L.k_k, L.k_a, v_first=vfirst_seq,
                v_gate=lora[3] if i > 0 else None, num_heads=H, head_dim=N, w_transform="log_decay",
                v_mode=1 if i == 0 else 2, v_out=rkv[2])
            shp = (B, T, H, N)
            if f16:
                # the fp16-state sequence recurrence on raw w (w0 already added),
                # -kk and kk*a as the reference forms them (native_jit_prefill.py:792-804)
                kk4 = kk.view(shp)
                y = native_fp16_sequence(rkv[0].view(shp), lora[0].view(shp), k_adj.view(shp), v_int.view(shp),
                                         torch.neg(kk4), kk4 * lora[1].view(shp), state[i], cache.fp16_elapsed)
            else:
                y, _ = _run_chunk(rkv[0].view(shp), w_log.view(shp), k_adj.view(shp), v_int.view(shp),
                                  kk.view(shp), lora[1].view(shp), state[i], w_is_log=1, chunk=16,
                                  state_out=state[i])
            prep = fused_attn_output_prepare(y.view(R, A), rkv[0], k_adj, v_int, lora[2], L.r_k, L.gn[0], L.gn[1],
                                             num_heads=H, head_dim=N, head_v_dim=N, eps=N * 1e-5)
            x2 = x.reshape(R, D)
            L.o_proj.apply(prep, x2, residual=x2)
            fk, new_prev_f = fused_ffn_sequence_shift_mix(x, xpf[i], L.fx_k, norm_weight=L.ln2[0],
                                                          norm_bias=L.ln2[1], eps=eps)
            xpf[i].copy_(new_prev_f)
            L.key.apply(fk.reshape(R, D), kf, act=3)
            L.value.apply(kf, x2, residual=x2)
        v_first.copy_(vfirst_seq.view(B, T, A)[:, -1])
        if f16:
            cache.fp16_elapsed.add_(T)  # the dither phase moves on by the prompt's tokens
        keep = T if logits_to_keep is None or int(logits_to_keep) <= 0 else min(int(logits_to_keep), T)
        h = layer_norm(x[:, T - keep:].reshape(B * keep, D).contiguous(), self.norm[0], self.norm[1], eps)
        logits = torch.empty(B * keep, cfg.vocab_size, device=dev, dtype=dt)
        self.lm_head.apply(h, logits)
        cache.seen_tokens = cache.seen_tokens + T
        cache._invalidate_native_graph_binding()
        if not torch.cuda.is_current_stream_capturing():
            # the chunk kernel's bounded inter-wave waits report a give-up in a
            # sticky status word; an eager prefill raises on it (one device
            # synchronisation per call).  A captured prefill is checked after
            # each replay (NativePrefillGraphRunner.replay).
            check_wkv7_chunk_status()
        return logits.view(B, keep, cfg.vocab_size)

    # ------------------------------------------------------------- API
    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor | None = None, attention_mask=None, inputs_embeds=None,
                past_key_values=None, use_cache: bool | None = None, output_hidden_states: bool | None = None,
                output_attentions: bool | None = None, return_dict: bool | None = None, labels=None,
                logits_to_keep=None, num_logits_to_keep=None, return_legacy_cache: bool | None = None,
                use_graph: bool = True, **kwargs):
        """The reference's ``NativeRWKV7ForCausalLM.forward`` contract
        (rwkv7_hf/native_model.py:618-853) on the native routes only.

        * Prefill (no cache, or a cache plus T > 1 tokens): chunked-scan prefill;
          logits of the last ``logits_to_keep`` tokens (all tokens when it is
          0, or when ``labels`` are given).
        * Decode (a cache and T == 1): the hipGraph-captured step of
          :class:`NativeGraphRunner` (``use_graph=False``: the same step eagerly).
        * ``labels``: shifted cross-entropy over all tokens, ignore index -100,
          no cache input (as the reference).
        * ``attention_mask``: all-ones masks are accepted (equivalent to none);
          a mask that drops tokens is refused with ``ValueError``: the native
          routes do not skip recurrent updates per row.
        * ``output_attentions`` / ``output_hidden_states``: refused (RWKV-7 has
          no attention maps; hidden states are not kept on the native route).

        Returns ``CausalLMOutputWithPast(loss, logits [B, keep, V], past_key_values)``,
        or the tuple form when ``return_dict`` is False.
        """
        if input_ids is not None and inputs_embeds is not None:
            raise ValueError("NativeRWKV7ForCausalLM accepts either input_ids or inputs_embeds, not both")
        if input_ids is None and inputs_embeds is None:
            raise ValueError("NativeRWKV7ForCausalLM requires input_ids or inputs_embeds")
        if input_ids is not None and input_ids.dim() == 1:
            input_ids = input_ids.view(1, -1)
        if input_ids is not None and input_ids.dim() != 2:
            raise ValueError("NativeRWKV7ForCausalLM expects input_ids shaped [batch, seq]")
        if inputs_embeds is not None and (inputs_embeds.dim() != 3
                                          or int(inputs_embeds.shape[-1]) != self.config.hidden_size):
            raise ValueError("NativeRWKV7ForCausalLM expects inputs_embeds shaped [batch, seq, hidden]")
        src = input_ids if input_ids is not None else inputs_embeds
        B, T = int(src.shape[0]), int(src.shape[1])
        if B <= 0 or T <= 0:
            raise ValueError("NativeRWKV7ForCausalLM requires a non-empty batch and sequence")
        if output_attentions:
            raise ValueError("RWKV-7 has no attention weights to output")
        if output_hidden_states:
            raise ValueError("rwkv7mi's native routes do not keep per-layer hidden states")
        cache = _as_native_cache(past_key_values)
        if cache is not None and cache.get_batch_size() not in (None, B):
            raise ValueError(f"NativeRWKV7 cache batch size must match inputs (cache batch="
                             f"{cache.get_batch_size()}, input batch={B})")
        _check_attention_mask(attention_mask, B, T, allow_trailing=cache is not None)
        use_cache = True if use_cache is None else bool(use_cache)
        return_dict = True if return_dict is None else bool(return_dict)
        keep = _resolve_logits_to_keep(logits_to_keep, num_logits_to_keep)
        loss = None
        if labels is not None:
            if labels.dim() == 1:
                labels = labels.view(1, -1)
            if tuple(labels.shape[:2]) != (B, T):
                raise ValueError("NativeRWKV7ForCausalLM labels must have the same shape as inputs")
            if cache is not None:
                raise ValueError("NativeRWKV7ForCausalLM does not support labels with past_key_values")
            keep = 0
        ids = None if input_ids is None else input_ids.to(self.device)
        if cache is not None and T == 1 and ids is not None:
            if use_graph:
                runner = self.graph_runner(B)
                logits = runner.replay(ids[:, 0], cache).clone().unsqueeze(1)
            else:
                self.reserve_workspace(B)
                lg = torch.empty(B, self.config.vocab_size, device=self.device, dtype=self.dtype)
                self.decode_step_(ids[:, 0].contiguous(), cache, lg)
                cache.seen_tokens = cache.seen_tokens + 1
                cache._invalidate_native_graph_binding()
                logits = lg.unsqueeze(1)
        else:
            if cache is None:
                cache = self.new_cache(B)
            elif not cache.is_initialized:
                seen = cache.seen_tokens
                fresh = self.new_cache(B)
                cache._state, cache._xpa, cache._xpf, cache._v_first = fresh._state, fresh._xpa, fresh._xpf, fresh._v_first
                cache.seen_tokens = seen
            else:
                # the prefill updates the state in place; a cache bound to a
                # graph runner keeps its tensors (they are the runner's buffers)
                pass
            logits = self.prefill_(ids, cache, logits_to_keep=1 if keep is None else keep,
                                   inputs_embeds=None if ids is not None else inputs_embeds)
        if loss is None and labels is not None:
            lab = labels.to(logits.device)
            shift_logits = logits[:, :-1].float()
            shift_labels = lab[:, 1:]
            if shift_logits.numel() == 0 or not bool((shift_labels != -100).any()):
                loss = logits.float().sum() * 0.0
            else:
                loss = torch.nn.functional.cross_entropy(shift_logits.reshape(-1, shift_logits.shape[-1]),
                                                         shift_labels.reshape(-1), ignore_index=-100)
        logits = _slice_logits(logits, keep)
        out_cache = cache if use_cache else None
        if out_cache is not None and return_legacy_cache is True:
            out_cache = out_cache.to_legacy_cache()
        if not return_dict:
            return tuple(v for v in (loss, logits, out_cache) if v is not None)
        return _CausalLMOutput(loss=loss, logits=logits, past_key_values=out_cache)

    __call__ = forward

    def prefill_graph_runner(self, batch: int, tokens: int, *, logits_to_keep: int = 1,
                             carry_state: bool = False) -> "NativePrefillGraphRunner":
        """The cached prefill graph for this shape (captured on first use)."""
        key = (int(batch), int(tokens), int(logits_to_keep), bool(carry_state))
        runners = self.__dict__.setdefault("_prefill_graph_runners", {})
        if key not in runners:
            runners[key] = NativePrefillGraphRunner(self, batch, tokens, logits_to_keep=logits_to_keep,
                                                    carry_state=carry_state)
        return runners[key]

    def graph_runner(self, batch: int) -> "NativeGraphRunner":
        r = self._graph_runners.get(batch)
        if r is None:
            r = NativeGraphRunner(self, batch)
            self._graph_runners[batch] = r
        return r

    # ------------------------------------------------ Hugging Face generation contract
    def prepare_inputs_for_generation(self, input_ids, past_key_values=None, inputs_embeds=None,
                                      return_legacy_cache: bool | None = None, **kwargs):
        """GenerationMixin's per-step inputs (rwkv7_hf/model_generation.py:38-97):
        the whole prompt on the first step, then only the last token with the
        recurrent cache (which the decode graph then replays)."""
        cached = _as_native_cache(past_key_values) is not None
        last = (lambda t: t[:, -1:]) if cached else (lambda t: t)
        out: dict = {}
        if inputs_embeds is not None and not cached:
            out["inputs_embeds"] = inputs_embeds
        elif input_ids is not None:
            out["input_ids"] = last(input_ids)
        else:
            out["inputs_embeds"] = last(inputs_embeds)
        use_cache = kwargs.get("use_cache", True)
        out["past_key_values"] = past_key_values
        out["use_cache"] = True if use_cache is None else use_cache
        if return_legacy_cache is not None:
            out["return_legacy_cache"] = return_legacy_cache
        if kwargs.get("attention_mask") is not None:
            out["attention_mask"] = last(kwargs["attention_mask"])
        for k in ("logits_to_keep", "num_logits_to_keep", "output_hidden_states", "output_attentions",
                  "return_dict"):
            if k in kwargs:
                out[k] = kwargs[k]
        return out

    @staticmethod
    def _reorder_cache(past_key_values, beam_idx: torch.LongTensor):
        """Beam reordering of the recurrent cache (rwkv7_hf/model_generation.py:15-35)."""
        cache = _as_native_cache(past_key_values)
        if cache is None:
            return None
        out = cache.reorder_cache(beam_idx)
        return out.to_legacy_cache() if isinstance(past_key_values, tuple) else out

    @classmethod
    def from_pretrained(cls, pretrained_model_name_or_path, *model_args, config=None, device=None,
                        device_map=None, torch_dtype=None, dtype=None, use_native_mm8: bool | None = None,
                        native_mm8_policy: str | None = None, native_mm8_min_params: int | None = None,
                        **kwargs):
        """A model from a converted directory (``config.json`` +
        ``*.safetensors``, or a prepacked MM8 directory with ``manifest.json``),
        as ``AutoModelForCausalLM.from_pretrained`` would give the reference's.
        ``dtype`` / ``torch_dtype``: ``"auto"`` reads ``config.json``;
        default fp16.  ``device`` / a single-device ``device_map``: default
        ``cuda``.  The ``use_native_mm8`` family overrides the config."""
        import json
        from pathlib import Path

        from .converter import load_pretrained

        path = Path(pretrained_model_name_or_path)
        want = dtype if dtype is not None else torch_dtype
        if want is None or want == "auto":
            name = json.loads((path / "config.json").read_text()).get("torch_dtype") if want == "auto" else None
            want = getattr(torch, name) if isinstance(name, str) else torch.float16
        elif isinstance(want, str):
            want = getattr(torch, want)
        if device is None:
            device = device_map if isinstance(device_map, (str, torch.device)) and device_map != "auto" else "cuda"
        if config is not None and use_native_mm8 is None:
            use_native_mm8 = getattr(config, "use_native_mm8", None)
        return load_pretrained(path, device=device, dtype=want, use_native_mm8=use_native_mm8,
                               native_mm8_policy=native_mm8_policy, native_mm8_min_params=native_mm8_min_params)

    def save_pretrained(self, save_directory, **kwargs):
        """Write a directory :meth:`from_pretrained` reads: a prepacked MM8
        directory when any projection is quantised, else ``config.json`` +
        ``model.safetensors``."""
        from .converter import save_hf_directory, save_prepacked

        if self._replaced:
            save_prepacked(self, save_directory)
        else:
            save_hf_directory(save_directory, self.config, self.dense_state_dict(),
                              dtype_name=str(self.dtype).replace("torch.", ""))

    @torch.no_grad()
    def generate_greedy(self, input_ids: torch.Tensor, max_new_tokens: int, *, use_graph: bool = True):
        """Greedy generation without GenerationMixin's per-step host work: the
        decode graph computes each step's argmax and feeds it to its own next
        replay.  Returns ``[B, T + max_new_tokens]``, the ids
        ``generate(input_ids, max_new_tokens=..., do_sample=False)`` gives
        with no end-of-sequence token."""
        B = int(input_ids.shape[0])
        out0 = self.forward(input_ids)
        logits, cache = out0.logits, out0.past_key_values
        nxt = argmax_rows(logits[:, -1])
        out = [input_ids, nxt[:, None]]
        runner = self.graph_runner(B) if use_graph else None
        for t in range(max_new_tokens - 1):
            if runner is not None:
                nxt = runner.replay_greedy(cache, nxt if t == 0 else None).clone()
            else:
                lg = self.forward(nxt[:, None], past_key_values=cache, use_graph=False).logits[:, -1]
                nxt = argmax_rows(lg)
            out.append(nxt[:, None])
        return torch.cat(out, 1)


class _LazyWeights(dict):
    """Generates each random parameter on first access (bounded peak memory)."""

    def __init__(self, cfg, seed, device, dtype):
        super().__init__()
        self._cfg, self._seed, self._device, self._dtype = cfg, seed, device, dtype
        self._shapes = parameter_shapes(cfg)

    def __contains__(self, name):
        return name in self._shapes

    def __getitem__(self, name):
        return random_weights(self._cfg, seed=self._seed, device=self._device, dtype=self._dtype, names=[name])[name]


# ------------------------------------------------------------------ graph runner
class NativeGraphRunner:
    """hipGraph-captured decode step for a fixed batch (rwkv7_hf/native_graph_runtime.py:212-711).

    The runner owns static cache tensors; ``replay`` copies a foreign cache in
    once, then binds it (the cache's tensors become the runner's buffers) so
    later steps run with no copies.  The graph ends with the greedy token of
    every row (``argmax_rows``), written both to ``next_tokens`` and to the
    graph's own input buffer, so :meth:`replay_greedy` runs a greedy step with
    no launch besides the graph.
    """

    def __init__(self, model: NativeRWKV7ForCausalLM, batch: int, *, warmup: int = 2):
        self.model = model
        self.batch = int(batch)
        dev = model.device
        model.reserve_workspace(self.batch)
        self.cache = model.new_cache(self.batch)
        self.tokens = torch.zeros(self.batch, dtype=torch.long, device=dev)
        self.logits = torch.empty(self.batch, model.config.vocab_size, device=dev, dtype=model.dtype)
        self.next_tokens = torch.zeros(self.batch, dtype=torch.long, device=dev)
        self.argmax_ws = torch.empty(argmax_workspace_bytes(self.batch, model.config.vocab_size, model.dtype),
                                     device=dev, dtype=torch.uint8)
        self.bufs = model._decode_buffers(self.batch)
        snapshot = self.cache.clone()
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self._step()
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()
        self._copy_into(snapshot)
        self.replays = 0
        self._bound_cache_ref = None

    def _step(self) -> None:
        """The captured work: one decode step, then the greedy tokens."""
        self.model.decode_step_(self.tokens, self.cache, self.logits, self.bufs)
        argmax_rows(self.logits, out=self.next_tokens, out2=self.tokens, workspace=self.argmax_ws)

    def _copy_into(self, cache: NativeRWKV7Cache) -> None:
        if cache.state_dtype not in (None, self.cache.state_dtype):
            raise ValueError(f"graph runner with a {self.cache.state_dtype} state got a cache with a "
                             f"{cache.state_dtype} state")
        for dst, src in zip(self.cache._all_tensors(), cache._all_tensors()):
            dst.copy_(src)

    def detach_bound_cache(self, keep: NativeRWKV7Cache | None = None) -> None:
        """Give the cache bound to this runner (unless it is ``keep``) its own
        copy of the runner's buffers and unbind it, before anything else
        writes those buffers: another cache's copy-in, or a state pool's
        gather (rwkv7_hf/native_graph_runtime.py:618-630).  The copy keeps the
        layer-major storage of :meth:`NativeRWKV7Cache.zeros`."""
        prev = self._bound_cache_ref() if self._bound_cache_ref is not None else None
        if prev is not None and prev is keep:
            return
        self._bound_cache_ref = None
        if prev is None or not prev._native_graph_bound_to(self):
            return
        s, a, f, v = self.cache
        prev._state = list(torch.stack(s).unbind(0))
        prev._xpa = list(torch.stack(a).unbind(0))
        prev._xpf = list(torch.stack(f).unbind(0))
        prev._v_first = v.clone()
        prev._elapsed = None if self.cache._elapsed is None else self.cache._elapsed.clone()
        prev._invalidate_native_graph_binding()

    def bind_cache(self, cache: NativeRWKV7Cache) -> None:
        """The cache's tensors become this runner's buffers (no copies per
        step).  A different cache bound before keeps its state as a copy."""
        self.detach_bound_cache(keep=cache)
        cache._state, cache._xpa, cache._xpf, cache._v_first = (
            list(self.cache._state), list(self.cache._xpa), list(self.cache._xpf), self.cache._v_first)
        cache._elapsed = self.cache._elapsed
        cache._invalidate_native_graph_binding()
        cache._bind_native_graph_runner(self)
        self._bound_cache_ref = weakref.ref(cache)

    def reorder_batch_inplace(self, indices: torch.Tensor) -> bool:
        """Permute the bound batch rows in place (beam search on a bound cache)."""
        idx = indices.to(device=self.model.device, dtype=torch.long)
        if int(idx.numel()) != self.batch:
            return False
        for t in self.cache._all_tensors():
            t.copy_(t.index_select(0, idx))
        return True

    def replay(self, tokens: torch.Tensor, cache: NativeRWKV7Cache) -> torch.Tensor:
        if cache.get_batch_size() not in (None, self.batch):
            raise ValueError(f"graph runner for batch {self.batch} got a cache of batch {cache.get_batch_size()}")
        if not cache._native_graph_bound_to(self):
            self.detach_bound_cache(keep=cache)
            self._copy_into(cache)
            self.bind_cache(cache)
        self.tokens.copy_(tokens.reshape(-1))
        self.graph.replay()
        self.replays += 1
        cache.seen_tokens = cache.seen_tokens + 1
        return self.logits

    def replay_greedy(self, cache: NativeRWKV7Cache, tokens: torch.Tensor | None = None) -> torch.Tensor:
        """One greedy step: feed ``tokens`` (default: the previous replay's greedy
        tokens, already in the graph's input buffer) and return the next greedy
        tokens ``[B]``, the runner's ``next_tokens`` buffer (clone it to keep
        it past the next replay).  ``self.logits`` holds the step's logits."""
        if tokens is not None:
            return self._greedy_from(tokens, cache)
        if not cache._native_graph_bound_to(self):
            raise ValueError("replay_greedy without tokens continues a cache bound to this runner")
        self.graph.replay()
        self.replays += 1
        cache.seen_tokens = cache.seen_tokens + 1
        return self.next_tokens

    def _greedy_from(self, tokens: torch.Tensor, cache: NativeRWKV7Cache) -> torch.Tensor:
        self.replay(tokens, cache)
        return self.next_tokens


class NativePrefillGraphRunner:
    """hipGraph-captured prefill for one shape ``(B, T, logits_to_keep)``
    (rwkv7_hf/model_prefill_graph.py:38-381): the whole layer stack of
    :meth:`NativeRWKV7ForCausalLM.prefill_` — embedding, mixes, MM8 GEMMs,
    LoRA, state prep, chunked scan, output prep — replays as one graph for
    repeated prompt shapes.

    Static buffers: ``ids [B, T]`` and a layer-major cache; intermediates
    live in the graph's private memory pool.  ``carry_state=False`` starts
    every replay from zeros (the static cache is cleared by fill kernels
    before the replay); ``carry_state=True`` copies ``initial_cache`` in
    first (cache continuation).  ``replay`` returns ``(logits, cache)``: new
    tensors by default (a later replay does not disturb them), or the
    runner's static buffers with ``copy=False``."""

    def __init__(self, model: "NativeRWKV7ForCausalLM", batch: int, tokens: int, *, logits_to_keep: int = 1,
                 carry_state: bool = False, warmup: int = 1):
        self.model = model
        self.batch, self.tokens_n = int(batch), int(tokens)
        self.logits_to_keep = int(logits_to_keep)
        self.carry_state = bool(carry_state)
        dev = model.device
        model.reserve_workspace(min(self.batch * self.tokens_n, 256))
        self.ids = torch.zeros(self.batch, self.tokens_n, dtype=torch.long, device=dev)
        self.cache = model.new_cache(self.batch)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(warmup):  # grows every workspace slot the body uses, before capture
                model.prefill_(self.ids, self.cache, logits_to_keep=self.logits_to_keep)
        torch.cuda.current_stream(dev).wait_stream(side)
        self._zero_state()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = model.prefill_(self.ids, self.cache, logits_to_keep=self.logits_to_keep)
        self.replays = 0

    def _zero_state(self) -> None:
        for t in self.cache._all_tensors():
            t.zero_()

    def matches(self, batch: int, tokens: int, logits_to_keep: int, carry_state: bool) -> bool:
        return (self.batch, self.tokens_n, self.logits_to_keep, self.carry_state) == (
            int(batch), int(tokens), int(logits_to_keep), bool(carry_state))

    def replay(self, input_ids: torch.Tensor, initial_cache: "NativeRWKV7Cache | None" = None, *, copy: bool = True):
        if tuple(input_ids.shape) != (self.batch, self.tokens_n):
            raise ValueError(f"prefill graph for [{self.batch}, {self.tokens_n}] got {tuple(input_ids.shape)}")
        if initial_cache is not None and not self.carry_state:
            raise ValueError("this prefill graph was captured without cache continuation (carry_state=False)")
        seen = 0
        if self.carry_state and initial_cache is not None and initial_cache.is_initialized:
            if initial_cache.get_batch_size() != self.batch:
                raise ValueError("initial cache batch differs from the captured batch")
            if initial_cache.state_dtype != self.cache.state_dtype:
                raise ValueError("initial cache state dtype differs from the captured one")
            for dst, src in zip(self.cache._all_tensors(), initial_cache._all_tensors()):
                dst.copy_(src)
            seen = initial_cache.seen_tokens
        else:
            self._zero_state()
        self.ids.copy_(input_ids)
        self.graph.replay()
        self.replays += 1
        check_wkv7_chunk_status()
        if not copy:
            out = NativeRWKV7Cache(list(self.cache._state), list(self.cache._xpa), list(self.cache._xpf),
                                   self.cache._v_first, seen + self.tokens_n)
            out._elapsed = self.cache._elapsed
            return self.logits, out
        out = self.model.new_cache(self.batch)
        for dst, src in zip(out._all_tensors(), self.cache._all_tensors()):
            dst.copy_(src)
        out.seen_tokens = seen + self.tokens_n
        return self.logits.clone(), out


try:  # AutoConfig / AutoModelForCausalLM resolve model_type "rwkv7_native" to these classes
    from transformers import AutoConfig as _AutoConfig
    from transformers import AutoModelForCausalLM as _AutoModelForCausalLM

    _AutoConfig.register(NativeRWKV7Config.model_type, NativeRWKV7Config, exist_ok=True)
    _AutoModelForCausalLM.register(NativeRWKV7Config, NativeRWKV7ForCausalLM, exist_ok=True)
except Exception:  # pragma: no cover - transformers absent or too old
    pass


__all__ = ["NativeRWKV7Config", "NativeRWKV7Cache", "NativeRWKV7ForCausalLM", "NativeGraphRunner",
           "NativePrefillGraphRunner", "random_weights", "parameter_shapes"]
