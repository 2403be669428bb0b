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
the embedding row gather and, for prefills with more than 64 rows, the dense
library GEMM that follows an MM8 dequantisation (rocBLAS through torch).
"""
from __future__ import annotations

import zlib
from dataclasses import dataclass, field

import torch

from . import _lib
from . import workspace as _ws
from .fused_decode_norm_mix import fused_attn_norm_mix6_decode, fused_ffn_add_norm_mix_decode, layer_norm
from .fused_lora import (ACT_NONE, ACT_SIGMOID, ACT_TANH, dense_multi, fused_lora_decode_supported,
                         fused_wavg_lora_output_prepare_raw, lora_multi, lora_workspace_bytes)
from .fused_output import fused_attn_output_prepare
from .fused_prefill import fused_prefill_state_prep
from .fused_recurrent_update import fused_recurrent_output_prepare_raw
from .fused_time_mix import fused_attn_sequence_shift_mix, fused_ffn_sequence_shift_mix
from .native_quant_mm8 import (GEMM_ROWS, GEMV_ROWS, MM8Linear, is_blocked, mm8_gemm_multi_into, mm8_gemm_workspace_bytes,
                               mm8_lnmix_multi_into, mm8_matmul_multi_into)
from .native_quant_policy import should_quantize_linear
from .self_chunk_rwkv7 import _run_chunk

EXP_HALF = 0.606531


@dataclass
class NativeRWKV7Config:
    """Subset of rwkv7_hf NativeRWKV7Config that shapes the inference path."""

    vocab_size: int = 65536
    hidden_size: int = 768
    num_hidden_layers: int = 12
    head_dim: int = 64
    num_heads: int | None = None
    intermediate_size: int | None = None
    decay_low_rank_dim: int = 64
    a_low_rank_dim: int = 64
    gate_low_rank_dim: int = 128
    v_low_rank_dim: int = 32
    norm_eps: float = 1e-5
    use_native_mm8: bool = False
    native_mm8_min_params: int = 8_000_000
    native_mm8_policy: str = "memory"
    extra: dict = field(default_factory=dict)

    def __post_init__(self):
        if self.num_heads is None:
            self.num_heads = self.hidden_size // self.head_dim
        if self.intermediate_size is None:
            self.intermediate_size = 4 * self.hidden_size
        if self.head_dim != 64:
            raise ValueError("rwkv7mi kernels require head_dim = 64")

    @property
    def attention_hidden_size(self) -> int:
        return self.num_heads * self.head_dim


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
    """fp16/bf16 Linear ``y = x W^T`` on the HIP dense kernel (decode sizes) or a
    library GEMM (long prefills)."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None = None):
        self.weight = weight.contiguous()
        self.bias = None if bias is None else bias.contiguous()
        self.out_features, self.in_features = (int(s) for s in self.weight.shape)

    def apply(self, x2, out, *, act=ACT_NONE, residual=None):
        rows = int(x2.shape[0])
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
    """MM8 Linear: the fused out-major dequant GEMV for up to ``GEMV_ROWS``
    rows, the 64-row MFMA tile GEMM (split K) up to ``GEMM_ROWS`` rows, and a
    dequantise + library GEMM route above that (long prefills, where the
    products are MFMA-bound and the library GEMM's tiling pays)."""

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
        if rows > self.GEMV_ROWS:
            m = self.m
            W = torch.empty((m.out_features, m.in_features), device=x2.device, dtype=x2.dtype)
            _lib.call("rwkv7mi_mm8t_dequant", _lib.ptr(m.w_blk), _lib.ptr(m.mx), _lib.ptr(m.rx), _lib.ptr(m.my),
                      _lib.ptr(m.ry), _lib.ptr(W), m.in_features, m.out_features, _lib.dtype_code(m.mx),
                      _lib.dtype_code(W), _lib.stream_of(x2))
            y = torch.nn.functional.linear(x2, W)
            if m.bias is not None:
                y = y + m.bias
            if act == 3:
                y = torch.relu(y).square()
            if residual is not None:
                y = y + residual
            out.copy_(y)
            return out
        epi = _lib.EPI_RELU2 if act == 3 else (_lib.EPI_RESIDUAL if residual is not None else _lib.EPI_NONE)
        return self.m._run(x2, out=out, residual=residual, epilogue=epi)

    @staticmethod
    def apply_group(lins, xs, outs):
        """The same as ``[l.apply(x, o) for ...]``; out-major MM8 modules of one
        shape run as one launch."""
        rows = int(xs[0].shape[0])
        if (all(isinstance(l, QuantLinear) for l in lins) and rows <= QuantLinear.GEMM_ROWS
                and len({(l.in_features, l.out_features) for l in lins}) == 1
                and all(is_blocked(l.m.w_blk) for l in lins)):
            if rows <= QuantLinear.GEMV_ROWS:
                mm8_matmul_multi_into(list(xs), [l.m for l in lins], list(outs))
            else:
                mm8_gemm_multi_into(list(xs), [l.m for l in lins], list(outs))
            return outs
        for l, x2, o in zip(lins, xs, outs):
            l.apply(x2, o)
        return outs


# ------------------------------------------------------------------ cache
class NativeRWKV7Cache:
    """Recurrent-state cache with the reference's contract (rwkv7_hf/model_cache.py:48).

    Iterable as ``(state, xpa, xpf, v_first)``; ``state[l]`` is ``[B,H,N,N]`` fp32.
    """

    def __init__(self, state=None, xpa=None, xpf=None, v_first=None, seen_tokens: int = 0):
        self._state, self._xpa, self._xpf, self._v_first = state, xpa, xpf, v_first
        self._seen_tokens = int(seen_tokens)
        self._rwkv7_cache_version = 0
        self._bound_runner = None

    @classmethod
    def zeros(cls, cfg: NativeRWKV7Config, batch: int, device, dtype=torch.float16):
        H, N, D, A, L = cfg.num_heads, cfg.head_dim, cfg.hidden_size, cfg.attention_hidden_size, cfg.num_hidden_layers
        return cls([torch.zeros(batch, H, N, N, device=device, dtype=torch.float32) for _ in range(L)],
                   [torch.zeros(batch, D, device=device, dtype=dtype) for _ in range(L)],
                   [torch.zeros(batch, D, device=device, dtype=dtype) for _ in range(L)],
                   torch.zeros(batch, A, device=device, dtype=dtype), 0)

    def __iter__(self):
        return iter((self._state, self._xpa, self._xpf, self._v_first))

    def __len__(self):
        return 0 if self._state is None else len(self._state)

    def __getitem__(self, idx):
        return (self._state[idx], self._xpa[idx], self._xpf[idx], self._v_first)

    @property
    def seen_tokens(self) -> int:
        return self._seen_tokens

    @seen_tokens.setter
    def seen_tokens(self, value: int) -> None:
        self._seen_tokens = int(value)

    def get_seq_length(self, layer_idx: int | None = 0, cache_position=None) -> int:
        return self._seen_tokens

    def get_batch_size(self) -> int | None:
        return None if self._v_first is None else int(self._v_first.shape[0])

    def is_initialized(self) -> bool:
        return self._state is not None

    def _invalidate(self):
        self._rwkv7_cache_version += 1
        self._bound_runner = None

    def clone(self) -> "NativeRWKV7Cache":
        c = NativeRWKV7Cache([s.clone() for s in self._state], [x.clone() for x in self._xpa],
                             [x.clone() for x in self._xpf], self._v_first.clone(), self._seen_tokens)
        return c

    def reset(self) -> None:
        for t in (*self._state, *self._xpa, *self._xpf, self._v_first):
            t.zero_()
        self._seen_tokens = 0
        self._invalidate()

    def to(self, device=None, dtype=None) -> "NativeRWKV7Cache":
        self._state = [s.to(device) for s in self._state]
        self._xpa = [x.to(device=device, dtype=dtype or x.dtype) for x in self._xpa]
        self._xpf = [x.to(device=device, dtype=dtype or x.dtype) for x in self._xpf]
        self._v_first = self._v_first.to(device=device, dtype=dtype or self._v_first.dtype)
        self._invalidate()
        return self

    def select_batch(self, indices: torch.LongTensor, *, inplace: bool = True) -> "NativeRWKV7Cache":
        idx = indices.to(self._v_first.device)
        target = self if inplace else NativeRWKV7Cache(seen_tokens=self._seen_tokens)
        target._state = [s.index_select(0, idx) for s in self._state]
        target._xpa = [x.index_select(0, idx) for x in self._xpa]
        target._xpf = [x.index_select(0, idx) for x in self._xpf]
        target._v_first = self._v_first.index_select(0, idx)
        target._invalidate()
        return target

    reorder_cache = select_batch

    def batch_repeat_interleave(self, repeats: int):
        self._state = [s.repeat_interleave(repeats, 0) for s in self._state]
        self._xpa = [x.repeat_interleave(repeats, 0) for x in self._xpa]
        self._xpf = [x.repeat_interleave(repeats, 0) for x in self._xpf]
        self._v_first = self._v_first.repeat_interleave(repeats, 0)
        self._invalidate()


# ------------------------------------------------------------------ model
class _Layer:
    pass


class NativeRWKV7ForCausalLM:
    """RWKV-7 causal LM (inference) over the HIP kernels; see the module docstring."""

    def __init__(self, config: NativeRWKV7Config, weights: dict[str, torch.Tensor], *, device="cuda",
                 dtype=torch.float16):
        self.config = cfg = config
        self.device = torch.device(device)
        self.dtype = dtype
        # run the decode LoRA projections on a second stream beside R/K/V
        self.lora_side_stream = False
        # decode: LoRA up projections inside the wkv kernel (when the shapes allow)
        self.fused_lora_decode = True
        # decode: LayerNorm + token-shift mixes inside the R/K/V and FFN-key GEMVs
        self.fused_mix_decode = True
        dev = self.device

        def get(name):
            return weights[name].to(device=dev, dtype=dtype).contiguous()

        def linear(name):
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

        self._replaced = 0
        self.emb = get("model.embeddings.weight")
        self.layers = []
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
        self._rwkv7_native_mm_quantization = "mm8" if cfg.use_native_mm8 else None
        self._rwkv7_native_mm_replaced_modules = self._replaced
        self._graph_runners: dict[int, "NativeGraphRunner"] = {}

    # ------------------------------------------------------------- helpers
    @classmethod
    def from_random(cls, config: NativeRWKV7Config, *, seed: int = 0, device="cuda", dtype=torch.float16):
        """Random-init model; weights are generated one tensor at a time on ``device``."""
        return cls(config, _LazyWeights(config, seed, device, dtype), device=device, dtype=dtype)

    def new_cache(self, batch: int) -> NativeRWKV7Cache:
        return NativeRWKV7Cache.zeros(self.config, batch, self.device, self.dtype)

    def reserve_workspace(self, rows: int) -> None:
        """Grow the per-device scratch slots for ``rows``-row decode steps (before capture)."""
        need = 0
        for lin in self._linears():
            if isinstance(lin, QuantLinear):
                need = max(need, lin.m.rwkv7_workspace_bytes(min(rows, 64)))
        if need:
            _ws.reserve(self.device, need)
        if QuantLinear.GEMV_ROWS < rows <= QuantLinear.GEMM_ROWS:
            gneed = 0
            for L in self.layers:
                gneed = max(gneed, mm8_gemm_workspace_bytes(3, rows, L.r_proj.in_features, L.r_proj.out_features))
            for lin in self._linears():
                if isinstance(lin, QuantLinear):
                    gneed = max(gneed, mm8_gemm_workspace_bytes(1, rows, lin.in_features, lin.out_features))
            if gneed:
                _ws.reserve(self.device, gneed, slot="mm8g")
        cfg = self.config
        ranks = [cfg.decay_low_rank_dim, cfg.a_low_rank_dim, cfg.gate_low_rank_dim, cfg.v_low_rank_dim]
        _ws.reserve(self.device, lora_workspace_bytes(ranks, rows, cfg.hidden_size), slot="lora")

    def _linears(self):
        for L in self.layers:
            yield from (L.r_proj, L.k_proj, L.v_proj, L.o_proj, L.key, L.value)
        yield self.lm_head

    def _lora(self, L, xw, xa, xg, xv, rows, outs, mids):
        """W, A (sigmoid applied), G, V-gate projections on the LoRA HIP kernels."""
        n = len(L.lora_down)
        xin = [xw, xa, xg, xv][:n]
        acts_down = [ACT_TANH, ACT_NONE, ACT_SIGMOID, ACT_NONE][:n]
        acts_up = [ACT_NONE, ACT_SIGMOID, ACT_NONE, ACT_SIGMOID][:n]
        if rows > 256:
            for q in range(n):
                h = xin[q] @ L.lora_down[q].t()
                if acts_down[q] == ACT_TANH:
                    h = torch.tanh(h)
                elif acts_down[q] == ACT_SIGMOID:
                    h = torch.sigmoid(h)
                y = torch.nn.functional.linear(h, L.lora_up[q], L.lora_bias[q])
                if acts_up[q] == ACT_SIGMOID:
                    y = torch.sigmoid(y)
                outs[q].copy_(y)
            return
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
        }

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
        x = bufs["x"]
        torch.index_select(self.emb, 0, tokens, out=x)
        state, xpa, xpf, v_first = cache
        H, N, eps = cfg.num_heads, cfg.head_dim, cfg.norm_eps
        mixb, rkv, lora, prep = bufs["mix"], bufs["rkv"], bufs["lora"], bufs["prep"]
        main = torch.cuda.current_stream(x.device)
        side, ev_in, ev_out = self._side(x.device) if self.lora_side_stream else (None, None, None)
        fmix = self._mix_fusable(B) and not self.lora_side_stream
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
                                            pre_norm_bias=L.pre[1] if L.pre else None)
            if (self.fused_lora_decode and not self.lora_side_stream
                    and fused_lora_decode_supported([int(d.shape[0]) for d in L.lora_down], B)):
                # LoRA down (split-K launch), then the up projections inside the wkv kernel
                if not fmix:
                    QuantLinear.apply_group((L.r_proj, L.k_proj, L.v_proj), (xr, xk, xv), (rkv[0], rkv[1], rkv[2]))
                fused_wavg_lora_output_prepare_raw(
                    rkv[0], rkv[1], rkv[2], [xw, xa, xg, xv][:n], L.lora_down, L.lora_up, L.lora_bias, state[i],
                    L.k_k, L.k_a, L.r_k, L.gn[0], L.gn[1], eps=N * 1e-5, out=prep, state_out=state[i],
                    v_first=v_first, v_mode=1 if i == 0 else 2, down_sums=bufs["ldown"] if fmix else None)
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
            L.value.apply(bufs["kf"], x, residual=x)
        if fmix:
            # the kernels read the shift inputs while writing this step's rows, so
            # the rows go to separate buffers and replace the cache's here
            torch._foreach_copy_(list(xpa) + list(xpf), list(bufs["hatt"].unbind(0)) + list(bufs["hffn"].unbind(0)))
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
    def prefill_(self, input_ids: torch.Tensor, cache: NativeRWKV7Cache) -> torch.Tensor:
        """Run ``input_ids [B, T]`` through every layer (chunked scan), update the cache,
        return the last token's logits ``[B, V]``."""
        cfg = self.config
        B, T = (int(s) for s in input_ids.shape)
        dev, dt = self.device, self.dtype
        D, A, H, N, F, eps = (cfg.hidden_size, cfg.attention_hidden_size, cfg.num_heads, cfg.head_dim,
                              cfg.intermediate_size, cfg.norm_eps)
        R = B * T
        state, xpa, xpf, v_first = cache
        x = torch.nn.functional.embedding(input_ids.reshape(-1), self.emb).reshape(B, T, D).contiguous()
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
            L.r_proj.apply(xr, rkv[0])
            L.k_proj.apply(xk, rkv[1])
            L.v_proj.apply(xv, rkv[2])
            self._lora(L, xw, xa, xg, xv, R, [lora[q] for q in range(4)], mids)
            w_log, k_adj, v_int, kk = fused_prefill_state_prep(
                lora[0], rkv[1], rkv[2], lora[1], L.k_k, L.k_a, v_first=vfirst_seq,
                v_gate=lora[3] if i > 0 else None, num_heads=H, head_dim=N, w_transform="log",
                v_mode=1 if i == 0 else 2)
            shp = (B, T, H, N)
            y, _ = _run_chunk(rkv[0].view(shp), w_log.view(shp), k_adj.view(shp), v_int.view(shp), kk.view(shp),
                              lora[1].view(shp), state[i], w_is_log=True, chunk=16, state_out=state[i])
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
        h = layer_norm(x[:, -1].contiguous(), self.norm[0], self.norm[1], eps)
        logits = torch.empty(B, cfg.vocab_size, device=dev, dtype=dt)
        self.lm_head.apply(h, logits)
        cache.seen_tokens = cache.seen_tokens + T
        cache._invalidate()
        return logits

    # ------------------------------------------------------------- API
    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, past_key_values: NativeRWKV7Cache | None = None, use_cache=True):
        """Returns ``(logits [B, 1, V], cache)``; prefill for T > 1, one decode step for T == 1."""
        B, T = (int(s) for s in input_ids.shape)
        cache = past_key_values if past_key_values is not None else self.new_cache(B)
        if T == 1:
            self.reserve_workspace(B)
            logits = torch.empty(B, self.config.vocab_size, device=self.device, dtype=self.dtype)
            self.decode_step_(input_ids[:, 0].contiguous(), cache, logits)
            cache.seen_tokens = cache.seen_tokens + 1
            cache._invalidate()
        else:
            logits = self.prefill_(input_ids, cache)
        return logits.unsqueeze(1), cache

    __call__ = forward

    def graph_runner(self, batch: int) -> "NativeGraphRunner":
        r = self._graph_runners.get(batch)
        if r is None:
            r = NativeGraphRunner(self, batch)
            self._graph_runners[batch] = r
        return r

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int, *, use_graph: bool = True):
        """Greedy generation; returns ``[B, T + max_new_tokens]``."""
        B = int(input_ids.shape[0])
        logits, cache = self.forward(input_ids)
        nxt = logits[:, -1].float().argmax(-1)
        out = [input_ids, nxt[:, None]]
        runner = self.graph_runner(B) if use_graph else None
        for _ in range(max_new_tokens - 1):
            if runner is not None:
                lg = runner.replay(nxt, cache)
            else:
                lg, cache = self.forward(nxt[:, None], cache)
                lg = lg[:, -1]
            nxt = lg.float().argmax(-1)
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
    later steps run with no copies.
    """

    def __init__(self, model: NativeRWKV7ForCausalLM, batch: int, *, warmup: int = 2):
        self.model = model
        self.batch = int(batch)
        dev = model.device
        model.reserve_workspace(self.batch)
        self.cache = model.new_cache(self.batch)
        self.tokens = torch.zeros(self.batch, dtype=torch.long, device=dev)
        self.logits = torch.empty(self.batch, model.config.vocab_size, device=dev, dtype=model.dtype)
        self.bufs = model._decode_buffers(self.batch)
        snapshot = self.cache.clone()
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                model.decode_step_(self.tokens, self.cache, self.logits, self.bufs)
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            model.decode_step_(self.tokens, self.cache, self.logits, self.bufs)
        self._copy_into(snapshot)
        self.replays = 0

    def _copy_into(self, cache: NativeRWKV7Cache) -> None:
        s, a, f, v = self.cache
        s2, a2, f2, v2 = cache
        for dst, src in zip((*s, *a, *f, v), (*s2, *a2, *f2, v2)):
            dst.copy_(src)

    def bind_cache(self, cache: NativeRWKV7Cache) -> None:
        cache._state, cache._xpa, cache._xpf, cache._v_first = (
            list(self.cache._state), list(self.cache._xpa), list(self.cache._xpf), self.cache._v_first)
        cache._bound_runner = self

    def replay(self, tokens: torch.Tensor, cache: NativeRWKV7Cache) -> torch.Tensor:
        if cache._bound_runner is not self:
            self._copy_into(cache)
            self.bind_cache(cache)
        self.tokens.copy_(tokens.reshape(-1))
        self.graph.replay()
        self.replays += 1
        cache.seen_tokens = cache.seen_tokens + 1
        return self.logits


__all__ = ["NativeRWKV7Config", "NativeRWKV7Cache", "NativeRWKV7ForCausalLM", "NativeGraphRunner",
           "random_weights", "parameter_shapes"]
