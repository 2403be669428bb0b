"""Native MM4 (4-bit affine and group-wise symmetric) with the reference's API.

Mirrors rwkv7_hf/native_quant_mm4.py (rwkv-rs/hf-adapter 0.8.1):
``quantize_mm4`` (:77), ``dequantize_mm4`` (:108), ``mm4_matmul`` (:125),
``mm4_linear`` (:133), the Triton-named entry points ``mm4_gemv_triton`` /
``mm4_batched_gemv_triton`` / ``mm4_matmul_triton`` (:545-578), ``MM4Linear``
(:581) with its group path (``group_size`` 128/256 -> the symmetric W4 format of
rwkv7_hf/sm70_quant.py:502), and ``quantize_model_mm4`` with the group
policies (:720-832).

Packing runs as gfx950 kernels that reproduce the reference's fp32 op sequence
bit for bit.  ``MM4Linear`` keeps its affine nibbles packed along the inputs
(``packed_t [out, in/2]``), the layout the fused HIP GEMV streams; its
``state_dict`` holds the reference's ``packed [in, ceil(out/2)]``, converted on
save and load.  The Triton-named functional calls run a fused MFMA kernel
straight over the reference layout (``rwkv7mi_mm4_matmul``); ``mm4_matmul``
dequantises and uses a library GEMM, as the reference's own does.  GPU
tensors only.
"""
from __future__ import annotations

import torch

from . import _lib
from . import workspace as _ws
from .native_quant_policy import normalize_native_mm_policy, should_quantize_linear
from .sm70_quant import quantize_w4_groupwise, w4_groupwise_linear, w4_groupwise_linear_into


def _pack(weight: torch.Tensor, out_major: bool):
    w = weight.contiguous()
    if out_major:
        m, n = (int(s) for s in w.shape)  # Linear.weight [out, in]
    else:
        n, m = (int(s) for s in w.shape)  # W = weight.T [in, out]
    mp = m + (m & 1)
    dev, dt = w.device, w.dtype
    packed = (torch.empty((mp, n // 2), device=dev, dtype=torch.uint8) if out_major
              else torch.empty((n, mp // 2), device=dev, dtype=torch.uint8))
    mx = torch.empty(mp, device=dev, dtype=dt)
    rx_s = torch.empty(mp, device=dev, dtype=dt)
    my = torch.empty((n, 1), device=dev, dtype=dt)
    ry_s = torch.empty((n, 1), device=dev, dtype=dt)
    ws = torch.empty(2 * n + 2 * mp, device=dev, dtype=torch.float32)
    _lib.call("rwkv7mi_mm4_pack_t" if out_major else "rwkv7mi_mm4_pack", _lib.ptr(w), n, m, _lib.dtype_code(w),
              _lib.ptr(packed), _lib.ptr(mx), _lib.ptr(rx_s), _lib.ptr(my), _lib.ptr(ry_s), _lib.ptr(ws),
              _lib.stream_of(w))
    return packed, mx, rx_s, my, ry_s, m, mp


def quantize_mm4(weight: torch.Tensor):
    """Quantize ``weight: [N, M]`` to the 4-bit affine format.

    Returns ``(packed [N, M_pad/2] uint8, mx [M_pad], rx_s [M_pad], my [N,1],
    ry_s [N,1], M_orig, M_pad)``, identical to the reference packer.
    """
    if weight.dim() != 2:
        raise ValueError("quantize_mm4 expects a 2-D weight")
    _lib.require_gpu(weight, name="quantize_mm4")
    return _pack(weight, out_major=False)


def quantize_mm4_outmajor(weight: torch.Tensor):
    """Quantize ``nn.Linear.weight [M, N]`` to the same values as
    ``quantize_mm4(weight.t())`` with nibbles paired along the inputs:
    ``(packed_t [M_pad, N/2], mx, rx_s, my, ry_s, M_orig, M_pad)`` (an odd M's
    pad column is the last row)."""
    if weight.dim() != 2 or int(weight.shape[1]) % 2:
        raise ValueError("quantize_mm4_outmajor expects a 2-D weight with an even in_features")
    _lib.require_gpu(weight, name="quantize_mm4_outmajor")
    return _pack(weight, out_major=True)


def dequantize_mm4(packed, mx, rx_s, my, ry_s, m_orig, out_dtype=None):
    """Materialise ``[N, M_orig]`` from the reference layout (fp32 math, one rounding)."""
    _lib.require_gpu(packed, mx, name="dequantize_mm4")
    dtype = out_dtype if out_dtype is not None else mx.dtype
    n = int(packed.shape[0])
    out = torch.empty((n, int(m_orig)), device=packed.device, dtype=dtype)
    meta = [t.reshape(-1).contiguous() for t in (mx, rx_s, my, ry_s)]
    _lib.call("rwkv7mi_mm4_dequant", _lib.ptr(packed.contiguous()), *(_lib.ptr(t) for t in meta), _lib.ptr(out), n,
              int(m_orig), _lib.dtype_code(meta[0]), _lib.dtype_code(out), _lib.stream_of(packed))
    return out


def mm4_matmul(x, packed, mx, rx_s, my, ry_s, m_orig):
    """``y = x @ dequant(W)`` from the reference layout (dequantise, then a library GEMM)."""
    deq = dequantize_mm4(packed, mx, rx_s, my, ry_s, m_orig, out_dtype=x.dtype)
    return x @ deq


def mm4_linear(x, packed, mx, rx_s, my, ry_s, m_orig):
    return mm4_matmul(x, packed, mx, rx_s, my, ry_s, m_orig)


def mm4_gemv_available(device=None) -> bool:
    """The fused path needs the HIP library and a GPU device."""
    try:
        _lib.load()
    except Exception:
        return False
    return torch.cuda.is_available()


# Rows above which the reference-layout matmul dequantises once and runs a
# library GEMM: the fused kernel streams the packed bytes once per 16 rows.
MM4_FUSED_MAX_ROWS = 64


def mm4_workspace_bytes(n: int, m_padded: int) -> int:
    """K-range partials of the reference-layout kernel (the ``"mm4"`` slot)."""
    return int(_lib.load().rwkv7mi_mm4_matmul_workspace_bytes(int(n), int(m_padded)))


def mm4_matmul_into(x2, packed, mx, rx_s, my, ry_s, out, *, bias=None, residual=None, epilogue=_lib.EPI_NONE):
    """Fused product over the reference layout ``packed [N, M_pad/2]``:
    ``out [rows, M] = epilogue(x2 [rows, N] @ dequant(W)[:, :M])``, M <= M_pad."""
    if x2.dim() != 2 or packed.dim() != 2:
        raise ValueError("mm4: x2 must be [rows, N] and packed [N, M_pad/2]")
    rows, n = (int(s) for s in x2.shape)
    if int(packed.shape[0]) != n:
        raise ValueError(f"input width {n} does not match quantized weight width {packed.shape[0]}")
    mp = 2 * int(packed.shape[1])
    m = int(out.shape[-1])
    if m > mp or int(mx.numel()) < m or int(rx_s.numel()) < m or int(my.numel()) != n or int(ry_s.numel()) != n:
        raise ValueError(f"mm4: scales do not match packed {tuple(packed.shape)} and {m} outputs")
    if tuple(out.shape) != (rows, m) or not out.is_contiguous() or out.dtype != x2.dtype:
        raise ValueError("mm4: out must be a contiguous [rows, M] tensor of x's dtype")
    if residual is not None:
        residual = residual.reshape(rows, m)
        if not residual.is_contiguous() or residual.dtype != x2.dtype:
            raise ValueError("mm4: residual must be contiguous with x's dtype")
    _lib.require_gpu(x2, packed, out, name="mm4_matmul")
    x2 = x2.contiguous()
    packed = packed.contiguous()
    mdt = mx.dtype
    meta = [t.reshape(-1).to(mdt).contiguous() for t in (mx, rx_s, my, ry_s)]
    if bias is not None:
        bias = bias.reshape(-1).to(mdt).contiguous()
    ws = _ws.reserve(x2.device, mm4_workspace_bytes(n, mp), slot="mm4")
    _lib.call("rwkv7mi_mm4_matmul", _lib.ptr(x2), _lib.ptr(packed), *(_lib.ptr(t) for t in meta), _lib.ptr(bias),
              _lib.ptr(residual), _lib.ptr(out), rows, n, m, mp, int(epilogue), _lib.dtype_code(x2),
              _lib.dtype_code(meta[0]), _lib.ptr(ws), int(ws.numel()), _lib.stream_of(x2))
    return out


def _fused(x2, packed, mx, rx_s, my, ry_s, m_orig):
    out = torch.empty((int(x2.shape[0]), int(m_orig)), device=x2.device, dtype=x2.dtype)
    return mm4_matmul_into(x2, packed, mx, rx_s, my, ry_s, out)


def mm4_gemv_triton(x, packed, mx, rx_s, my, ry_s, m_orig, *, block_pairs=None, block_n=None):
    """Fused dequant GEMV ``x [N] -> [M_orig]`` (rwkv7_hf/native_quant_mm4.py:458-471).
    ``block_pairs`` / ``block_n`` are the reference's Triton tile knobs and are
    accepted for signature parity; the HIP kernel picks its own tiling."""
    _lib.require_gpu(x, packed, name="mm4_gemv_triton")
    return _fused(x.reshape(1, -1), packed, mx, rx_s, my, ry_s, m_orig).reshape(-1)


def mm4_batched_gemv_triton(x, packed, mx, rx_s, my, ry_s, m_orig, *, block_pairs=None, block_n=None):
    """Fused GEMV for a small ``[B, N]`` decode batch (rwkv7_hf/native_quant_mm4.py:474-491)."""
    if not (x.is_cuda and x.dim() == 2):
        raise RuntimeError("mm4_batched_gemv_triton requires a 2-D CUDA input")
    return _fused(x, packed, mx, rx_s, my, ry_s, m_orig)


def mm4_batched_dot_triton(x, packed, mx, rx_s, my, ry_s, m_orig, *, block_b=None, block_pairs=None, block_n=None,
                           num_warps=None):
    """The fp16 matrix-core batch path (rwkv7_hf/native_quant_mm4.py:494-542);
    the same MFMA kernel as every other row count here."""
    if not (x.is_cuda and x.dim() == 2):
        raise RuntimeError("mm4_batched_dot_triton requires a 2-D CUDA input")
    if x.dtype != torch.float16:
        raise TypeError("mm4_batched_dot_triton currently requires fp16 input")
    return _fused(x, packed, mx, rx_s, my, ry_s, m_orig)


def mm4_matmul_triton(x, packed, mx, rx_s, my, ry_s, m_orig, *, max_gemv_rows: int | None = None):
    """Routed matmul (rwkv7_hf/native_quant_mm4.py:545-578): 1-D and 2-D inputs
    of at most ``max_gemv_rows`` rows (default ``MM4_FUSED_MAX_ROWS``) run the
    fused kernel; more rows, or more than two dimensions, dequantise once and
    run a library GEMM."""
    _lib.require_gpu(x, packed, name="mm4_matmul_triton")
    if x.dim() == 1:
        return mm4_gemv_triton(x, packed, mx, rx_s, my, ry_s, m_orig)
    if x.dim() != 2:
        return mm4_matmul(x, packed, mx, rx_s, my, ry_s, m_orig)
    limit = MM4_FUSED_MAX_ROWS if max_gemv_rows is None else min(max(1, int(max_gemv_rows)), 65536)
    if int(x.shape[0]) > limit:
        return mm4_matmul(x, packed, mx, rx_s, my, ry_s, m_orig)
    return _fused(x, packed, mx, rx_s, my, ry_s, m_orig)


def mm4t_matmul_into(x2, packed_t, mx, rx_s, my, ry_s, out, *, bias=None, residual=None, epilogue=_lib.EPI_NONE):
    """Fused GEMV/GEMM over inputs-paired nibbles: ``out = epilogue(x2 @ dequant(W))``."""
    rows, n = (int(s) for s in x2.shape)
    m = int(out.shape[-1])
    if int(packed_t.shape[1]) * 2 != n or int(packed_t.shape[0]) < m:
        raise ValueError(f"mm4: x has {n} features but packed_t is {tuple(packed_t.shape)}")
    if tuple(out.shape) != (rows, m) or not out.is_contiguous() or out.dtype != x2.dtype:
        raise ValueError("mm4: out must be a contiguous [rows, M] tensor of x's dtype")
    if residual is not None:
        residual = residual.reshape(rows, m)
        if not residual.is_contiguous() or residual.dtype != x2.dtype:
            raise ValueError("mm4: residual must be contiguous with x's dtype")
    _lib.require_gpu(x2, packed_t, out, name="mm4_matmul")
    _lib.call("rwkv7mi_mm4t_matmul", _lib.ptr(x2), _lib.ptr(packed_t), _lib.ptr(mx), _lib.ptr(rx_s), _lib.ptr(my),
              _lib.ptr(ry_s), _lib.ptr(bias), _lib.ptr(residual), _lib.ptr(out), rows, n, m, int(epilogue),
              _lib.dtype_code(x2), _lib.dtype_code(mx), _lib.stream_of(x2))
    return out


def _unpack_pairs(p: torch.Tensor, axis_len: int) -> torch.Tensor:
    """[R, C] bytes -> [R, 2C] nibbles (low first), cut to axis_len columns."""
    u = torch.stack((p & 15, p >> 4), dim=-1).reshape(p.shape[0], -1)
    return u[:, :axis_len]


def _pack_pairs(u: torch.Tensor) -> torch.Tensor:
    """[R, 2C] nibbles -> [R, C] bytes (low nibble = even column)."""
    return (u[:, 0::2] | (u[:, 1::2] << 4)).to(torch.uint8).contiguous()


def outmajor_to_reference(packed_t: torch.Tensor, in_features: int) -> torch.Tensor:
    """``packed_t [M_pad, N/2]`` -> the reference's ``packed [N, M_pad/2]``."""
    u = _unpack_pairs(packed_t, in_features).t()  # [N, M_pad]
    return _pack_pairs(u)


def reference_to_outmajor(packed: torch.Tensor, out_features: int) -> torch.Tensor:
    """The reference's ``packed [N, M_pad/2]`` -> ``packed_t [M_pad, N/2]``."""
    mp = int(packed.shape[1]) * 2
    u = _unpack_pairs(packed, mp).t().contiguous()  # [M_pad, N]
    return _pack_pairs(u)


class MM4Linear(torch.nn.Module):
    """Drop-in for ``nn.Linear`` with 4-bit weights (rwkv7_hf/native_quant_mm4.py:581-718).

    ``group_size`` 0: affine MM4 (fused out-major GEMV); 128/256 with
    ``in_features % group_size == 0``: symmetric group W4 (``packed_group``,
    ``group_scales``; fused GEMV as well).
    """

    def __init__(self, linear, *, fused=True, group_size=0):
        super().__init__()
        self.in_features, self.out_features = int(linear.weight.shape[1]), int(linear.weight.shape[0])
        self.group_size = int(group_size)
        if self.group_size not in {0, 128, 256}:
            raise ValueError("native MM4 group_size must be 0, 128, or 256")
        self.groupwise = bool(self.group_size in {128, 256} and self.in_features % self.group_size == 0)
        self.sm70_rowwise = False
        if self.groupwise:
            packed_group, group_scales, packed_inputs = quantize_w4_groupwise(linear.weight.data,
                                                                              group_size=self.group_size)
            self.register_buffer("packed_group", packed_group)
            self.register_buffer("group_scales", group_scales)
            self.packed_inputs = int(packed_inputs)
            self.m_orig = self.out_features
        else:
            if self.in_features % 32:
                raise ValueError("affine MM4 on gfx950 needs in_features divisible by 32")
            packed_t, mx, rx_s, my, ry_s, m_orig, _ = quantize_mm4_outmajor(linear.weight.data)
            self.m_orig = m_orig
            self.register_buffer("packed_t", packed_t)
            self.register_buffer("mx", mx)
            self.register_buffer("rx_s", rx_s)
            self.register_buffer("my", my)
            self.register_buffer("ry_s", ry_s)
        if linear.bias is not None:
            self.register_buffer("bias", linear.bias.data.clone())
        else:
            self.bias = None
        self.fused = bool(fused)

    # the reference's buffer name and layout in state dicts
    @property
    def packed(self) -> torch.Tensor:
        return outmajor_to_reference(self.packed_t, self.in_features)

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        super()._save_to_state_dict(destination, prefix, keep_vars)
        if not self.groupwise:
            destination.pop(prefix + "packed_t", None)
            destination[prefix + "packed"] = self.packed

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                              error_msgs):
        key = prefix + "packed"
        if not self.groupwise and key in state_dict:
            state_dict = dict(state_dict)
            ref = state_dict.pop(key)
            state_dict[prefix + "packed_t"] = reference_to_outmajor(ref.to(self.packed_t.device), self.out_features)
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                                      error_msgs)

    def _run(self, x, out=None, residual=None, epilogue=_lib.EPI_NONE):
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        rows = int(x2.shape[0])
        out2 = (torch.empty((rows, self.out_features), device=x.device, dtype=x.dtype) if out is None
                else out.reshape(rows, self.out_features))
        if self.groupwise:
            w4_groupwise_linear_into(x2, self.packed_group, self.group_scales, out2, group_size=self.group_size,
                                     bias=self.bias, residual=residual, epilogue=epilogue)
        else:
            mm4t_matmul_into(x2, self.packed_t, self.mx, self.rx_s, self.my.reshape(-1), self.ry_s.reshape(-1), out2,
                             bias=self.bias, residual=residual, epilogue=epilogue)
        return out2.reshape(*lead, self.out_features) if out is None else out

    def forward(self, x):
        return self._run(x)

    def rwkv7_forward_into(self, x, out):
        return self._run(x, out=out)

    def rwkv7_forward_relu2(self, x):
        return self._run(x, epilogue=_lib.EPI_RELU2)

    def rwkv7_forward_add(self, x, residual):
        return self._run(x, residual=residual.contiguous(), epilogue=_lib.EPI_RESIDUAL)

    def extra_repr(self):
        return (f"in={self.in_features}, out={self.out_features}, "
                f"mm4(fused={self.fused}, group_size={self.group_size}, hip=gfx950)")


NATIVE_MM4_GROUP_POLICIES = ("all", "lm_head", "ffn_key", "ffn_value", "lm_head_and_key", "lm_head_and_value")


def normalize_native_mm4_group_policy(policy: str | None) -> str:
    value = (policy or "all").strip().lower().replace("-", "_")
    if value not in NATIVE_MM4_GROUP_POLICIES:
        raise ValueError(f"unsupported native MM4 group policy {policy!r}; expected: "
                         + ", ".join(NATIVE_MM4_GROUP_POLICIES))
    return value


def native_mm4_group_size_for_module(name: str, group_size: int, group_policy: str) -> int:
    """Group size for one module under the policy (rwkv7_hf/native_quant_mm4.py:741-758)."""
    if int(group_size) == 0:
        return 0
    policy = normalize_native_mm4_group_policy(group_policy)
    is_head = name == "lm_head" or name.endswith(".lm_head")
    is_key = name.endswith(".ffn.key")
    is_value = name.endswith(".ffn.value")
    enabled = {"all": True, "lm_head": is_head, "ffn_key": is_key, "ffn_value": is_value,
               "lm_head_and_key": is_head or is_key, "lm_head_and_value": is_head or is_value}[policy]
    return int(group_size) if enabled else 0


def quantize_model_mm4(model, *, min_params: int = 8_000_000, fused: bool = True, policy: str = "memory",
                       group_size: int = 0, group_policy: str = "all") -> int:
    """Swap eligible ``nn.Linear`` modules for :class:`MM4Linear`; returns the count."""
    policy = normalize_native_mm_policy(policy)
    group_policy = normalize_native_mm4_group_policy(group_policy)
    targets = [n for n, m in model.named_modules()
               if isinstance(m, torch.nn.Linear)
               and should_quantize_linear(n, int(m.weight.numel()), min_params=min_params, policy=policy)]
    for full_name in targets:
        parent_name, _, attr = full_name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, attr, MM4Linear(getattr(parent, attr), fused=fused,
                                        group_size=native_mm4_group_size_for_module(full_name, group_size,
                                                                                    group_policy)))
    setattr(model, "_rwkv7_native_mm_quantization", "mm4")
    setattr(model, "_rwkv7_native_mm_replaced_modules", len(targets))
    setattr(model, "_rwkv7_native_mm4_group_size", int(group_size))
    setattr(model, "_rwkv7_native_mm4_group_policy", group_policy)
    setattr(model, "_rwkv7_native_mm_block_replaced_modules", sum(n.startswith("model.layers.") for n in targets))
    return len(targets)


__all__ = [
    "quantize_mm4", "quantize_mm4_outmajor", "dequantize_mm4", "mm4_matmul", "mm4_linear", "mm4_gemv_available",
    "mm4_gemv_triton", "mm4_batched_gemv_triton", "mm4_batched_dot_triton", "mm4_matmul_triton", "mm4_matmul_into",
    "mm4_workspace_bytes", "MM4_FUSED_MAX_ROWS", "mm4t_matmul_into", "MM4Linear",
    "quantize_model_mm4", "normalize_native_mm4_group_policy", "native_mm4_group_size_for_module",
    "NATIVE_MM4_GROUP_POLICIES", "outmajor_to_reference", "reference_to_outmajor",
]
