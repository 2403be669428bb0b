"""Module-selection policy for native MM8/MM4 quantization.

Same policy names, aliases and decisions as rwkv7_hf/native_quant_policy.py:8-42:
``memory`` replaces every Linear with at least ``min_params`` weights,
``speed`` replaces only ``lm_head``.
"""
from __future__ import annotations

NATIVE_MM_POLICIES = ("memory", "speed")

_ALIASES = {
    "default": "memory", "all": "memory", "size": "memory", "size_gated": "memory",
    "fast": "speed", "head": "speed", "head_only": "speed", "lm_head": "speed", "lm_head_only": "speed",
}


def normalize_native_mm_policy(policy: str | None) -> str:
    value = (policy or "memory").strip().lower().replace("-", "_")
    value = _ALIASES.get(value, value)
    if value not in NATIVE_MM_POLICIES:
        allowed = ", ".join(NATIVE_MM_POLICIES)
        raise ValueError(f"unsupported native MM quantization policy {policy!r}; expected one of: {allowed}")
    return value


def should_quantize_linear(name: str, weight_numel: int, *, min_params: int, policy: str | None = "memory") -> bool:
    if int(weight_numel) < int(min_params):
        return False
    if normalize_native_mm_policy(policy) == "memory":
        return True
    return name == "lm_head" or name.endswith(".lm_head")


__all__ = ["NATIVE_MM_POLICIES", "normalize_native_mm_policy", "should_quantize_linear"]
