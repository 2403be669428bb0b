"""fp64 per-token RWKV-7 model oracle — TEST INFRASTRUCTURE ONLY.

Restates the reference's eager per-token path (rwkv7_hf/native.py:180-265
``attn_step_batched``, :268-273 ``ffn_step_batched``, embedding + layer-0
pre-norm + final norm + LM head as in rwkv7_hf/native_model.py) in numpy fp64
over a dict of weights named like the converted checkpoints.  Quantised
linears are passed in already dequantised (``linear_override``), so the oracle
checks the kernels, not the quantisation.  Only tests and bench.py's CPU
baseline may import it.
"""
from __future__ import annotations

import numpy as np

EXP_HALF = 0.606531


def _ln(x, w, b, eps=1e-5):
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * w + b


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


class ModelOracle:
    def __init__(self, cfg, weights: dict, linear_override: dict | None = None, dtype=np.float64):
        """weights: name -> array; linear_override: linear name (without .weight)
        -> W_hat [in, out] used as x @ W_hat.  dtype: fp64 (checker) or fp32 (CPU baseline)."""
        self.cfg = cfg
        self.dtype = dtype
        self.w = {k: np.asarray(v, dtype=dtype) for k, v in weights.items()}
        self.lin = {k: np.asarray(v, dtype=dtype) for k, v in (linear_override or {}).items()}

    def _linear(self, name, x):
        if name in self.lin:
            return x @ self.lin[name]
        return x @ self.w[name + ".weight"].T

    def new_state(self, B):
        c = self.cfg
        H, N, D, A, L = c.num_heads, c.head_dim, c.hidden_size, c.attention_hidden_size, c.num_hidden_layers
        dt = self.dtype
        return {
            "state": [np.zeros((B, H, N, N), dt) for _ in range(L)],
            "xpa": [np.zeros((B, D), dt) for _ in range(L)],
            "xpf": [np.zeros((B, D), dt) for _ in range(L)],
            "v_first": np.zeros((B, A), dt),
        }

    def head(self, x):
        """Final norm + LM head of one hidden row batch (used to time the head alone)."""
        w = self.w
        return self._linear("lm_head", _ln(x, w["model.norm.weight"], w["model.norm.bias"], self.cfg.norm_eps))

    def step(self, tokens, st):
        """One token per row (tokens [B]); updates st in place; returns logits [B, V]."""
        c, w = self.cfg, self.w
        H, N = c.num_heads, c.head_dim
        B = len(tokens)
        x = w["model.embeddings.weight"][np.asarray(tokens)]
        for i in range(c.num_hidden_layers):
            p = f"model.layers.{i}."
            if i == 0:
                x = _ln(x, w[p + "pre_norm.weight"], w[p + "pre_norm.bias"], c.norm_eps)
            # --- time mix (rwkv7_hf/native.py:180-265)
            h = _ln(x, w[p + "attn_norm.weight"], w[p + "attn_norm.bias"], c.norm_eps)
            xx = st["xpa"][i] - h
            xr, xw, xk, xv, xa, xg = (h + xx * w[p + "attn." + m].reshape(1, -1)
                                      for m in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"))
            st["xpa"][i] = h
            r = self._linear(p + "attn.r_proj", xr)
            k = self._linear(p + "attn.k_proj", xk)
            v = self._linear(p + "attn.v_proj", xv)
            lw = lambda n, q: q @ w[p + f"attn.{n}.lora.0.weight"].T
            up = lambda n, q: q @ w[p + f"attn.{n}.lora.2.weight"].T + w.get(p + f"attn.{n}.lora.2.bias", 0.0)
            wd = up("w_lora", np.tanh(lw("w_lora", xw)))
            a = _sigmoid(up("a_lora", lw("a_lora", xa)))
            g = up("g_lora", _sigmoid(lw("g_lora", xg)))
            kk = (k * w[p + "attn.k_k"].reshape(1, -1)).reshape(B, H, N)
            kk = kk / np.maximum(np.linalg.norm(kk, axis=-1, keepdims=True), 1e-12)
            k = k * (1 + (a - 1) * w[p + "attn.k_a"].reshape(1, -1))
            if i == 0:
                st["v_first"] = v.copy()
            else:
                v = v + (st["v_first"] - v) * _sigmoid(up("v_lora", lw("v_lora", xv)))
            dec = np.exp(-EXP_HALF * _sigmoid(wd))
            S = st["state"][i]
            kk3, a3, k3, v3, r3, d3 = (t.reshape(B, H, N) for t in (kk, a, k, v, r, dec))
            dot = np.einsum("bhij,bhj->bhi", S, kk3)
            S = S * d3[:, :, None, :] - dot[..., None] * (kk3 * a3)[:, :, None, :] + v3[..., None] * k3[:, :, None, :]
            st["state"][i] = S
            y = np.einsum("bhij,bhj->bhi", S, r3)
            mu = y.mean(-1, keepdims=True)
            var = ((y - mu) ** 2).mean(-1, keepdims=True)
            y = ((y - mu) / np.sqrt(var + N * 1e-5)).reshape(B, H * N)
            y = y * w[p + "attn.g_norm.weight"] + w[p + "attn.g_norm.bias"]
            sk = (r3 * k3 * w[p + "attn.r_k"].reshape(1, H, N)).sum(-1, keepdims=True)
            y = y + (sk * v3).reshape(B, H * N)
            x = x + self._linear(p + "attn.o_proj", y * g)
            # --- channel mix (rwkv7_hf/native.py:268-273)
            h2 = _ln(x, w[p + "ffn_norm.weight"], w[p + "ffn_norm.bias"], c.norm_eps)
            fk = h2 + (st["xpf"][i] - h2) * w[p + "ffn.x_k"].reshape(1, -1)
            st["xpf"][i] = h2
            kf = np.maximum(self._linear(p + "ffn.key", fk), 0.0) ** 2
            x = x + self._linear(p + "ffn.value", kf)
        hN = _ln(x, w["model.norm.weight"], w["model.norm.bias"], c.norm_eps)
        return self._linear("lm_head", hN)

    def run_seq(self, ids, st=None, keep: int = 1):
        """The same model as :meth:`step`, with every token-parallel product
        (norms, shift mixes, projections, LoRAs, GroupNorm, FFN) taken over
        the whole sequence at once and only the DPLR recurrence per token, as
        the reference's sequence prefill orders it
        (rwkv7_hf/native_jit_prefill.py:223-1057); fp64 like :meth:`step`.
        Feeds ids [B, T]; returns (logits of the last ``keep`` tokens
        [B, keep, V], state)."""
        c, w = self.cfg, self.w
        H, N, D = c.num_heads, c.head_dim, c.hidden_size
        ids = np.asarray(ids)
        B, T = ids.shape
        st = st if st is not None else self.new_state(B)
        x = w["model.embeddings.weight"][ids]  # [B, T, D]
        for i in range(c.num_hidden_layers):
            p = f"model.layers.{i}."
            if i == 0:
                x = _ln(x, w[p + "pre_norm.weight"], w[p + "pre_norm.bias"], c.norm_eps)
            h = _ln(x, w[p + "attn_norm.weight"], w[p + "attn_norm.bias"], c.norm_eps)
            prev = np.concatenate([st["xpa"][i][:, None], h[:, :-1]], 1)
            st["xpa"][i] = h[:, -1].copy()
            xr, xw, xk, xv, xa, xg = (h + (prev - h) * w[p + "attn." + m].reshape(1, 1, -1)
                                      for m in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"))
            r = self._linear(p + "attn.r_proj", xr)
            k = self._linear(p + "attn.k_proj", xk)
            v = self._linear(p + "attn.v_proj", xv)
            lw = lambda n, q: q @ w[p + f"attn.{n}.lora.0.weight"].T
            up = lambda n, q: q @ w[p + f"attn.{n}.lora.2.weight"].T + w.get(p + f"attn.{n}.lora.2.bias", 0.0)
            wd = up("w_lora", np.tanh(lw("w_lora", xw)))
            a = _sigmoid(up("a_lora", lw("a_lora", xa)))
            g = up("g_lora", _sigmoid(lw("g_lora", xg)))
            kk = (k * w[p + "attn.k_k"].reshape(1, 1, -1)).reshape(B, T, H, N)
            kk = kk / np.maximum(np.linalg.norm(kk, axis=-1, keepdims=True), 1e-12)
            k = k * (1 + (a - 1) * w[p + "attn.k_a"].reshape(1, 1, -1))
            if i == 0:
                st["v_first"] = v[:, -1].copy()
                vfirst = v.copy()
            else:
                v = v + (vfirst - v) * _sigmoid(up("v_lora", lw("v_lora", xv)))
            dec = np.exp(-EXP_HALF * _sigmoid(wd))
            kk4, a4, k4, v4, r4, d4 = (t.reshape(B, T, H, N) for t in (kk, a, k, v, r, dec))
            S = st["state"][i]
            y = np.empty((B, T, H, N), S.dtype)
            for t in range(T):
                dot = np.einsum("bhij,bhj->bhi", S, kk4[:, t])
                S = (S * d4[:, t, :, None, :] - dot[..., None] * (kk4[:, t] * a4[:, t])[:, :, None, :]
                     + v4[:, t, :, :, None] * k4[:, t, :, None, :])
                y[:, t] = np.einsum("bhij,bhj->bhi", S, r4[:, t])
            st["state"][i] = S
            mu = y.mean(-1, keepdims=True)
            var = ((y - mu) ** 2).mean(-1, keepdims=True)
            y = ((y - mu) / np.sqrt(var + N * 1e-5)).reshape(B, T, H * N)
            y = y * w[p + "attn.g_norm.weight"] + w[p + "attn.g_norm.bias"]
            sk = (r4 * k4 * w[p + "attn.r_k"].reshape(1, 1, H, N)).sum(-1, keepdims=True)
            y = y + (sk * v4).reshape(B, T, H * N)
            x = x + self._linear(p + "attn.o_proj", y * g)
            h2 = _ln(x, w[p + "ffn_norm.weight"], w[p + "ffn_norm.bias"], c.norm_eps)
            prev2 = np.concatenate([st["xpf"][i][:, None], h2[:, :-1]], 1)
            st["xpf"][i] = h2[:, -1].copy()
            fk = h2 + (prev2 - h2) * w[p + "ffn.x_k"].reshape(1, 1, -1)
            kf = np.maximum(self._linear(p + "ffn.key", fk), 0.0) ** 2
            x = x + self._linear(p + "ffn.value", kf)
        hN = _ln(x[:, T - keep:], w["model.norm.weight"], w["model.norm.bias"], c.norm_eps)
        return self._linear("lm_head", hN), st

    def run(self, ids, st=None):
        """Feed ids [B, T] token by token; returns (logits [B, T, V], state)."""
        ids = np.asarray(ids)
        B, T = ids.shape
        st = st if st is not None else self.new_state(B)
        out = [self.step(ids[:, t], st) for t in range(T)]
        return np.stack(out, 1) if out else np.zeros((B, 0, self.cfg.vocab_size)), st
