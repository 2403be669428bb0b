#!/usr/bin/env python3
"""Benchmark of the rwkv7mi hot path on one MI355X (BASELINE.json metric:
"decode tok/s 7.2B MM8 bsz1/8; wkv7 prefill tok/s; % HBM roofline").

Workloads (synthetic inputs, random-init weights; nothing is downloaded):
  decode  : BASELINE configs[4], the RWKV-7 7.2B architecture (L=32, D=4096,
            H=64, N=64, F=16384, V=65536, LoRA 64/64/128/32) with MM8 weights
            (memory policy: every Linear with >= 8M weights, 193 modules), fp16
            activations, fp32 state; a 16-token prefill, then hipGraph-replayed
            greedy decode steps at bsz 1 (the headline ``value``), 8 and 64.
            One step = one token for every row through the full model.
  scan    : configs[1], the wkv7 chunked prefill scan B=8, T=4096, N=64 at
            H=32 and H=64: r,k,v ~ N(0,1) fp16, k L2-normalised, kk = k,
            a = sigmoid(N(0,1)), w = exp(-exp(x)), x ~ N(-0.5, 0.5), fp32 state;
            and its decode form, one single-token update (B=8, H=32) with the
            state in HBM.
  gemv    : configs[2], MM8 GEMV/GEMM at the 1.5B shapes x batch 1/8/32, and
            configs[3], group-128 W4 (asymmetric min/max affine, and the
            reference's symmetric form) at the 7.2B shapes x batch 1/4/16.
  prefill : configs[4]'s prefill, B=8 x T=4096 through the 7.2B model.
  fp16state: the opt-in fp16-state lane: its sequence kernel at B=8, T=4096,
            H=64 and its decode kernel at H=64 for bsz 1/8/64.
The default run measures all of them and prints ONE JSON line.

    python bench.py [--steps K] [--warmup W] [--workload all|decode|scan|gemv|prefill|...] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "hf-adapter_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def _log(msg):
    print(msg, file=sys.stderr, flush=True)


def host_cores() -> int:
    """Host threads this process may use: its CPU affinity, capped by OMP_NUM_THREADS."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    return min(n, int(omp)) if omp and omp.isdigit() and int(omp) > 0 else n


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ------------------------------------------------------------------ byte models
def scan_bytes(B, T, H, N):
    """Algorithmic HBM bytes of one scan call: per (token, head, channel)
    r,k,v,kk,a fp16 (10 B) + w fp32 (4 B) in, y fp16 (2 B) out; plus the fp32
    state read and written once."""
    return B * T * H * N * 16 + 2 * B * H * N * N * 4


def decode_step_bytes(cfg, B, quantized: set[str], shapes: dict, state_bytes: int = 4):
    """Algorithmic HBM bytes of one decode step: every weight read once (MM8:
    1 B/weight + fp16 row/col metadata; others fp16), the recurrent state read +
    written (``state_bytes`` per element), shift states read + written,
    embedding rows and logits."""
    total = 0
    for name, shp in shapes.items():
        if name == "model.embeddings.weight":
            total += B * shp[1] * 2
            continue
        n = 1
        for s in shp:
            n *= s
        base = name[: -len(".weight")] if name.endswith(".weight") else None
        if base is not None and base in quantized:
            o, i = shp
            total += o * i + 2 * (i + o) * 2
        else:
            total += n * 2
    L, H, N, D = cfg.num_hidden_layers, cfg.num_heads, cfg.head_dim, cfg.hidden_size
    total += L * B * H * N * N * state_bytes * 2  # state read + write
    total += L * 2 * B * D * 2 * 2               # xpa / xpf read + write
    total += B * cfg.vocab_size * 2               # logits
    return total


def mm8_bytes(I, O, rows):
    """One MM8 product: weights (1 B each), fp16 row/column metadata, activations in and out."""
    return I * O + 2 * (I + O) * 2 + rows * (I + O) * 2


def w4_bytes(I, O, rows, group=128, affine=True):
    """One group W4 product: nibbles, fp16 scales (and biases), activations in and out."""
    return I * O // 2 + (I * O // group) * 2 * (2 if affine else 1) + rows * (I + O) * 2


# ------------------------------------------------------------------ timing
def time_events(fn, steps, warmup):
    """W untimed calls, then K timed ones between HIP events on the current
    stream, with a device synchronisation on both sides; returns (mean ms per
    call, wall seconds of the timed region)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        ev[2 * i].record(stream)
        fn()
        ev[2 * i + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [ev[2 * i].elapsed_time(ev[2 * i + 1]) for i in range(steps)]
    return sum(per) / len(per), wall


def time_graph(calls, reps=20):
    """Capture ``calls`` (a list of launch closures) in one hipGraph, replay it
    ``reps`` times back to back between two HIP events on the launch stream;
    returns the mean ms per call."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for c in calls:
            c()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for c in calls:
            c()
    graph.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        graph.replay()
    e1.record(st)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (reps * len(calls))
    del graph
    return ms


# ------------------------------------------------------------------ scan
def make_scan_inputs(B, T, H, N, seed=0, device="cuda"):
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    r = torch.randn(B, T, H, N, generator=g, device=device).half()
    k = torch.randn(B, T, H, N, generator=g, device=device)
    k = (k / k.norm(dim=-1, keepdim=True).clamp_min(1e-12)).half()
    v = torch.randn(B, T, H, N, generator=g, device=device).half()
    kk = k.clone()
    a = torch.sigmoid(torch.randn(B, T, H, N, generator=g, device=device)).half()
    x = torch.randn(B, T, H, N, generator=g, device=device) * 0.5 - 0.5
    w = torch.exp(-torch.exp(x)).float()
    state = torch.zeros(B, H, N, N, device=device, dtype=torch.float32)
    return r, w, k, v, kk, a, state


def run_scan(B=8, T=4096, H=32, steps=20, warmup=3):
    from rwkv7mi import self_chunk_rwkv7

    N = 64
    inputs = make_scan_inputs(B, T, H, N)
    ms, wall = time_events(lambda: self_chunk_rwkv7(*inputs, chunk_size=16), steps, warmup)
    nbytes = scan_bytes(B, T, H, N)
    gbs = nbytes / (ms / 1e3) / 1e9
    return {"tok_s": B * T / (ms / 1e3), "ms": ms, "wall_s": wall, "bytes": nbytes, "gbs": gbs,
            "frac": gbs / HBM_PEAK_GBS, "config": f"B={B} T={T} H={H} N={N} chunk=16"}


def run_decode_form_step(B=8, H=32, reps=20):
    """configs[1]'s decode form: one single-token DPLR update per launch with
    the state read from and written to HBM (16 state buffers in rotation, 64 MB,
    so the state is not cache-resident between launches)."""
    import torch
    from rwkv7mi import fused_recurrent_update

    N = 64
    r, w, k, v, kk, a, _ = make_scan_inputs(B, 1, H, N)
    one = [t[:, 0].contiguous() for t in (r, w, k, v, kk, a)]
    states = [torch.zeros(B, H, N, N, device="cuda") for _ in range(16)]
    outs = [torch.empty(B, H, N, device="cuda", dtype=torch.float16) for _ in range(16)]
    calls = [(lambda s=s, o=o: fused_recurrent_update(*one, s, state_out=s, out=o)) for s, o in zip(states, outs)]
    ms = time_graph(calls, reps)
    nbytes = B * H * (2 * N * N * 4 + N * 2 * 5 + N * 4 + N * 2)
    gbs = nbytes / (ms / 1e3) / 1e9
    return {"us_per_step": round(ms * 1e3, 3), "bytes": nbytes, "gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "tok_s": round(B / (ms / 1e3), 1),
            "config": f"B={B} H={H} N={N}, one token, fp32 state in HBM"}


def fp16_sequence_bytes(B, T, H, N):
    """Algorithmic HBM bytes of one fp16-state sequence call: per (token, head,
    channel) r, w, k, v, -kk, kk*a in and y out, fp16 (14 B); plus the fp16
    state read and written once."""
    return B * T * H * N * 14 + 2 * B * H * N * N * 2


def fp16_decode_bytes(B, H, N):
    """One fp16-state decode launch: the fp16 state read and written, six fp16
    vectors in (r, w, k, v, a, g) and out, five fp16 per-channel parameters."""
    return B * H * (2 * N * N * 2 + 7 * N * 2) + 5 * H * N * 2 + 4 * B


def run_fp16_state(steps=20, warmup=3):
    """The opt-in fp16-state lane: the sequence kernel at the scan benchmark's
    shape (B=8, T=4096, H=64) and the decode kernel at a 7.2B layer's heads
    (H=64) for bsz 1/8/64, hipGraph-replayed over 16 rotating states."""
    import torch
    from rwkv7mi import native_fp16_recurrent_output_prepare_raw, native_fp16_sequence

    N, H = 64, 64
    res = {}
    B, T = 8, 4096
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    rn = lambda *s: torch.randn(*s, generator=g, device="cuda")
    r, v = rn(B, T, H, N).half(), rn(B, T, H, N).half()
    w = (rn(B, T, H, N) * 0.5 - 0.5).half()
    k = (rn(B, T, H, N) * 0.3).half()
    kk = torch.nn.functional.normalize(rn(B, T, H, N), dim=-1)
    a = torch.sigmoid(rn(B, T, H, N))
    nkk, kka = (-kk).half().contiguous(), (kk * a).half().contiguous()
    st = torch.zeros(B, H, N, N, device="cuda", dtype=torch.float16)
    el = torch.zeros(B, device="cuda", dtype=torch.int32)
    ms, _ = time_events(lambda: native_fp16_sequence(r, w, k, v, nkk, kka, st, el), steps, warmup)
    nbytes = fp16_sequence_bytes(B, T, H, N)
    gbs = nbytes / (ms / 1e3) / 1e9
    res["sequence"] = {"config": f"B={B} T={T} H={H} N={N}, fp16 state", "ms_per_call": round(ms, 4),
                       "tok_s": round(B * T / (ms / 1e3), 1), "ns_per_token_per_head": round(ms * 1e6 / T, 2),
                       "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                    "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": nbytes,
                                    "kernel": "wkv7_f16_sequence_kernel"}}
    del r, v, w, k, kk, a, nkk, kka
    dec = {}
    for B in (1, 8, 64):
        vec = lambda: rn(B, H, N).half()
        rr, ww, kr, vv, aa, gg = vec(), vec(), vec(), vec(), torch.sigmoid(rn(B, H, N)).half(), vec()
        par = lambda: (1.0 + 0.1 * rn(H * N)).half()
        kk_, ka_, rk_, gw_, gb_ = par(), par(), par(), par(), par()
        states = [torch.zeros(B, H, N, N, device="cuda", dtype=torch.float16) for _ in range(16)]
        elapsed = torch.zeros(B, device="cuda", dtype=torch.int32)
        calls = [(lambda s=s: native_fp16_recurrent_output_prepare_raw(
            rr, ww, kr, vv, aa, s, gg, kk_, ka_, rk_, gw_, gb_, elapsed, advance_elapsed=False, eps=1e-5))
            for s in states]
        ms = time_graph(calls, 20)
        nbytes = fp16_decode_bytes(B, H, N)
        gbs = nbytes / (ms / 1e3) / 1e9
        dec[str(B)] = {"us_per_launch": round(ms * 1e3, 3), "bytes": nbytes, "gbs": round(gbs, 1),
                       "frac": round(gbs / HBM_PEAK_GBS, 4)}
        del states
    res["decode_H64"] = dec
    return res


def cpu_scan_baseline(B=8, H=32, N=64, T_sample=1024, seed=0, min_seconds=10.0):
    """The build's fp32 C restatement (OpenMP over heads), repeated for >= min_seconds."""
    import numpy as np
    from oracle import oracle

    oracle.build()
    rng = np.random.default_rng(seed)
    shape = (B, T_sample, H, N)
    r = rng.standard_normal(shape).astype(np.float32)
    k = rng.standard_normal(shape).astype(np.float32)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal(shape).astype(np.float32)
    a = (1 / (1 + np.exp(-rng.standard_normal(shape)))).astype(np.float32)
    w = np.exp(-np.exp(rng.normal(-0.5, 0.5, shape))).astype(np.float32)
    st = np.zeros((B, H, N, N), np.float32)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.wkv7_scan_f32(r, w, k, v, k, a, st)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds:
            break
    return {"value": round(B * T_sample * reps / dt, 1), "unit": "tok/s", "cores": oracle.num_threads(),
            "kind": "port", "cpu": cpu_model(),
            "sample": f"wkv7 scan: fp32 C sequential restatement (OpenMP over heads), B={B} T={T_sample} H={H} "
                      f"N={N}, {reps} reps in {dt:.1f} s"}


# ------------------------------------------------------------------ decode
def config_7p2b():
    from rwkv7mi.model import NativeRWKV7Config

    return NativeRWKV7Config(vocab_size=65536, hidden_size=4096, num_hidden_layers=32, intermediate_size=16384,
                             decay_low_rank_dim=64, a_low_rank_dim=64, gate_low_rank_dim=128, v_low_rank_dim=32,
                             use_native_mm8=True, native_mm8_min_params=8_000_000, native_mm8_policy="memory")


def build_7p2b():
    import torch
    from rwkv7mi.model import NativeRWKV7ForCausalLM, QuantLinear

    cfg = config_7p2b()
    t0 = time.perf_counter()
    model = NativeRWKV7ForCausalLM.from_random(cfg, seed=0, device="cuda", dtype=torch.float16)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    named = {"lm_head": model.lm_head}
    for L in model.layers:
        p = f"model.layers.{L.idx}."
        named.update({p + "attn.r_proj": L.r_proj, p + "attn.k_proj": L.k_proj, p + "attn.v_proj": L.v_proj,
                      p + "attn.o_proj": L.o_proj, p + "ffn.key": L.key, p + "ffn.value": L.value})
    quantized = {n for n, lin in named.items() if isinstance(lin, QuantLinear)}
    _log(f"bench: 7.2B MM8 model built in {build_s:.1f} s ({len(quantized)} MM8 modules)")
    return cfg, model, quantized


def run_decode(model, cfg, quantized, batches=(1, 8, 64), steps=64, warmup=5):
    import torch
    from rwkv7mi import argmax_rows
    from rwkv7mi.model import parameter_shapes

    shapes = parameter_shapes(cfg)
    sbytes = torch.empty(0, dtype=model.state_dtype).element_size()
    res = {}
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    for B in batches:
        prompt = torch.randint(0, cfg.vocab_size, (B, 16), generator=g, device="cuda")
        out = model(prompt)
        cache = out.past_key_values
        runner = model.graph_runner(B)
        # the graph ends with the greedy tokens (argmax of the logits), which it
        # feeds to its own next replay: a timed step is one whole greedy step
        runner.replay_greedy(cache, argmax_rows(out.logits[:, -1]))

        def step():
            runner.replay_greedy(cache)

        ms, wall = time_events(step, steps, warmup)
        nbytes = decode_step_bytes(cfg, B, quantized, shapes, sbytes)
        gbs = nbytes / (ms / 1e3) / 1e9
        res[B] = {"tok_s": B / (ms / 1e3), "ms": ms, "wall_s": wall, "bytes": nbytes, "gbs": gbs,
                  "frac": gbs / HBM_PEAK_GBS}
        _log(f"bench: decode bsz {B} ({'fp16' if sbytes == 2 else 'fp32'} state): {ms:.3f} ms/step, {B / (ms / 1e3):.1f} tok/s, {gbs:.0f} GB/s "
             f"({100 * gbs / HBM_PEAK_GBS:.1f}% of the step roofline)")
        del model._graph_runners[B]
    return res


def run_mm8_roofline(model, cfg, reps=20):
    """The MM8 launches of one bsz-1 decode step (the same modules, shapes and
    buffers) recorded from an eager step, captured alone in a hipGraph and
    replayed back to back between two HIP events on the launch stream: the
    average launch duration and its algorithmic bytes."""
    import torch
    import rwkv7mi.model as model_mod
    from rwkv7mi.model import QuantLinear

    B = 1
    cache = model.new_cache(B)
    toks = torch.zeros(B, dtype=torch.long, device="cuda")
    logits = torch.empty(B, cfg.vocab_size, device="cuda", dtype=torch.float16)
    bufs = model._decode_buffers(B)
    calls, nbytes = [], []
    orig_apply, orig_group, orig_lnmix = QuantLinear.apply, QuantLinear.apply_group, model_mod.mm8_lnmix_multi_into

    def rec_apply(self, x2, out, **kw):
        calls.append(lambda: orig_apply(self, x2, out, **kw))
        nbytes.append(mm8_bytes(self.in_features, self.out_features, int(x2.shape[0])))
        return orig_apply(self, x2, out, **kw)

    def rec_group(lins, xs, outs):
        calls.append(lambda: orig_group(lins, xs, outs))
        nbytes.append(sum(mm8_bytes(l.in_features, l.out_features, int(x.shape[0])) for l, x in zip(lins, xs)))
        return orig_group(lins, xs, outs)

    def rec_lnmix(x, prev, ln_w, ln_b, eps, mixes, mods, outs, **kw):
        # the LN-mix prologue launches (R/K/V and FFN key at one row): weights and
        # metadata, plus the prologue's vectors (x, prev, LN weight and bias,
        # mixes), its extra outputs (h, extra mixes) and, on the R/K/V launch,
        # the LoRA down-projection weights it reads and the fp32 sums it writes
        calls.append(lambda: orig_lnmix(x, prev, ln_w, ln_b, eps, mixes, mods, outs, **kw))
        rows, i = (int(v) for v in x.shape)
        naux = len(kw.get("aux_outs", ()))
        extra = (rows * i + 2 * i + len(mixes) * i + rows * i * (1 if kw.get("h_out") is not None else 0)
                 + naux * (i + rows * i)) * 2
        if kw.get("lora_downs") is not None:
            ranks = sum(int(d.shape[0]) for d in kw["lora_downs"])
            extra += ranks * i * 2 + rows * ranks * 4
        nbytes.append(sum(mm8_bytes(m.in_features, m.out_features, rows) for m in mods) + extra)
        return orig_lnmix(x, prev, ln_w, ln_b, eps, mixes, mods, outs, **kw)

    QuantLinear.apply = rec_apply
    QuantLinear.apply_group = staticmethod(rec_group)
    model_mod.mm8_lnmix_multi_into = rec_lnmix
    try:
        model.decode_step_(toks, cache, logits, bufs)
    finally:
        QuantLinear.apply, QuantLinear.apply_group = orig_apply, staticmethod(orig_group)
        model_mod.mm8_lnmix_multi_into = orig_lnmix
    ms = time_graph(calls, reps)
    per = sum(nbytes) / len(nbytes)
    return {"launches": len(calls), "avg_us": 1e3 * ms, "bytes_per_launch": per, "gbs": per / (ms / 1e3) / 1e9}


def run_prefill(model, cfg, B=8, T=4096, steps=2, warmup=1):
    """configs[4]'s prefill: B x T random tokens through the 7.2B model (the
    chunked scan, the projections, the LoRA and the head on the last token)."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(3)
    ids = torch.randint(0, cfg.vocab_size, (B, T), device="cuda", generator=g)
    ms, wall = time_events(lambda: model(ids), steps, warmup)
    # matmul flops per token: every projection's weights (MM8 and the fp16 LoRA), twice
    D, A, F, L = cfg.hidden_size, cfg.attention_hidden_size, cfg.intermediate_size, cfg.num_hidden_layers
    ranks = cfg.decay_low_rank_dim + cfg.a_low_rank_dim + cfg.gate_low_rank_dim + cfg.v_low_rank_dim
    per_tok = L * (4 * D * A + 2 * D * F + 2 * D * ranks)
    flops = 2 * per_tok * B * T + 2 * B * D * cfg.vocab_size
    tflops = flops / (ms / 1e3) / 1e12
    return {"tok_s": round(B * T / (ms / 1e3), 1), "ms": round(ms, 2), "config": f"B={B} T={T}",
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                         "flops_per_call": flops}}


def cpu_decode_baseline(min_seconds=12.0, max_tokens=64):
    """The fp32 numpy restatement of the per-token model (oracle/model_oracle.py)
    over the whole 7.2B architecture (all 32 layers and the head; fp32 weights,
    29 GB of host memory), bsz 1, timed over whole tokens for about
    ``min_seconds`` after one warm-up token."""
    import numpy as np
    import torch
    from oracle.model_oracle import ModelOracle
    from rwkv7mi.model import parameter_shapes, random_weights

    cfg = config_7p2b()
    w = {}
    for name in parameter_shapes(cfg):  # generated on the GPU one tensor at a time, kept on the host
        w[name] = random_weights(cfg, seed=0, device="cuda", dtype=torch.float32, names=[name])[name].cpu().numpy()
    ora = ModelOracle(cfg, w, dtype=np.float32)
    del w
    st = ora.new_state(1)
    ora.step(np.array([1]), st)
    n, t0 = 0, time.perf_counter()
    while n < max_tokens and (n < 3 or time.perf_counter() - t0 < min_seconds):
        ora.step(np.array([(17 * n) % cfg.vocab_size]), st)
        n += 1
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": host_cores(), "kind": "port", "cpu": cpu_model(),
            "sample": f"7.2B decode bsz 1, all 32 layers + head: fp32 numpy per-token restatement "
                      f"(oracle/model_oracle.py), {n} tokens in {dt:.1f} s"}


# ------------------------------------------------------------------ GEMV legs
def _mods_for(I, O, count, seed):
    import torch
    from rwkv7mi import MM8Linear

    torch.manual_seed(seed)
    mods = []
    for _ in range(count):
        lin = torch.nn.Linear(I, O, bias=False, device="cuda", dtype=torch.float16)
        with torch.no_grad():
            lin.weight.normal_(0.0, 0.02)
        mods.append(MM8Linear(lin))
        del lin
    return mods


def _distinct(nbytes_one):
    """Copies of a weight that keep the rotation beyond the 256 MB last-level cache."""
    return max(2, min(64, -(-(512 << 20) // nbytes_one)))


def run_gemv_c3(reps=20):
    """MM8 at the 1.5B shapes x batch 1 / 8 / 32: per shape and
    batch, a hipGraph of launches over distinct weight copies (so no copy is
    cache-resident), average launch time, algorithmic bytes and HBM fraction."""
    import torch
    from rwkv7mi import workspace as ws
    from rwkv7mi.native_quant_mm8 import GEMV_ROWS, mm8_gemm_workspace_bytes

    out = {}
    for I, O in ((2048, 2048), (2048, 8192), (8192, 2048), (2048, 65536)):
        mods = _mods_for(I, O, _distinct(I * O), seed=I + O)
        for rows in (1, 8, 32):
            if rows > GEMV_ROWS:
                ws.reserve(torch.device("cuda", 0), mm8_gemm_workspace_bytes(1, rows, I, O), slot="mm8g")
            x = torch.randn(rows, I, device="cuda", dtype=torch.float16)
            ys = [torch.empty(rows, O, device="cuda", dtype=torch.float16) for _ in mods]
            calls = [(lambda m=m, y=y: m.rwkv7_forward_into(x, y)) for m, y in zip(mods, ys)]
            torch.cuda.nvtx.range_push(f"MM8 {I}x{O} b{rows}")  # labels the cell in a profiler trace
            ms = time_graph(calls, reps)
            torch.cuda.nvtx.range_pop()
            nb = mm8_bytes(I, O, rows)
            gbs = nb / (ms / 1e3) / 1e9
            out[f"{I}x{O}/b{rows}"] = {"us": round(ms * 1e3, 2), "gbs": round(gbs, 1),
                                       "frac": round(gbs / HBM_PEAK_GBS, 4)}
        del mods
        torch.cuda.empty_cache()
    return out


def run_gemv_c4(reps=20):
    """Group-128 W4 at the 7.2B shapes x batch 1 / 4 / 16, the
    asymmetric (min/max affine) form and the reference's symmetric form."""
    import torch
    from rwkv7mi.sm70_quant import (quantize_w4_affine_groupwise, quantize_w4_groupwise, w4_affine_groupwise_linear,
                                    w4_groupwise_linear)

    out = {}
    for I, O in ((4096, 4096), (4096, 16384), (16384, 4096), (4096, 65536)):
        n = _distinct(I * O // 2)
        g = torch.Generator(device="cuda").manual_seed(I + O)
        packs_a, packs_s = [], []
        for _ in range(n):
            W = torch.randn(O, I, device="cuda", dtype=torch.float16, generator=g) * 0.02
            packs_a.append(quantize_w4_affine_groupwise(W))
            packs_s.append(quantize_w4_groupwise(W))
            del W
        for rows in (1, 4, 16):
            x = torch.randn(rows, I, device="cuda", dtype=torch.float16)
            ys = [torch.empty(rows, O, device="cuda", dtype=torch.float16) for _ in range(n)]
            calls = [(lambda p=p, y=y: w4_affine_groupwise_linear(x, p[0], p[1], p[2], O, I, out=y))
                     for p, y in zip(packs_a, ys)]
            torch.cuda.nvtx.range_push(f"W4 asym {I}x{O} b{rows}")
            ms = time_graph(calls, reps)
            torch.cuda.nvtx.range_pop()
            gbs = w4_bytes(I, O, rows, affine=True) / (ms / 1e3) / 1e9
            calls_s = [(lambda p=p, y=y: w4_groupwise_linear(x, p[0], p[1], O, I, out=y)) for p, y in zip(packs_s, ys)]
            torch.cuda.nvtx.range_push(f"W4 sym {I}x{O} b{rows}")
            ms_s = time_graph(calls_s, reps)
            torch.cuda.nvtx.range_pop()
            gbs_s = w4_bytes(I, O, rows, affine=False) / (ms_s / 1e3) / 1e9
            out[f"{I}x{O}/b{rows}"] = {"asym_us": round(ms * 1e3, 2), "asym_gbs": round(gbs, 1),
                                       "asym_frac": round(gbs / HBM_PEAK_GBS, 4), "sym_us": round(ms_s * 1e3, 2),
                                       "sym_frac": round(gbs_s / HBM_PEAK_GBS, 4)}
        del packs_a, packs_s
        torch.cuda.empty_cache()
    return out


def cpu_gemv_baseline(shapes, batch=1, kind="mm8", min_seconds=1.0):
    """The reference's CPU forms, restated in fp32 numpy and timed on the host
    cores: mm8_matmul dequantises the whole weight and multiplies
    (rwkv7_hf/native_quant_mm8.py:100-119); the sm70 W4 torch fallback does the
    same for the symmetric group format (sm70_quant.py:598-610).  Each shape is
    repeated for about ``min_seconds``; returns microseconds per call."""
    import numpy as np

    rng = np.random.default_rng(0)
    out = {}
    for I, O in shapes:
        x = rng.standard_normal((batch, I)).astype(np.float32)
        if kind == "mm8":
            q = rng.integers(0, 256, (I, O), dtype=np.uint8)
            mx, rx = (rng.random(O, dtype=np.float32) * 0.01 for _ in range(2))
            my, ry = (rng.random((I, 1), dtype=np.float32) * 0.01 for _ in range(2))
            call = lambda: x @ ((q.astype(np.float32) + np.float32(0.5)) * ry * rx + my + mx)
        else:
            pk = rng.integers(0, 256, (O, I // 2), dtype=np.uint8)
            sc = rng.random((O, I // 128), dtype=np.float32) * 0.01

            def call():
                w = np.empty((O, I), np.float32)
                w[:, 0::2] = (pk & 15).astype(np.float32) - 8
                w[:, 1::2] = (pk >> 4).astype(np.float32) - 8
                w *= np.repeat(sc, 128, axis=1)
                return x @ w.T
        call()
        n, t0 = 0, time.perf_counter()
        while n < 2 or time.perf_counter() - t0 < min_seconds:
            call()
            n += 1
        out[f"{I}x{O}/b{batch}"] = round((time.perf_counter() - t0) / n * 1e6, 1)
    return out


def run_c1(prompt=512, steps=64):
    """the RWKV-7 0.1B architecture (L=12, D=768, H=12, FFN 3072,
    vocab 65536), random init seed 0, fp32, bsz 1: a 512-token uniform-random
    prompt, then 64 greedy steps (the decode graph).  Times the prefill and the
    greedy steps separately on the GPU, and the same work with the fp32 numpy
    restatement (oracle/model_oracle.py: sequence-form prefill, per-token
    steps) on the host."""
    import numpy as np
    import torch
    from rwkv7mi.model import NativeRWKV7Config, NativeRWKV7ForCausalLM, parameter_shapes, random_weights

    cfg = NativeRWKV7Config(vocab_size=65536, hidden_size=768, num_hidden_layers=12, intermediate_size=3072,
                            decay_low_rank_dim=64, a_low_rank_dim=64, gate_low_rank_dim=128, v_low_rank_dim=32)
    w = random_weights(cfg, seed=0, device="cpu", dtype=torch.float32)
    model = NativeRWKV7ForCausalLM(cfg, w, device="cuda", dtype=torch.float32)
    ids = torch.tensor(np.random.default_rng(0).integers(0, cfg.vocab_size, (1, prompt)), device="cuda")
    out = model.generate_greedy(ids, steps)  # warm-up: captures the graphs
    torch.cuda.synchronize()
    pre_ms, _ = time_events(lambda: model(ids), 5, 1)
    o = model(ids)
    cache, nxt = o.past_key_values, o.logits[:, -1].argmax(-1)
    runner = model.graph_runner(1)
    runner.replay_greedy(cache, nxt)
    dec_ms, _ = time_events(lambda: runner.replay_greedy(cache), steps, 3)
    shapes = parameter_shapes(cfg)
    nbytes = sum(int(np.prod(s)) * 4 for n, s in shapes.items() if n != "model.embeddings.weight")
    nbytes += cfg.hidden_size * 4 + cfg.num_hidden_layers * (cfg.num_heads * 64 * 64 * 4 * 2
                                                              + 2 * cfg.hidden_size * 4 * 2) + cfg.vocab_size * 4
    gbs = nbytes / (dec_ms / 1e3) / 1e9
    total_ms = pre_ms + steps * dec_ms
    res = {"config": f"0.1B fp32, bsz 1, prompt {prompt} + {steps} greedy steps",
           "prefill_ms": round(pre_ms, 3), "prefill_tok_s": round(prompt / (pre_ms / 1e3), 1),
           "decode_ms_per_step": round(dec_ms, 4), "decode_tok_s": round(1e3 / dec_ms, 1),
           "generate_ms": round(total_ms, 2), "generate_tok_s": round(steps / (total_ms / 1e3), 1),
           "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "decode step (graph)",
                        "step_bytes": nbytes},
           "greedy_ids_head": out[0, prompt:prompt + 8].tolist()}
    del model
    torch.cuda.empty_cache()
    # host: the fp32 restatement, same prompt and step count
    from oracle.model_oracle import ModelOracle

    ora = ModelOracle(cfg, {k: v.numpy() for k, v in w.items()}, dtype=np.float32)
    del w
    t0 = time.perf_counter()
    lg, st = ora.run_seq(ids.cpu().numpy(), keep=1)
    t1 = time.perf_counter()
    tok = np.array([int(lg[0, -1].argmax())])
    for _ in range(steps):
        tok = np.array([int(ora.step(tok, st)[0].argmax())])
    t2 = time.perf_counter()
    res["cpu_baseline"] = {"value": round(steps / (t2 - t0), 2), "unit": "generated tok/s", "cores": host_cores(),
                           "kind": "port", "cpu": cpu_model(),
                           "sample": f"the whole configs[0] run: fp32 numpy restatement (oracle/model_oracle.py), "
                                     f"prefill {prompt} tokens in {t1 - t0:.2f} s, {steps} greedy steps in "
                                     f"{t2 - t1:.2f} s"}
    return res


# ------------------------------------------------------------------ counter workloads
TRAFFIC_JSON = ROOT / "profiles" / "traffic.json"
COPY_BYTES = 256 << 20


def _traffic_gemv(key):
    """HBM bytes per launch of a configs[2]/[3] head cell from profiles/traffic_gemv.json, or None."""
    try:
        return json.loads((ROOT / "profiles" / "traffic_gemv.json").read_text())["traffic_bytes_per_launch"][key]
    except (OSError, ValueError, KeyError):
        return None


def _traffic():
    """HBM bytes per MM8 launch measured by the counter runs (profiles/traffic.json), or None."""
    try:
        return json.loads(TRAFFIC_JSON.read_text())["traffic_bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        return None


def _calibration_copy():
    import torch

    src = torch.ones(COPY_BYTES // 2, device="cuda", dtype=torch.float16)
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()


def run_traffic():
    """Kernels for the HBM-traffic counters: two eager bsz-1 decode steps of the
    7.2B MM8 model (the second is the measured one) and one elementwise copy of
    COPY_BYTES (read and written once) that calibrates FETCH_SIZE / WRITE_SIZE.
    Run under ``rocprofv3 --pmc FETCH_SIZE`` and then ``--pmc WRITE_SIZE``."""
    import torch

    cfg, model, _ = build_7p2b()
    cache = model.new_cache(1)
    toks = torch.zeros(1, dtype=torch.long, device="cuda")
    logits = torch.empty(1, cfg.vocab_size, device="cuda", dtype=torch.float16)
    bufs = model._decode_buffers(1)
    for _ in range(2):
        model.decode_step_(toks, cache, logits, bufs)
    _calibration_copy()
    _log("bench: traffic workload done (2 decode steps + calibration copy)")


def run_scan_traffic(H=32):
    """Kernels for the scan's counter runs: two chunked-scan calls at B=8,
    T=4096 (the second is the measured one) and the COPY_BYTES calibration copy."""
    from rwkv7mi import self_chunk_rwkv7

    inputs = make_scan_inputs(8, 4096, H, 64)
    for _ in range(2):
        self_chunk_rwkv7(*inputs, chunk_size=16)
    _calibration_copy()
    _log(f"bench: scan traffic workload done (H={H}: 2 scan calls + calibration copy)")


def _counter_rows(path):
    import csv

    with open(path) as f:
        return list(csv.DictReader(f))


def summarize_traffic(fetch_csv, write_csv, out=TRAFFIC_JSON, kernel="mm8t_kernel"):
    """Per-launch HBM bytes of ``kernel``'s launches in the second half of the
    run (the second of its two identical passes) from the two counter runs,
    scaled by what the counters read for the copy kernel of known size; writes ``out``."""
    def per_dispatch(path, counter):
        rows = [r for r in _counter_rows(path) if r.get("Counter_Name") == counter]
        rows.sort(key=lambda r: int(r["Dispatch_Id"]))
        ks = [float(r["Counter_Value"]) * 1024 for r in rows if kernel in r["Kernel_Name"]]
        copy = [float(r["Counter_Value"]) * 1024 for r in rows if "neg" in r["Kernel_Name"]]
        return ks[len(ks) // 2:], copy[-1]
    f_k, f_copy = per_dispatch(fetch_csv, "FETCH_SIZE")
    w_k, w_copy = per_dispatch(write_csv, "WRITE_SIZE")
    ff, fw = COPY_BYTES / f_copy, COPY_BYTES / w_copy
    n = len(f_k)
    res = {"kernel": kernel, "launches": n, "traffic_bytes_per_launch": round((sum(f_k) * ff + sum(w_k) * fw) / n),
           "fetch_bytes_per_launch": round(sum(f_k) * ff / n), "write_bytes_per_launch": round(sum(w_k) * fw / n),
           "fetch_scale": ff, "write_scale": fw, "copy_bytes": COPY_BYTES,
           "source": f"rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs ({Path(fetch_csv).parent.name}, "
                     f"{Path(write_csv).parent.name})"}
    try:  # the kernels' source revision, when summarised inside the git checkout
        import subprocess

        res["kernels_at_commit"] = subprocess.run(["git", "rev-parse", "--short", "HEAD"], cwd=ROOT, check=True,
                                                  capture_output=True, text=True).stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        pass
    Path(out).parent.mkdir(parents=True, exist_ok=True)
    Path(out).write_text(json.dumps(res, indent=1) + "\n")
    print(json.dumps(res))
    return res


# ------------------------------------------------------------------ main
def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="all",
                    choices=["all", "decode", "scan", "gemv", "prefill", "c1", "fp16state", "traffic",
                             "scan_traffic"])
    ap.add_argument("--summarize-traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write a traffic summary from two rocprofv3 --pmc counter CSVs and exit")
    ap.add_argument("--traffic-kernel", default="mm8t_kernel")
    ap.add_argument("--traffic-out", default=str(TRAFFIC_JSON))
    ap.add_argument("--heads", default="32,64", help="scan head counts (configs[1]: 32; north star: 64)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--batches", default="1,8,64", help="decode batch sizes (1 is the headline)")
    args = ap.parse_args(argv)
    if args.summarize_traffic:
        summarize_traffic(*args.summarize_traffic, out=args.traffic_out, kernel=args.traffic_kernel)
        return 0
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is described in DESIGN.md and not run.", file=sys.stderr)
        return 2

    import torch

    torch.cuda.set_device(0)
    heads = [int(h) for h in args.heads.split(",")]
    if args.workload == "traffic":
        run_traffic()
        return 0
    if args.workload == "scan_traffic":
        run_scan_traffic(heads[0])
        return 0
    wl = args.workload
    scans = {}
    step = None
    if wl in ("all", "scan"):
        for H in heads:
            s = run_scan(H=H, steps=min(args.steps, 20), warmup=min(args.warmup, 3))
            scans[H] = s
            _log(f"bench: scan {s['config']}: {s['ms']:.3f} ms, {s['tok_s'] / 1e6:.1f} M tok/s, "
                 f"{100 * s['frac']:.1f}% of HBM roofline")
        step = run_decode_form_step()
        _log(f"bench: decode-form step {step['config']}: {step['us_per_step']} us ({100 * step['frac']:.1f}%)")
    dec = mk = pre = dec16 = None
    if wl in ("all", "decode", "prefill"):
        cfg, model, quantized = build_7p2b()
        if wl in ("all", "decode"):
            dec = run_decode(model, cfg, quantized, tuple(int(b) for b in args.batches.split(",")), args.steps,
                             args.warmup)
            mk = run_mm8_roofline(model, cfg)
            _log(f"bench: MM8 launches of a bsz-1 step: {mk['avg_us']:.2f} us avg, {mk['gbs']:.0f} GB/s")
            # the opt-in fp16-state lane through the same model (the reference's
            # own comparison is 7.2B B8 decode with fp32 vs fp16 state)
            model.state_dtype = torch.float16
            dec16 = run_decode(model, cfg, quantized, tuple(int(b) for b in args.batches.split(",")),
                               min(args.steps, 32), min(args.warmup, 3))
            model.state_dtype = torch.float32
        if wl in ("all", "prefill"):
            pre = run_prefill(model, cfg)
            _log(f"bench: prefill {pre['config']}: {pre['ms']:.1f} ms, {pre['tok_s']:.0f} tok/s, "
                 f"{pre['roofline']['achieved']} TFLOP/s")
        del model
        torch.cuda.empty_cache()
    c3 = c4 = c1 = None
    if wl in ("all", "gemv"):
        c3 = run_gemv_c3()
        _log("bench: configs[2] MM8: " + ", ".join(f"{k} {v['us']}us" for k, v in c3.items()))
        c4 = run_gemv_c4()
        _log("bench: configs[3] W4: " + ", ".join(f"{k} {v['asym_us']}us" for k, v in c4.items()))
    f16 = None
    if wl in ("all", "fp16state"):
        f16 = run_fp16_state()
        _log(f"bench: fp16-state sequence {f16['sequence']['config']}: {f16['sequence']['ms_per_call']} ms "
             f"({100 * f16['sequence']['roofline']['frac']:.1f}% of HBM); decode H=64: "
             + ", ".join(f"bsz{b} {d['us_per_launch']}us" for b, d in f16["decode_H64"].items()))
    if wl in ("all", "c1"):
        c1 = run_c1()
        _log(f"bench: configs[0] 0.1B fp32: prefill {c1['prefill_ms']} ms, decode {c1['decode_ms_per_step']} ms/step, "
             f"generate {c1['generate_tok_s']} tok/s (host restatement {c1['cpu_baseline']['value']} tok/s)")

    out: dict = {}
    if dec is not None and 1 in dec:
        d1 = dec[1]
        out = {
            "metric": "decode tok/s 7.2B MM8 bsz1 (bsz 8 and 64, wkv7 prefill tok/s and the other configs alongside)",
            "value": round(d1["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(d1["ms"], 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f16 activations / u8 MM8 weights / f32 state",
            "data": "synthetic: random-init weights (seed 0), random token ids",
            "config": {"workload": "RWKV-7 7.2B MM8 hipGraph decode (BASELINE.json configs[4])", "layers": 32,
                       "hidden": 4096, "heads": 64, "ffn": 16384, "vocab": 65536, "global_batch": 1,
                       "parallelism": "single-gpu"},
            "roofline": {"bound": "hbm", "achieved": round(mk["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(mk["gbs"] / HBM_PEAK_GBS, 4), "traffic": _traffic(), "kernel": "mm8t_kernel",
                         "avg_launch_us": round(mk["avg_us"], 3), "bytes_per_launch": round(mk["bytes_per_launch"]),
                         "launches_per_step": mk["launches"]},
            "decode": {str(b): {"tok_s": round(dec[b]["tok_s"], 2), "ms_per_step": round(dec[b]["ms"], 4),
                                "step_bytes": dec[b]["bytes"], "step_gbs": round(dec[b]["gbs"], 1),
                                "step_roofline_frac": round(dec[b]["frac"], 4)} for b in dec},
        }
    elif dec is not None:
        out = {"decode": {str(b): {"tok_s": round(dec[b]["tok_s"], 2), "ms_per_step": round(dec[b]["ms"], 4),
                                   "step_roofline_frac": round(dec[b]["frac"], 4)} for b in dec}}
    if scans:
        scan_out = {f"H{H}": {"tok_s": round(s["tok_s"], 1), "ms_per_call": round(s["ms"], 4), "config": s["config"],
                              "roofline": {"bound": "hbm", "achieved": round(s["gbs"], 1), "peak": HBM_PEAK_GBS,
                                           "unit": "GB/s", "frac": round(s["frac"], 4),
                                           "algorithmic_bytes": s["bytes"], "kernel": "wkv7_chunk_kernel"}}
                    for H, s in scans.items()}
        if not out:
            s = scans[heads[0]]
            out = {"metric": "wkv7 prefill tok/s (chunked DPLR scan, BASELINE.json configs[1])",
                   "value": round(s["tok_s"], 1), "unit": "tok/s", "n_gpus": 1, "steps": min(args.steps, 20),
                   "warmup": min(args.warmup, 3), "ms_per_step": round(s["ms"], 4), "higher_is_better": True,
                   "scaling": "weak", "vs_baseline": None, "dtype": "f16 in / f32 state",
                   "data": "synthetic (configs[1] distribution, seed 0)",
                   "config": {"workload": f"wkv7_scan_op {s['config']}", "parallelism": "single-gpu"},
                   "roofline": scan_out[f"H{heads[0]}"]["roofline"]}
        out["wkv7_prefill"] = scan_out
    if step:
        out["wkv7_decode_form_step"] = step
    if pre:
        out["prefill_c5"] = pre
    c3_shapes = ((2048, 2048), (2048, 8192), (8192, 2048), (2048, 65536))
    c4_shapes = ((4096, 4096), (4096, 16384), (16384, 4096), (4096, 65536))
    if c3:
        head = c3["2048x65536/b1"]
        out["mm8_c3"] = {"shapes": c3, "roofline": {
            "bound": "hbm", "achieved": head["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": head["frac"],
            "traffic": _traffic_gemv("mm8t_kernel MM8 2048x65536 b1"), "kernel": "mm8t_kernel", "shape": "2048x65536/b1",
            "bytes_per_launch": mm8_bytes(2048, 65536, 1), "avg_launch_us": head["us"]}}
    if c4:
        head = c4["4096x65536/b1"]
        out["w4_c4"] = {"shapes": c4, "roofline": {
            "bound": "hbm", "achieved": head["asym_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": head["asym_frac"], "traffic": _traffic_gemv("w4t_kernel W4 asym 4096x65536 b1"), "kernel": "w4t_kernel",
            "shape": "4096x65536/b1 asymmetric",
            "bytes_per_launch": w4_bytes(4096, 65536, 1, affine=True), "avg_launch_us": head["asym_us"]}}
    if c1:
        out["c1_0p1b"] = c1
    if f16 or dec16:
        out["wkv7_fp16_state"] = dict(f16 or {})
        if dec16:
            out["wkv7_fp16_state"]["decode_7p2b"] = {
                str(b): {"tok_s": round(d["tok_s"], 2), "ms_per_step": round(d["ms"], 4),
                         "fp32_state_ms_per_step": round(dec[b]["ms"], 4) if dec and b in dec else None,
                         "step_roofline_frac": round(d["frac"], 4)} for b, d in dec16.items()}
    if not args.no_cpu and out:
        for key, shapes, kind, bytes_of in (("mm8_c3", c3_shapes, "mm8", lambda i, o: mm8_bytes(i, o, 1)),
                                            ("w4_c4", c4_shapes, "w4", lambda i, o: w4_bytes(i, o, 1, affine=False))):
            if key in out:
                us = cpu_gemv_baseline(shapes, kind=kind)
                tot = sum(us.values())
                out[key]["cpu_baseline"] = {
                    "value": round(sum(bytes_of(i, o) for i, o in shapes) / (tot / 1e6) / 1e9, 2), "unit": "GB/s",
                    "cores": host_cores(), "kind": "port", "cpu": cpu_model(), "us_per_call": us,
                    "sample": ("fp32 numpy dequantise + matmul per call (the reference's CPU form), each shape "
                               "at batch 1 for about 1 s" + ("" if kind == "mm8" else "; symmetric group-128 W4"))}
        if dec is not None:
            out["cpu_baseline"] = cpu_decode_baseline()
        if scans:
            cs = cpu_scan_baseline()
            if dec is None:
                out["cpu_baseline"] = cs
            else:
                out["wkv7_prefill"]["cpu_baseline"] = cs
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
