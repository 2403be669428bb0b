#!/usr/bin/env python3
"""Benchmark of the rwkv7mi hot path on one MI355X (BASELINE.json metric:
"decode tok/s 7.2B MM8 bsz1/8; wkv7 prefill tok/s; % HBM roofline").

Workloads (synthetic inputs, random-init weights; nothing is downloaded):
  decode : RWKV-7 7.2B architecture (L=32, D=4096,
           H=64, N=64, F=16384, V=65536, LoRA 64/64/128/32) with MM8 weights
           (memory policy: every Linear >= 8M weights), fp16 activations, fp32
           state; a 16-token prefill, then hipGraph-replayed greedy decode steps
           at bsz 1, 8 and 64.  One step = one token for every row, the full model.
  scan   : the wkv7 chunked prefill scan: B=8, T=4096, H=32, N=64,
           r,k,v ~ N(0,1) fp16, k L2-normalised, kk = k, a = sigmoid(N(0,1)),
           w = exp(-exp(x)), x ~ N(-0.5, 0.5), fp32 state from zero.
The default run measures both and prints ONE JSON line whose ``value`` is the
bsz-1 decode throughput; bsz 8 and 64 and the scan are reported alongside.

    python bench.py [--steps K] [--warmup W] [--workload decode|scan|all] [--no-cpu]
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


# ------------------------------------------------------------------ byte models
def scan_bytes(B, T, H, N):
    """Algorithmic HBM bytes of one scan call: per (token, head, channel)
    r,k,v,kk,a fp16 (10 B) + w fp32 (4 B) in, y fp16 (2 B) out; plus the fp32
    state read and written once."""
    return B * T * H * N * 16 + 2 * B * H * N * N * 4


def decode_step_bytes(cfg, B, quantized: set[str], shapes: dict):
    """Algorithmic HBM bytes of one decode step: every weight read once (MM8:
    1 B/weight + fp16 row/col metadata; others fp16), the recurrent state read +
    written, shift states read + written, embedding rows and logits."""
    total = 0
    mm8 = 0
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
            b = o * i + 2 * (i + o) * 2
            mm8 += b + B * (i + o) * 2
            total += b
        else:
            total += n * 2
    L, H, N, D = cfg.num_hidden_layers, cfg.num_heads, cfg.head_dim, cfg.hidden_size
    total += L * B * H * N * N * 4 * 2          # state read + write
    total += L * 2 * B * D * 2 * 2               # xpa / xpf read + write
    total += B * cfg.vocab_size * 2               # logits
    return total, mm8


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


def time_events(fn, steps, warmup):
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


def run_scan(B=8, T=4096, H=32, steps=20, warmup=3):
    from rwkv7mi import self_chunk_rwkv7

    N = 64
    inputs = make_scan_inputs(B, T, H, N)
    ms, wall = time_events(lambda: self_chunk_rwkv7(*inputs, chunk_size=16), steps, warmup)
    nbytes = scan_bytes(B, T, H, N)
    gbs = nbytes / (ms / 1e3) / 1e9
    return {"tok_s": B * T / (ms / 1e3), "ms": ms, "wall_s": wall, "bytes": nbytes, "gbs": gbs,
            "frac": gbs / HBM_PEAK_GBS, "config": f"B={B} T={T} H={H} N={N} chunk=16"}


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
    return {"value": B * T_sample * reps / dt, "unit": "tok/s", "cores": oracle.num_threads(), "kind": "port",
            "sample": f"wkv7 scan: fp32 C sequential restatement (OpenMP over heads), B={B} T={T_sample} H={H} "
                      f"N={N}, {reps} reps in {dt:.1f} s"}


# ------------------------------------------------------------------ decode
def config_7p2b():
    from rwkv7mi.model import NativeRWKV7Config

    return NativeRWKV7Config(vocab_size=65536, hidden_size=4096, num_hidden_layers=32, intermediate_size=16384,
                             decay_low_rank_dim=64, a_low_rank_dim=64, gate_low_rank_dim=128, v_low_rank_dim=32,
                             use_native_mm8=True, native_mm8_min_params=8_000_000, native_mm8_policy="memory")


def run_decode(batches=(1, 8), steps=64, warmup=5, log=print):
    import torch
    from rwkv7mi.model import NativeRWKV7ForCausalLM, QuantLinear, parameter_shapes

    cfg = config_7p2b()
    t0 = time.perf_counter()
    model = NativeRWKV7ForCausalLM.from_random(cfg, seed=0, device="cuda", dtype=torch.float16)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    log(f"bench: 7.2B MM8 model built in {build_s:.1f} s ({model._rwkv7_native_mm_replaced_modules} MM8 modules)")
    shapes = parameter_shapes(cfg)
    quantized = set()
    named = {"lm_head": model.lm_head}
    for L in model.layers:
        p = f"model.layers.{L.idx}."
        named.update({p + "attn.r_proj": L.r_proj, p + "attn.k_proj": L.k_proj, p + "attn.v_proj": L.v_proj,
                      p + "attn.o_proj": L.o_proj, p + "ffn.key": L.key, p + "ffn.value": L.value})
    for n, lin in named.items():
        if isinstance(lin, QuantLinear):
            quantized.add(n)
    res = {"build_s": build_s, "mm8_modules": len(quantized)}
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    for B in batches:
        prompt = torch.randint(0, cfg.vocab_size, (B, 16), generator=g, device="cuda")
        out = model(prompt)
        logits, cache = out.logits, out.past_key_values
        runner = model.graph_runner(B)
        tok = logits[:, -1].argmax(-1)
        state = {"tok": tok}

        def step():
            lg = runner.replay(state["tok"], cache)
            state["tok"] = lg.argmax(-1)

        ms, wall = time_events(step, steps, warmup)
        nbytes, mm8b = decode_step_bytes(cfg, B, quantized, shapes)
        gbs = nbytes / (ms / 1e3) / 1e9
        res[B] = {"tok_s": B / (ms / 1e3), "ms": ms, "wall_s": wall, "bytes": nbytes, "gbs": gbs,
                  "frac": gbs / HBM_PEAK_GBS}
        log(f"bench: decode bsz {B}: {ms:.3f} ms/step, {B / (ms / 1e3):.1f} tok/s, {gbs:.0f} GB/s")
    # MM8 GEMV roofline: the MM8 launches of one bsz-1 decode step (the same
    # modules, shapes and buffers), captured alone in a hipGraph and replayed
    # back to back between two HIP events on the launch stream; the average
    # launch duration is the elapsed time over all launches.
    B = 1
    cache = model.new_cache(B)
    toks = torch.zeros(B, dtype=torch.long, device="cuda")
    logits = torch.empty(B, cfg.vocab_size, device="cuda", dtype=torch.float16)
    bufs = model._decode_buffers(B)
    calls, nbytes = [], []
    orig_apply, orig_group = QuantLinear.apply, QuantLinear.apply_group

    def mm8_bytes(lin, rows):
        i, o = lin.in_features, lin.out_features
        return o * i + 2 * (i + o) * 2 + rows * (i + o) * 2

    def rec_apply(self, x2, out, **kw):
        calls.append(lambda: orig_apply(self, x2, out, **kw))
        nbytes.append(mm8_bytes(self, int(x2.shape[0])))
        return orig_apply(self, x2, out, **kw)

    def rec_group(lins, xs, outs):
        calls.append(lambda: orig_group(lins, xs, outs))
        nbytes.append(sum(mm8_bytes(l, int(x.shape[0])) for l, x in zip(lins, xs)))
        return orig_group(lins, xs, outs)

    import rwkv7mi.model as model_mod
    orig_lnmix = model_mod.mm8_lnmix_multi_into

    def rec_lnmix(x, prev, ln_w, ln_b, eps, mixes, mods, outs, **kw):
        # the LN-mix prologue launches (R/K/V and FFN key at one row): weights and
        # metadata as above, plus the prologue's vectors (x, prev, LN weight and
        # bias, mixes) and its extra outputs (h, extra mixes)
        calls.append(lambda: orig_lnmix(x, prev, ln_w, ln_b, eps, mixes, mods, outs, **kw))
        rows, i = (int(v) for v in x.shape)
        naux = len(kw.get("aux_outs", ()))
        extra = (rows * i + 2 * i + len(mixes) * i + rows * i * (1 if kw.get("h_out") is not None else 0)
                 + naux * (i + rows * i)) * 2
        nbytes.append(sum(mm8_bytes(m, rows) for m in mods) + extra)
        return orig_lnmix(x, prev, ln_w, ln_b, eps, mixes, mods, outs, **kw)

    QuantLinear.apply = rec_apply
    QuantLinear.apply_group = staticmethod(rec_group)
    model_mod.mm8_lnmix_multi_into = rec_lnmix
    try:
        model.decode_step_(toks, cache, logits, bufs)
    finally:
        QuantLinear.apply, QuantLinear.apply_group = orig_apply, staticmethod(orig_group)
        model_mod.mm8_lnmix_multi_into = orig_lnmix
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
    reps = 20
    graph.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        graph.replay()
    e1.record(st)
    torch.cuda.synchronize()
    tot_ms = e0.elapsed_time(e1)
    n = reps * len(calls)
    tot_b = reps * sum(nbytes)
    res["mm8_kernel"] = {"launches": len(calls), "avg_us": 1e3 * tot_ms / n,
                         "bytes_per_launch": tot_b / n, "gbs": tot_b / (tot_ms / 1e3) / 1e9}
    del graph
    return res


def cpu_decode_baseline(min_seconds=10.0):
    """fp32 numpy restatement of the per-token model (oracle/model_oracle.py) on a
    bounded slice of the 7.2B shapes: 2 of the 32 layers + head, bsz 1; the
    per-token time is scaled to 32 layers."""
    import numpy as np
    import torch
    from oracle.model_oracle import ModelOracle
    from rwkv7mi.model import NativeRWKV7Config, random_weights

    full = config_7p2b()
    cfg = NativeRWKV7Config(vocab_size=full.vocab_size, hidden_size=full.hidden_size, num_hidden_layers=2,
                            intermediate_size=full.intermediate_size)
    w = random_weights(cfg, seed=0, device="cpu", dtype=torch.float32)
    ora = ModelOracle(cfg, {k: v.numpy() for k, v in w.items()}, dtype=np.float32)
    del w
    st = ora.new_state(1)
    ora.step(np.array([1]), st)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < min_seconds:
        ora.step(np.array([n % 1000]), st)
        n += 1
    per_tok = (time.perf_counter() - t0) / n
    xh = np.ones((1, cfg.hidden_size), np.float32)
    m, t0 = 0, time.perf_counter()
    while m < 3 or time.perf_counter() - t0 < 1.0:
        ora.head(xh)
        m += 1
    t_head = (time.perf_counter() - t0) / m
    t_layer = max(per_tok - t_head, 0.0) / cfg.num_hidden_layers
    est = t_layer * full.num_hidden_layers + t_head
    return {"value": 1.0 / est, "unit": "tok/s", "cores": int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)),
            "kind": "port",
            "sample": f"7.2B decode bsz 1: fp32 numpy per-token restatement (oracle/model_oracle.py) of 2 of 32 "
                      f"layers + head, {n} tokens ({per_tok * 1e3:.0f} ms/token, head {t_head * 1e3:.0f} ms); "
                      f"per-layer time scaled to 32 layers"}


TRAFFIC_JSON = Path(__file__).resolve().parent / "profiles" / "traffic.json"


def _traffic():
    """HBM bytes per MM8 launch measured by the counter runs (profiles/traffic.json), or None."""
    try:
        return json.loads(TRAFFIC_JSON.read_text())["traffic_bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        return None
COPY_BYTES = 256 << 20


def run_traffic():
    """Kernels for the HBM-traffic counters: two eager bsz-1 decode steps of the
    7.2B MM8 model (the second is the measured one) and one elementwise copy of
    COPY_BYTES (read and written once) that calibrates FETCH_SIZE / WRITE_SIZE.
    Run under ``rocprofv3 --pmc FETCH_SIZE`` and then ``--pmc WRITE_SIZE``."""
    import torch
    from rwkv7mi.model import NativeRWKV7ForCausalLM

    cfg = config_7p2b()
    model = NativeRWKV7ForCausalLM.from_random(cfg, seed=0, device="cuda", dtype=torch.float16)
    cache = model.new_cache(1)
    toks = torch.zeros(1, dtype=torch.long, device="cuda")
    logits = torch.empty(1, cfg.vocab_size, device="cuda", dtype=torch.float16)
    bufs = model._decode_buffers(1)
    for _ in range(2):
        model.decode_step_(toks, cache, logits, bufs)
    src = torch.ones(COPY_BYTES // 2, device="cuda", dtype=torch.float16)
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print("bench: traffic workload done (2 decode steps + calibration copy)", file=sys.stderr, flush=True)


def run_scan_traffic(H=32):
    """Kernels for the scan's counter runs: two chunked-scan calls at B=8,
    T=4096 (the second is the measured one) and the COPY_BYTES calibration copy."""
    import torch
    from rwkv7mi import self_chunk_rwkv7

    inputs = make_scan_inputs(8, 4096, H, 64)
    for _ in range(2):
        self_chunk_rwkv7(*inputs, chunk_size=16)
    src = torch.ones(COPY_BYTES // 2, device="cuda", dtype=torch.float16)
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(f"bench: scan traffic workload done (H={H}: 2 scan calls + calibration copy)", file=sys.stderr, flush=True)


def _counter_rows(path):
    import csv

    with open(path) as f:
        return list(csv.DictReader(f))


def summarize_traffic(fetch_csv, write_csv, out=TRAFFIC_JSON):
    """Per-launch HBM bytes of the decode step's MM8 GEMV launches from the two
    counter runs, scaled by the copy kernel's known bytes; writes ``out``."""
    def per_dispatch(path, counter):
        rows = [r for r in _counter_rows(path) if r.get("Counter_Name") == counter]
        rows.sort(key=lambda r: int(r["Dispatch_Id"]))
        mm8 = [float(r["Counter_Value"]) * 1024 for r in rows if "mm8t_kernel" in r["Kernel_Name"]]
        copy = [float(r["Counter_Value"]) * 1024 for r in rows if "neg" in r["Kernel_Name"]]
        half = len(mm8) // 2  # two decode steps: keep the second
        return mm8[half:], copy[-1]
    f_mm8, f_copy = per_dispatch(fetch_csv, "FETCH_SIZE")
    w_mm8, w_copy = per_dispatch(write_csv, "WRITE_SIZE")
    ff, fw = COPY_BYTES / f_copy, COPY_BYTES / w_copy
    n = len(f_mm8)
    traffic = (sum(f_mm8) * ff + sum(w_mm8) * fw) / n
    res = {"kernel": "mm8t_kernel", "launches_per_step": n, "traffic_bytes_per_launch": round(traffic),
           "fetch_bytes_per_launch": round(sum(f_mm8) * ff / n), "write_bytes_per_launch": round(sum(w_mm8) * fw / n),
           "fetch_scale": ff, "write_scale": fw, "copy_bytes": COPY_BYTES,
           "source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of bench.py --workload traffic"}
    Path(out).parent.mkdir(parents=True, exist_ok=True)
    Path(out).write_text(json.dumps(res, indent=1) + "\n")
    print(json.dumps(res))
    return res


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=["all", "decode", "scan", "traffic", "scan_traffic"], default="all")
    ap.add_argument("--summarize-traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write profiles/traffic.json from two rocprofv3 --pmc counter CSVs and exit")
    ap.add_argument("--heads", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--batches", default="1,8,64", help="decode batch sizes (1 is the headline)")
    args = ap.parse_args(argv)
    if args.summarize_traffic:
        summarize_traffic(*args.summarize_traffic)
        return 0
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is described in DESIGN.md and not run.", file=sys.stderr)
        return 2

    import torch

    torch.cuda.set_device(0)
    log = lambda m: print(m, file=sys.stderr, flush=True)
    if args.workload == "traffic":
        run_traffic()
        return 0
    if args.workload == "scan_traffic":
        run_scan_traffic(args.heads)
        return 0
    out: dict = {}
    scan = dec = None
    if args.workload in ("all", "scan"):
        scan = run_scan(H=args.heads, steps=min(args.steps, 20), warmup=min(args.warmup, 3))
        log(f"bench: scan {scan['config']}: {scan['ms']:.3f} ms, {scan['tok_s'] / 1e6:.1f} M tok/s, "
            f"{100 * scan['frac']:.1f}% of HBM roofline")
    if args.workload in ("all", "decode"):
        dec = run_decode(batches=tuple(int(b) for b in args.batches.split(",")), steps=args.steps,
                         warmup=args.warmup, log=log)
    if dec is not None and 1 not in dec:  # a partial sweep without the headline batch size
        print(json.dumps({"decode": {str(b): {"tok_s": round(dec[b]["tok_s"], 2), "ms_per_step": round(dec[b]["ms"], 4),
                                              "step_roofline_frac": round(dec[b]["frac"], 4)}
                                     for b in dec if isinstance(b, int)}}), flush=True)
        return 0
    if dec is not None:
        d1 = dec[1]
        mk = dec["mm8_kernel"]
        out = {
            "metric": "decode tok/s 7.2B MM8 bsz1 (bsz 8 and 64 and wkv7 prefill tok/s alongside)",
            "value": round(d1["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(d1["ms"], 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f16 activations / u8 MM8 weights / f32 state",
            "data": "synthetic: random-init weights (seed 0), random token ids",
            "config": {"workload": "RWKV-7 7.2B MM8 hipGraph decode (BASELINE.json configs[4])", "layers": 32,
                       "hidden": 4096, "heads": 64, "ffn": 16384, "vocab": 65536, "global_batch": 1,
                       "parallelism": "single-gpu"},
            "roofline": {"bound": "hbm", "achieved": round(mk["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(mk["gbs"] / HBM_PEAK_GBS, 4), "traffic": _traffic(), "kernel": "mm8t_kernel",
                         "avg_launch_us": round(mk["avg_us"], 3),
                         "bytes_per_launch": round(mk["bytes_per_launch"]), "launches_per_step": mk["launches"]},
            "decode": {str(b): {"tok_s": round(dec[b]["tok_s"], 2), "ms_per_step": round(dec[b]["ms"], 4),
                                "step_bytes": dec[b]["bytes"], "step_gbs": round(dec[b]["gbs"], 1),
                                "step_roofline_frac": round(dec[b]["frac"], 4)}
                       for b in dec if isinstance(b, int)},
        }
    if scan is not None:
        s = {"tok_s": round(scan["tok_s"], 1), "ms_per_call": round(scan["ms"], 4), "config": scan["config"],
             "roofline": {"bound": "hbm", "achieved": round(scan["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(scan["frac"], 4), "algorithmic_bytes": scan["bytes"],
                          "kernel": "wkv7_chunk_kernel"}}
        if not out:
            out = {"metric": "wkv7 prefill tok/s (chunked DPLR scan, BASELINE.json configs[1])",
                   "value": s["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": min(args.steps, 20),
                   "warmup": min(args.warmup, 3), "ms_per_step": s["ms_per_call"], "higher_is_better": True,
                   "scaling": "weak", "vs_baseline": None, "dtype": "f16 in / f32 state",
                   "data": "synthetic (configs[1] distribution, seed 0)",
                   "config": {"workload": f"wkv7_scan_op {scan['config']}", "parallelism": "single-gpu"},
                   "roofline": s["roofline"]}
        else:
            out["wkv7_prefill"] = s
    if not args.no_cpu:
        if dec is not None:
            out["cpu_baseline"] = cpu_decode_baseline()
            if scan is not None:
                out["wkv7_prefill"]["cpu_baseline"] = cpu_scan_baseline()
        else:
            out["cpu_baseline"] = cpu_scan_baseline()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
