#!/usr/bin/env python3
"""Benchmark of the MI355X MoE expert path: one GLM-5.3-style K4 trellis MoE layer, batch-1 decode.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu] [--no-prefill] [--config 0..4]

Default (--config 0): one step = one token through the whole layer (router GEMV, bias-corrected top-8, eight routed
experts plus the shared expert as K4-trellis decode GEMVs with SwiGLU, weighted combine and
residual) -- one launch of the fused decode kernel.  Inputs and weights are resident in HBM before
timing starts.  Several independently seeded layers (expert and router weights) are rotated, and
tokens vary, so consecutive steps stream different bytes instead of re-reading the 256 MB
last-level cache.

Prints ONE JSON line.  `value` is decode tokens/s; `us_per_token`, achieved algorithmic HBM GB/s
and the roofline of the fused layer kernel (timed with HIP events on its launch stream) are
reported beside it.  The same line carries the metric's prefill half (`prefill`: a 512-token
chunk through the joined-MXFP4 layer, tokens/s) and the CPU baseline (the C restatement with fp32
accumulation, built with -march=native for this host, timed on all its cores).

The other workloads of the same path are measured with --config N (same JSON shape, whole-step
timing with HIP events):
  1  joined-MXFP4 layer, batch-1 decode (router + MXFP4 gate_up/down GEMVs + combine)
  2  8-token speculative-verify batch through the K4 layer (correlated rows, experts deduplicated)
  3  512-token prefill chunk through the joined-MXFP4 layer (Zipf-skewed routing, grouped GEMMs)
  4  20 consecutive K4 layers (RMSNorm'd residual each), batch-1 decode
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

H, M, E = 6144, 2048, 257
TRELLIS = H * M // 2                      # bytes per expert projection (K4 = 4 bits/weight)
# Algorithmic bytes per token (batch 1): 9 experts x 3 projections of trellis + router weight +
# side vectors + bias + activations in/out.
BYTES_TOKEN = 9 * 3 * TRELLIS + 256 * H * 4 + 9 * 3 * (H + M) * 2 + 256 * 4 + 3 * H * 2
HBM_PEAK_GBPS = 8000.0
METRIC = "MoE-layer decode µs/token + HBM GB/s (K4 trellis, b=1); prefill tok/s"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--layers", type=int, default=4, help="independently seeded layers rotated per step")
    p.add_argument("--tokens", type=int, default=16, help="distinct tokens rotated per step")
    p.add_argument("--seed", type=int, default=2026)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-prefill", action="store_true", help="skip the prefill measurement of the default line")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--config", type=int, default=0, choices=range(5),
                   help="workload: 0 K4 b=1 (default), 1 MXFP4 b=1, 2 K4 8-token verify, 3 MXFP4 512-token "
                        "prefill, 4 20-layer K4 stack")
    p.add_argument("--k4-prefill", action="store_true",
                   help="instead: the K4 grouped prefill MLP (values of 512 Zipf-routed rows x 9 slots)")
    p.add_argument("--k3", action="store_true",
                   help="instead: the K3 layer (the multi-token-prediction layer's width) at batch-1 decode")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="also run a plain 1 GiB device copy (reference point for rocprofv3 FETCH/WRITE_SIZE)")
    return p.parse_args()


def traffic_from_profiles(name="k4_layer_b1_pmc.txt"):
    """HBM bytes per layer launch from a committed rocprofv3 PMC summary, if present."""
    path = ROOT / "profiles" / name
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1].split()[0])
            except ValueError:
                return None
    return None


def cpu_baseline(layer, w, bias, xs, rs, seconds, runs=5):
    """The CPU restatement of the reference operator chain, timed on this host: the oracle's C source
    built here with fp32 accumulation and -march=native (OpenMP over all cores); the float64 oracle
    if that build is not possible.  One warm-up token, then `runs` runs of the same token count
    (sized so the runs take about `seconds` together); the value is the median run's tokens/s."""
    import statistics
    import tempfile

    import numpy as np
    import torch
    from oracle import lib as oracle_lib, native_f32

    orc = native_f32(Path(tempfile.gettempdir()) / "moe_cpu_baseline")
    kind = "C restatement built here: -O3 -march=native -fopenmp, fp32 accumulation"
    if orc is None:
        orc = oracle_lib()
        kind = "C oracle (prebuilt -O3 -march=x86-64-v3 -fopenmp), float64 accumulation"
    host = {p: t.cpu().numpy() for p, t in layer["packed"].items()}
    sc = {p: tuple(v.contiguous().view(torch.int16).cpu().numpy().view(np.uint16) for v in pair)
          for p, pair in layer["scales"].items()}
    wh, bh = w.cpu().numpy(), bias.cpu().numpy()
    bits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    xb = [bits(x) for x in xs]
    rb = [bits(r) for r in rs]

    def token(i):
        i %= len(xb)
        logits = orc.router_logits(xb[i], wh)
        ids, scores = orc.route(logits, bh)
        orc.k4_moe(xb[i], ids, scores, rb[i], H, M, host["gate"], host["up"], host["down"],
                   sc["gate"][0], sc["gate"][1], sc["up"][0], sc["up"][1], sc["down"][0], sc["down"][1])

    t0 = time.perf_counter()
    token(0)  # warm-up (page-in, thread pool start)
    warm = time.perf_counter() - t0
    per_run = max(1, int(round(seconds / runs / max(warm, 1e-3))))
    rates = []
    done = 0
    for r in range(runs):
        t0 = time.perf_counter()
        for i in range(per_run):
            token(1 + done + i)
        rates.append(per_run / (time.perf_counter() - t0))
        done += per_run
    return {"value": round(statistics.median(rates), 3), "unit": "tokens/s", "cores": orc.num_threads(),
            "kind": "port",
            "runs": [round(v, 3) for v in rates],
            "sample": f"{runs} runs of {per_run} tokens after one warm-up token, median reported: the same batch-1 "
                      f"K4 layer (router GEMV + route + 9-expert MLP + combine), rotating {len(xb)} tokens; {kind}"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported (this path has no "
              "multi-GPU collectives: experts would be sharded across GPUs by expert id, one GPU's share per rank)", file=sys.stderr)
        sys.exit(2)
    if args.k4_prefill:
        print(json.dumps(bench_k4_prefill(args)), flush=True)
        return
    if args.k3:
        print(json.dumps(bench_k3_decode(args)), flush=True)
        return
    if args.config != 0:
        print(json.dumps(OTHER[args.config](args)), flush=True)
        return
    import torch
    from mlxlr8_amd import synth
    from mlxlr8_amd._lib import lib
    from mlxlr8_amd.experts import ExpertLayer

    dev = torch.device("cuda:0")
    layers, raw = [], []
    for i in range(args.layers):
        L = synth.k4_layer(dev, args.seed + 17 * i)
        raw.append(L)
        layers.append(ExpertLayer(L["packed"], L["scales"], H, M))
    # each rotated layer has its own router weights (6.3 MB per step, streamed like the experts)
    routers = [synth.router(dev, args.seed + 17 * i) for i in range(args.layers)]
    xs, rs = [], []
    for t in range(args.tokens):
        x, r = synth.activations(dev, args.seed + 1000 + t, 1)
        xs.append(x)
        rs.append(r)
    torch.cuda.synchronize()

    # one prepared C call per (layer, token) pair: no per-step tensor work on the host
    calls = [[layer.prepare_decode(xs[t], rs[t], *routers[k]) for t in range(len(xs))]
             for k, layer in enumerate(layers)]

    def step(i):
        return calls[i % len(layers)][i % len(xs)].run()

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # timed region: K steps, nothing else on the stream
    n = args.steps
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for i in range(n):
        step(args.warmup + i)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_step_ms = start.elapsed_time(end) / n
    us_tok = per_step_ms * 1e3

    # one step = one launch of the fused layer kernel on this stream, back to back: the timed
    # region's per-step time is the kernel's average duration (a rocprofv3 kernel trace of the same
    # command agrees: profiles/k4_layer_b1_kernel_trace.txt)
    from mlxlr8_amd._lib import stalled_launches
    wait_errors = stalled_launches()
    achieved = BYTES_TOKEN / (us_tok * 1e-6) / 1e9
    hbm = achieved
    traffic = traffic_from_profiles()

    result = {
        "metric": METRIC,
        "value": round(1e3 / per_step_ms, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": n,
        "warmup": args.warmup,
        "ms_per_step": round(per_step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "GLM-5.3-style K4-trellis MoE layer, batch-1 decode: hidden 6144, 256 routed + 1 shared "
                        "expert, top-8, intermediate 2048, bf16 activations, fp32 accumulate",
            "global_batch": 1, "seq_len": 1, "parallelism": "none (1 GPU)",
            "layers_rotated": args.layers, "tokens_rotated": args.tokens, "seed": args.seed,
        },
        "us_per_token": round(us_tok, 2),
        "hbm_GBps": round(hbm, 1),
        "hbm_frac": round(hbm / HBM_PEAK_GBPS, 4),
        "bytes_per_token": BYTES_TOKEN,
        "wait_errors": wait_errors,
        "roofline": {"kernel": "k4_layer_kernel<1, false, 4> (router, top-8, shared and routed gate/up and down decode "
                               "GEMVs, finishes and combine in one persistent launch)",
                     "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "traffic_source": "committed rocprofv3 PMC summary profiles/k4_layer_b1_pmc.txt (FETCH_SIZE, "
                                       "WRITE_SIZE per launch, copy-calibrated), not measured in this run",
                     "algorithmic_bytes": BYTES_TOKEN},
        "wall_s": round(wall, 3),
    }
    if args.calibrate_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        result["calibration_copy_bytes"] = 1 << 30
    if not args.no_prefill:
        pf = bench_prefill(args, steps=20, warmup=3)
        result["prefill"] = {"metric": "prefill tok/s", "value": pf["value"], "unit": "tokens/s",
                             "ms_per_chunk": pf["ms_per_step"], "workload": pf["config"]["workload"],
                             "touched_experts": pf["config"]["touched_experts"],
                             "hbm_GBps": pf["roofline"]["achieved"],
                             "mfma_util_fp4_peak": pf["mfma_util_fp4_peak"], "steps": pf["steps"]}
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(raw[0], *routers[0], xs, rs, args.cpu_seconds)
    print(json.dumps(result), flush=True)


def _time_steps(step, steps, warmup):
    """HIP events around `steps` calls of step(i) after `warmup` untimed ones; ms per step."""
    import torch
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        step(warmup + i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def _line(args, value, unit, ms, dtype, workload, extra, algo_bytes, kernel):
    gbps = algo_bytes / (ms * 1e-3) / 1e9
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": unit, "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dtype, "data": "synthetic",
        "config": dict({"workload": workload, "parallelism": "none (1 GPU)", "seed": args.seed}, **extra),
        "roofline": {"kernel": kernel, "bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "algorithmic_bytes": int(algo_bytes)},
    }
    return out


def _stalls():
    """Fused decode launches of this run whose bounded cross-wave waits ran out (should be 0)."""
    from mlxlr8_amd._lib import stalled_launches
    return stalled_launches()


MX_EXPERT_BYTES = 2 * M * H // 2 + 2 * M * H // 32 + H * M // 2 + H * M // 32   # 20,054,016


def _mx_layers(dev, seed, n):
    from mlxlr8_amd import synth
    from mlxlr8_amd.joined_mxfp4 import JoinedMXFP4
    out = []
    for i in range(n):
        L = synth.mxfp4_layer(dev, seed + 31 * i)
        side = L["side"]
        out.append(JoinedMXFP4(L["weights"], L["unit"], {"gate": (None, side["out_gate"]), "up": (None, side["out_up"]),
                                                         "down": (side["in_down"], side["out_down"])}, H, M))
    return out


def bench_mxfp4_decode(args):
    import torch
    from mlxlr8_amd import synth
    dev = torch.device("cuda:0")
    layers = _mx_layers(dev, args.seed, min(args.layers, 3))
    w, bias = synth.router(dev, args.seed)
    toks = [synth.activations(dev, args.seed + 1000 + t, 1) for t in range(args.tokens)]
    calls = [[l.prepare_decode(x, r, w, bias) for (x, r) in toks] for l in layers]
    ms = _time_steps(lambda i: calls[i % len(calls)][i % len(toks)].run(), args.steps, args.warmup)
    algo = 9 * MX_EXPERT_BYTES + 256 * H * 4 + 9 * (3 * M + H) * 2 + H * 2 + 256 * 4 + 3 * H * 2
    line = _line(args, 1e3 / ms, "tokens/s", ms, "f32",
                 "GLM-5.3-style joined-MXFP4 MoE layer, batch-1 decode: hidden 6144, 256 routed + 1 shared, "
                 "top-8, intermediate 2048 (e2m1 + e8m0 per 32), bf16 activations, fp32 accumulate",
                 {"global_batch": 1, "seq_len": 1, "layers_rotated": len(layers)}, algo,
                 "mx_layer_kernel: router, both projections of the nine slots and the combine in one launch")
    line["roofline"]["traffic"] = traffic_from_profiles("mxfp4_layer_b1_pmc.txt")
    if line["roofline"]["traffic"] is not None:
        line["roofline"]["traffic_source"] = "committed rocprofv3 PMC summary profiles/mxfp4_layer_b1_pmc.txt"
    from mlxlr8_amd._lib import stalled_launches
    return dict(line, us_per_token=round(ms * 1e3, 2), wait_errors=stalled_launches())


def bench_k3_decode(args):
    """The routed K3 block, batch 1: K3 trellis experts (3 bits per weight) at the K4 layer's shape."""
    import torch
    from mlxlr8_amd import synth
    from mlxlr8_amd.experts import ExpertLayer
    dev = torch.device("cuda:0")
    layers = []
    for i in range(min(args.layers, 3)):
        L = synth.k4_layer(dev, args.seed + 17 * i, k=3)
        layers.append(ExpertLayer(L["packed"], L["scales"], H, M, k=3, number=78))
    w, bias = synth.router(dev, args.seed)
    toks = [synth.activations(dev, args.seed + 1000 + t, 1) for t in range(args.tokens)]
    calls = [[l.prepare_decode(x, r, w, bias) for (x, r) in toks] for l in layers]
    ms = _time_steps(lambda i: calls[i % len(calls)][i % len(toks)].run(), args.steps, args.warmup)
    algo = 9 * 3 * (TRELLIS * 3 // 4) + 256 * H * 4 + 9 * 3 * (H + M) * 2 + 256 * 4 + 3 * H * 2
    line = _line(args, 1e3 / ms, "tokens/s", ms, "f32",
                 "GLM-5.3-style MoE layer with K3 trellis experts (the multi-token-prediction layer's width), "
                 "batch-1 decode: hidden 6144, 256 routed + 1 shared, top-8, intermediate 2048",
                 {"global_batch": 1, "seq_len": 1, "layers_rotated": len(layers)}, algo,
                 "k4_layer_kernel<1, false, 3>: router, the nine slots' K3 projections and the combine in one launch")
    return dict(line, us_per_token=round(ms * 1e3, 2), wait_errors=_stalls())


def bench_k4_verify(args):
    import torch
    from mlxlr8_amd import synth
    from mlxlr8_amd.experts import ExpertLayer
    dev = torch.device("cuda:0")
    layers = [ExpertLayer(**{k: v for k, v in synth.k4_layer(dev, args.seed + 17 * i).items()}, hidden=H,
                          intermediate=M) for i in range(min(args.layers, 3))]
    w, bias = synth.router(dev, args.seed)
    batches = [synth.activations(dev, args.seed + 2000 + t, 8, correlated=True) for t in range(4)]
    calls = [[l.prepare_decode(x, r, w, bias) for (x, r) in batches] for l in layers]
    for c in calls[0]:
        c.run()
    torch.cuda.synchronize()
    uniq = [len(set(c.ids.cpu().numpy().ravel().tolist())) for c in calls[0]]
    U = sum(uniq) / len(uniq)
    ms = _time_steps(lambda i: calls[i % len(calls)][i % len(batches)].run(), args.steps, args.warmup)
    algo = U * (3 * TRELLIS + 3 * (H + M) * 2) + 256 * H * 4 + 256 * 4 + 8 * 3 * H * 2
    return dict(_line(args, 8e3 / ms, "tokens/s", ms, "f32",
                      "8-token speculative-verify batch through the K4-trellis MoE layer (correlated rows, "
                      "distinct experts streamed once)",
                      {"global_batch": 8, "seq_len": 1, "distinct_experts": U, "layers_rotated": len(layers)},
                      algo, "k4_layer_kernel<8, false, 4>: router, the distinct experts' projections and the combine in one launch"),
                us_per_step=round(ms * 1e3, 2), wait_errors=_stalls())


def bench_prefill(args, steps=None, warmup=None):
    import torch
    from mlxlr8_amd import synth
    dev = torch.device("cuda:0")
    layers = _mx_layers(dev, args.seed, 2)
    w, bias = synth.router(dev, args.seed + 1, zipf=True)
    x, res = synth.activations(dev, args.seed + 3000, 512)
    _, ids, _ = layers[0].prefill(x, res, w, bias)
    torch.cuda.synchronize()
    touched = len(set(ids.cpu().numpy().ravel().tolist()))
    steps = steps if steps is not None else max(1, min(args.steps, 40))
    warmup = warmup if warmup is not None else min(args.warmup, 5)
    ms = _time_steps(lambda i: layers[i % 2].prefill(x, res, w, bias), steps, warmup)
    algo = touched * MX_EXPERT_BYTES + 256 * H * 4 + 3 * 512 * H * 2
    out = _line(args, 512e3 / ms, "tokens/s", ms, "f32",
                "512-token prefill chunk through the joined-MXFP4 MoE layer (Zipf(1.1)-skewed routing, "
                "sort-by-expert grouped GEMMs on the MX matrix cores, weighted combine)",
                {"global_batch": 512, "seq_len": 512, "touched_experts": touched}, algo,
                "whole step: router + sort + grouped gate_up/down GEMMs + combine")
    out["steps"] = steps
    flops = 512 * 9 * 3 * 2 * H * M
    out["mfma_util_fp4_peak"] = round(flops / (ms * 1e-3) / 10.1e15, 4)
    return out


def bench_k4_prefill(args):
    """K4 grouped prefill MLP (exlr8/fast_prefill.py:188-211): values of 512 rows x 9 slots, ids from
    the Zipf-skewed router of the 512-token prefill workload, two K4 layers rotated."""
    import torch
    from mlxlr8_amd import synth
    from mlxlr8_amd.fast_prefill import grouped_expert_mlp
    from mlxlr8_amd.fast_router import route, router_logits
    dev = torch.device("cuda:0")
    layers = [synth.k4_layer(dev, args.seed + 41 * i) for i in range(2)]
    w, bias = synth.router(dev, args.seed + 1, zipf=True)
    x, _ = synth.activations(dev, args.seed + 3000, 512)
    ids, _ = route(router_logits(x, w), bias)
    torch.cuda.synchronize()
    touched = len(set(ids.cpu().numpy().ravel().tolist()))
    run = lambda i: grouped_expert_mlp(x, ids, layers[i % 2]["packed"], layers[i % 2]["scales"], 4, H, M)
    steps = max(1, min(args.steps, 20))
    ms = _time_steps(run, steps, min(args.warmup, 3))
    algo = touched * 3 * TRELLIS + touched * 6 * H * 2 + 512 * H * 2 + 512 * 9 * H * 2
    out = _line(args, 512e3 / ms, "tokens/s", ms, "f32",
                "K4-trellis grouped prefill MLP, 512 Zipf(1.1)-routed rows x 9 slots (values; sort-by-expert "
                "blocks, trellis decoded next to the fp16 matrix cores)",
                {"global_batch": 512, "seq_len": 512, "touched_experts": touched}, algo,
                "whole step: segment table + prep + grouped gate/up and down GEMMs + finishes")
    out["steps"] = steps
    return out


def bench_stack(args):
    import torch
    from mlxlr8_amd import synth
    from mlxlr8_amd.experts import ExpertLayer
    dev = torch.device("cuda:0")
    n = 20
    calls, x = [], synth.activations(dev, args.seed + 4000, 1)[0].contiguous()
    for i in range(n):
        spec, w, bias, norm = synth.stack_layer(dev, args.seed, i)
        lay = ExpertLayer(**spec, hidden=H, intermediate=M)
        c = lay.prepare_layer_decode(x, norm, w, bias)
        calls.append(c)
        x = c.out
    steps = max(1, min(args.steps, 50))
    ms = _time_steps(lambda i: [c.run() for c in calls], steps, min(args.warmup, 5))
    algo = n * (BYTES_TOKEN + H * 2)
    out = _line(args, 1e3 / ms, "tokens/s", ms, "f32",
                "20 consecutive GLM-5.3-style K4-trellis MoE layers (independent seeded weights, Zipf-skewed "
                "router biases, RMSNorm'd residual per layer), batch-1 decode",
                {"global_batch": 1, "seq_len": 1, "layers": n}, algo, "20 x (residual + RMSNorm launch, fused K4 block launch)")
    out["steps"] = steps
    out["us_per_token_stack"] = round(ms * 1e3, 2)
    out["wait_errors"] = _stalls()
    return out


OTHER = {1: bench_mxfp4_decode, 2: bench_k4_verify, 3: bench_prefill, 4: bench_stack}


if __name__ == "__main__":
    main()
