#!/usr/bin/env python3
"""Benchmark of the MI355X MoE expert path: one GLM-5.3-style K4 trellis MoE layer, batch-1 decode.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu]

One step = one token through the whole layer (router GEMV, bias-corrected top-8, eight routed
experts plus the shared expert as K4-trellis decode GEMVs with SwiGLU, weighted combine and
residual).  Inputs and weights are resident in HBM before timing starts.  Weights of several
independently seeded layers are rotated (and tokens vary) so consecutive steps stream
different expert bytes instead of re-reading the 256 MB last-level cache.

Prints ONE JSON line.  `value` is tokens/s; `us_per_token`, achieved algorithmic HBM GB/s and
the roofline of the dominant kernel (the fused gate/up decode GEMV, timed with HIP events on
its own stream) are reported beside it, with the CPU oracle timed on this host's cores.
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
# side vectors + bias + activations in/out ("Measurement").
BYTES_TOKEN = 9 * 3 * TRELLIS + 256 * H * 4 + 9 * 3 * (H + M) * 2 + 256 * 4 + 3 * H * 2
# Dominant kernel: gate/up GEMV of 9 experts (2 projections each) + its side vectors and input.
BYTES_GATEUP = 9 * 2 * TRELLIS + 9 * 2 * H * 2 + 9 * 2 * M * 2 + 9 * M * 2 + H * 2
BYTES_DOWN = 9 * TRELLIS + 9 * M * 4 + 9 * H * 2 + 2 * H * 2
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
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--calibrate-copy", action="store_true",
                   help="also run a plain 1 GiB device copy (reference point for rocprofv3 FETCH/WRITE_SIZE)")
    return p.parse_args()


def traffic_from_profiles():
    """HBM bytes per gate/up launch from the committed rocprofv3 PMC summary, if present."""
    path = ROOT / "profiles" / "k4_gateup_b1_pmc.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1].split()[0])
            except ValueError:
                return None
    return None


def cpu_baseline(layer, w, bias, xs, rs, seconds):
    """The CPU oracle (C restatement of the reference operator chain, OpenMP) on this host."""
    import numpy as np
    import torch
    from oracle import lib as oracle_lib

    orc = oracle_lib()
    host = {p: t.cpu().numpy() for p, t in layer["packed"].items()}
    sc = {p: tuple(v.contiguous().view(torch.int16).cpu().numpy().view(np.uint16) for v in pair)
          for p, pair in layer["scales"].items()}
    wh, bh = w.cpu().numpy(), bias.cpu().numpy()
    bits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    done, t0 = 0, time.perf_counter()
    while True:
        i = done % len(xs)
        logits = orc.router_logits(bits(xs[i]), wh)
        ids, scores = orc.route(logits, bh)
        orc.k4_moe(bits(xs[i]), ids, scores, bits(rs[i]), H, M, host["gate"], host["up"], host["down"],
                   sc["gate"][0], sc["gate"][1], sc["up"][0], sc["up"][1], sc["down"][0], sc["down"][1])
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": done / el, "unit": "tokens/s", "cores": orc.num_threads(), "kind": "port",
            "sample": f"{done} tokens of the same batch-1 K4 layer (router GEMV + route + 9-expert MLP + combine), "
                      f"{el:.1f} s, C oracle -O3 -fopenmp, float64 accumulation"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported (this path has no "
              "multi-GPU collectives; see DESIGN.md for how it would shard)", file=sys.stderr)
        sys.exit(2)
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
    w, bias = synth.router(dev, args.seed)
    xs, rs = [], []
    for t in range(args.tokens):
        x, r = synth.activations(dev, args.seed + 1000 + t, 1)
        xs.append(x)
        rs.append(r)
    torch.cuda.synchronize()

    # one prepared C call per (layer, token) pair: no per-step tensor work on the host
    calls = [[layer.prepare_decode(xs[t], rs[t], w, bias) for t in range(len(xs))] for layer in layers]

    def step(i):
        return calls[i % len(layers)][i % len(xs)].run()

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # timed region: every step also records per-kernel HIP events on the launch stream
    import ctypes
    n = args.steps
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(n)]
    L = lib()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # torch creates an event's HIP handle on its first record(): record each once first
    for row in evs:
        for e in row:
            e.record()
    handles = [(ctypes.c_void_p * 4)(*[ctypes.c_void_p(e.cuda_event) for e in row]) for row in evs]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for i in range(n):
        L.moe_profile_events(handles[i], 4)
        step(args.warmup + i)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end)
    per_step_ms = ms / n
    us_tok = per_step_ms * 1e3
    router_us = sum(evs[i][0].elapsed_time(evs[i][1]) for i in range(n)) / n * 1e3
    gateup_us = sum(evs[i][1].elapsed_time(evs[i][2]) for i in range(n)) / n * 1e3
    down_us = sum(evs[i][2].elapsed_time(evs[i][3]) for i in range(n)) / n * 1e3
    achieved = BYTES_GATEUP / (gateup_us * 1e-6) / 1e9
    hbm = BYTES_TOKEN / (us_tok * 1e-6) / 1e9
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
        "kernels_us": {"router": round(router_us, 2), "gate_up": round(gateup_us, 2), "down": round(down_us, 2)},
        "roofline": {"kernel": "k4_gemv_kernel<prep,gate> (fused gate/up decode GEMV, 9 experts)",
                     "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "algorithmic_bytes": BYTES_GATEUP},
        "wall_s": round(wall, 3),
    }
    if args.calibrate_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        result["calibration_copy_bytes"] = 1 << 30
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(raw[0], w, bias, xs, rs, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
