#!/usr/bin/env python3
"""Benchmark: one 27B-shape q4_k_m decode layer of linears, M = 1, on one MI355X.

Workload (Qwen-27B shapes, seeded synthetic weights ~ N(0, 0.02) quantized by
the oracle's block generators; x ~ N(0, 1)):
    Q4_K q 6144x5120, k 1024x5120, v 1024x5120  (one launch, shared activation)
    Q4_K o 5120x6144                            (fused quantization of its output)
    Q4_K gate, up 17408x5120 + SwiGLU           (one launch, fused output quantization)
    Q6_K down 5120x17408
in dependency order.  A step is one such layer pass.  Weights rotate over
enough distinct device copies (>= 2 x the 256 MB Infinity Cache) that every
step streams its weights from HBM; a warm (cache-resident) figure is reported
beside it.  The whole step sequence is captured once in a HIP graph.

value = weight bytes of the layer (GGUF, unpadded: 214,671,360 B) / step time.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

HBM_PEAK_GBS = 8000.0
METRIC = "Q4_K/Q6_K matvec weight-GB/s (% of HBM peak) + µs per decode layer, M=1"
LAYER = [  # name, type, rows, K
    ("q", "Q4_K", 6144, 5120), ("k", "Q4_K", 1024, 5120), ("v", "Q4_K", 1024, 5120),
    ("o", "Q4_K", 5120, 6144), ("gate", "Q4_K", 17408, 5120), ("up", "Q4_K", 17408, 5120),
    ("down", "Q6_K", 5120, 17408),
]
MALL_BYTES = 256 << 20


def load_pkg():
    from conftest import load_package
    return load_package().m27q


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def build_layers(m27q, ora, dev, copies):
    import torch
    host = {}
    for i, (name, tname, rc, k) in enumerate(LAYER):
        t = getattr(ora, tname)
        host[name] = (t, rc, k, ora.synth_weights(t, rc, k, seed=10 + i))
    layers = []
    first = {}
    for name, (t, rc, k, blocks) in host.items():
        rb = k // 256
        first[name] = m27q.Weight.upload(blocks.reshape(-1), t, rb, rc, m27q.TILED, dev)
    layers.append(first)
    for _ in range(1, copies):
        layers.append({n: m27q.Weight(w.data.clone(), w.type, w.rb, w.rc, w.layout) for n, w in first.items()})
    torch.cuda.synchronize()
    return layers, host


class Buffers:
    def __init__(self, m27q, dev):
        import torch
        self.x = torch.from_numpy(np.random.default_rng(1).standard_normal(5120).astype(np.float32)).to(dev)
        self.q = torch.empty(6144, dtype=torch.float32, device=dev)
        self.k = torch.empty(1024, dtype=torch.float32, device=dev)
        self.v = torch.empty(1024, dtype=torch.float32, device=dev)
        self.h = torch.empty(5120, dtype=torch.float32, device=dev)
        self.f = torch.empty(17408, dtype=torch.float32, device=dev)
        self.fq = m27q.Act(1, 17408, dev)
        self.out = torch.empty(5120, dtype=torch.float32, device=dev)


# The layer's products in dependency order.  fp32 activations are quantized
# inside each product; the SwiGLU product hands its output to down already
# quantized.  o consumes the 6144-vector q in place of the attention output.
STAGES = {
    "qkv": lambda m27q, L, B, s: m27q.matvec_multi([L["q"], L["k"], L["v"]], B.x, [B.q, B.k, B.v], stream=s),
    "o": lambda m27q, L, B, s: m27q.matvec(L["o"], B.q, B.h, residual=B.x, stream=s),
    "gate_up": lambda m27q, L, B, s: m27q.ffn_swiglu(L["gate"], L["up"], B.h, B.f, yq=B.fq, stream=s),
    "down": lambda m27q, L, B, s: m27q.matvec_q8(L["down"], B.fq, B.out, residual=B.h, stream=s),
}
STAGE_WEIGHTS = {"qkv": ("q", "k", "v"), "o": ("o",), "gate_up": ("gate", "up"), "down": ("down",)}


def stage_bytes(m27q, name):
    """Algorithmic HBM bytes of one product: GGUF weight bytes (unpadded) + fp32
    activation in + fp32 output (+ residual read, + quantized output)."""
    w = {n: (m27q.BLOCK_BYTES[getattr(m27q, t)] * rc * k // 256, rc, k) for n, t, rc, k in LAYER}
    wb = sum(w[n][0] for n in STAGE_WEIGHTS[name])
    k = w[STAGE_WEIGHTS[name][0]][2]
    rows = sum(w[n][1] for n in STAGE_WEIGHTS[name])
    if name == "qkv":
        return wb + 4 * k + 4 * rows
    if name == "o":
        return wb + 4 * k + 4 * rows + 4 * rows          # + residual
    if name == "gate_up":
        n = w["gate"][1]
        return wb + 4 * k + 4 * n + (n + 8 * (n // 32))  # + quantized output
    n = w["down"][1]
    return wb + (k + 8 * (k // 32)) + 4 * n + 4 * n      # quantized input, + residual


def measured_traffic(kernel_label):
    """HBM bytes per launch of one product as measured by rocprofv3 --pmc
    (FETCH_SIZE and WRITE_SIZE, scaled by a kernel of known size), read from
    the committed summary; None where that summary is absent."""
    path = os.path.join(ROOT, "profiles", "gemv_decode_layer_hbm_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith(kernel_label + ":"):
            return int(line.split()[-3])
    return None


def layer_pass(m27q, L, B, stream):
    for fn in STAGES.values():
        fn(m27q, L, B, stream)


def capture(torch, fn):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(s)  # eager warm pass on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        fn(torch.cuda.current_stream())
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, reps):
    """Average ms per replay, HIP events on the replay stream."""
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(s)
    for _ in range(reps):
        g.replay()
    e1.record(s)
    e1.synchronize()
    return e0.elapsed_time(e1) / reps


def cpu_baseline(ora, host, budget_s=12.0):
    """The oracle's restatement of ggml's CPU path (q8_K activations, q4_K x q8_K /
    q6_K x q8_K dots), rows split over host threads, on the same layer weights."""
    nthreads = max(1, min(16, os.cpu_count() or 1))
    x = np.random.default_rng(1).standard_normal(17408).astype(np.float32)
    xq = {k: ora.quant_cpu_act(ora.Q4_K, x[:k]) for k in (5120, 6144, 17408)}
    total_bytes = sum(b.nbytes for (_, _, _, b) in host.values())
    reps, t0 = 0, time.perf_counter()
    while True:
        for name, (t, rc, k, blocks) in host.items():
            ora.gemv_cpu(t, blocks, k // 256, rc, xq[k], nthreads=nthreads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or (reps >= 3 and el * (reps + 1) / reps > budget_s):
            break
    sec = el / reps
    return {"value": round(total_bytes / sec / 1e9, 3), "unit": "GB/s", "cores": nthreads, "kind": "port",
            "sample": f"{reps} full layer passes (7 matvecs, {total_bytes} weight bytes) in {el:.2f} s, "
                      f"{sec * 1e6:.0f} us/layer; oracle restatement of ggml q4_K/q6_K x q8_K CPU dots "
                      f"(not ggml itself: the vendored ref/llama.cpp is empty)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--copies", type=int, default=0, help="distinct weight copies (0: auto, >= 2x MALL)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calib", action="store_true",
                    help="also run a plain 512 MiB device copy (the reference point that scales the "
                         "FETCH_SIZE / WRITE_SIZE counters of a rocprofv3 --pmc run)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build is single-GPU by design); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import oracle as ora
    m27q = load_pkg()
    dev = torch.device("cuda:0")
    layer_bytes = sum(m27q.BLOCK_BYTES[getattr(m27q, t)] * rc * k // 256 for _, t, rc, k in LAYER)
    copies = args.copies or max(2, -(-2 * MALL_BYTES // layer_bytes) + 1)
    log(f"building {copies} layer copies ({layer_bytes * copies / 2**20:.0f} MiB)")
    layers, host = build_layers(m27q, ora, dev, copies)
    B = Buffers(m27q, dev)

    def cold_pass(s):
        for L in layers:
            layer_pass(m27q, L, B, s)

    def warm_pass(s):
        for _ in range(copies):
            layer_pass(m27q, layers[0], B, s)

    log("capturing graphs")
    g_cold = capture(torch, cold_pass)
    g_warm = capture(torch, warm_pass)
    reps = max(1, args.steps // copies)
    wreps = max(1, args.warmup // copies)
    for _ in range(wreps):
        g_cold.replay()
    torch.cuda.synchronize()
    log(f"timing {reps * copies} layer passes")
    ms_cold = time_graph(torch, g_cold, reps) / copies
    ms_warm = time_graph(torch, g_warm, reps) / copies

    # Each product on its own, over the same rotated copies: average launch
    # duration from HIP events on the replay stream.
    stages = {}
    for name, fn in STAGES.items():
        g = capture(torch, lambda st, fn=fn: [fn(m27q, L, B, st) for L in layers])
        g.replay()
        ms = time_graph(torch, g, reps) / copies
        nbytes = stage_bytes(m27q, name)
        stages[name] = {"us": round(ms * 1e3, 3), "bytes": nbytes, "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)}
        log(f"{name}: {ms * 1e3:.2f} us, {stages[name]['GBps']} GB/s")
    dom = stages["gate_up"]  # the dominant product: 100 MB of the layer's 215 MB

    # Plain streaming read of 1 GiB (torch's sum kernel) for the measured peak.
    big = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    big.sum()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        big.sum()
    e1.record()
    e1.synchronize()
    read_gbs = big.numel() * 4 * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del big
    if args.calib:
        src = torch.ones(1 << 27, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    gbs = layer_bytes / (ms_cold * 1e-3) / 1e9
    rec = {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": reps * copies, "warmup": wreps * copies, "ms_per_step": round(ms_cold, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "qwen27b_q4km_decode_layer_linears_m1",
                   "layer": {n: f"{t} {rc}x{k}" for n, t, rc, k in LAYER},
                   "weight_bytes": layer_bytes, "layout": "tiled", "activation": "int8 per-32, fp32 scale",
                   "cold_copies": copies, "graph": True},
        "us_per_layer": round(ms_cold * 1e3, 2),
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
        "lower_bound_us": round(layer_bytes / HBM_PEAK_GBS / 1e3, 2),
        "x_lower_bound": round(ms_cold * 1e3 / (layer_bytes / HBM_PEAK_GBS / 1e3), 3),
        "warm_us_per_layer": round(ms_warm * 1e3, 2),
        "hbm_read_GBps_measured": round(read_gbs, 1),
        "stages": stages,
        "roofline": {"bound": "hbm", "kernel": "k_gemv_q8<Q4K,TILED,SWIGLU> (gate+up 17408x5120, fp32 x in, "
                                               "fp32 + quantized out)",
                     "achieved": dom["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic("gate_up"),
                     "traffic_source": "profiles/gemv_decode_layer_hbm_traffic.txt",
                     "avg_launch_us": dom["us"], "algorithmic_bytes": dom["bytes"]},
    }
    if not args.no_cpu:
        log("cpu baseline")
        rec["cpu_baseline"] = cpu_baseline(ora, host)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
