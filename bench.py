#!/usr/bin/env python3
"""Benchmark: one 27B-shape q4_k_m decode layer of linears, M = 1, on one MI355X.

Workload (Qwen-27B shapes, seeded synthetic weights ~ N(0, 0.02) quantized by
the oracle's block generators; x ~ N(0, 1)):
    Q4_K q 6144x5120, k 1024x5120, v 1024x5120  (one launch on the fp32 x)
    Q4_K o 5120x6144                            (on the q vector, + residual)
    Q4_K gate, up 17408x5120 + SwiGLU           (one launch, fp32 output)
    Q6_K down 5120x17408                        (on that fp32 output, + residual)
in dependency order; every product quantizes its fp32 input inside the
kernel.  A step is one such layer pass.  Weights rotate over enough distinct
device copies (>= 2 x the 256 MB Infinity Cache) that every step streams its
weights from HBM; a warm (cache-resident) figure is reported beside it.  The
K timed passes replay from one HIP graph of exactly K layer passes (past
1024 passes, 1024-pass graphs and one for the rest), as a decode step
replays one graph for all its layers.  Before the W warmup passes
(their own graph), 100 ms of untimed layer passes let the GPU's clocks
settle; each product timed alone
rotates over copies of its own weights (>= 2 x the Infinity Cache) after 30 ms
of untimed replays.

value = weight bytes of the layer (GGUF, unpadded: 214,671,360 B) / step time.
"""
import argparse
import hashlib
import json
import os
import re
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
# GGUF bytes of one 256-weight block of each type in the layer
_BLOCK = {"Q4_K": 144, "Q6_K": 210}
LAYER_BYTES = sum(_BLOCK[t] * rc * k // 256 for _, t, rc, k in LAYER)  # 214,671,360


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


def cold_pool(m27q, torch, layers, names):
    """Copies of the named weights, enough of them (>= 2 x the 256 MB Infinity
    Cache per rotation, and at least the layer copies) that every launch of a
    product timed alone streams its weights from HBM: the layer copies first,
    then device clones of them."""
    per = sum(layers[0][n].data.numel() for n in names)
    n = max(len(layers), -(-2 * MALL_BYTES // per) + 1)
    pool = [{k: L[k] for k in names} for L in layers]
    while len(pool) < n:
        src = layers[len(pool) % len(layers)]
        pool.append({k: m27q.Weight(src[k].data.clone(), src[k].type, src[k].rb, src[k].rc, src[k].layout)
                     for k in names})
    torch.cuda.synchronize()
    return pool


class Buffers:
    def __init__(self, m27q, dev):
        import torch
        self.x = torch.from_numpy(np.random.default_rng(1).standard_normal(5120).astype(np.float32)).to(dev)
        # the attention layer's Wo input: the attention output (q stands in)
        # gated by sigmoid(gate), quantized by m27q_quant_act_gated into qa
        self.gate = torch.from_numpy(np.random.default_rng(2).standard_normal(6144).astype(np.float32)).to(dev)
        self.qa = m27q.Act(1, 6144, dev)
        self.q = torch.empty(6144, dtype=torch.float32, device=dev)
        self.k = torch.empty(1024, dtype=torch.float32, device=dev)
        self.v = torch.empty(1024, dtype=torch.float32, device=dev)
        self.h = torch.empty(5120, dtype=torch.float32, device=dev)
        self.f = torch.empty(17408, dtype=torch.float32, device=dev)
        self.out = torch.empty(5120, dtype=torch.float32, device=dev)


# The layer's products in dependency order.  Every product takes an fp32
# activation and quantizes it inside the kernel (down's 17408-vector included:
# balanced tiling makes that 1 us faster per layer than a quantizer launch
# between the SwiGLU product and down).  o consumes the 6144-vector q in place
# of the attention output.
STAGES = {
    "qkv": lambda m27q, L, B, s: m27q.matvec_multi([L["q"], L["k"], L["v"]], B.x, [B.q, B.k, B.v], stream=s),
    "o": lambda m27q, L, B, s: m27q.matvec(L["o"], B.q, B.h, residual=B.x, stream=s),
    "gate_up": lambda m27q, L, B, s: m27q.ffn_swiglu(L["gate"], L["up"], B.h, B.f, stream=s),
    "down": lambda m27q, L, B, s: m27q.matvec(L["down"], B.f, B.out, residual=B.h, stream=s),
}
STAGE_WEIGHTS = {"qkv": ("q", "k", "v"), "o": ("o",), "gate_up": ("gate", "up"), "down": ("down",),
                 "cfg1": ("gate",)}

# The attention layer's form of the same products (exec:2451-2464): Wo's input
# is the attention output gated by sigmoid(gate), quantized by a separate
# launch (m27q_quant_act_gated, as k_quant_q8_1_fused_gate), then the product
# on those codes with the residual (m27q_matvec_q8, as l_mv_q8_on).
STAGES_ATTN = dict(STAGES)
STAGES_ATTN["o"] = lambda m27q, L, B, s: (m27q.quant_act(B.q, B.qa, gate=B.gate, stream=s),
                                          m27q.matvec_q8(L["o"], B.qa, B.h, residual=B.x, stream=s))

# Config 4: the same products on M quantized activation rows (A[K] holds the M
# rows of length K; Y[name] is [M][rows]).
STAGES_M = {
    "qkv": lambda m27q, L, A, Y, s: m27q.matmul_q8_multi([L["q"], L["k"], L["v"]], A[5120], [Y["q"], Y["k"], Y["v"]],
                                                         stream=s),
    "o": lambda m27q, L, A, Y, s: m27q.matmul_q8(L["o"], A[6144], Y["o"], stream=s),
    "gate_up": lambda m27q, L, A, Y, s: m27q.matmul_q8_multi([L["gate"], L["up"]], A[5120], [Y["gate"], Y["up"]],
                                                             stream=s),
    "down": lambda m27q, L, A, Y, s: m27q.matmul_q8(L["down"], A[17408], Y["down"], stream=s),
}


def stage_bytes(m27q, name):
    """Algorithmic HBM bytes of one product: GGUF weight bytes (unpadded) + fp32
    activation in + fp32 output (+ residual read)."""
    w = {n: (m27q.BLOCK_BYTES[getattr(m27q, t)] * rc * k // 256, rc, k) for n, t, rc, k in LAYER}
    wb = sum(w[n][0] for n in STAGE_WEIGHTS[name])
    k = w[STAGE_WEIGHTS[name][0]][2]
    rows = w[STAGE_WEIGHTS[name][0]][1] if name == "gate_up" else sum(w[n][1] for n in STAGE_WEIGHTS[name])
    res = 4 * rows if name in ("o", "down") else 0
    return wb + 4 * k + 4 * rows + res


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


def source_hash():
    """sha256 (first 16 hex digits) of the library's sources: what a committed
    profile is stamped with, so a figure read from it is used only while the
    kernels it measured are the ones built here."""
    h = hashlib.sha256()
    pkg = os.path.join(ROOT, "mono-qwen27_amd")
    files = sorted(os.path.join("csrc", f) for f in os.listdir(os.path.join(pkg, "csrc"))) + ["Makefile"]
    for f in files:
        h.update(f.encode())
        h.update(open(os.path.join(pkg, f), "rb").read())
    h.update(open(os.path.join(ROOT, "include", "m27q.h"), "rb").read())
    return h.hexdigest()[:16]


def profiled_kernel_us(kernel_label):
    """Average kernel duration (us) of one product inside the layer graph, from
    the committed rocprofv3 --kernel-trace summary, and whether that summary's
    source stamp matches the sources here (None where it is absent)."""
    path = os.path.join(ROOT, "profiles", "gemv_decode_layer_kernel_trace.txt")
    if not os.path.exists(path):
        return None, False
    us, stamp = None, None
    for line in open(path):
        if line.startswith("sources:"):
            stamp = line.split()[1]
        m = re.match(r"\s+" + re.escape(kernel_label) + r":.* avg\s+([0-9.]+) us", line)
        if m and us is None:
            us = float(m.group(1))
    return us, stamp == source_hash()


def rand_weight(m27q, torch, dev, t, rc, k, layout=None):
    """Random valid-size weight bytes (timing only; parity is the tests' job).
    fp16 scales are forced finite."""
    layout = m27q.TILED if layout is None else layout
    rb = k // m27q.BLOCK_ELEMS[t]
    raw = torch.randint(0, 256, (rc * rb, m27q.BLOCK_BYTES[t]), dtype=torch.uint8, device=dev)
    if t == m27q.Q6_K:
        raw[:, 209] = 0x0a
    else:
        raw[:, 1] = 0x0a
        if t in (m27q.Q4_K, m27q.Q5_K):
            raw[:, 3] = 0x0a
    if layout == m27q.GGUF:
        return m27q.Weight(raw.reshape(-1), t, rb, rc, layout)
    host = m27q.repack(t, rb, rc, raw.cpu().numpy().reshape(-1))
    return m27q.Weight(torch.from_numpy(host).to(dev), t, rb, rc, layout)


SETTLE_MS = 30.0
SETTLE_MS_LAYER = 100.0


def settle(torch, g, ms=SETTLE_MS, min_replays=3):
    """Untimed replays of g until the GPU has run it for at least ms.  After the
    host has left the GPU idle (capturing graphs, cloning weights), its first
    ~10 ms of work run slower: gate/up 20.4-21.2 us per launch against 18.4-19.0
    once settled, the LM head 181 us against 163."""
    t0 = time.perf_counter()
    n = 0
    while n < min_replays or (time.perf_counter() - t0) * 1e3 < ms:
        g.replay()
        n += 1
        if n % 2 == 0:
            torch.cuda.synchronize()  # host time then tracks the GPU's
    torch.cuda.synchronize()


def timed(torch, fn, ncopies, reps, warm=3, calls=32):
    """Average us per call of fn(c, stream) over ncopies rotated inputs, captured in a
    graph of at least `calls` calls (whole rotations), so graph launch boundaries
    stay rare; at least `warm` untimed replays and SETTLE_MS of them first."""
    rot = max(1, -(-calls // ncopies))
    g = capture(torch, lambda st: [fn(c, st) for _ in range(rot) for c in range(ncopies)])
    settle(torch, g, min_replays=warm)
    return time_graph(torch, g, max(1, reps // rot)) / (rot * ncopies) * 1e3


SECTIONS = ("cfg1", "cfg2", "cfg3", "types", "cfg4", "cfg5", "decode")


def suite(m27q, torch, dev, layers, host, reps, sections=SECTIONS):
    """The other configurations of the path, each timed cold (rotated copies >= 2 x MALL)."""
    out = {}
    rng = np.random.default_rng(5)
    x5120 = torch.from_numpy(rng.standard_normal(5120).astype(np.float32)).to(dev)
    if "cfg3" in sections:
        # config 3 in the integration-faithful forms: (a) the attention layer,
        # whose Wo takes the gated attention output through the separate
        # gated quantizer; (b) the layer on weights in GGUF layout, uploaded
        # verbatim as the reference's loader does (exec:1695-1716), no re-tiling
        B = Buffers(m27q, dev)
        us = timed(torch, lambda c, st: layer_pass(m27q, layers[c], B, st, STAGES_ATTN), len(layers), reps)
        out["cfg3_attention_layer_gated_wo"] = {"us": round(us, 3), "GBps": round(LAYER_BYTES / us / 1e3, 1)}
        log(f"attention layer (gated Wo): {us:.2f} us")
    # the layer copies in GGUF layout, uploaded verbatim (config 3 and config 4)
    gl = None
    if "cfg3" in sections or "cfg4" in sections:
        first = {}
        for name, (t, rc, k, blocks) in host.items():
            first[name] = m27q.Weight.upload(blocks.reshape(-1), t, k // 256, rc, m27q.GGUF, dev)
        gl = [first] + [{n: m27q.Weight(w.data.clone(), w.type, w.rb, w.rc, w.layout) for n, w in first.items()}
                        for _ in range(1, len(layers))]
        del first
        torch.cuda.synchronize()
    if "cfg3" in sections:
        us = timed(torch, lambda c, st: layer_pass(m27q, gl[c], B, st), len(gl), reps)
        out["cfg3_layer_gguf_layout"] = {"us": round(us, 3), "GBps": round(LAYER_BYTES / us / 1e3, 1)}
        log(f"layer on GGUF-layout weights: {us:.2f} us")
    # config 1: Q4_K 17408 x 5120 alone, fp32 x
    if "cfg1" in sections:
        y = torch.empty(17408, dtype=torch.float32, device=dev)
        pool = cold_pool(m27q, torch, layers, STAGE_WEIGHTS["cfg1"])
        us = timed(torch, lambda c, st: m27q.matvec(pool[c]["gate"], x5120, y, stream=st), len(pool), reps)
        del pool
        out["cfg1_q4k_17408x5120_m1"] = {"us": round(us, 3), "GBps": round(50135040 / us / 1e3, 1)}
        log(f"config 1: {us:.2f} us")
    # the further weight types at the shapes the reference's UD-Q4_K_XL file
    # gives them: the SSM layer's pair on one activation (l_mv_pair,
    # exec:2106-2125: wqkv Q6_K 10240 x 5120 and wqkv_gate Q5_K 6144 x 5120,
    # one launch per type), Q5_K alone, and IQ4_XS at the FFN's 17408 x 5120
    if "types" in sections:
        for key, spec in (("ssm_pair_q6k_10240_q5k_6144_x5120_m1", ((m27q.Q6_K, 10240), (m27q.Q5_K, 6144))),
                          ("q5k_6144x5120_m1", ((m27q.Q5_K, 6144),)),
                          ("iq4xs_17408x5120_m1", ((m27q.IQ4_XS, 17408),))):
            nbytes = sum(rc * 20 * m27q.BLOCK_BYTES[t] for t, rc in spec)
            nc = max(2, -(-2 * MALL_BYTES // nbytes) + 1)
            ws = [[rand_weight(m27q, torch, dev, t, rc, 5120) for t, rc in spec] for _ in range(nc)]
            ys = [torch.empty(rc, dtype=torch.float32, device=dev) for _, rc in spec]
            if len(spec) == 1:
                us = timed(torch, lambda c, st: m27q.matvec(ws[c][0], x5120, ys[0], stream=st), nc, reps)
            else:
                us = timed(torch, lambda c, st: m27q.matvec_multi(ws[c], x5120, ys, stream=st), nc, reps)
            out[key] = {"us": round(us, 3), "GBps": round(nbytes / us / 1e3, 1), "bytes": nbytes}
            log(f"{key}: {us:.2f} us")
            del ws
    # config 2: Q8_0 draft shapes, fp32 x
    for rc, k in ((2048, 2048), (6144, 2048), (2048, 6144)) if "cfg2" in sections else ():
        nbytes = rc * k // 32 * 34
        nc = max(2, -(-2 * MALL_BYTES // nbytes) + 1)
        ws = [rand_weight(m27q, torch, dev, m27q.Q8_0, rc, k) for _ in range(nc)]
        xx = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(dev)
        yy = torch.empty(rc, dtype=torch.float32, device=dev)
        us = timed(torch, lambda c, st: m27q.matvec(ws[c], xx, yy, stream=st), nc, reps)
        out[f"cfg2_q80_{rc}x{k}_m1"] = {"us": round(us, 3), "GBps": round(nbytes / us / 1e3, 1)}
        del ws
    if "cfg2" in sections:
        log("config 2 done")
    # config 4: the layer's products on M quantized activation rows
    for M in (2, 4, 8, 16) if "cfg4" in sections else ():
        acts = {k: m27q.Act(M, k, dev) for k in (5120, 6144, 17408)}
        for k, a in acts.items():
            m27q.quant_act(torch.from_numpy(rng.standard_normal((M, k)).astype(np.float32)).to(dev), a)
        Ys = {n: torch.empty((M, rc), dtype=torch.float32, device=dev) for n, _, rc, _ in LAYER}

        def layer_m(c, st, L=layers):
            for fn in STAGES_M.values():
                fn(m27q, L[c], acts, Ys, st)
        us = timed(torch, layer_m, len(layers), reps)
        out[f"cfg4_layer_m{M}"] = {"us": round(us, 3), "GBps": round(LAYER_BYTES / us / 1e3, 1)}
        # the same on the GGUF-layout copies
        us_g = timed(torch, lambda c, st: layer_m(c, st, gl), len(gl), reps)
        out[f"cfg4_layer_m{M}_gguf_layout"] = {"us": round(us_g, 3), "GBps": round(LAYER_BYTES / us_g / 1e3, 1)}
        log(f"config 4 M={M}: {us:.2f} us, GGUF layout {us_g:.2f} us")
    del gl
    # config 5: LM head GEMV, exact top-64, 512-row gather
    if "cfg5" in sections or "decode" in sections:
        lm = rand_weight(m27q, torch, dev, m27q.Q6_K, 248320, 5120)
        logits = torch.empty(248320, dtype=torch.float32, device=dev)
        k = 64
        scratch = torch.empty(m27q.topk_scratch_bytes(248320, k), dtype=torch.uint8, device=dev)
        idx = torch.empty(k, dtype=torch.int32, device=dev)
        val = torch.empty(k, dtype=torch.float32, device=dev)
    if "cfg5" in sections:
        # 8 launches per graph replay (the 1 GB table is 4x the MALL, so every
        # launch streams it from HBM), so the host's replay cost stays hidden
        us = timed(torch, lambda c, st: m27q.matvec(lm, x5120, logits, stream=st), 8, max(8, reps // 8))
        out["cfg5_lm_head_q6k_248320x5120"] = {"us": round(us, 3), "GBps": round(248320 * 4200 / us / 1e3, 1)}
        # 16 calls per graph replay, so the host's replay cost stays hidden behind the GPU
        us = timed(torch, lambda c, st: m27q.topk(logits, k, idx, val, scratch, stream=st), 16, reps)
        out["cfg5_topk64_of_248320"] = {"us": round(us, 3), "GBps": round(248320 * 4 / us / 1e3, 1)}
        # 256 id sets (2.15 MB of rows each, 550 MB over a rotation: >= 2 x the
        # Infinity Cache), so the rows stream from HBM as in a cold prefill
        nsets = -(-2 * MALL_BYTES // (512 * 4200)) + 1
        ids = [torch.from_numpy(rng.integers(0, 248320, 512).astype(np.int32)).to(dev) for _ in range(nsets)]
        rows = torch.empty((512, 5120), dtype=torch.float32, device=dev)
        us = timed(torch, lambda c, st: m27q.embed_rows(lm, ids[c], rows, stream=st), nsets, reps)
        out["cfg5_gather_512_q6k_rows"] = {"us": round(us, 3),
                                           "GBps": round((512 * 4200 + 512 * 5120 * 4) / us / 1e3, 1)}
        log("config 5 done")
    if "decode" not in sections:
        return out
    # A decode step of linears, one graph with nothing on the host in between:
    # the embedding row of one token id (the 248320 x 5120 Q6_K table stands in
    # for token_embd), 64 layers of the layer's four products over the rotated
    # cold copies (every fourth layer, il % 4 == 3, is an attention layer whose
    # Wo takes the gated quantizer's codes, exec:2451-2464), the LM head, the
    # exact top-64 and the on-device sample.
    B = Buffers(m27q, dev)
    tok_id = torch.tensor([12345], dtype=torch.int32, device=dev)
    u = torch.full((1,), 0.3, dtype=torch.float32, device=dev)
    tok = torch.empty(1, dtype=torch.int32, device=dev)

    def decode_step(c, st):
        m27q.embed_rows(lm, tok_id, B.x.view(1, 5120), stream=st)
        for li in range(64):
            layer_pass(m27q, layers[li % len(layers)], B, st, STAGES_ATTN if li % 4 == 3 else STAGES)
        m27q.matvec(lm, B.out, logits, stream=st)
        m27q.topk(logits, k, idx, val, scratch, stream=st)
        m27q.sample(idx, val, k, 0.8, 0.05, 0.95, u, tok, stream=st)
    us = timed(torch, decode_step, 1, max(4, reps // 10), calls=1)
    out["decode_step_linears_64_layers"] = {"us": round(us, 1), "tokens_per_s": round(1e6 / us, 1)}
    log(f"decode step of linears: {us:.1f} us")
    return out


def layer_pass(m27q, L, B, stream, stages=STAGES):
    for fn in stages.values():
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


def replay_times(torch, g, reps):
    """ms of each replay, from HIP events between consecutive replays."""
    s = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    torch.cuda.synchronize()
    ev[0].record(s)
    for i in range(reps):
        g.replay()
        ev[i + 1].record(s)
    ev[-1].synchronize()
    return [ev[i].elapsed_time(ev[i + 1]) for i in range(reps)]


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


STREAM_SIZES_MB = (4.456, 13.37, 17.76, 21.63, 23.65, 47.35, 50.14, 64.63, 73.22, 100.36, 200.0, 1000.0)


def stream_lib():
    """The plain streaming read of libm27q_stream.so (the measured HBM read peak)."""
    import ctypes as C
    L = C.CDLL(os.path.join(ROOT, "mono-qwen27_amd", "libm27q_stream.so"))
    L.m27q_stream_read.restype = C.c_int
    L.m27q_stream_read.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p]
    return L


def stream_read_peak(torch, dev, reps):
    """GB/s of the plain streaming read at each size (the Q8_0 draft products'
    sizes, the layer's product sizes, the further weight types' products, 200
    MB and 1 GB), from HIP events over graph replays that rotate through
    >= 2 x the 256 MB Infinity Cache of distinct bytes (each read streams from
    HBM).  Every launch includes its dispatch, as the products' figures do."""
    L = stream_lib()
    total = 1100 << 20
    buf = torch.zeros(total // 4, dtype=torch.float32, device=dev)
    sink = torch.zeros(1 << 17, dtype=torch.float32, device=dev)
    out = {}
    for mb in STREAM_SIZES_MB:
        nbytes = int(mb * 1e6) // 16 * 16
        ncopy = max(1, min(total // nbytes, -(-2 * MALL_BYTES // nbytes) + 1))
        per = max(1, 64 // ncopy) if mb < 200 else 4

        def body(st, nbytes=nbytes, ncopy=ncopy, per=per):
            for _ in range(per):
                for c in range(ncopy):
                    rc = L.m27q_stream_read(buf.data_ptr() + c * nbytes, nbytes, sink.data_ptr(), st.cuda_stream)
                    assert rc == 0, rc
        g = capture(torch, body)
        settle(torch, g)
        us = time_graph(torch, g, max(3, reps // 10)) / (per * ncopy) * 1e3
        out[f"{mb:g}MB"] = round(nbytes / us / 1e3, 1)
        log(f"stream read {mb:g} MB: {us:.2f} us, {out[f'{mb:g}MB']} GB/s")
    del buf
    return out


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(ora, host, budget_s=8.0, single_budget_s=3.0):
    """The oracle's restatement of ggml's CPU path (q8_K activations, q4_K x q8_K /
    q6_K x q8_K dots), rows split over host threads, on the same layer weights:
    the AVX2 build and the scalar C build, each at up to 16 threads (the box's
    CPU share) and at one thread.  value is the AVX2 build at all threads."""
    nthreads = max(1, min(16, os.cpu_count() or 1))
    x = np.random.default_rng(1).standard_normal(17408).astype(np.float32)
    xq = {k: ora.quant_cpu_act(ora.Q4_K, x[:k]) for k in (5120, 6144, 17408)}
    total_bytes = sum(b.nbytes for (_, _, _, b) in host.values())

    def passes(nt, budget, simd):
        reps, t0 = 0, time.perf_counter()
        while True:
            for name, (t, rc, k, blocks) in host.items():
                ora.gemv_cpu(t, blocks, k // 256, rc, xq[k], nthreads=nt, simd=simd)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget or (reps >= 1 and el * (reps + 1) / reps > budget):
                return reps, el

    res = {}
    for simd in (True, False):
        for nt, budget in ((nthreads, budget_s), (1, single_budget_s)):
            reps, el = passes(nt, budget, simd)
            res[(simd, nt)] = (reps, el, el / reps)
    gbs = {k: round(total_bytes / v[2] / 1e9, 3) for k, v in res.items()}
    desc = "; ".join(f"{'AVX2' if sm else 'scalar'} {nt} thread{'s' if nt > 1 else ''}: {r} layer passes in "
                     f"{el:.2f} s ({sec * 1e6:.0f} us/layer)" for (sm, nt), (r, el, sec) in res.items())
    return {"value": gbs[(True, nthreads)], "unit": "GB/s", "cores": nthreads, "kind": "port",
            "single_thread_value": gbs[(True, 1)],
            "scalar_value": gbs[(False, nthreads)], "scalar_single_thread_value": gbs[(False, 1)],
            "cpu_model": cpu_model(), "nproc": os.cpu_count(),
            "sample": f"full layer passes (7 matvecs, {total_bytes} weight bytes): {desc}; the oracle's "
                      f"restatement of ggml's q4_K/q6_K x q8_K CPU dots in AVX2 and in scalar C (not ggml "
                      f"itself: the vendored ref/llama.cpp is empty)"}


def wave_timeline(m27q, torch, dev, layers, B, trials=3):
    """Per-wave timeline of each M = 1 product, one launch on cold weights per
    trial (the last of a run of back-to-back launches), from the measurement build (libm27q_timeline.so: the same kernels
    recording, per wave, the real-time counter at start, once the activation is
    staged in LDS, and at the end, with the wave's CU).  Prints one summary per
    launch: quantiles (p0/p10/p50/p90/p100, microseconds) of wave start,
    staging time, compute time and end; the mean time CUs sit idle between
    their last wave's end and the launch's end; and the CUs' end times grouped
    by how many workgroups each CU ran."""
    import collections
    import ctypes as C
    L = m27q.lib()
    L.m27q_timeline_read.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    y = torch.empty(17408, dtype=torch.float32, device=dev)
    prods = dict(STAGES)
    prods["cfg1"] = lambda m27q, Lw, B, s: m27q.matvec(Lw["gate"], B.x, y, stream=s)
    N = 1 << 16
    q = lambda a: "/".join(f"{np.percentile(a, p):.2f}" for p in (0, 10, 50, 90, 100))
    for name, fn in prods.items():
        pool = cold_pool(m27q, torch, layers, STAGE_WEIGHTS[name])
        for trial in range(trials):
            if L.m27q_timeline_clear() != 0:
                raise RuntimeError("m27q_timeline_clear failed")
            # The recorded launch follows other launches with nothing in
            # between, as in a decode step: a launch that follows a host copy
            # or an idle queue starts its waves on the 8 XCDs up to ~4 us
            # apart, one that follows a kernel within ~0.2 us.  Every launch
            # writes the same slots, so the records are the last launch's.
            for r in range(len(pool) + trial + 1):
                fn(m27q, pool[r % len(pool)], B, None)
            torch.cuda.synchronize()
            t = np.zeros((N, 3), np.uint64)
            hw = np.zeros((N, 3), np.uint32)
            if L.m27q_timeline_read(t.ctypes.data, hw.ctypes.data, N) != 0:
                raise RuntimeError("m27q_timeline_read failed")
            used = t[:, 0] > 0
            ts, h = t[used].astype(np.int64), hw[used]
            st, sg, en = [(ts[:, j] - ts[:, 0].min()) / 100.0 for j in range(3)]  # 100 MHz counter
            hid = h[:, 0].astype(np.int64)
            cu = ((h[:, 1].astype(np.int64) & 0xf) << 8) | (((hid >> 13) & 7) << 5) | (((hid >> 12) & 1) << 4) | ((hid >> 8) & 0xf)
            blk = h[:, 2] >> 8
            cu_blocks, cu_end = collections.defaultdict(set), collections.defaultdict(float)
            for c, b, e in zip(cu.tolist(), blk.tolist(), en.tolist()):
                cu_blocks[c].add(b)
                cu_end[c] = max(cu_end[c], e)
            span = float(en.max())
            by = collections.defaultdict(list)
            for c, b in cu_blocks.items():
                by[len(b)].append(cu_end[c])
            idle = float(np.mean([span - e for e in cu_end.values()]))
            print(f"{name:8s} launch {trial}: waves {len(ts)} on {len(cu_blocks)} CUs, span {span:.2f} us | "
                  f"start {q(st)} | staging {q(sg - st)} | compute {q(en - sg)} | end {q(en)} | "
                  f"mean CU idle at the end {idle:.2f} us ({100 * idle / span:.0f}%)", flush=True)
            print("    CU end by workgroups per CU {n: (CUs, mean us, max us)}:",
                  {k: (len(v), round(float(np.mean(v)), 2), round(float(np.max(v)), 2)) for k, v in sorted(by.items())},
                  flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--copies", type=int, default=0, help="distinct weight copies (0: auto, >= 2x MALL)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-suite", action="store_true", help="skip the configurations other than the layer")
    ap.add_argument("--only", default="",
                    help="comma-separated suite sections (cfg1,cfg2,cfg3,types,cfg4,cfg5,decode) to run alone, without the "
                         "layer timing; prints their figures (for profiler runs), not the benchmark line")
    ap.add_argument("--timeline", action="store_true",
                    help="per-wave timeline of each M = 1 product from the measurement build "
                         "(libm27q_timeline.so); prints summaries, not the benchmark line")
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
    if args.timeline:
        m27q.LIB_PATH = os.path.join(os.path.dirname(m27q.LIB_PATH), "libm27q_timeline.so")
    dev = torch.device("cuda:0")
    layer_bytes = LAYER_BYTES
    copies = args.copies or max(2, -(-2 * MALL_BYTES // layer_bytes) + 1)
    log(f"building {copies} layer copies ({layer_bytes * copies / 2**20:.0f} MiB)")
    layers, host = build_layers(m27q, ora, dev, copies)
    if args.only:
        secs = tuple(x for x in args.only.split(",") if x)
        bad = [x for x in secs if x not in SECTIONS]
        if bad:
            print(f"unknown sections {bad}; known: {SECTIONS}", file=sys.stderr)
            sys.exit(2)
        print(json.dumps({"only": secs,
                          "suite": suite(m27q, torch, dev, layers, host, max(1, args.steps // copies), secs)}))
        return
    B = Buffers(m27q, dev)
    if args.timeline:
        wave_timeline(m27q, torch, dev, layers, B)
        return

    # A decode step replays one graph for all its layers, so the K timed layer
    # passes replay one captured graph of exactly K passes (pass i on copy
    # i mod copies, continuing after the W warmup passes; past MAXG passes, a
    # graph of MAXG is replayed and a last one holds the remainder): the
    # timed region has one graph launch boundary, as a decode step does.
    MAXG = max(copies, 1024 // copies * copies)

    def passes(st, first, n):
        for i in range(first, first + n):
            layer_pass(m27q, layers[i % copies], B, st)

    def pass_graphs(first, n):
        """[(graph, replays)] running passes first .. first + n - 1."""
        if n <= 0:
            return []
        q, r = divmod(n, MAXG)
        out = []
        if q:
            out.append((capture(torch, lambda st: passes(st, first, MAXG)), q))
        if r:
            out.append((capture(torch, lambda st: passes(st, first + q * MAXG, r)), 1))
        return out

    def replay(gs):
        for g, n in gs:
            for _ in range(n):
                g.replay()

    log("capturing graphs")
    g_settle = capture(torch, lambda st: passes(st, 0, 8 * copies))
    g_warmup = pass_graphs(0, args.warmup)
    g_timed = pass_graphs(args.warmup, args.steps)
    PG = 8 * copies
    g_warm = capture(torch, lambda st: [layer_pass(m27q, layers[0], B, st) for _ in range(PG)])

    # The GPU's clocks settle first (untimed layer passes, SETTLE_MS_LAYER of
    # them), then the W warmup passes run, then the K timed ones.
    settle(torch, g_settle, SETTLE_MS_LAYER)
    replay(g_warmup)
    torch.cuda.synchronize()
    log(f"timing {args.steps} layer passes")
    s0 = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(s0)
    replay(g_timed)
    e1.record(s0)
    e1.synchronize()
    ms_cold = e0.elapsed_time(e1) / args.steps
    reps = max(1, args.steps // copies)
    ms_warm = time_graph(torch, g_warm, max(1, args.steps // PG)) / PG
    # Spread: the timed graph (its first, or only, graph) replayed alone ten
    # times, each replay timed by one event pair, as the headline is.
    g0, _ = g_timed[0]
    n0 = min(args.steps, MAXG)
    per = [time_graph(torch, g0, 1) / n0 * 1e3 for _ in range(10)]

    # Each product on its own, over copies of its own weights that exceed the
    # Infinity Cache twice over (graphs of at least 32 launches): average launch
    # duration from HIP events on the replay stream.
    stages = {}
    for name, fn in STAGES.items():
        pool = cold_pool(m27q, torch, layers, STAGE_WEIGHTS[name])
        rot = max(1, -(-32 // len(pool)))
        g = capture(torch, lambda st, fn=fn: [fn(m27q, L, B, st) for _ in range(rot) for L in pool])
        settle(torch, g)
        ms = time_graph(torch, g, max(3, args.steps // (rot * len(pool)))) / (rot * len(pool))
        del g, pool
        nbytes = stage_bytes(m27q, name)
        stages[name] = {"us": round(ms * 1e3, 3), "bytes": nbytes, "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)}
        log(f"{name}: {ms * 1e3:.2f} us, {stages[name]['GBps']} GB/s")
    # The dominant kernel is the SwiGLU product (100 MB of the layer's 215 MB),
    # the gate/up stage.
    dom = stages["gate_up"]

    # The plain streaming read at the products' sizes: the measured peak.
    read_gbs = stream_read_peak(torch, dev, reps)
    if args.calib:
        # kernels of known size for scaling the FETCH_SIZE / WRITE_SIZE counters:
        # a 1 GiB streaming read and a 512 MiB device copy
        L = stream_lib()
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        sink = torch.zeros(1 << 17, dtype=torch.float32, device=dev)
        for _ in range(3):
            assert L.m27q_stream_read(src.data_ptr(), 1 << 30, sink.data_ptr(),
                                      torch.cuda.current_stream().cuda_stream) == 0
        dst = torch.empty(1 << 27, dtype=torch.float32, device=dev)
        for _ in range(3):
            dst.copy_(src[:1 << 27])
        torch.cuda.synchronize()
        del src, dst

    gbs = layer_bytes / (ms_cold * 1e-3) / 1e9
    prof_us, prof_current = profiled_kernel_us("gate_up")
    ach = dom["GBps"]
    rec = {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_cold, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "qwen27b_q4km_decode_layer_linears_m1",
                   "layer": {n: f"{t} {rc}x{k}" for n, t, rc, k in LAYER},
                   "weight_bytes": layer_bytes, "layout": "tiled", "activation": "int8 per-32, fp32 scale",
                   "cold_copies": copies, "graph": True, "layer_passes_per_graph": n0,
                   "untimed_settle_ms_before_warmup": SETTLE_MS_LAYER},
        "us_per_layer": round(ms_cold * 1e3, 2),
        "us_per_layer_batches_p10_median_p90": [round(float(np.percentile(per, q)), 2) for q in (10, 50, 90)],
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
        "lower_bound_us": round(layer_bytes / HBM_PEAK_GBS / 1e3, 2),
        "x_lower_bound": round(ms_cold * 1e3 / (layer_bytes / HBM_PEAK_GBS / 1e3), 3),
        "warm_us_per_layer": round(ms_warm * 1e3, 2),
        "hbm_read_GBps_measured": read_gbs,
        "stages": stages,
        "roofline": {"bound": "hbm", "kernel": "k_gemv_q8<Q4K,TILED,GemvCfg<4,1,1>,SWIGLU> (gate+up 17408x5120, "
                                               "fp32 x in, fp32 y out)",
                     "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": measured_traffic("gate_up"),
                     "achieved_source": "HIP events of this run: the product alone, graphs of >= 32 launches over "
                                        "cold copies, on the replay stream (dispatch gap to the next launch included)",
                     "avg_launch_us_events": dom["us"],
                     # the kernel inside the layer graph, from the committed
                     # rocprofv3 trace; null when that trace was taken from
                     # other sources than the ones built here
                     "rocprof_kernel_avg_us_in_layer": prof_us if prof_current else None,
                     "rocprof_source_stamp": source_hash(),
                     "measured_read_GBps_100MB_events": read_gbs.get("100.36MB"),
                     "frac_of_measured_read": (round(ach / read_gbs["100.36MB"], 4)
                                               if read_gbs.get("100.36MB") else None),
                     "traffic_source": "profiles/gemv_decode_layer_hbm_traffic.txt",
                     "algorithmic_bytes": dom["bytes"]},
    }
    if not args.no_suite:
        rec["suite"] = suite(m27q, torch, dev, layers, host, reps)
    if not args.no_cpu:
        log("cpu baseline")
        rec["cpu_baseline"] = cpu_baseline(ora, host)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
