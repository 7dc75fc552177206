"""A decode step recorded into one HIP graph and replayed: every replay must
equal the same calls run eagerly on the same inputs, bit for bit.

The library allocates, clears and synchronizes nothing (the top-k counter is
reset by a kernel), so the whole step -- embedding gather, q/k/v, o with
residual, gate/up with the fused output quantization, down, the small-M
products (the resident-activation kernel included), the LM head, top-k and
sampling -- can be captured, as the
reference captures its step (exec:2353-2360).  Between replays the inputs are
rewritten by eager copies and the outputs read back, with synchronizations in
between, so stale state carried from one replay to the next would show."""
import numpy as np
import pytest

from gpu_util import say, to_dev, to_host

pytestmark = pytest.mark.gpu


def bits(t):
    a = to_host(t)
    return a.view(np.uint8).copy()


def test_decode_step_graph_replays_match_eager(m27q, ora, dev):
    import torch
    W = {}
    for name, t, rc, k, seed in (("emb", m27q.Q6_K, 4096, 5120, 1), ("q", m27q.Q4_K, 1024, 5120, 2),
                                 ("o", m27q.Q4_K, 5120, 1024, 3), ("gate", m27q.Q4_K, 2048, 5120, 4),
                                 ("up", m27q.Q4_K, 2048, 5120, 5), ("down", m27q.Q6_K, 5120, 2048, 6),
                                 ("lm", m27q.Q6_K, 8192, 5120, 7),
                                 ("big", m27q.Q4_K, 16400, 5120, 8)):  # resident activation rows at M = 16
        W[name] = m27q.Weight.upload(ora.synth_weights(t, rc, k, seed=seed).reshape(-1), t,
                                     k // m27q.BLOCK_ELEMS[t], rc, m27q.TILED, dev)
    k = 40
    ids = torch.zeros(2, dtype=torch.int32, device=dev)
    u = torch.zeros(1, dtype=torch.float32, device=dev)
    x = torch.empty((2, 5120), dtype=torch.float32, device=dev)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    qv = torch.empty(1024, dtype=torch.float32, device=dev)
    h = torch.empty(5120, dtype=torch.float32, device=dev)
    f = torch.empty(2048, dtype=torch.float32, device=dev)
    fq = m27q.Act(1, 2048, dev)
    out = torch.empty(5120, dtype=torch.float32, device=dev)
    out2 = torch.empty(5120, dtype=torch.float32, device=dev)
    act2 = m27q.Act(2, 5120, dev)
    Y2 = torch.empty((2, 1024), dtype=torch.float32, device=dev)
    act16 = m27q.Act(16, 5120, dev)
    X16 = torch.empty((16, 5120), dtype=torch.float32, device=dev)
    Y16 = torch.empty((16, 2048), dtype=torch.float32, device=dev)
    Y16b = torch.empty((16, 16400), dtype=torch.float32, device=dev)
    act5 = m27q.Act(5, 5120, dev)
    X5 = torch.empty((5, 5120), dtype=torch.float32, device=dev)
    Y5 = torch.empty((5, 8192), dtype=torch.float32, device=dev)      # two row sets per tile
    Y5q = torch.empty((5, 1024), dtype=torch.float32, device=dev)
    Y5g = torch.empty((5, 2048), dtype=torch.float32, device=dev)
    logits = torch.empty(8192, dtype=torch.float32, device=dev)
    scratch = torch.empty(m27q.topk_scratch_bytes(8192, k), dtype=torch.uint8, device=dev)
    idx = torch.empty(k, dtype=torch.int32, device=dev)
    val = torch.empty(k, dtype=torch.float32, device=dev)
    tok = torch.empty(1, dtype=torch.int32, device=dev)
    outs = [x, qv, h, f, fq.buf, out, out2, Y2, Y16, Y16b, Y5, Y5q, Y5g, logits, idx, val, tok]

    def step(s):
        m27q.embed_rows(W["emb"], ids, x, bad, stream=s)
        m27q.matvec(W["q"], x[0], qv, stream=s)
        m27q.matvec(W["o"], qv, h, residual=x[1], stream=s)
        m27q.ffn_swiglu(W["gate"], W["up"], h, f, yq=fq, stream=s)
        m27q.matvec_q8(W["down"], fq, out, residual=h, stream=s)
        m27q.matvec(W["down"], f, out2, residual=h, stream=s)  # the fp32 hand-off to down
        m27q.quant_act(x, act2, stream=s)
        m27q.matmul_q8(W["q"], act2, Y2, stream=s)
        m27q.quant_act(X16, act16, stream=s)
        m27q.matmul_q8(W["gate"], act16, Y16, stream=s)
        m27q.matmul_q8(W["big"], act16, Y16b, stream=s)
        m27q.quant_act(X5, act5, stream=s)
        m27q.matmul_q8(W["lm"], act5, Y5, stream=s)
        m27q.matmul_q8_multi([W["q"], W["gate"]], act5, [Y5q, Y5g], stream=s)
        m27q.matvec(W["lm"], out, logits, stream=s)
        m27q.topk(logits, k, idx, val, scratch, stream=s)
        m27q.sample(idx, val, k, 0.8, 0.05, 0.95, u, tok, stream=s)

    rng = np.random.default_rng(0)

    def set_inputs(i):
        ids.copy_(torch.from_numpy(np.array([7 + 13 * i, 4000 - 5 * i], np.int32)))
        u.fill_(0.15 + 0.3 * i)
        X16.copy_(torch.from_numpy(rng.standard_normal((16, 5120)).astype(np.float32)))
        X5.copy_(torch.from_numpy(rng.standard_normal((5, 5120)).astype(np.float32)))
        torch.cuda.synchronize()

    # eager reference results for three input sets
    want = []
    for i in range(3):
        set_inputs(i)
        X16_i, X5_i = X16.clone(), X5.clone()
        say("graph eager", i)
        step(torch.cuda.current_stream())
        torch.cuda.synchronize()
        want.append(([bits(t) for t in outs], X16_i, X5_i))
    assert to_host(bad)[0] == 0

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(s)  # warm pass on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(torch.cuda.current_stream())
    torch.cuda.synchronize()
    for rep in range(2):
        for i in range(3):
            set_inputs(i)
            X16.copy_(want[i][1])
            X5.copy_(want[i][2])
            for t in outs:
                t.zero_()
            torch.cuda.synchronize()
            say("graph replay", rep, i)
            g.replay()
            torch.cuda.synchronize()
            for j, (t, w) in enumerate(zip(outs, want[i][0])):
                assert np.array_equal(bits(t), w), (rep, i, j)
