"""Every launch bench.py times, at its benched shape, layout and activation
form, against the oracle: the decode layer's four products (TILED, fp32
activations, residuals), the Q4_K 17408 x 5120 product alone, the Q8_0 draft
shapes, the layer at M = 2, 4, 8 and 16 rows, the 248320 x 5120 Q6_K LM head
on a TILED table with an fp32 hidden state (exact top-64 and sampled rows) and
the 512-row gather from that table.  The launches are bench.py's own (its
STAGES / STAGES_M and rand_weight)."""
import numpy as np
import pytest

from gpu_util import act_host, int_dot_tol, say, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def bench():
    import importlib.util
    import os
    from conftest import ROOT
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="module")
def layer(bench, m27q, ora, dev):
    """One copy of the benched layer (bench.build_layers: the same seeds), and
    the GGUF blocks it was made from."""
    layers, host = bench.build_layers(m27q, ora, dev, 1)
    return layers[0], host


def check_rows(ora, t, blocks, rb, rc, x, got, residual=None):
    """got (fp32 [rc]) against the integer-dot oracle on x's quantization."""
    q, d, s = ora.quant_act(x)
    want, nrm = ora.gemv_act(t, blocks, rb, rc, q, d, s)
    g = got.astype(np.float64)
    tol = int_dot_tol(nrm)
    if residual is not None:
        g = g - residual
        tol = tol + 1e-6 * np.abs(residual)
    bad = np.abs(g - want) > tol
    assert not bad.any(), (np.flatnonzero(bad)[:5], g[bad][:5], want[bad][:5])


def test_decode_layer_stages_as_benched(bench, layer, m27q, ora, dev):
    """The four products of bench.layer_pass, in order, each checked on the
    GPU's own input to it: q/k/v on x; o on q (+ x); SwiGLU gate/up on h; down
    on f (+ h)."""
    L, host = layer
    B = bench.Buffers(m27q, dev)
    for name, fn in bench.STAGES.items():
        say("bench stage", name)
        fn(m27q, L, B, None)
    x, q, h, f, out = (to_host(t) for t in (B.x, B.q, B.h, B.f, B.out))
    for name, y in (("q", q), ("k", to_host(B.k)), ("v", to_host(B.v))):
        t, rc, k, blocks = host[name]
        check_rows(ora, t, blocks, k // 256, rc, x, y)
    t, rc, k, blocks = host["o"]
    check_rows(ora, t, blocks, k // 256, rc, q, h, residual=x.astype(np.float64))
    # SwiGLU: silu(g) u from the oracle's g and u (fp32 error of each carried through)
    tg, rc, k, gb = host["gate"]
    _, _, _, ub = host["up"]
    qq, dd, ss = ora.quant_act(h)
    g, gn = ora.gemv_act(tg, gb, k // 256, rc, qq, dd, ss)
    u, un = ora.gemv_act(tg, ub, k // 256, rc, qq, dd, ss)
    sg = g / (1 + np.exp(-g))
    tol = 1.1 * int_dot_tol(gn) * np.abs(u) + np.abs(sg) * int_dot_tol(un) + 4e-7 * np.abs(sg * u) + 1e-30
    assert (np.abs(f.astype(np.float64) - sg * u) <= tol).all()
    t, rc, k, blocks = host["down"]
    check_rows(ora, t, blocks, k // 256, rc, f, out, residual=h.astype(np.float64))


def test_config1_alone_as_benched(layer, m27q, ora, dev):
    """Config 1: the Q4_K 17408 x 5120 product alone on an fp32 x."""
    import torch
    L, host = layer
    x = np.random.default_rng(5).standard_normal(5120).astype(np.float32)
    y = torch.empty(17408, dtype=torch.float32, device=dev)
    say("config 1")
    m27q.matvec(L["gate"], to_dev(x, dev), y)
    t, rc, k, blocks = host["gate"]
    check_rows(ora, t, blocks, 20, rc, x, to_host(y))


@pytest.mark.parametrize("rc,k", [(2048, 2048), (6144, 2048), (2048, 6144)])
def test_config2_q80_draft_as_benched(bench, m27q, ora, dev, rc, k):
    """Config 2: Q8_0 draft shapes, TILED, fp32 x (bench.rand_weight bytes)."""
    import torch
    w = bench.rand_weight(m27q, torch, dev, m27q.Q8_0, rc, k)
    gguf = m27q.unpack(m27q.Q8_0, w.rb, rc, to_host(w.data))
    x = np.random.default_rng(rc + k).standard_normal(k).astype(np.float32)
    y = torch.empty(rc, dtype=torch.float32, device=dev)
    say("config 2", rc, k)
    m27q.matvec(w, to_dev(x, dev), y)
    check_rows(ora, m27q.Q8_0, gguf, w.rb, rc, x, to_host(y))


@pytest.mark.parametrize("M", [2, 4, 8, 16])
def test_config4_layer_as_benched(bench, layer, m27q, ora, dev, M):
    """Config 4: bench.STAGES_M on M quantized rows; every token row of q/k/v,
    o, gate, up and down against the integer-dot oracle."""
    import torch
    L, host = layer
    rng = np.random.default_rng(100 + M)
    X = {k: rng.standard_normal((M, k)).astype(np.float32) for k in (5120, 6144, 17408)}
    A = {k: m27q.Act(M, k, dev) for k in X}
    for k, a in A.items():
        m27q.quant_act(to_dev(X[k], dev), a)
    Y = {n: torch.empty((M, rc), dtype=torch.float32, device=dev) for n, _, rc, _ in bench.LAYER}
    for name, fn in bench.STAGES_M.items():
        say("config 4", M, name)
        fn(m27q, L, A, Y, None)
    rows = range(M)
    for n, _, rc, k in bench.LAYER:
        t, _, _, blocks = host[n]
        q, d, s = act_host(m27q, A[k])
        got = to_host(Y[n]).astype(np.float64)
        for m in rows:
            want, nrm = ora.gemv_act(t, blocks, k // 256, rc, q[m], d[m], s[m])
            assert (np.abs(got[m] - want) <= int_dot_tol(nrm)).all(), (n, m)


@pytest.fixture(scope="module")
def lm_head(bench, m27q, dev):
    """The benched 248320 x 5120 Q6_K table: bench.rand_weight's random blocks
    (finite d) re-tiled on the host, TILED on the device."""
    import torch
    torch.manual_seed(20)
    return bench.rand_weight(m27q, torch, dev, m27q.Q6_K, 248320, 5120)


def gguf_rows(m27q, w, rows):
    """GGUF bytes of the given rows of a TILED weight, unpacked tile by tile."""
    unit = m27q.weight_bytes(w.type, w.rb, 8, m27q.TILED)  # one 8-row tile
    data = w.data
    out = []
    for r in rows:
        t = int(r) // 8
        tile = to_host(data[t * unit:(t + 1) * unit])
        g = m27q.unpack(w.type, w.rb, 8, tile).reshape(8, -1)
        out.append(g[int(r) % 8])
    return np.stack(out)


def test_config5_lm_head_tiled_fp32(m27q, ora, dev, lm_head):
    """LM head as benched (TILED, fp32 hidden state): exact top-64 of the GPU
    logits, and 256 sampled rows against the integer-dot oracle."""
    import torch
    from test_gpu_topk import run_topk
    h = np.random.default_rng(22).standard_normal(5120).astype(np.float32)
    logits = torch.empty(248320, dtype=torch.float32, device=dev)
    say("lm head tiled fp32")
    m27q.matvec(lm_head, to_dev(h, dev), logits)
    lg = to_host(logits)
    idx, val = run_topk(m27q, dev, lg, 64)
    oi, ov = ora.topk(lg, 64)
    assert np.array_equal(idx, oi) and np.array_equal(val.view(np.uint32), ov.view(np.uint32))
    rows = np.concatenate([np.random.default_rng(23).integers(0, 248320, 254), [0, 248319]])
    host = gguf_rows(m27q, lm_head, rows)
    q, d, s = ora.quant_act(h)
    want, nrm = ora.gemv_act(m27q.Q6_K, host, 20, rows.size, q, d, s)
    assert (np.abs(lg[rows].astype(np.float64) - want) <= int_dot_tol(nrm)).all()


def test_config5_gather_tiled(m27q, ora, dev, lm_head):
    """512-row gather from the TILED table, bit-exact."""
    import torch
    ids = np.random.default_rng(21).integers(0, 248320, 512).astype(np.int32)
    ids[:2] = [0, 248319]
    out = torch.empty((512, 5120), dtype=torch.float32, device=dev)
    say("gather 512 tiled")
    m27q.embed_rows(lm_head, to_dev(ids, dev), out)
    want = ora.dequant(m27q.Q6_K, gguf_rows(m27q, lm_head, ids), 20, 512)
    assert np.array_equal(to_host(out).view(np.uint32), want.view(np.uint32))
