"""Exact top-k on the GPU vs the oracle's total order (value desc, index asc)."""
import numpy as np
import pytest

from gpu_util import say, to_dev, to_host

pytestmark = pytest.mark.gpu


def run_topk(m27q, dev, v, k):
    import torch
    n = v.size
    idx = torch.empty(k, dtype=torch.int32, device=dev)
    val = torch.empty(k, dtype=torch.float32, device=dev)
    scratch = torch.empty(m27q.topk_scratch_bytes(n, k), dtype=torch.uint8, device=dev)
    m27q.topk(to_dev(v, dev), k, idx, val, scratch)
    return to_host(idx), to_host(val)


@pytest.mark.parametrize("n,k", [(248320, 64), (248320, 1), (1000, 40), (64, 64), (65, 7), (1, 1), (4097, 64)])
def test_topk_random(m27q, ora, dev, n, k):
    v = np.random.default_rng(n + k).standard_normal(n).astype(np.float32)
    say("topk", n, k)
    idx, val = run_topk(m27q, dev, v, k)
    oi, ov = ora.topk(v, k)
    assert np.array_equal(idx, oi)
    assert np.array_equal(val.view(np.uint32), ov.view(np.uint32))


def test_topk_ties_zeros_nan_inf(m27q, ora, dev):
    rng = np.random.default_rng(5)
    v = np.round(rng.standard_normal(50000)).astype(np.float32)  # heavy ties
    v[rng.integers(0, v.size, 300)] = -0.0
    v[rng.integers(0, v.size, 50)] = np.nan
    v[[7, 49999]] = np.inf
    v[[8, 9]] = -np.inf
    for k in (1, 64):
        say("topk ties", k)
        idx, val = run_topk(m27q, dev, v, k)
        oi, ov = ora.topk(v, k)
        assert np.array_equal(idx, oi)
        assert np.array_equal(val.view(np.uint32), ov.view(np.uint32))
    # all equal: the first k indices, in order, each value with its own sign
    z = np.zeros(3000, np.float32)
    z[::2] = -0.0
    idx, val = run_topk(m27q, dev, z, 64)
    assert list(idx) == list(range(64))
    assert np.array_equal(val.view(np.uint32), z[:64].view(np.uint32))
    # NaN only beats padding: with n = k everything is returned, NaN last, each
    # NaN with its own payload
    w = np.array([np.nan, 1.0, -np.inf, np.nan], np.float32)
    w.view(np.uint32)[3] = 0xFFC00123
    idx, val = run_topk(m27q, dev, w, 4)
    assert list(idx) == [1, 2, 0, 3]
    assert np.array_equal(val.view(np.uint32), w[[1, 2, 0, 3]].view(np.uint32))


@pytest.mark.parametrize("case,k", [("equal", 8), ("equal", 64), ("descending", 64), ("ascending", 33)])
def test_topk_candidate_paths(m27q, ora, dev, case, k):
    """The filter's and the select's paths at the vocab size.  The bound is the
    k-th largest chunk maximum (chunks of 1024): with all values equal, k = 8
    leaves 7 full chunks above it, each reduced to its own top 8 (57 candidates,
    ranked directly), and k = 64 leaves 63, reduced to 63 x 64 + 1 = 4033
    candidates (radix select over the list); sorted inputs put all the
    candidates in a few chunks."""
    n = 248320
    if case == "equal":
        v = np.full(n, 0.5, np.float32)
    else:
        v = np.linspace(-3.0, 3.0, n, dtype=np.float32)
        if case == "descending":
            v = v[::-1].copy()
    say("topk path", case, k)
    idx, val = run_topk(m27q, dev, v, k)
    oi, ov = ora.topk(v, k)
    assert np.array_equal(idx, oi)
    assert np.array_equal(val.view(np.uint32), ov.view(np.uint32))


def test_vocab_scoring_full_size(m27q, ora, dev):
    """Config 5 scoring: Q6_K 248320 x 5120 LM head GEMV of a N(0,1) hidden state,
    exact top-64 on the GPU logits vs the oracle on the same logits, and a row
    sample of the logits vs the integer-dot oracle."""
    import torch
    rb, rc, k = 20, 248320, 5120
    g = torch.Generator(device=dev)
    g.manual_seed(20)
    raw = torch.randint(0, 256, (rc * rb, 210), dtype=torch.uint8, device=dev, generator=g)
    raw[:, 208] = 0x1f
    raw[:, 209] = 0x0a
    w = m27q.Weight(raw.reshape(-1), m27q.Q6_K, rb, rc, m27q.GGUF)
    h = np.random.default_rng(22).standard_normal(k).astype(np.float32)
    act = m27q.Act(1, k, dev)
    m27q.quant_act(to_dev(h, dev), act)
    logits = torch.empty(rc, dtype=torch.float32, device=dev)
    say("vocab gemv")
    m27q.matvec_q8(w, act, logits)
    lg = to_host(logits)
    say("vocab topk")
    idx, val = run_topk(m27q, dev, lg, 64)
    oi, ov = ora.topk(lg, 64)
    assert np.array_equal(idx, oi) and np.array_equal(val.view(np.uint32), ov.view(np.uint32))
    rows = np.random.default_rng(1).integers(0, rc, 256)
    host = raw.view(rc, rb * 210)[torch.from_numpy(rows).long().to(dev)].cpu().numpy()
    codes, d, s = act.parts()
    want, nrm = ora.gemv_act(m27q.Q6_K, host, rb, rows.size, to_host(codes)[0], to_host(d)[0],
                             to_host(s)[0].view(np.uint32))
    assert (np.abs(lg[rows] - want) <= 1e-5 * nrm + 1e-30).all()


@pytest.mark.parametrize("T,min_p,top_p", [(0.8, 0.05, 0.95), (1.0, 0.0, 1.0), (0.3, 0.1, 0.6), (0.0, 0.05, 0.95)])
def test_sample_matches_oracle(m27q, ora, dev, T, min_p, top_p):
    """m27q_sample on m27q_topk's candidates (k = 40, the reference's default
    top_k) against the oracle's restatement of sample(), over a grid of u and
    at u just below and above each pick boundary: both sides use the same exp
    and the same float sums in candidate order, so every pick agrees."""
    import torch
    lg = (np.random.default_rng(4).standard_normal(248320) * 3).astype(np.float32)
    k = 40
    idx, val = run_topk(m27q, dev, lg, k)
    di, dv = to_dev(idx, dev), to_dev(val, dev)
    tok = torch.empty(1, dtype=torch.int32, device=dev)
    us = list(np.linspace(0.0, 0.999, 200, dtype=np.float32))
    grid = np.linspace(0.0, 0.999, 2000, dtype=np.float32)
    picks = [ora.sample(idx, val, T, min_p, top_p, float(u)) for u in grid]
    for i in range(1, grid.size):  # the grid points on both sides of every change of pick
        if picks[i] != picks[i - 1]:
            us += [grid[i - 1], grid[i]]
    say("sample", T, min_p, top_p, len(us))
    for u in us:
        want = ora.sample(idx, val, T, min_p, top_p, float(u))
        m27q.sample(di, dv, k, T, min_p, top_p, to_dev(np.array([u], np.float32), dev), tok)
        assert int(to_host(tok)[0]) == want, float(u)
