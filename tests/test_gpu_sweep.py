"""Seeded random shapes through every product entry point, against the
integer-dot oracle: random type, layout, row count (ragged tiles), K (whole
blocks, ragged Q8_0 units), token count M up to the entry points' 64 (the few-token GEMV, both MFMA
packings, 16-token launches and their remainders), fp32 or quantized
activations, residual, multi-weight launches of mixed types and the SwiGLU
epilogue.  Those draw at most 3000 rows, too few for the resident-activation
kernel (16-token launches over >= 4 row sets of 16 per CU: 16369 rows on 256
CUs); a third set of seeds draws 16400-20000 rows and 16-40 tokens for it,
every token row checked.  The fixed cases elsewhere pin the
benched shapes and the edges the kernels were written for; these cover the
combinations between them (any layout, except multi-weight launches of
several tokens, which take TILED weights).  A second set of seeds draws the
weights as random bytes in every field (6-bit scales and mins at their
extremes, Q6_K's int8 scales down to -128, IQ4_XS's split scale bits, zero,
subnormal and negative fp16 scales) instead of the quantizer's output."""
import numpy as np
import pytest

from gpu_util import act_host, int_dot_tol, say, to_dev, to_host
from test_oracle import random_blocks

pytestmark = pytest.mark.gpu

TYPES = ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "IQ4_XS"]
MS = [1, 1, 1, 2, 2, 3, 4, 7, 8, 9, 16, 17, 24, 33, 47, 64]


def draw(seed):
    r = np.random.default_rng(1000 + seed)
    t = TYPES[r.integers(len(TYPES))]
    k = int(32 * r.integers(1, 97)) if t == "Q8_0" else int(256 * r.integers(1, 25))
    rc = int(r.integers(1, 3001))
    return dict(type=t, k=k, rc=rc, M=int(MS[r.integers(len(MS))]), layout=int(r.integers(2)),
                fp32x=bool(r.integers(2)), res=bool(r.integers(2)), kind=int(r.integers(4)), r=r)


def weight(m27q, ora, dev, t, rc, k, layout, seed, raw=False):
    """Quantizer-made blocks, or (raw) random bytes with finite fp16 scales."""
    tid = getattr(m27q, t)
    rb = k // m27q.BLOCK_ELEMS[tid]
    if raw:
        wb = random_blocks(ora, tid, rb * rc, np.random.default_rng(7000 + seed))
    else:
        wb = ora.synth_weights(tid, rc, k, seed=seed)
    return tid, wb, rb, m27q.Weight.upload(wb.reshape(-1), tid, rb, rc, layout, dev)


@pytest.mark.parametrize("seed", range(256))
def test_random_product_vs_oracle(m27q, ora, dev, seed):
    run_case(m27q, ora, dev, seed, raw=False)


@pytest.mark.parametrize("seed", range(5000, 5096))
def test_random_bytes_vs_oracle(m27q, ora, dev, seed):
    run_case(m27q, ora, dev, seed, raw=True)


@pytest.mark.parametrize("seed", range(9000, 9006))
def test_random_resident_vs_oracle(m27q, ora, dev, seed):
    """Random type and layout, 16400-20000 rows (ragged last set), small K,
    16-40 tokens (resident 16-token launches, then the remainder on the
    per-unit kernel; GGUF-layout Q8_0 / IQ4_XS on the VALU kernel), one or
    two weights of one K; every token row against the oracle."""
    import torch
    r = np.random.default_rng(3000 + seed)
    t = TYPES[r.integers(len(TYPES))]
    k = int(128 * r.integers(2, 9)) if t == "Q8_0" else int(256 * r.integers(1, 5))
    M = int(r.integers(16, 41))
    n = int(r.integers(1, 3))
    layout = m27q.GGUF if r.integers(2) else m27q.TILED
    mats = []
    for i in range(n):
        rc = int(r.integers(16400, 20001))
        tid, wb, rb, w = weight(m27q, ora, dev, t, rc, k, layout, seed + 100 * i)
        mats.append((tid, wb, rb, w, rc))
    X = r.standard_normal((M, k)).astype(np.float32)
    act = m27q.Act(M, k, dev)
    m27q.quant_act(to_dev(X, dev), act)
    q, d, s = act_host(m27q, act)
    Ys = [torch.empty((M, m[4]), dtype=torch.float32, device=dev) for m in mats]
    say("sweep resident", seed, t, [m[4] for m in mats], k, M, layout)
    if n == 1:
        m27q.matmul_q8(mats[0][3], act, Ys[0])
    else:
        m27q.matmul_q8_multi([m[3] for m in mats], act, Ys)
    for (tid, wb, rb, _, rc), Y in zip(mats, Ys):
        got = to_host(Y).astype(np.float64)
        for m in range(M):
            want, nrm = ora.gemv_act(tid, wb, rb, rc, q[m], d[m], s[m])
            assert (np.abs(got[m] - want) <= int_dot_tol(nrm)).all(), (seed, rc, m)


def run_case(m27q, ora, dev, seed, raw):
    import torch
    c = draw(seed)
    t, k, rc, M, layout, r = c["type"], c["k"], c["rc"], c["M"], c["layout"], c["r"]
    tid, wb, rb, w = weight(m27q, ora, dev, t, rc, k, layout, seed, raw)
    X = r.standard_normal((M, k)).astype(np.float32)
    act = m27q.Act(M, k, dev)
    xd = to_dev(X, dev)
    m27q.quant_act(xd, act)
    q, d, s = act_host(m27q, act)
    rows = sorted({0, M // 2, M - 1})

    if c["kind"] == 3 and M == 1:
        # SwiGLU: a second weight of the same type, shape and layout
        _, ub, _, uw = weight(m27q, ora, dev, t, rc, k, layout, seed + 500, raw)
        y = torch.empty(rc, dtype=torch.float32, device=dev)
        say("sweep swiglu", "raw" if raw else "", seed, t, rc, k, layout, "fp32 x" if c["fp32x"] else "q8 x")
        if c["fp32x"]:
            m27q.ffn_swiglu(w, uw, xd.view(-1), y)
        else:
            m27q.ffn_swiglu_q8(w, uw, act, y)
        check_swiglu_rb(ora, tid, wb, ub, rb, rc, q[0], d[0], s[0], to_host(y))
        return

    if c["kind"] == 2:
        # two or three weights of one K, types drawn independently, one call
        n = int(r.integers(2, 4))
        mats = [(tid, wb, rb, w, rc)]
        for i in range(1, n):
            ti = TYPES[r.integers(len(TYPES))]
            if (ti == "Q8_0") != (t == "Q8_0") and k % 256:
                ti = t  # K must be whole blocks of every type
            rci = int(r.integers(1, 3001))
            tj, wbj, rbj, wj = weight(m27q, ora, dev, ti, rci, k, layout, seed + 100 * i, raw)
            mats.append((tj, wbj, rbj, wj, rci))
        Ys = [torch.empty((M, m[4]), dtype=torch.float32, device=dev) for m in mats]
        say("sweep multi", "raw" if raw else "", seed, [(m[0], m[4]) for m in mats], k, M, layout)
        if M == 1 and c["fp32x"]:
            m27q.matvec_multi([m[3] for m in mats], xd.view(-1), [Y.view(-1) for Y in Ys])
        elif M == 1:
            m27q.matvec_q8_multi([m[3] for m in mats], act, [Y.view(-1) for Y in Ys])
        else:
            m27q.matmul_q8_multi([m[3] for m in mats], act, Ys)
        for (tj, wbj, rbj, _, rci), Y in zip(mats, Ys):
            got = to_host(Y).astype(np.float64).reshape(M, rci)
            for m in rows:
                want, nrm = ora.gemv_act(tj, wbj, rbj, rci, q[m], d[m], s[m])
                assert (np.abs(got[m] - want) <= int_dot_tol(nrm)).all(), (seed, tj, rci, m)
        return

    res = r.standard_normal((M, rc)).astype(np.float32) if c["res"] else None
    resd = to_dev(res, dev) if res is not None else None
    Y = torch.empty((M, rc), dtype=torch.float32, device=dev)
    say("sweep", "raw" if raw else "", seed, t, rc, k, M, layout, "fp32 x" if c["fp32x"] else "q8 x", "res" if c["res"] else "")
    if M == 1 and c["fp32x"]:
        m27q.matvec(w, xd.view(-1), Y.view(-1), residual=None if resd is None else resd.view(-1))
    elif M == 1:
        m27q.matvec_q8(w, act, Y.view(-1), residual=None if resd is None else resd.view(-1))
    else:
        m27q.matmul_q8(w, act, Y, residual=resd)
    got = to_host(Y).astype(np.float64)
    base = res.astype(np.float64) if res is not None else np.zeros((M, rc))
    for m in rows:
        want, nrm = ora.gemv_act(tid, wb, rb, rc, q[m], d[m], s[m])
        tol = int_dot_tol(nrm) + 1e-6 * np.abs(base[m])
        assert (np.abs(got[m] - base[m] - want) <= tol).all(), (seed, m)


def check_swiglu_rb(ora, tid, gb, ub, rb, rc, q, d, s, y):
    """check_swiglu for any K: the same bound with this product's blocks per row."""
    g, ng = ora.gemv_act(tid, gb, rb, rc, q, d, s)
    u, nu = ora.gemv_act(tid, ub, rb, rc, q, d, s)
    with np.errstate(over="ignore"):  # e^-g overflows below g = -709: silu(g) is then -0
        sg = g / (1 + np.exp(-g))
    want = sg * u
    tol = 1.1 * np.abs(u) * int_dot_tol(ng) + np.abs(sg) * int_dot_tol(nu) + 4e-7 * np.abs(want) + 1e-30
    err = np.abs(y.astype(np.float64) - want)
    assert (err <= tol).all(), (np.flatnonzero(err > tol)[:5], err.max())
