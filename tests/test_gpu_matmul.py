"""Small-M products (speculative-verify / prefill rows) vs M independent rows."""
import numpy as np
import pytest

from gpu_util import act_host, int_dot_tol, say, to_dev, to_host

pytestmark = pytest.mark.gpu

_cache = {}

CASES = [  # type, rows, K, M, layout
    ("Q4_K", 6144, 5120, 1, 1), ("Q4_K", 6144, 5120, 2, 1), ("Q4_K", 6144, 5120, 4, 1),
    ("Q4_K", 6144, 5120, 8, 1), ("Q4_K", 6144, 5120, 16, 1), ("Q4_K", 6144, 5120, 23, 0),
    ("Q4_K", 40, 512, 5, 0), ("Q4_K", 40, 512, 64, 1),
    ("Q6_K", 5120, 17408, 16, 1), ("Q6_K", 5120, 17408, 3, 0), ("Q6_K", 24, 768, 9, 1),
    ("Q8_0", 2048, 6144, 16, 1), ("Q8_0", 2048, 6144, 2, 0), ("Q8_0", 13, 160, 7, 1),
    # few tokens: M = 2 on the GEMV-structured kernel (TILED Q4_K / Q5_K: on
    # MFMA with direct weight operands), M = 3 and 4 on MFMA (padding tokens,
    # partial 8-row tiles), each type
    ("Q6_K", 5120, 17408, 2, 1), ("Q6_K", 24, 768, 4, 1), ("Q4_K", 40, 512, 3, 1), ("Q8_0", 13, 160, 3, 1),
    ("Q8_0", 2048, 6144, 4, 1),
    # Q5_K on each path: few-token GEMV, MFMA, GGUF VALU
    ("Q5_K", 6144, 5120, 2, 1), ("Q5_K", 6144, 5120, 16, 1), ("Q5_K", 40, 512, 9, 1), ("Q5_K", 40, 512, 3, 0),
    # IQ4_XS likewise
    ("IQ4_XS", 6144, 5120, 2, 1), ("IQ4_XS", 6144, 5120, 16, 1), ("IQ4_XS", 40, 512, 9, 1),
    ("IQ4_XS", 40, 512, 3, 0),
    # MFMA with two 16-row sets per tile (M <= 8 and >= 128 sets of 32 rows):
    # a partial last set (8200 rows), a partial Q8_0 unit (K = 160), every
    # type, and 24 tokens (one 16-token launch, then one packed 8-token launch)
    ("Q4_K", 8200, 512, 5, 1), ("Q4_K", 8192, 512, 8, 1), ("Q4_K", 8192, 512, 24, 1),
    ("Q6_K", 8200, 768, 7, 1), ("Q8_0", 8200, 160, 6, 1), ("Q5_K", 8192, 512, 8, 1),
    ("IQ4_XS", 8200, 512, 6, 1),
    # gate-sized rows at M = 3 (two sets per tile), the down shape at M = 12
    # (padding tokens in a 16-token launch), 17 tokens (16, then 1 on two sets)
    ("Q4_K", 17408, 5120, 3, 1), ("Q6_K", 5120, 17408, 12, 1), ("Q4_K", 8192, 512, 17, 1),
    # few tokens with balanced tiling on 256 CUs (rows under 40 units) on the
    # GEMV-structured kernel (Q6_K), and the same shapes on MFMA with direct
    # operands (Q4_K): o, a ragged last tile
    ("Q4_K", 5120, 6144, 2, 1), ("Q6_K", 4100, 2048, 2, 1), ("Q4_K", 6141, 2048, 2, 1),
    # direct weight operands at M = 2: a single partial tile, a partial last
    # two-set tile, and gate-sized rows (544 workgroups: K over 4 waves)
    ("Q4_K", 13, 256, 2, 1), ("Q5_K", 8200, 512, 2, 1), ("Q4_K", 17408, 1024, 2, 1),
    # resident activation rows (16-token launches with >= 4 row sets per CU:
    # 1025 sets of 16 rows on 256 CUs), every type, a partial last set, a
    # partial Q8_0 unit (K = 1056), and 16 + 9 tokens (the resident launch,
    # then the per-unit staging one)
    ("Q4_K", 16390, 1024, 16, 1), ("Q6_K", 16390, 1024, 16, 1), ("Q8_0", 16390, 1056, 16, 1),
    ("Q5_K", 16390, 1024, 25, 1), ("IQ4_XS", 16390, 1024, 32, 1),
    # two row sets per tile over 1025 sets of 32 rows (a last set of 8 rows),
    # every type, padding tokens
    ("Q4_K", 32776, 512, 8, 1), ("Q6_K", 32776, 768, 5, 1), ("Q8_0", 32776, 160, 7, 1),
    ("Q5_K", 32776, 512, 3, 1), ("IQ4_XS", 32776, 512, 8, 1),
    # GGUF-layout K-quants on the MFMA kernel, staged from the row blocks:
    # from M = 2, two-set tiles with a partial last set, 16-token resident
    # launches (Q6_K: the per-unit kernel) and padding tokens; Q6_K rows of an
    # odd block count (K = 768, 2304: every other row starts 2 bytes past a
    # multiple of 4) and the down shape
    ("Q4_K", 6144, 5120, 2, 0), ("Q4_K", 8200, 512, 6, 0), ("Q4_K", 16390, 1024, 16, 0), ("Q4_K", 4100, 1024, 19, 0),
    ("Q5_K", 6144, 5120, 2, 0), ("Q5_K", 8200, 512, 8, 0), ("Q5_K", 16390, 1024, 25, 0),
    ("Q6_K", 24, 768, 2, 0), ("Q6_K", 8200, 768, 7, 0), ("Q6_K", 16390, 1024, 16, 0), ("Q6_K", 1030, 2304, 11, 0),
    ("Q6_K", 5120, 17408, 16, 0), ("Q6_K", 33, 2304, 4, 0),
    # GGUF-layout weights at M = 2 on the few-token kernel: o's shape (balanced
    # over one workgroup per CU), IQ4_XS and Q8_0 (its 34-byte blocks)
    ("Q4_K", 5120, 6144, 2, 0), ("IQ4_XS", 40, 512, 2, 0), ("Q8_0", 13, 160, 2, 0),
]


@pytest.mark.parametrize("type_name,rc,k,M,layout", CASES)
def test_matmul_vs_oracle(m27q, ora, dev, type_name, rc, k, M, layout):
    import torch
    t = getattr(m27q, type_name)
    rb = k // m27q.BLOCK_ELEMS[t]
    key = (type_name, rc, k)
    if key not in _cache:
        _cache[key] = ora.synth_weights(t, rc, k, seed=40)
    wb = _cache[key]
    w = m27q.Weight.upload(wb.reshape(-1), t, rb, rc, layout, dev)
    X = np.random.default_rng(M).standard_normal((M, k)).astype(np.float32)
    act = m27q.Act(M, k, dev)
    m27q.quant_act(to_dev(X, dev), act)
    res = np.random.default_rng(M + 1).standard_normal((M, rc)).astype(np.float32)
    Y = torch.empty((M, rc), dtype=torch.float32, device=dev)
    say("matmul", type_name, rc, k, M, layout)
    m27q.matmul_q8(w, act, Y, residual=to_dev(res, dev))
    got = to_host(Y).astype(np.float64) - res
    q, d, s = act_host(m27q, act)
    for m in range(M):
        want, nrm = ora.gemv_act(t, wb, rb, rc, q[m], d[m], s[m])
        assert (np.abs(got[m] - want) <= int_dot_tol(nrm) + 1e-6 * np.abs(res[m])).all(), m


@pytest.mark.parametrize("M", [2, 5, 16, 19])
def test_matmul_multi_vs_oracle(m27q, ora, dev, M):
    """q/k/v-shaped weights on one activation in one launch, each against the
    integer-dot oracle (row subsets), across the 16-token launch boundary."""
    import torch
    k, shapes = 5120, [6144, 1024, 1024]
    wbs = [ora.synth_weights(m27q.Q4_K, rc, k, seed=60 + i) for i, rc in enumerate(shapes)]
    ws = [m27q.Weight.upload(wb.reshape(-1), m27q.Q4_K, 20, rc, m27q.TILED, dev) for wb, rc in zip(wbs, shapes)]
    X = np.random.default_rng(M + 7).standard_normal((M, k)).astype(np.float32)
    act = m27q.Act(M, k, dev)
    m27q.quant_act(to_dev(X, dev), act)
    Ys = [torch.empty((M, rc), dtype=torch.float32, device=dev) for rc in shapes]
    say("matmul multi", M)
    m27q.matmul_q8_multi(ws, act, Ys)
    q, d, s = act_host(m27q, act)
    for wb, rc, Y in zip(wbs, shapes, Ys):
        got = to_host(Y).astype(np.float64)
        for m in sorted({0, M // 2, M - 1}):
            want, nrm = ora.gemv_act(m27q.Q4_K, wb, 20, rc, q[m], d[m], s[m])
            assert (np.abs(got[m] - want) <= int_dot_tol(nrm)).all(), (rc, m)


@pytest.mark.parametrize("M,rows", [(16, 8200), (32, 8200), (7, 16400)])
def test_matmul_multi_resident_vs_oracle(m27q, ora, dev, M, rows):
    """Two weights of one K in one launch over 1026 row sets: at M = 16 and 32
    the resident-activation kernel (the second matrix's sets following the
    first's in the workgroups' runs), at M = 7 the two-set per-unit kernel;
    each against the integer-dot oracle."""
    import torch
    k, shapes = 1024, [rows, rows]
    wbs = [ora.synth_weights(m27q.Q4_K, rc, k, seed=70 + i) for i, rc in enumerate(shapes)]
    ws = [m27q.Weight.upload(wb.reshape(-1), m27q.Q4_K, 4, rc, m27q.TILED, dev) for wb, rc in zip(wbs, shapes)]
    X = np.random.default_rng(M + 9).standard_normal((M, k)).astype(np.float32)
    act = m27q.Act(M, k, dev)
    m27q.quant_act(to_dev(X, dev), act)
    Ys = [torch.empty((M, rc), dtype=torch.float32, device=dev) for rc in shapes]
    say("matmul multi resident", M)
    m27q.matmul_q8_multi(ws, act, Ys)
    q, d, s = act_host(m27q, act)
    for wb, rc, Y in zip(wbs, shapes, Ys):
        got = to_host(Y).astype(np.float64)
        for m in range(M):
            want, nrm = ora.gemv_act(m27q.Q4_K, wb, 4, rc, q[m], d[m], s[m])
            assert (np.abs(got[m] - want) <= int_dot_tol(nrm)).all(), (rc, m)


@pytest.mark.parametrize("M", [2, 9, 16])
def test_matmul_multi_gguf_vs_oracle(m27q, ora, dev, M):
    """GGUF-layout weights through the multi entry point: Q4_K q/k/v-shaped
    weights in one MFMA launch, then a mixed group (Q6_K on the MFMA kernel,
    Q8_0 on the per-weight VALU kernel) on the same activation; every token
    row of each output against the integer-dot oracle."""
    import torch
    k = 1536
    spec = [("Q4_K", 6144, 80), ("Q4_K", 1024, 81), ("Q4_K", 1024, 82)]
    mixed = [("Q6_K", 1030, 83), ("Q8_0", 515, 84)]
    X = np.random.default_rng(M + 11).standard_normal((M, k)).astype(np.float32)
    act = m27q.Act(M, k, dev)
    m27q.quant_act(to_dev(X, dev), act)
    q, d, s = act_host(m27q, act)
    for group in (spec, mixed):
        wbs, ws, rbs = [], [], []
        for name, rc, seed in group:
            t = getattr(m27q, name)
            rb = k // m27q.BLOCK_ELEMS[t]
            wb = ora.synth_weights(t, rc, k, seed=seed)
            wbs.append(wb)
            rbs.append(rb)
            ws.append(m27q.Weight.upload(wb.reshape(-1), t, rb, rc, m27q.GGUF, dev))
        Ys = [torch.empty((M, rc), dtype=torch.float32, device=dev) for _, rc, _ in group]
        say("matmul multi gguf", M, [g[0] for g in group])
        m27q.matmul_q8_multi(ws, act, Ys)
        for (name, rc, _), wb, rb, Y in zip(group, wbs, rbs, Ys):
            got = to_host(Y).astype(np.float64)
            for m in range(M):
                want, nrm = ora.gemv_act(getattr(m27q, name), wb, rb, rc, q[m], d[m], s[m])
                assert (np.abs(got[m] - want) <= int_dot_tol(nrm)).all(), (name, rc, m)


@pytest.mark.parametrize("type_name,rc,k", [("Q6_K", 1030, 2304), ("Q6_K", 8200, 768), ("Q6_K", 4098, 6144),
                                            ("Q8_0", 515, 1056)])
def test_gguf_two_byte_aligned_base(m27q, ora, dev, type_name, rc, k):
    """GGUF Q6_K and Q8_0 weights need only 2-byte alignment: the matrix placed
    2 bytes past a multiple of 4 (a view into a larger buffer).  The M = 1
    products (quantized and fp32 x; one- and two-tile waves read Q6_K's fields
    as shifted dwords or halfwords) and the small-M products (Q6_K: the MFMA
    kernel with one- and two-set tiles, whose staging reads dwords from the
    4-aligned address below each chunk; Q8_0: the VALU kernel), every token
    row against the integer-dot oracle."""
    import torch
    t = getattr(m27q, type_name)
    rb = k // m27q.BLOCK_ELEMS[t]
    wb = ora.synth_weights(t, rc, k, seed=90)
    raw = torch.from_numpy(wb.reshape(-1).copy()).to(dev)
    buf = torch.zeros(raw.numel() + 2, dtype=torch.uint8, device=dev)
    buf[2:] = raw
    w = m27q.Weight(buf[2:], t, rb, rc, m27q.GGUF)
    assert w.data.data_ptr() % 4 == 2
    rng = np.random.default_rng(91)
    for M in (1, 2, 7, 16):
        X = rng.standard_normal((M, k)).astype(np.float32)
        act = m27q.Act(M, k, dev)
        m27q.quant_act(to_dev(X, dev), act)
        q, d, s = act_host(m27q, act)
        Y = torch.empty((M, rc), dtype=torch.float32, device=dev)
        say("gguf 2-byte base", type_name, rc, k, M)
        m27q.matmul_q8(w, act, Y)
        got = to_host(Y).astype(np.float64)
        for m in range(M):
            want, nrm = ora.gemv_act(t, wb, rb, rc, q[m], d[m], s[m])
            assert (np.abs(got[m] - want) <= int_dot_tol(nrm)).all(), (M, m)
        if M == 1:
            y = torch.empty(rc, dtype=torch.float32, device=dev)
            m27q.matvec(w, to_dev(X[0], dev), y)
            qf, df, sf = ora.quant_act(X[0])
            want, nrm = ora.gemv_act(t, wb, rb, rc, qf, df, sf)
            assert (np.abs(to_host(y).astype(np.float64) - want) <= int_dot_tol(nrm)).all(), "fp32 x"
