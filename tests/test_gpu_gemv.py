"""M = 1 products on the GPU vs the oracle.

int8-activation path: against the oracle's integer-dot formula evaluated in
fp64 (tolerance 1e-5 x the sum of |per-group terms|: fp32 reassociation only),
and against the fp64 dequant-then-dot oracle, no worse than the ggml q8_K CPU
path on the same inputs.  fp32-activation path: within 1e-3 relative of the
fp64 dequant-then-dot oracle (it lands near 1e-6 of sum |w x|).
"""
import numpy as np
import pytest

from gpu_util import act_host, int_dot_tol, say, to_dev, to_host

pytestmark = pytest.mark.gpu

SHAPES = {  # (type, rows, K)
    "q4k_small": ("Q4_K", 40, 512),
    "q4k_ffn": ("Q4_K", 17408, 5120),
    "q4k_o": ("Q4_K", 5120, 6144),
    "q5k_gate": ("Q5_K", 6144, 5120),
    "q5k_small": ("Q5_K", 24, 768),
    "iq4_gate": ("IQ4_XS", 6144, 5120),
    "iq4_small": ("IQ4_XS", 24, 768),
    "q6k_down": ("Q6_K", 5120, 17408),
    "q6k_small": ("Q6_K", 24, 768),
    "q80_2048": ("Q8_0", 2048, 2048),
    "q80_down": ("Q8_0", 2048, 6144),
    "q80_ragged": ("Q8_0", 13, 160),
}

_cache = {}


def weights(ora, type_name, rc, k, seed):
    key = (type_name, rc, k, seed)
    if key not in _cache:
        t = getattr(ora, type_name)
        _cache[key] = ora.synth_weights(t, rc, k, seed)
    return _cache[key]


def quantized_x(m27q, dev, k, seed):
    x = np.random.default_rng(seed).standard_normal(k).astype(np.float32)
    act = m27q.Act(1, k, dev)
    m27q.quant_act(to_dev(x, dev), act)
    return x, act


@pytest.mark.parametrize("shape", list(SHAPES))
@pytest.mark.parametrize("layout", [0, 1])
def test_matvec_q8_vs_int_oracle(m27q, ora, dev, shape, layout):
    import torch
    type_name, rc, k = SHAPES[shape]
    t = getattr(m27q, type_name)
    rb = k // m27q.BLOCK_ELEMS[t]
    wb = weights(ora, type_name, rc, k, 10)
    w = m27q.Weight.upload(wb.reshape(-1), t, rb, rc, layout, dev)
    x, act = quantized_x(m27q, dev, k, 1)
    q, d, s = act_host(m27q, act)
    y = torch.empty(rc, dtype=torch.float32, device=dev)
    say("matvec_q8", shape, "layout", layout)
    m27q.matvec_q8(w, act, y)
    got = to_host(y).astype(np.float64)
    want, nrm = ora.gemv_act(t, wb, rb, rc, q[0], d[0], s[0])
    bad = np.abs(got - want) > int_dot_tol(nrm)
    assert not bad.any(), (np.flatnonzero(bad)[:5], got[bad][:5], want[bad][:5])


@pytest.mark.parametrize("type_name,rc,k", [("Q4_K", 17408, 5120), ("Q6_K", 5120, 17408), ("Q8_0", 6144, 2048)])
def test_q8_path_no_worse_than_q8K_cpu_path(m27q, ora, dev, type_name, rc, k):
    import torch
    t = getattr(m27q, type_name)
    rb = k // m27q.BLOCK_ELEMS[t]
    wb = weights(ora, type_name, rc, k, 10)
    w = m27q.Weight.upload(wb.reshape(-1), t, rb, rc, m27q.TILED, dev)
    x, act = quantized_x(m27q, dev, k, 1)
    y = torch.empty(rc, dtype=torch.float32, device=dev)
    say("no-worse-than-q8K", type_name)
    m27q.matvec_q8(w, act, y)
    got = to_host(y).astype(np.float64)
    exact = ora.gemv_f64(t, wb, rb, rc, x)
    cpu = ora.gemv_cpu(t, wb, rb, rc, ora.quant_cpu_act(t, x), nthreads=8).astype(np.float64)
    e_gpu = np.sqrt(np.mean((got - exact) ** 2))
    e_cpu = np.sqrt(np.mean((cpu - exact) ** 2))
    print(f"rms err gpu(per-32 int8)={e_gpu:.3e} cpu(q8_K/q8_0)={e_cpu:.3e} ratio={e_gpu / e_cpu:.3f}")
    # the accuracy bar: no worse than the reference's own q8_K-activation path
    assert e_gpu <= e_cpu, f"rms error ratio gpu/cpu = {e_gpu / e_cpu:.4f}"


@pytest.mark.parametrize("layout", [0, 1])
def test_layouts_agree_and_residual(m27q, ora, dev, layout):
    import torch
    rc, k = 6144, 5120
    wb = weights(ora, "Q4_K", rc, k, 12)
    w = m27q.Weight.upload(wb.reshape(-1), m27q.Q4_K, 20, rc, layout, dev)
    x, act = quantized_x(m27q, dev, k, 2)
    res = torch.from_numpy(np.random.default_rng(3).standard_normal(rc).astype(np.float32)).to(dev)
    y0 = torch.empty(rc, dtype=torch.float32, device=dev)
    y1 = torch.empty(rc, dtype=torch.float32, device=dev)
    say("residual", layout)
    m27q.matvec_q8(w, act, y0)
    m27q.matvec_q8(w, act, y1, residual=res)
    a, b, r = to_host(y0), to_host(y1), to_host(res)
    assert np.array_equal((a + r).view(np.uint32), b.view(np.uint32))


def test_fused_output_quant_matches_standalone(m27q, ora, dev):
    import torch
    rc, k = 5120, 6144
    wb = weights(ora, "Q4_K", rc, k, 13)
    w = m27q.Weight.upload(wb.reshape(-1), m27q.Q4_K, 24, rc, m27q.TILED, dev)
    x, act = quantized_x(m27q, dev, k, 4)
    y = torch.empty(rc, dtype=torch.float32, device=dev)
    yq = m27q.Act(1, rc, dev)
    say("fused output quant")
    m27q.matvec_q8(w, act, y, yq=yq)
    ref = m27q.Act(1, rc, dev)
    m27q.quant_act(y, ref)
    for a, b in zip(act_host(m27q, yq), act_host(m27q, ref)):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    qo, do, so = ora.quant_act(to_host(y))
    assert np.array_equal(act_host(m27q, yq)[0][0], qo)


@pytest.mark.parametrize("type_name,rc,k", [("Q4_K", 17408, 5120), ("Q4_K", 5120, 6144), ("Q8_0", 2048, 6144),
                                             ("Q6_K", 5120, 17408), ("Q4_K", 1024, 5120)])
@pytest.mark.parametrize("layout", [0, 1])
def test_fused_output_quant_shapes(m27q, ora, dev, type_name, rc, k, layout):
    """The fused output quantization at every workgroup shape the products pick
    for these sizes; two calls in a row on one buffer both match the standalone
    quantizer."""
    import torch
    t = getattr(m27q, type_name)
    rb = k // m27q.BLOCK_ELEMS[t]
    wb = weights(ora, type_name, rc, k, 14)
    w = m27q.Weight.upload(wb.reshape(-1), t, rb, rc, layout, dev)
    y = torch.empty(rc, dtype=torch.float32, device=dev)
    yq = m27q.Act(1, rc, dev)
    ref = m27q.Act(1, rc, dev)
    for call in range(2):
        x = to_dev(np.random.default_rng(50 + call).standard_normal(k).astype(np.float32), dev)
        say("fused output quant", type_name, rc, k, "call", call)
        m27q.matvec(w, x, y, yq=yq)
        m27q.quant_act(y, ref)
        for a, b in zip(act_host(m27q, yq), act_host(m27q, ref)):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), call


def test_multi_matches_single(m27q, ora, dev):
    import torch
    k = 5120
    shapes = [6144, 1024, 1024]
    ws, wbs = [], []
    for i, rc in enumerate(shapes):
        wb = weights(ora, "Q4_K", rc, k, 20 + i)
        wbs.append(wb)
        ws.append(m27q.Weight.upload(wb.reshape(-1), m27q.Q4_K, 20, rc, m27q.TILED, dev))
    x, act = quantized_x(m27q, dev, k, 5)
    ys = [torch.empty(rc, dtype=torch.float32, device=dev) for rc in shapes]
    say("multi q/k/v")
    m27q.matvec_q8_multi(ws, act, ys)
    q, d, s = act_host(m27q, act)
    for wb, rc, y in zip(wbs, shapes, ys):
        want, nrm = ora.gemv_act(m27q.Q4_K, wb, 20, rc, q[0], d[0], s[0])
        assert (np.abs(to_host(y) - want) <= int_dot_tol(nrm)).all()


@pytest.mark.parametrize("type_name", ["Q4_K", "Q5_K", "Q6_K", "IQ4_XS"])
def test_ffn_swiglu(m27q, ora, dev, type_name):
    import torch
    t = getattr(m27q, type_name)
    rc, k = 17408, 5120
    gb = weights(ora, type_name, rc, k, 30)
    ub = weights(ora, type_name, rc, k, 31)
    gw = m27q.Weight.upload(gb.reshape(-1), t, 20, rc, m27q.TILED, dev)
    uw = m27q.Weight.upload(ub.reshape(-1), t, 20, rc, m27q.TILED, dev)
    x, act = quantized_x(m27q, dev, k, 6)
    y = torch.empty(rc, dtype=torch.float32, device=dev)
    yq = m27q.Act(1, rc, dev)
    g = torch.empty(rc, dtype=torch.float32, device=dev)
    u = torch.empty(rc, dtype=torch.float32, device=dev)
    say("swiglu", type_name)
    m27q.ffn_swiglu_q8(gw, uw, act, y, yq=yq)
    q, d, s = act_host(m27q, act)
    check_swiglu(ora, t, gb, ub, rc, q[0], d[0], s[0], to_host(y))
    ref = m27q.Act(1, rc, dev)
    m27q.quant_act(y, ref)
    for a, b in zip(act_host(m27q, yq), act_host(m27q, ref)):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))


def check_swiglu(ora, t, gb, ub, rc, q, d, s, y):
    """y = silu(g) u against the fp64 integer-dot oracle: the fp32 error of g and
    u (int_dot_tol each) propagated through silu(g) u (|silu'| < 1.1), plus the
    rounding of the epilogue itself."""
    g, ng = ora.gemv_act(t, gb, 20, rc, q, d, s)
    u, nu = ora.gemv_act(t, ub, 20, rc, q, d, s)
    sg = g / (1 + np.exp(-g))
    want = sg * u
    tol = 1.1 * np.abs(u) * int_dot_tol(ng) + np.abs(sg) * int_dot_tol(nu) + 4e-7 * np.abs(want) + 1e-30
    err = np.abs(y.astype(np.float64) - want)
    assert (err <= tol).all(), (np.flatnonzero(err > tol)[:5], err.max())


@pytest.mark.parametrize("shape", ["q4k_ffn", "q6k_down", "q80_down", "q4k_small", "q80_ragged", "q5k_gate", "q5k_small",
                                   "iq4_gate", "iq4_small"])
@pytest.mark.parametrize("layout", [0, 1])
def test_matvec_f32_vs_fp64(m27q, ora, dev, shape, layout):
    import torch
    type_name, rc, k = SHAPES[shape]
    t = getattr(m27q, type_name)
    rb = k // m27q.BLOCK_ELEMS[t]
    wb = weights(ora, type_name, rc, k, 10)
    w = m27q.Weight.upload(wb.reshape(-1), t, rb, rc, layout, dev)
    x = np.random.default_rng(8).standard_normal(k).astype(np.float32)
    y = torch.empty(rc, dtype=torch.float32, device=dev)
    say("matvec_f32", shape, layout)
    m27q.matvec_f32(w, to_dev(x, dev), y)
    got = to_host(y).astype(np.float64)
    want = ora.gemv_f64(t, wb, rb, rc, x)
    scale = np.abs(ora.dequant(t, wb, rb, rc)).astype(np.float64) @ np.abs(x).astype(np.float64)
    assert (np.abs(got - want) <= 1e-5 * scale).all()
    rel = np.abs(got - want) / np.maximum(np.abs(want), 1e-3 * scale)
    assert rel.max() <= 1e-3


@pytest.mark.parametrize("type_name", ["F16", "F32"])
def test_matvec_dense(m27q, ora, dev, type_name):
    import torch
    t = getattr(m27q, type_name)
    rc, k = 48, 5120
    w32 = np.random.default_rng(2).standard_normal((rc, k)).astype(np.float32)
    raw = ora.quantize(t, w32)
    w = m27q.Weight.upload(raw.reshape(-1), t, k, rc, m27q.GGUF, dev)
    x = np.random.default_rng(9).standard_normal(k).astype(np.float32)
    y = torch.empty(rc, dtype=torch.float32, device=dev)
    say("matvec dense", type_name)
    m27q.matvec_f32(w, to_dev(x, dev), y)
    want = ora.gemv_f64(t, raw, k, rc, x)
    scale = np.abs(ora.dequant(t, raw, k, rc)).astype(np.float64) @ np.abs(x)
    assert (np.abs(to_host(y) - want) <= 1e-5 * scale).all()


@pytest.mark.parametrize("type_name,rc,k", [("Q6_K", 5120, 17408), ("Q4_K", 4096, 6144), ("Q4_K", 17408, 5120),
                                             ("Q8_0", 2048, 6144), ("Q5_K", 4096, 6144), ("IQ4_XS", 4096, 6144)])
def test_fp32_input_equals_two_step(m27q, ora, dev, type_name, rc, k):
    """In-kernel quantization of fp32 x gives the codes of m27q_quant_act, so at
    shapes where both input forms split K alike the product is bit-identical to
    quant_act followed by the quantized-input product.  (The down shape: both
    forms take balanced tiling and split K four ways; at 5120 x 6144 the two
    forms split it four and eight ways, so 4096 rows stand in there.)"""
    import torch
    t = getattr(m27q, type_name)
    rb = k // m27q.BLOCK_ELEMS[t]
    wb = weights(ora, type_name, rc, k, 10)
    w = m27q.Weight.upload(wb.reshape(-1), t, rb, rc, m27q.TILED, dev)
    from test_gpu_act import edge_rows
    res = to_dev(np.random.default_rng(2).standard_normal(rc).astype(np.float32), dev)
    # random x, then the quantizer's edge rows (ties, values beside 0.5,
    # subnormal scales) laid end to end
    for xi, x in enumerate((np.random.default_rng(1).standard_normal(k).astype(np.float32),
                            np.resize(edge_rows(256).reshape(-1), k).astype(np.float32))):
        xd = to_dev(x, dev)
        y0 = torch.empty(rc, dtype=torch.float32, device=dev)
        y1 = torch.empty(rc, dtype=torch.float32, device=dev)
        say("matvec fp32 input", type_name, xi)
        m27q.matvec(w, xd, y0, residual=res)
        act = m27q.Act(1, k, dev)
        m27q.quant_act(xd, act)
        m27q.matvec_q8(w, act, y1, residual=res)
        assert np.array_equal(to_host(y0).view(np.uint32), to_host(y1).view(np.uint32)), xi


@pytest.mark.parametrize("type_name,rc,k", [("Q4_K", 6144, 5120), ("Q8_0", 13, 160), ("Q4_K", 40, 512),
                                             ("Q5_K", 6144, 5120)])
def test_fp32_input_vs_oracle(m27q, ora, dev, type_name, rc, k):
    """Shapes where the fp32-input product launches its own workgroup shape:
    against the integer-dot oracle on the codes of the standalone quantizer."""
    import torch
    t = getattr(m27q, type_name)
    rb = k // m27q.BLOCK_ELEMS[t]
    wb = weights(ora, type_name, rc, k, 10)
    w = m27q.Weight.upload(wb.reshape(-1), t, rb, rc, m27q.TILED, dev)
    x = np.random.default_rng(3).standard_normal(k).astype(np.float32)
    y = torch.empty(rc, dtype=torch.float32, device=dev)
    say("matvec fp32 input vs oracle", type_name, rc, k)
    m27q.matvec(w, to_dev(x, dev), y)
    q, d, s = ora.quant_act(x)
    want, nrm = ora.gemv_act(t, wb, rb, rc, q, d, s)
    assert (np.abs(to_host(y) - want) <= int_dot_tol(nrm)).all()


@pytest.mark.parametrize("type_name,rc,k", [("Q6_K", 4100, 10240), ("Q4_K", 6141, 10240)])
@pytest.mark.parametrize("layout", [0, 1])
def test_balanced_tiling_edges(m27q, ora, dev, type_name, rc, k, layout):
    """Balanced tiling at the ends of its range on 256 CUs: 513 tiles (one
    workgroup with 3, the rest with 2, which reread their last tile) and 768
    (3 each), both with a ragged last tile.  The quantized-input product
    against the integer-dot oracle; the fp32-input product (balanced too from
    10240 columns) bit-identical to it; the rows past row_count untouched."""
    import torch
    t = getattr(m27q, type_name)
    rb = k // m27q.BLOCK_ELEMS[t]
    wb = weights(ora, type_name, rc, k, 12)
    w = m27q.Weight.upload(wb.reshape(-1), t, rb, rc, layout, dev)
    x = np.random.default_rng(13).standard_normal(k).astype(np.float32)
    xd = to_dev(x, dev)
    act = m27q.Act(1, k, dev)
    m27q.quant_act(xd, act)
    guard = np.float32(-7.25)
    y0 = torch.full((rc + 8,), float(guard), dtype=torch.float32, device=dev)
    y1 = torch.full((rc + 8,), float(guard), dtype=torch.float32, device=dev)
    say("balanced tiling", type_name, rc, k, layout)
    m27q.matvec_q8(w, act, y1[:rc])
    q, d, s = ora.quant_act(x)
    want, nrm = ora.gemv_act(t, wb, rb, rc, q, d, s)
    got = to_host(y1)
    assert (np.abs(got[:rc] - want) <= int_dot_tol(nrm)).all()
    assert (got[rc:] == guard).all()
    m27q.matvec(w, xd, y0[:rc])
    assert np.array_equal(to_host(y0).view(np.uint32), got.view(np.uint32))


@pytest.mark.parametrize("layout_name", ["TILED", "GGUF"])
@pytest.mark.parametrize("type_name", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "IQ4_XS"])
@pytest.mark.parametrize("rc,units", [(4098, 24), (5117, 2), (5120, 68), (1030, 9), (17001, 20)])
def test_single_product_edges_every_type(m27q, ora, dev, layout_name, type_name, rc, units):
    """Single products around the balanced-tiling rule, every integer-dot type
    and both layouts: 513 tiles with a last tile of 2 rows (24 units), 640
    tiles with a last tile of 5 rows and a single unit pair (fewer units than
    K slices: waves with nothing to stream), the 68-unit down shape (balanced
    tiling on quantized input), and rows of an odd unit count (GGUF Q6_K: every
    other row starts 2 bytes past a multiple of 4; one-tile waves read its
    fields as shifted dwords), and 2126 tiles with a last tile of one row
    (8-9 tiles per CU: balanced tiling with up to 9 tiles per workgroup,
    three per wave).  The quantized-input and the fp32-input
    products, each with a residual, against the integer-dot oracle (in-kernel
    quantization gives the same codes), the rows past row_count untouched."""
    import torch
    t = getattr(m27q, type_name)
    k = units * (128 if type_name == "Q8_0" else 256)
    rb = k // m27q.BLOCK_ELEMS[t]
    wb = weights(ora, type_name, rc, k, 21)
    w = m27q.Weight.upload(wb.reshape(-1), t, rb, rc, getattr(m27q, layout_name), dev)
    rng = np.random.default_rng(17)
    x = rng.standard_normal(k).astype(np.float32)
    res = rng.standard_normal(rc).astype(np.float32)
    xd, rd = to_dev(x, dev), to_dev(res, dev)
    act = m27q.Act(1, k, dev)
    m27q.quant_act(xd, act)
    guard = np.float32(-7.25)
    y0 = torch.full((rc + 8,), float(guard), dtype=torch.float32, device=dev)
    y1 = torch.full((rc + 8,), float(guard), dtype=torch.float32, device=dev)
    say("single product edges", layout_name, type_name, rc, k)
    m27q.matvec_q8(w, act, y1[:rc], residual=rd)
    q, d, s = ora.quant_act(x)
    want, nrm = ora.gemv_act(t, wb, rb, rc, q, d, s)
    m27q.matvec(w, xd, y0[:rc], residual=rd)
    for form, y in (("q8 x", y1), ("fp32 x", y0)):
        got = to_host(y)
        bad = np.abs(got[:rc].astype(np.float64) - (want + res)) > int_dot_tol(nrm) + 1e-6 * np.abs(res)
        assert not bad.any(), (form, np.flatnonzero(bad)[:5], got[:rc][bad][:5], (want + res)[bad][:5])
        assert (got[rc:] == guard).all(), form


def test_fp32_input_multi_and_swiglu(m27q, ora, dev):
    import torch
    k = 5120
    shapes = [6144, 1024, 1024]
    wbs = [weights(ora, "Q4_K", rc, k, 40 + i) for i, rc in enumerate(shapes)]
    ws = [m27q.Weight.upload(wb.reshape(-1), m27q.Q4_K, 20, rc, m27q.TILED, dev) for wb, rc in zip(wbs, shapes)]
    xh = np.random.default_rng(11).standard_normal(k).astype(np.float32)
    x = to_dev(xh, dev)
    ya = [torch.empty(rc, dtype=torch.float32, device=dev) for rc in shapes]
    say("multi fp32 input")
    m27q.matvec_multi(ws, x, ya)
    q, d, s = ora.quant_act(xh)
    for wb, rc, y in zip(wbs, shapes, ya):
        want, nrm = ora.gemv_act(m27q.Q4_K, wb, 20, rc, q, d, s)
        assert (np.abs(to_host(y) - want) <= int_dot_tol(nrm)).all()
    rc = 17408
    gb, ub = weights(ora, "Q4_K", rc, k, 30), weights(ora, "Q4_K", rc, k, 31)
    gw = m27q.Weight.upload(gb.reshape(-1), m27q.Q4_K, 20, rc, m27q.TILED, dev)
    uw = m27q.Weight.upload(ub.reshape(-1), m27q.Q4_K, 20, rc, m27q.TILED, dev)
    y0 = torch.empty(rc, dtype=torch.float32, device=dev)
    q0, ref = m27q.Act(1, rc, dev), m27q.Act(1, rc, dev)
    say("swiglu fp32 input")
    m27q.ffn_swiglu(gw, uw, x, y0, yq=q0)
    check_swiglu(ora, m27q.Q4_K, gb, ub, rc, q, d, s, to_host(y0))
    m27q.quant_act(y0, ref)
    assert np.array_equal(to_host(q0.buf), to_host(ref.buf))


@pytest.mark.parametrize("type_name,rc,k", [("Q4_K", 17408, 5120), ("Q6_K", 5120, 17408)])
def test_properties_full_size(m27q, ora, dev, type_name, rc, k):
    """Zero input -> exact zeros; x = 127 e_j -> 127 x column j of the dequantized matrix."""
    import torch
    t = getattr(m27q, type_name)
    rb = k // 256
    wb = weights(ora, type_name, rc, k, 10)
    w = m27q.Weight.upload(wb.reshape(-1), t, rb, rc, m27q.TILED, dev)
    y = torch.empty(rc, dtype=torch.float32, device=dev)
    act = m27q.Act(1, k, dev)
    say("zero input", type_name)
    m27q.quant_act(torch.zeros(k, dtype=torch.float32, device=dev), act)
    m27q.matvec_q8(w, act, y)
    assert (to_host(y) == 0).all()
    deq = torch.empty((rc, 256), dtype=torch.float32, device=dev)
    for j in (0, 37, k // 2 + 131, k - 1):
        x = torch.zeros(k, dtype=torch.float32, device=dev)
        x[j] = 127.0
        say("one-hot", type_name, j)
        m27q.quant_act(x, act)
        m27q.matvec_q8(w, act, y)
        blk = j // 256
        # column j of the dequantized matrix, via the GPU dequant (bit-exact, tested separately)
        wcol = m27q.Weight.upload(np.ascontiguousarray(wb.reshape(rc, rb, -1)[:, blk]).reshape(-1), t, 1, rc,
                                  m27q.GGUF, dev)
        m27q.dequant_rows(wcol, 0, rc, deq)
        col = to_host(deq)[:, j % 256].astype(np.float64)
        got = to_host(y).astype(np.float64)
        assert np.allclose(got, 127.0 * col, rtol=1e-6, atol=1e-6 * np.abs(127.0 * col).max())


@pytest.mark.parametrize("layout", [0, 1])
def test_mixed_type_pair_ssm_shapes(m27q, ora, dev, layout):
    """l_mv_pair's SSM-layer pair (exec:2106-2125, :2492): wqkv Q6_K 10240 x 5120
    and wqkv_gate Q5_K 6144 x 5120 on one activation, through the multi entry
    points (one launch per type); each output matches the integer-dot oracle
    and is bit-identical to the single product on the same activation."""
    import torch
    k = 5120
    spec = [("Q6_K", 10240, 31), ("Q5_K", 6144, 32)]
    ws, bl = [], []
    for name, rc, seed in spec:
        t = getattr(m27q, name)
        wb = weights(ora, name, rc, k, seed)
        bl.append(wb)
        ws.append(m27q.Weight.upload(wb.reshape(-1), t, k // 256, rc, layout, dev))
    x, act = quantized_x(m27q, dev, k, 33)
    q, d, s = act_host(m27q, act)
    xd = to_dev(x, dev)
    for form in ("q8", "fp32"):
        ys = [torch.empty(rc, dtype=torch.float32, device=dev) for _, rc, _ in spec]
        one = [torch.empty(rc, dtype=torch.float32, device=dev) for _, rc, _ in spec]
        say("mixed pair", form, "layout", layout)
        if form == "q8":
            m27q.matvec_q8_multi(ws, act, ys)
            for w, y in zip(ws, one):
                m27q.matvec_q8(w, act, y)
        else:
            m27q.matvec_multi(ws, xd, ys)
            for w, y in zip(ws, one):
                m27q.matvec(w, xd, y)
        for (name, rc, _), w, wb, y, y1 in zip(spec, ws, bl, ys, one):
            got = to_host(y)
            want, nrm = ora.gemv_act(w.type, wb, w.rb, rc, q[0], d[0], s[0])
            assert (np.abs(got.astype(np.float64) - want) <= int_dot_tol(nrm)).all(), (form, name)
            assert np.array_equal(got.view(np.uint32), to_host(y1).view(np.uint32)), (form, name)
