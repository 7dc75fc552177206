"""Pins the CPU oracle against checks independent of its own formulas.

- fp16 conversion: numpy's float16 implementation, all 65536 inputs.
- Q4_K dequant: the reference's known-answer block (official_dequant.c bytes ->
  the values the reference's GPU embed wrote), and dequantize_row_q4_K compiled
  from the reference's debug/official_dequant.c (oracle/_ref) on random blocks.
- Q4_K / Q5_K / Q6_K / Q8_0 dequant: the reference's *other* formulation of
  each format, its dp4a vec-dot (exec:250-310, :421-495, :586-628, :535-580),
  driven with a one-hot activation so that it returns one dequantized weight
  per position.
- Q5_K dequant also reduces to the pinned Q4_K dequant when qh = 0.
- int-dot oracle: numpy fp64 matmul of dequantized weights and activations.
- activation quantizer: closed-form properties and constructed ties.
- top-k: numpy lexsort.
"""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN

RNG = np.random.default_rng(1234)


def random_blocks(ora, type_, nblocks, rng=RNG):
    """Random block bytes with finite fp16 scales (subnormals and negatives allowed)."""
    ts = ora.TYPE_SIZE[type_]
    b = rng.integers(0, 256, size=(nblocks, ts), dtype=np.uint8)
    f16 = lambda n: (rng.standard_normal(n) * 0.05).astype(np.float16).view(np.uint16)
    if type_ in (ora.Q4_K, ora.Q5_K):
        b[:, 0:2] = f16(nblocks).view(np.uint8).reshape(nblocks, 2)
        b[:, 2:4] = f16(nblocks).view(np.uint8).reshape(nblocks, 2)
    elif type_ == ora.Q6_K:
        b[:, 208:210] = f16(nblocks).view(np.uint8).reshape(nblocks, 2)
    elif type_ in (ora.Q8_0, ora.IQ4_XS):
        b[:, 0:2] = f16(nblocks).view(np.uint8).reshape(nblocks, 2)
    # a few subnormal / zero scales
    sub = np.array([0x0001, 0x03ff, 0x8001, 0x0000, 0x8000], np.uint16).view(np.uint8).reshape(5, 2)
    for i in range(min(5, nblocks)):
        off = {ora.Q4_K: 0, ora.Q5_K: 0, ora.Q6_K: 208, ora.Q8_0: 0, ora.IQ4_XS: 0}[type_]
        b[i, off:off + 2] = sub[i]
    return b


def test_fp16_to_fp32_all_inputs(ora):
    h = np.arange(65536, dtype=np.uint16)
    got = ora.fp16_to_fp32(h)
    want = h.view(np.float16).astype(np.float32)
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.isnan(got[~fin]).all()


def test_fp32_to_fp16_rne(ora):
    f = (RNG.standard_normal(200000) * 10.0 ** RNG.integers(-9, 6, 200000)).astype(np.float32)
    edge = np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 1e-9,
                     np.inf, -np.inf], np.float32)
    f = np.concatenate([f, edge])
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(ora.fp32_to_fp16(f), want)


def test_q4k_known_answer_from_reference(ora):
    kat = json.load(open(os.path.join(GOLDEN, "q4k_kat.json")))
    block = np.zeros(144, np.uint8)
    prefix = np.frombuffer(bytes.fromhex(kat["block_prefix_hex"]), np.uint8)
    block[:32] = prefix
    y = ora.dequant(ora.Q4_K, block, 1, 1)[0]
    want = np.array(kat["expected_first16"], np.float32)
    assert np.array_equal(y[:16].view(np.uint32), want.view(np.uint32))


def test_q4k_matches_reference_c_build(ora):
    ref = ora.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (needs the reference checkout at build time)")
    blocks = random_blocks(ora, ora.Q4_K, 512)
    got = ora.dequant(ora.Q4_K, blocks, 512, 1)[0]
    want = np.empty(512 * 256, np.float32)
    ref.dequantize_row_q4_K(blocks.ctypes.data, want.ctypes.data, 512 * 256)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("type_name", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "IQ4_XS"])
def test_dequant_matches_reference_vecdot_formulation(ora, type_name):
    """x = 127 e_j quantizes to d = 1, code 127 at j: the reference's dp4a dot then
    returns 127 * W[j] (rounded once or twice), which pins every position's
    nibble/bit/scale index of the dequant restatement."""
    t = getattr(ora, type_name)
    be = ora.BLOCK_ELEMS[t]
    rb = 2 if t != ora.Q8_0 else 8
    k = rb * be

    def f16(b, off):
        return abs(float(np.frombuffer(b[off:off + 2].tobytes(), np.float16)[0]))

    def term_bound(b):
        # largest |term| the fp32 combine of the reference's formulation can round:
        # 127 x (max scale) x (max code) x (block scale), per block
        if t in (ora.Q4_K, ora.Q5_K):
            qmax = 15 if t == ora.Q4_K else 31
            return 127.0 * 63 * (qmax * f16(b, 0) + f16(b, 2))
        if t == ora.Q6_K:
            return 127.0 * 128 * 32 * f16(b, 208)
        if t == ora.IQ4_XS:
            return 127.0 * 127 * 32 * f16(b, 0)
        return 127.0 * 128 * f16(b, 0)

    for trial in range(3):
        blocks = random_blocks(ora, t, rb, np.random.default_rng(trial))
        deq = ora.dequant(t, blocks, rb, 1)[0].astype(np.float64)
        for j in range(k):
            x = np.zeros(k, np.float32)
            x[j] = 127.0
            xq = ora.quant_q8_1(x)
            v = ora.ref_vec_dot_q8_1(t, blocks.reshape(-1), xq, rb)
            tol = max(4e-7 * abs(127.0 * deq[j]), 2.0 ** -22 * term_bound(blocks[j // be])) + 1e-30
            assert abs(v - 127.0 * deq[j]) <= tol, (type_name, trial, j)


def test_q6k_single_bit_layout(ora):
    """Hand-set bits land where the ggml Q6_K layout puts them."""
    blk = np.zeros(210, np.uint8)
    blk[208:210] = np.array([0x3C00], np.uint16).view(np.uint8)  # d = 1.0
    blk[192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8)  # scales 1..16
    blk[0] = 0x0F        # ql[0] low nibble -> q0 at position 0
    blk[32 + 5] = 0xF0   # ql[37] high nibble -> q3 at position 96 + 5
    blk[128 + 40] = 0xC0  # qh[40]: bits 6-7 -> q3 of half 1, l = 8 -> position 128 + 96 + 8
    y = ora.dequant(ora.Q6_K, blk, 1, 1)[0]
    want = np.full(256, -32.0, np.float32) * np.repeat(np.arange(1, 17, dtype=np.float32), 16)
    want[0] = 1.0 * (15 - 32)
    want[96 + 5] = 7.0 * (15 - 32)
    want[128 + 96 + 8] = 15.0 * (48 - 32)
    assert np.array_equal(y, want)


def test_q5k_without_high_bits_is_q4k(ora):
    """A Q5_K block with qh = 0 holds the same values as the Q4_K block with the
    same d, dmin, scales and qs (Q4_K is pinned to the reference's C above)."""
    q4 = random_blocks(ora, ora.Q4_K, 64)
    q5 = np.zeros((64, 176), np.uint8)
    q5[:, :16] = q4[:, :16]      # d, dmin, scales
    q5[:, 48:176] = q4[:, 16:144]  # qs after qh[32]
    a = ora.dequant(ora.Q4_K, q4, 64, 1)[0]
    b = ora.dequant(ora.Q5_K, q5, 64, 1)[0]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q5k_high_bit_positions(ora):
    """Bit j of qh[l] adds 16 to the code of position l of 32-group j, and only
    there (the index map of exec:955-969)."""
    rng = np.random.default_rng(3)
    base = random_blocks(ora, ora.Q5_K, 1, rng)[0]
    base[5:] = base[5:]  # keep random scales
    base[16:48] = 0       # qh = 0
    y0 = ora.dequant(ora.Q5_K, base, 1, 1)[0]
    q4 = np.concatenate([base[:16], base[48:]])
    for j in range(8):
        for l in (0, 7, 31):
            blk = base.copy()
            blk[16 + l] |= np.uint8(1 << j)
            y = ora.dequant(ora.Q5_K, blk, 1, 1)[0]
            changed = np.flatnonzero(y.view(np.uint32) != y0.view(np.uint32))
            pos = 32 * j + l
            assert set(changed) <= {pos}
            # the changed value: the Q4_K value of a block whose nibble is 16 larger
            # cannot be written in Q4_K, so compare with d*sc*(q+16) - dmin*m
            d = np.float32(np.frombuffer(q4[0:2].tobytes(), np.float16)[0])
            dm = np.float32(np.frombuffer(q4[2:4].tobytes(), np.float16)[0])
            sc, m = scale_min(q4[4:16], j)
            nib = (q4[16 + 32 * (j // 2) + l] >> (4 * (j & 1))) & 15
            want = np.float32(d * np.float32(sc)) * np.float32(nib + 16) - np.float32(dm * np.float32(m))
            assert y[pos].view(np.uint32) == np.float32(want).view(np.uint32) or (np.isnan(y[pos]) and np.isnan(want))


def scale_min(q, j):
    """get_scale_min_k4 from the reference's byte description (exec:690-693)."""
    q = [int(v) for v in q]
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def test_iq4xs_hand_set_block(ora):
    """d = 1, group scales ls_j = 32 + j + 1 (6 bits over scales_l / scales_h),
    index pattern (i + j) % 16: every value is (j + 1) kv[(i + j) % 16], with kv the
    table of exec:51-55, low nibbles at positions 0..15 of a group, high 16..31."""
    kv = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)
    blk = np.zeros(136, np.uint8)
    blk[0:2] = np.array([0x3C00], np.uint16).view(np.uint8)  # d = 1.0
    sh = 0
    for j in range(8):
        ls = 32 + j + 1
        blk[4 + j // 2] |= (ls & 15) << (4 * (j % 2))
        sh |= ((ls >> 4) & 3) << (2 * j)
        for i in range(16):
            blk[8 + 16 * j + i] = ((i + j) % 16) | (((i + j + 5) % 16) << 4)
    blk[2:4] = np.array([sh], np.uint16).view(np.uint8)
    y = ora.dequant(ora.IQ4_XS, blk, 1, 1)[0]
    want = np.zeros(256, np.float32)
    for j in range(8):
        for i in range(16):
            want[32 * j + i] = (j + 1) * kv[(i + j) % 16]
            want[32 * j + 16 + i] = (j + 1) * kv[(i + j + 5) % 16]
    assert np.array_equal(y, want)


@pytest.mark.parametrize("source", ["quantized", "random bytes"])
@pytest.mark.parametrize("type_name", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "IQ4_XS"])
def test_int_dot_oracle_vs_numpy_bruteforce(ora, type_name, source):
    t = getattr(ora, type_name)
    be = ora.BLOCK_ELEMS[t]
    rb, rc = (3, 16) if t != ora.Q8_0 else (24, 16)
    k = rb * be
    if source == "quantized":
        w = ora.synth_weights(t, rc, k, seed=5)
    else:
        w = random_blocks(ora, t, rb * rc, np.random.default_rng(55))
    x = RNG.standard_normal(k).astype(np.float32)
    q, d, s = ora.quant_act(x)
    y, nrm = ora.gemv_act(t, w, rb, rc, q, d, s)
    wd = ora.dequant(t, w, rb, rc).astype(np.float64)
    xd = q.astype(np.float64) * np.repeat(d.astype(np.float64), 32)
    want = wd @ xd
    # dequant rounds each weight once to fp32 (d*sc*q - dmin*m: exact products,
    # one rounded difference), which random scales and mins of unrelated
    # exponents expose; the oracle's integer dot has no such rounding
    tol = 1e-12 * np.abs(wd).sum(1).max() * np.abs(xd).max() + 2.0 ** -24 * (np.abs(wd) @ np.abs(xd))
    assert (np.abs(y - want) <= tol).all()
    assert (nrm >= np.abs(y) * (1 - 1e-12)).all()


def test_int_dot_oracle_special_cases(ora):
    w = ora.synth_weights(ora.Q4_K, 8, 512, seed=9)
    q, d, s = ora.quant_act(np.zeros(512, np.float32))
    y, _ = ora.gemv_act(ora.Q4_K, w, 2, 8, q, d, s)
    assert np.array_equal(y, np.zeros(8))
    assert (q == 0).all() and (d == 0).all() and (s == 0).all()


def test_quant_act_properties(ora):
    x = (RNG.standard_normal((4, 1024)) * 10.0 ** RNG.integers(-6, 6, (4, 1))).astype(np.float32)
    q, d, s = ora.quant_act(x)
    g = x.reshape(4, -1, 32)
    qg = q.reshape(4, -1, 32).astype(np.int64)
    amax = np.abs(g).max(-1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float32))
    assert (np.abs(qg) <= 127).all()
    assert (np.abs(qg).max(-1) == 127).all()
    err = np.abs(g.astype(np.float64) - qg * d[..., None].astype(np.float64))
    assert (err <= 0.5 * d[..., None] * (1 + 2.0 ** -22) + 1e-45).all()
    lo = qg[..., :16].sum(-1)
    hi = qg[..., 16:].sum(-1)
    s = s.astype(np.int64)
    assert np.array_equal(((s & 0xFFFF) ^ 0x8000) - 0x8000, lo)
    assert np.array_equal(((s >> 16) ^ 0x8000) - 0x8000, hi)


def test_quant_act_matches_numpy_restatement(ora):
    """The documented rule restated in numpy: float32 d = amax / 127, id = 1 / d
    (0 when d == 0), t = float32(x * id), code = round half away from zero of t
    (evaluated exactly in float64), clamped to +-127."""
    x = (RNG.standard_normal((8, 2048)) * 10.0 ** RNG.integers(-8, 8, (8, 1))).astype(np.float32)
    x[0, :32] = 0.0
    x[1, 32:64] = np.float32(1e-44)  # d underflows to 0: every code 0
    q, d, s = ora.quant_act(x)
    g = x.reshape(8, -1, 32)
    amax = np.abs(g).max(-1)
    dd = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(dd != 0, np.float32(1) / dd, np.float32(0)).astype(np.float32)
    t = (g * idv[..., None]).astype(np.float32).astype(np.float64)
    want = np.clip(np.sign(t) * np.floor(np.abs(t) + 0.5), -127, 127).astype(np.int64)
    assert np.array_equal(d, dd)
    assert np.array_equal(q.reshape(8, -1, 32).astype(np.int64), want)
    assert (q[0, :32] == 0).all() and (q[1, 32:64] == 0).all()


def test_quant_act_nan_rule(ora):
    """NaN values stay out of the group's amax and take code 0; a group of
    NaNs has d = 0 and all codes 0 (the GPU's maxNum and float-to-int rules)."""
    x = RNG.standard_normal(96).astype(np.float32)
    x[3], x[17] = np.nan, -np.nan
    x[64:96] = np.nan
    q, d, s = ora.quant_act(x)
    fin = x[:32][~np.isnan(x[:32])]
    assert d[0] == np.float32(np.abs(fin).max() / np.float32(127))
    assert q[3] == 0 and q[17] == 0 and (q[64:96] == 0).all() and d[2] == 0 and s[2] == 0
    # the finite values of the group quantize as they would with the NaNs at 0
    x0 = x.copy()
    x0[[3, 17]] = 0.0
    q0, d0, _ = ora.quant_act(x0[:32])
    assert np.array_equal(q[:32], q0) and d[0] == d0[0]


def test_quant_act_rounds_half_away_from_zero(ora):
    x = np.zeros(32, np.float32)
    x[0] = 127.0  # d = 1 exactly
    x[1:7] = [2.5, -2.5, 0.5, -0.5, 1.5, 126.5]
    q, d, _ = ora.quant_act(x)
    assert d[0] == 1.0
    assert list(q[1:7]) == [3, -3, 1, -1, 2, 127]


def test_topk_matches_lexsort(ora):
    v = np.round(RNG.standard_normal(5000) * 4).astype(np.float32)  # many ties
    v[10], v[20], v[30] = -0.0, 0.0, np.nan
    v[40], v[50] = np.inf, -np.inf
    idx, val = ora.topk(v, 64)
    key = np.where(np.isnan(v), -np.inf, v)
    nan_last = np.isnan(v).astype(np.int8)
    order = np.lexsort((np.arange(v.size), -key, nan_last))
    assert np.array_equal(idx, order[:64])
    assert np.array_equal(val.view(np.uint32), v[order[:64]].view(np.uint32))
    # -0.0 and +0.0 compare equal: index order decides
    z = np.array([0.0, -0.0, 0.0, -0.0], np.float32)
    assert list(ora.topk(z, 4)[0]) == [0, 1, 2, 3]


def test_q8k_cpu_path_is_a_sane_approximation(ora):
    """The ggml-semantics CPU path (parity unpinned) stays within its quantization error."""
    for t in (ora.Q4_K, ora.Q6_K, ora.Q8_0):
        k = 1024
        w = ora.synth_weights(t, 32, k, seed=3)
        x = RNG.standard_normal(k).astype(np.float32)
        rb = k // ora.BLOCK_ELEMS[t]
        y = ora.gemv_cpu(t, w, rb, 32, ora.quant_cpu_act(t, x), nthreads=2)
        ref = ora.gemv_f64(t, w, rb, 32, x)
        scale = np.abs(ora.dequant(t, w, rb, 32)).sum(1) * np.abs(x).max()
        assert (np.abs(y - ref) <= 0.02 * scale).all()


def test_sample_properties(ora):
    """sample() after its top-k: first candidate for temperature <= 0, for u = 0,
    for top_p -> 0 and for min_p = 1 (distinct values); over a fine grid of u
    the share of each token equals its kept probability."""
    rng = np.random.default_rng(11)
    val = np.sort(rng.standard_normal(40).astype(np.float32))[::-1].copy()
    idx = rng.permutation(1000)[:40].astype(np.int32)
    assert ora.sample(idx, val, 0.0, 0.05, 0.95, 0.7) == idx[0]
    assert ora.sample(idx, val, 0.8, 0.05, 0.95, 0.0) == idx[0]
    assert ora.sample(idx, val, 0.8, 0.0, 1e-9, 0.99) == idx[0]
    assert ora.sample(idx, val, 0.8, 1.0, 1.0, 0.99) == idx[0]
    for T, min_p, top_p in ((0.8, 0.05, 0.95), (1.5, 0.0, 1.0), (0.3, 0.2, 0.5)):
        p = np.exp((val.astype(np.float64) - val[0]) / T)
        p /= p.sum()
        keep = p >= p[0] * min_p
        ks = np.flatnonzero(keep)
        if top_p < 1:
            c = np.cumsum(p[ks])
            ks = ks[: int(np.searchsorted(c, top_p * (1 - 1e-6))) + 1]
        q = p[ks] / p[ks].sum()
        N = 20000
        us = (np.arange(N) + 0.5) / N
        got = np.array([ora.sample(idx, val, T, min_p, top_p, float(u)) for u in us])
        for i, want in zip(ks, q):
            assert abs((got == idx[i]).mean() - want) <= 2.0 / N + 1e-6
        assert set(got) <= set(idx[ks])


# ------------------------------------------ the fixed exp and the gate --

def _ulps(got, want64):
    """|got - want| in units of the float32 spacing at want."""
    w32 = want64.astype(np.float32)
    return np.abs(got.astype(np.float64) - want64) / np.spacing(np.abs(w32)).astype(np.float64)


def test_exp_cw_within_2_ulp(ora):
    """ora_exp_cw (Cody-Waite reduction + degree-7 Taylor polynomial) against
    float64 exp: every 97th float in [-87, 87], plus the clamp ends."""
    lo = np.float32(-87.0).view(np.uint32)
    hi = np.float32(87.0).view(np.uint32)
    pos = np.arange(0, int(hi) + 1, 97, dtype=np.uint32).view(np.float32)
    neg = np.arange(0x80000000, int(lo) + 1, 97, dtype=np.uint32).view(np.float32)
    t = np.concatenate([pos, neg, np.float32([87.0, -87.0, 0.5, -0.5, 1e-30, -1e-30])])
    got = ora.exp_cw(t)
    assert np.all(np.isfinite(got)) and np.all(got > 0)
    assert _ulps(got, np.exp(t.astype(np.float64))).max() <= 2.0
    assert ora.exp_cw(np.float32([0.0, -0.0]))[0] == 1.0
    ends = ora.exp_cw(np.float32([-1e4, -88.0, -np.inf, 1e4, 88.0, np.inf]))
    e_lo, e_hi = ora.exp_cw(np.float32([-87.0, 87.0]))
    assert np.array_equal(ends, np.float32([e_lo] * 3 + [e_hi] * 3))
    # NaN comes back as NaN, so a NaN gate propagates through gated() instead
    # of letting x through
    assert np.isnan(ora.exp_cw(np.float32([np.nan]))).all()
    assert np.isnan(ora.gated(np.float32([1.5, -2.0]), np.float32([np.nan, np.nan]))).all()
    # monotone over a fine sorted sweep (an off coefficient would show as a step)
    s = np.sort(t)
    assert np.all(np.diff(ora.exp_cw(s).astype(np.float64)) >= 0)


def test_gated_against_float64_sigmoid(ora):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(200000) * 10.0 ** rng.integers(-3, 4, 200000)).astype(np.float32)
    g = (rng.standard_normal(200000) * 8).astype(np.float32)
    got = ora.gated(x, g).astype(np.float64)
    want = x.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))
    # exp within 2 ulp, then an add, a divide and a multiply: a few ulp at most
    assert (np.abs(got - want) <= 8 * 2.0 ** -24 * np.abs(want) + 1e-45).all()
    # saturation: the gate is 1 far to the right, and x e^-87 / (1 + ...) far to the left
    assert np.array_equal(ora.gated(np.float32([3.0, -2.0]), np.float32([40.0, 1e4])), np.float32([3.0, -2.0]))
    far = ora.gated(np.float32([1.0]), np.float32([-1e4]))[0]
    assert 0 < far <= np.float32(1.7e-38)


def test_quant_act_subnormal_scale_groups(ora):
    """A group whose 1/d is not finite (d subnormal below 2^-128) gets all-zero
    codes and keeps its d; a subnormal d with a finite 1/d quantizes normally."""
    x = np.zeros(96, np.float32)
    x[0:32] = np.float32(1e-40) * np.arange(1, 33, dtype=np.float32)   # amax 3.2e-39: 1/d inf
    x[32:64] = np.float32(5e-37) * np.linspace(-1, 1, 32, dtype=np.float32)  # d ~ 3.9e-39: 1/d finite
    x[64:96] = RNG.standard_normal(32).astype(np.float32)
    q, d, s = ora.quant_act(x)
    assert d[0] == np.float32(np.float32(3.2e-39) / np.float32(127)) and d[0] > 0
    assert (q[0:32] == 0).all() and s[0] == 0
    assert np.isfinite(np.float32(1) / d[1])
    assert q[32] == -127 and q[63] == 127
    q2, d2, _ = ora.quant_act(x[64:96].copy())
    assert np.array_equal(q[64:96], q2) and d[2] == d2[0]


# ------------------------------ ggml CPU path (q8_K / q8_0): the pins --

def _oracle_variant(plant, tmp):
    """The oracle built with ORA_PLANT = plant (one planted mistake), as ctypes."""
    import ctypes as C
    import subprocess
    src = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "m27q_oracle.c")
    so = os.path.join(tmp, f"libora_plant{plant}.so")
    subprocess.run(["gcc", "-O2", "-march=x86-64-v3", "-ffp-contract=off", "-fPIC", "-std=c11", "-pthread",
                    "-shared", f"-DORA_PLANT={plant}", "-o", so, src, "-lm"], check=True)
    return C.CDLL(so)


def q8k_pin_failures(ora, L, dots="ora_vec_dot"):
    """Names of the checks that the ggml-path routines of library L fail:
    the quantize_row_q8_K properties fixed by its definition, and each vec-dot
    against the fp64 sum of the pinned dequantized weights times the values
    (d q) its activation blocks stand for."""
    import ctypes as C
    P = C.c_void_p
    L.ora_quantize_row_q8_K.argtypes = [P, P, C.c_int64]
    L.ora_quantize_row_q8_0_act.argtypes = [P, P, C.c_int64]
    for f in ("q4_K_q8_K", "q6_K_q8_K", "q8_0_q8_0"):
        getattr(L, f"{dots}_{f}").argtypes = [C.c_int, P, P]
        getattr(L, f"{dots}_{f}").restype = C.c_float

    def q8k(x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(x.size // 256 * 292, np.uint8)
        L.ora_quantize_row_q8_K(x.ctypes.data, out.ctypes.data, x.size)
        return out

    fails = []
    rng = np.random.default_rng(77)
    x = (rng.standard_normal(4096) * 3).astype(np.float32)
    x[256:512] = 0.0
    b = np.frombuffer(q8k(x).tobytes(), ora.Q8_K_DTYPE)
    q = b["qs"].astype(np.int64)
    d = b["d"].astype(np.float64)
    xb = x.reshape(-1, 256)
    live = np.abs(xb).max(1) > 0
    if np.abs(q).max() > 127:
        fails.append("q8_K codes within +-127")
    am = np.abs(xb).argmax(1)
    if not (q[live, am[live]] == -127).all():
        fails.append("q8_K argmax code -127")
    if not np.array_equal(b["bsums"].astype(np.int64), q.reshape(-1, 16, 16).sum(-1)):
        fails.append("q8_K bsums are the 16-value code sums")
    if not (np.abs(xb[live] - d[live, None] * q[live]) <= np.abs(d[live, None]) * (0.5 + 2.0 ** -16)).all():
        fails.append("q8_K |x - d q| <= |d| / 2")
    if not ((q[~live] == 0).all() and (d[~live] == 0).all()):
        fails.append("q8_K zero block")
    t = np.zeros(256, np.float32)
    t[0] = -127.0  # iscale = -127 / vmax = 1 exactly
    t[1:8] = [2.5, 3.5, -2.5, 0.5, -0.5, 1.5, 126.5]
    bt = np.frombuffer(q8k(t).tobytes(), ora.Q8_K_DTYPE)[0]
    if list(bt["qs"][:8]) != [-127, 2, 4, -2, 0, 0, 2, 126] or bt["d"] != 1.0:
        fails.append("q8_K round half to even")

    K, rc = 2048, 24
    xs = rng.standard_normal(K).astype(np.float32)
    for t_ in (ora.Q4_K, ora.Q6_K, ora.Q8_0):
        rb = K // ora.BLOCK_ELEMS[t_]
        w = ora.synth_weights(t_, rc, K, seed=40 + t_)
        if t_ == ora.Q8_0:
            xq = np.zeros(K // 32 * 34, np.uint8)
            L.ora_quantize_row_q8_0_act(xs.ctypes.data, xq.ctypes.data, K)
        else:
            xq = q8k(xs)
        xv = ora.cpu_act_values(t_, xq)
        W = ora.dequant(t_, w, rb, rc).astype(np.float64)
        want = W @ xv
        nrm = np.abs(W) @ np.abs(xv)
        if t_ == ora.Q4_K:  # the d sc q and dmin m terms separately: zero the quants
            w0 = w.reshape(rc, rb, 144).copy()
            w0[:, :, 16:] = 0
            nrm = nrm + 2 * np.abs(ora.dequant(t_, w0.reshape(rc, -1), rb, rc).astype(np.float64)) @ np.abs(xv)
        fn = getattr(L, f"{dots}_" + {ora.Q4_K: "q4_K_q8_K", ora.Q6_K: "q6_K_q8_K", ora.Q8_0: "q8_0_q8_0"}[t_])
        got = np.array([fn(K, np.ascontiguousarray(w[r]).ctypes.data, xq.ctypes.data) for r in range(rc)])
        if not (np.abs(got - want) <= K * 2.0 ** -24 * nrm).all():
            fails.append(f"vec_dot type {t_} = sum dequant(W) d q")
    return fails


def test_q8k_cpu_path_pinned(ora):
    """ggml's q8_K / q8_0 CPU path as restated: every pin holds."""
    assert q8k_pin_failures(ora, ora.lib()) == []


def test_q8k_cpu_path_avx2_build_pinned(ora):
    """The AVX2 build of the same dots (the CPU baseline's SIMD leg) meets the
    same pins, and its rows equal the scalar restatement's within fp32
    reassociation."""
    assert q8k_pin_failures(ora, ora.lib(), dots="ora_simd_vec_dot") == []
    for t in (ora.Q4_K, ora.Q6_K, ora.Q8_0):
        k, rc = 5120, 64
        w = ora.synth_weights(t, rc, k, seed=9)
        x = RNG.standard_normal(k).astype(np.float32)
        xq = ora.quant_cpu_act(t, x)
        rb = k // ora.BLOCK_ELEMS[t]
        a = ora.gemv_cpu(t, w, rb, rc, xq, nthreads=3)
        b = ora.gemv_cpu(t, w, rb, rc, xq, nthreads=2, simd=True)
        W = np.abs(ora.dequant(t, w, rb, rc).astype(np.float64))
        nrm = W @ np.abs(ora.cpu_act_values(t, xq))
        assert (np.abs(a.astype(np.float64) - b) <= 64 * 2.0 ** -24 * nrm + 1e-30).all(), t


@pytest.mark.parametrize("plant,check", [
    (1, "vec_dot type 12"),           # min paired with the wrong bsums
    (2, "bsums"),                     # bsums over the wrong 16 codes
    (3, "half to even"),              # q8_K rounds half away from zero
    (4, "vec_dot type 14"),           # Q6_K scale of the wrong 16-group
    (5, "vec_dot type 8"),            # Q8_0 codes paired in the wrong order
    (6, "vec_dot type 12"),           # Q4_K scale of the neighbouring group
])
def test_q8k_pins_catch_planted_mistakes(ora, tmp_path, plant, check):
    fails = q8k_pin_failures(ora, _oracle_variant(plant, str(tmp_path)))
    assert any(check in f for f in fails), fails
