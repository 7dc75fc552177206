"""C-ABI checks that need no GPU: exports, host-side pack-time functions, and
argument validation (every check returns before the first HIP call, so bogus
device pointers are never dereferenced here)."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

RNG = np.random.default_rng(7)
FAKE = 0x10000  # a 64 KiB-aligned non-null "device" address, never dereferenced


def test_library_exports_every_header_symbol(m27q):
    syms = m27q.header_symbols()
    assert len(syms) >= 20
    out = subprocess.run(["nm", "-D", "--defined-only", m27q.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [s for s in syms if s not in exported]
    assert not missing, missing
    lib = m27q.lib()
    for s in syms:
        assert getattr(lib, s) is not None


def test_status_strings(m27q):
    for code in range(8):
        assert m27q.lib().m27q_status_string(code)


def test_row_size_matches_gguf_block_table(m27q, ora):
    # src/mono27b_gguf.cpp:375-382: whole blocks only, 0 otherwise
    for t in (m27q.Q4_K, m27q.Q5_K, m27q.Q6_K, m27q.Q8_0, m27q.IQ4_XS, m27q.F16, m27q.F32):
        be, bb = m27q.BLOCK_ELEMS[t], m27q.BLOCK_BYTES[t]
        assert m27q.row_size(t, 5120) == 5120 // be * bb
        assert m27q.row_size(t, 0) == 0
        if be > 1:
            assert m27q.row_size(t, be + 1) == 0
        assert bb == ora.TYPE_SIZE[t]
    assert m27q.row_size(99, 256) == 0


@pytest.mark.parametrize("type_name", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "IQ4_XS"])
@pytest.mark.parametrize("rb,rc", [(1, 1), (3, 13), (20, 64), (5, 9)])
def test_repack_roundtrip(m27q, type_name, rb, rc):
    t = getattr(m27q, type_name)
    raw = RNG.integers(0, 256, rb * rc * m27q.BLOCK_BYTES[t], dtype=np.uint8)
    tiled = m27q.repack(t, rb, rc, raw)
    assert tiled.size == m27q.weight_bytes(t, rb, rc, m27q.TILED)
    assert tiled.size % 16 == 0
    assert np.array_equal(m27q.unpack(t, rb, rc, tiled), raw)
    # every byte kept, padding is zero
    assert np.sort(tiled)[-raw.size:].sum() >= 0  # shape check only
    assert np.count_nonzero(tiled) == np.count_nonzero(raw)


def test_tiled_layout_offsets(m27q):
    """Bytes of block (row r, col b) land at the documented TILED offsets."""
    rb, rc = 3, 16
    t = m27q.Q4_K
    raw = RNG.integers(0, 256, (rc, rb, 144), dtype=np.uint8)
    tiled = m27q.repack(t, rb, rc, raw.reshape(-1))
    r, b = 11, 2
    unit = ((r // 8) * rb + b) * 1152
    i = r % 8
    assert np.array_equal(tiled[unit + 16 * i: unit + 16 * i + 16], raw[r, b, :16])
    for g in range(4):  # qs chunk pair g of row i at 128 + 256 g + 32 i
        assert np.array_equal(tiled[unit + 128 + 256 * g + 32 * i: unit + 160 + 256 * g + 32 * i],
                              raw[r, b, 16 + 32 * g: 48 + 32 * g])
    t = m27q.Q5_K
    raw = RNG.integers(0, 256, (rc, rb, 176), dtype=np.uint8)
    tiled = m27q.repack(t, rb, rc, raw.reshape(-1))
    unit = ((r // 8) * rb + b) * 1408
    assert np.array_equal(tiled[unit + 16 * i: unit + 16 * i + 16], raw[r, b, :16])
    for g in range(4):
        assert np.array_equal(tiled[unit + 128 + 256 * g + 32 * i: unit + 160 + 256 * g + 32 * i],
                              raw[r, b, 48 + 32 * g: 80 + 32 * g])
    assert np.array_equal(tiled[unit + 1152 + 32 * i: unit + 1184 + 32 * i], raw[r, b, 16:48])
    t = m27q.IQ4_XS
    raw = RNG.integers(0, 256, (rc, rb, 136), dtype=np.uint8)
    tiled = m27q.repack(t, rb, rc, raw.reshape(-1))
    unit = ((r // 8) * rb + b) * 1088
    assert np.array_equal(tiled[unit + 128 * i: unit + 128 * i + 128], raw[r, b, 8:])
    assert np.array_equal(tiled[unit + 1024 + 8 * i: unit + 1032 + 8 * i], raw[r, b, :8])
    t = m27q.Q6_K
    raw = RNG.integers(0, 256, (rc, rb, 210), dtype=np.uint8)
    tiled = m27q.repack(t, rb, rc, raw.reshape(-1))
    unit = ((r // 8) * rb + b) * 1680
    assert np.array_equal(tiled[unit + 128 * i: unit + 128 * i + 128], raw[r, b, :128])
    assert np.array_equal(tiled[unit + 1024 + 64 * i: unit + 1024 + 64 * i + 64], raw[r, b, 128:192])
    assert np.array_equal(tiled[unit + 1536 + 16 * i: unit + 1536 + 16 * i + 16], raw[r, b, 192:208])
    assert np.array_equal(tiled[unit + 1664 + 2 * i: unit + 1664 + 2 * i + 2], raw[r, b, 208:210])
    t = m27q.Q8_0
    rb = 6
    raw = RNG.integers(0, 256, (rc, rb, 34), dtype=np.uint8)
    tiled = m27q.repack(t, rb, rc, raw.reshape(-1))
    b = 5
    unit = ((r // 8) * 2 + b // 4) * 1088
    k = b % 4
    assert np.array_equal(tiled[unit + 128 * i + 32 * k: unit + 128 * i + 32 * k + 32], raw[r, b, 2:])
    assert np.array_equal(tiled[unit + 1024 + 8 * i + 2 * k: unit + 1024 + 8 * i + 2 * k + 2], raw[r, b, :2])


def test_act_buffer_geometry(m27q):
    assert m27q.act_bytes(1, 5120) >= 5120 + 2 * 160 * 4
    d_off, s_off = m27q.act_offsets(3, 6144)
    assert d_off >= 3 * 6144 and d_off % 256 == 0
    assert s_off >= d_off + 3 * 192 * 4 and s_off % 256 == 0
    assert m27q.act_bytes(1, 33) == 0
    assert m27q.act_bytes(0, 64) == 0


def W(m27q, ptr=FAKE, t=None, rb=20, rc=64, layout=None):
    return m27q.WeightDesc(ptr, m27q.Q4_K if t is None else t, rb, rc, m27q.TILED if layout is None else layout)


def test_validation_matvec_q8(m27q):
    L = m27q.lib()
    ok = W(m27q)
    assert L.m27q_matvec_q8(None, FAKE, FAKE, None, None, None) == 1
    assert L.m27q_matvec_q8(C.byref(W(m27q, ptr=None)), FAKE, FAKE, None, None, None) == 1
    assert L.m27q_matvec_q8(C.byref(ok), None, FAKE, None, None, None) == 1
    assert L.m27q_matvec_q8(C.byref(ok), FAKE, None, None, None, None) == 1
    assert L.m27q_matvec_q8(C.byref(W(m27q, t=99)), FAKE, FAKE, None, None, None) == 3
    assert L.m27q_matvec_q8(C.byref(W(m27q, t=m27q.F16, layout=m27q.GGUF)), FAKE, FAKE, None, None, None) == 3
    assert L.m27q_matvec_q8(C.byref(W(m27q, rb=0)), FAKE, FAKE, None, None, None) == 2
    assert L.m27q_matvec_q8(C.byref(W(m27q, rc=0)), FAKE, FAKE, None, None, None) == 2
    assert L.m27q_matvec_q8(C.byref(W(m27q, rc=(1 << 24) + 1)), FAKE, FAKE, None, None, None) == 2
    assert L.m27q_matvec_q8(C.byref(W(m27q, rb=(1 << 20) // 256 + 1)), FAKE, FAKE, None, None, None) == 2
    assert L.m27q_matvec_q8(C.byref(W(m27q, layout=7)), FAKE, FAKE, None, None, None) == 4
    assert L.m27q_matvec_q8(C.byref(W(m27q, ptr=FAKE + 2)), FAKE, FAKE, None, None, None) == 4
    assert L.m27q_matvec_q8(C.byref(ok), FAKE + 4, FAKE, None, None, None) == 4
    # fused output quantization needs rows in whole 32-row groups
    assert L.m27q_matvec_q8(C.byref(W(m27q, rc=40)), FAKE, FAKE, None, FAKE, None) == 2
    # GGUF Q6_K only needs halfword alignment; a byte-offset pointer is rejected
    assert L.m27q_matvec_q8(C.byref(W(m27q, ptr=FAKE + 1, t=m27q.Q6_K, layout=m27q.GGUF)), FAKE, FAKE,
                            None, None, None) == 4


def test_validation_multi_and_swiglu(m27q):
    L = m27q.lib()
    ws = (m27q.WeightDesc * 2)(W(m27q), W(m27q, rb=24))
    ys = (C.c_void_p * 2)(FAKE, FAKE)
    assert L.m27q_matvec_q8_multi(2, ws, FAKE, ys, None) == 2       # row_blocks differ
    assert L.m27q_matvec_q8_multi(0, ws, FAKE, ys, None) == 2
    assert L.m27q_matvec_q8_multi(5, ws, FAKE, ys, None) == 2
    # types may differ (one launch per type) but K may not: Q8_0 with 20 blocks is K = 640
    ws2 = (m27q.WeightDesc * 2)(W(m27q), W(m27q, t=m27q.Q8_0))
    assert L.m27q_matvec_q8_multi(2, ws2, FAKE, ys, None) == 2
    assert L.m27q_matvec_multi(2, ws2, FAKE, ys, None) == 2
    # every member is checked before the first launch: a bad second-type member stops both
    ws4 = (m27q.WeightDesc * 2)(W(m27q), W(m27q, t=m27q.Q6_K, ptr=0))
    assert L.m27q_matvec_q8_multi(2, ws4, FAKE, ys, None) == 1
    ws5 = (m27q.WeightDesc * 2)(W(m27q), W(m27q, t=m27q.Q6_K, layout=m27q.GGUF, ptr=FAKE + 1))
    assert L.m27q_matvec_q8_multi(2, ws5, FAKE, ys, None) == 4
    assert L.m27q_matmul_q8_multi(2, ws2, 4, FAKE, ys, None) == 2
    ys0 = (C.c_void_p * 2)(FAKE, None)
    ws3 = (m27q.WeightDesc * 2)(W(m27q), W(m27q))
    assert L.m27q_matvec_q8_multi(2, ws3, FAKE, ys0, None) == 1
    assert L.m27q_matvec_multi(2, ws, FAKE, ys, None) == 2
    assert L.m27q_matvec_multi(2, ws3, None, ys, None) == 1
    assert L.m27q_matvec_multi(2, ws3, FAKE + 4, ys, None) == 4          # fp32 x: 16-byte aligned
    for fn in (L.m27q_ffn_swiglu, L.m27q_ffn_swiglu_q8):
        g, u = W(m27q), W(m27q, rc=32)
        assert fn(C.byref(g), C.byref(u), FAKE, FAKE, None, None) == 2
        u = W(m27q, layout=m27q.GGUF)
        assert fn(C.byref(g), C.byref(u), FAKE, FAKE, None, None) == 4
        u = W(m27q, t=m27q.Q6_K)
        assert fn(C.byref(g), C.byref(u), FAKE, FAKE, None, None) == 3
        assert fn(C.byref(g), None, FAKE, FAKE, None, None) == 1
        assert fn(C.byref(g), C.byref(g), None, FAKE, None, None) == 1
        assert fn(C.byref(W(m27q, rc=40)), C.byref(W(m27q, rc=40)), FAKE, FAKE, FAKE, None) == 2


def test_validation_activation_and_scratch(m27q):
    L = m27q.lib()
    assert L.m27q_quant_act(None, 1, 64, FAKE, None) == 1
    assert L.m27q_quant_act(FAKE, 1, 48, FAKE, None) == 2
    assert L.m27q_quant_act(FAKE, 0, 64, FAKE, None) == 2
    assert L.m27q_quant_act(FAKE, 1, 64, FAKE + 8, None) == 4
    assert L.m27q_quant_act_gated(FAKE, None, 1, 64, FAKE, None) == 1
    w = W(m27q)
    assert L.m27q_matvec(C.byref(w), None, FAKE, None, None, None) == 1
    assert L.m27q_matvec(C.byref(w), FAKE, None, None, None, None) == 1
    assert L.m27q_matvec(C.byref(W(m27q, rc=40)), FAKE, FAKE, None, FAKE, None) == 2
    f16 = W(m27q, t=m27q.F16, rb=5120, layout=m27q.GGUF)
    assert L.m27q_matvec(C.byref(f16), FAKE, FAKE, None, FAKE, None) == 3   # no fused quant on fp32 paths
    assert L.m27q_matmul_q8(C.byref(w), 0, FAKE, FAKE, None, None) == 2
    assert L.m27q_matmul_q8(C.byref(w), 65, FAKE, FAKE, None, None) == 2


def test_validation_gather_and_topk(m27q):
    L = m27q.lib()
    w = W(m27q, rc=100)
    assert L.m27q_embed_token(C.byref(w), -1, FAKE, None) == 6
    assert L.m27q_embed_token(C.byref(w), 100, FAKE, None) == 6
    assert L.m27q_embed_rows(C.byref(w), None, 4, FAKE, None, None) == 1
    assert L.m27q_embed_rows(C.byref(w), FAKE, 0, FAKE, None, None) == 2
    assert L.m27q_dequant_rows(C.byref(w), 90, 11, FAKE, None) == 6
    assert L.m27q_dequant_rows(C.byref(w), 0, 1, FAKE + 4, None) == 4
    f16 = W(m27q, t=m27q.F16, rb=12, layout=m27q.GGUF)
    assert L.m27q_dequant_rows(C.byref(f16), 0, 1, FAKE, None) == 2  # F16 rows must be a multiple of 8
    assert L.m27q_topk(FAKE, 100, 65, FAKE, FAKE, FAKE, 1 << 20, None) == 6
    assert L.m27q_topk(FAKE, 10, 11, FAKE, FAKE, FAKE, 1 << 20, None) == 6
    assert L.m27q_topk(FAKE, 10, 0, FAKE, FAKE, FAKE, 1 << 20, None) == 6
    assert L.m27q_topk(FAKE, 248320, 64, FAKE, FAKE, FAKE, 64, None) == 5
    assert L.m27q_topk(None, 10, 1, FAKE, FAKE, FAKE, 1 << 20, None) == 1
    assert m27q.topk_scratch_bytes(248320, 64) >= 64 * 8
    assert L.m27q_sample(FAKE, FAKE, 0, 1.0, 0.05, 0.9, FAKE, FAKE, None) == 6
    assert L.m27q_sample(FAKE, FAKE, 65, 1.0, 0.05, 0.9, FAKE, FAKE, None) == 6
    assert L.m27q_sample(FAKE, FAKE, 40, 1.0, 0.05, 0.0, FAKE, FAKE, None) == 6
    assert L.m27q_sample(None, FAKE, 40, 1.0, 0.05, 0.9, FAKE, FAKE, None) == 1
    assert m27q.topk_scratch_bytes(10, 11) == 0


C_CALLER = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_abi", "_build", "abi_caller")


def test_c_caller_cpu(m27q):
    """A C99 program that includes include/m27q.h and links libm27q.so (as the
    reference's host code would) runs the host-side entry points and the host
    validation of the device entry points."""
    if not os.path.exists(C_CALLER):
        subprocess.run(["make", "-C", os.path.dirname(os.path.dirname(C_CALLER))], check=True,
                       capture_output=True)
    r = subprocess.run([C_CALLER, "--cpu"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "abi_caller: ok" in r.stdout
