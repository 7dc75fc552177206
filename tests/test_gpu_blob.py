"""The loader of re-tiled .m27b blobs (m27q_blob_tensors / m27q_blob_load) on
the GPU: a blob written by the reference's own writer (mono27b_write_stub_blob,
built into oracle/_ref from the reference checkout) with Q4_K, Q5_K, Q6_K, Q8_0
and IQ4_XS matrices is re-tiled, its tensors are uploaded by the loader, and
every product on them matches the oracle; the un-tiled blob loads as GGUF
layout and gives the same products."""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import ROOT
from gpu_util import int_dot_tol, say, to_dev, to_host

pytestmark = pytest.mark.gpu

REF = os.path.join(ROOT, "oracle", "_ref", "libref_blob.so")
ENTRY = np.dtype([("name", "S64"), ("ggml_type", "<u4"), ("source_model", "<u4"), ("role", "<u4"),
                  ("row_elems", "<u4"), ("row_count", "<u4"), ("reserved", "<u4"),
                  ("data_offset", "<u8"), ("data_bytes", "<u8")])

# name, type, row_elems (K), row_count
MATS = [("blk.0.attn_q.weight", 12, 1024, 64), ("blk.0.ffn_down.weight", 14, 768, 40),
        ("blk.0.attn_gate.weight", 13, 512, 24), ("draft.blk.0.ffn_up.weight", 8, 2048, 24),
        ("blk.0.ffn_gate.weight", 23, 512, 16), ("output.weight", 14, 256, 72)]


def write_blob(ora, path):
    L = C.CDLL(REF)
    L.refblob_write.argtypes = [C.c_char_p, C.c_int, C.c_void_p, C.c_void_p, C.c_ulonglong, C.c_char_p, C.c_int]
    n = len(MATS)
    ents = np.zeros(n, ENTRY)
    datas, off = [], 16 + n * ENTRY.itemsize
    for i, (name, t, k, rc) in enumerate(MATS):
        d = ora.synth_weights(t, rc, k, seed=60 + i).reshape(-1)
        ents[i] = (name.encode(), t, 1, 1, k, rc, 0, off, d.size)
        datas.append(d)
        off += d.size
    payload = np.concatenate(datas)
    err = C.create_string_buffer(256)
    assert L.refblob_write(path.encode(), n, ents.ctypes.data, payload.ctypes.data, payload.size, err, 256) == 0, \
        err.value
    return datas


def test_loader_products_match_oracle(m27q, ora, dev, tmp_path):
    if not os.path.exists(REF):
        pytest.skip("oracle/_ref/libref_blob.so not built (needs the reference checkout at build time)")
    import torch
    src, dst = str(tmp_path / "in.m27b"), str(tmp_path / "tiled.m27b")
    datas = write_blob(ora, src)
    m27q.retile_blob(src, dst)
    rng = np.random.default_rng(61)
    for path, layout in ((dst, m27q.TILED), (src, m27q.GGUF)):
        ts = m27q.blob_tensors(path)
        assert [t.name.decode() for t in ts] == [m[0] for m in MATS]
        for t, d, (name, ty, k, rc) in zip(ts, datas, MATS):
            assert t.layout == layout and t.ggml_type == ty and t.row_count == rc
            say("blob load", name, layout)
            w = m27q.blob_load(path, t, dev)
            assert (w.type, w.rb, w.rc, w.layout) == (ty, k // ora.BLOCK_ELEMS[ty], rc, layout)
            x = rng.standard_normal(k).astype(np.float32)
            y = torch.empty(rc, dtype=torch.float32, device=dev)
            m27q.matvec(w, to_dev(x, dev), y)
            q, dd, s = ora.quant_act(x)
            want, nrm = ora.gemv_act(ty, d, w.rb, rc, q, dd, s)
            assert (np.abs(to_host(y) - want) <= int_dot_tol(nrm)).all(), name
            # the uploaded bytes are the blob's: unpacking them gives the GGUF rows back
            raw = to_host(w.data)
            back = m27q.unpack(ty, w.rb, rc, raw) if layout == m27q.TILED else raw[:d.size]
            assert np.array_equal(back, d), name
