"""Pack-time re-tiling of a .m27b blob (m27q_retile_blob), checked with the
reference's own blob code: blobs are written by mono27b_write_stub_blob and the
packer's output is read back by mono27b_validate_blob_file and
mono27b_read_weights_section (src/mono27b_blob.cpp, built into oracle/_ref from
the reference checkout; the test is skipped where that build is absent)."""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import ROOT

REF = os.path.join(ROOT, "oracle", "_ref", "libref_blob.so")

ENTRY = np.dtype([("name", "S64"), ("ggml_type", "<u4"), ("source_model", "<u4"), ("role", "<u4"),
                  ("row_elems", "<u4"), ("row_count", "<u4"), ("reserved", "<u4"),
                  ("data_offset", "<u8"), ("data_bytes", "<u8")])

# name, type, role (1 target matvec, 2 draft matvec, 3 output head, 0 other), row_elems, row_count
TENSORS = [
    ("blk.0.attn_q.weight", 12, 1, 512, 24),
    ("blk.0.ffn_down.weight", 14, 1, 768, 16),
    ("output.weight", 14, 3, 256, 40),
    ("blk.0.attn_norm.weight", 0, 0, 512, 1),
    ("draft.blk.0.ffn_up.weight", 8, 2, 96, 13),
    ("blk.1.attn_gate.weight", 13, 1, 256, 9),
    ("blk.2.ffn_gate.weight", 23, 1, 512, 8),
]


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF):
        pytest.skip("oracle/_ref/libref_blob.so not built (needs the reference checkout at build time)")
    L = C.CDLL(REF)
    L.refblob_write.argtypes = [C.c_char_p, C.c_int, C.c_void_p, C.c_void_p, C.c_ulonglong, C.c_char_p, C.c_int]
    L.refblob_validate.argtypes = [C.c_char_p, C.c_char_p, C.c_int]
    L.refblob_read_entries.argtypes = [C.c_char_p, C.c_void_p, C.c_int, C.c_char_p, C.c_int]
    L.refblob_weights_offset.argtypes = [C.c_char_p]
    assert L.refblob_entry_size() == ENTRY.itemsize
    return L


def write_blob(ref, m27q, path, rng):
    n = len(TENSORS)
    ents = np.zeros(n, ENTRY)
    datas, off = [], 16 + n * ENTRY.itemsize  # payload after the section header and entries
    for i, (name, t, role, re, rc) in enumerate(TENSORS):
        nb = m27q.row_size(t, re) * rc if t not in (0, 1) else re * rc * (4 if t == 0 else 2)
        d = rng.integers(0, 256, nb, dtype=np.uint8)
        ents[i] = (name.encode(), t, 2 if role == 2 else 1, role, re, rc, 0, off, nb)
        datas.append(d)
        off += nb
    payload = np.concatenate(datas)
    err = C.create_string_buffer(256)
    assert ref.refblob_write(path.encode(), n, ents.ctypes.data, payload.ctypes.data, payload.size, err, 256) == 0, err.value
    return ents, datas


def read_entries(ref, path):
    out = np.zeros(64, ENTRY)
    err = C.create_string_buffer(256)
    n = ref.refblob_read_entries(path.encode(), out.ctypes.data, 64, err, 256)
    assert n > 0, err.value
    return out[:n]


def tensor_bytes(path, ref, e):
    base = ref.refblob_weights_offset(path.encode())
    with open(path, "rb") as f:
        f.seek(base + int(e["data_offset"]))
        return np.frombuffer(f.read(int(e["data_bytes"])), np.uint8)


def test_retile_blob_reads_back_with_the_reference_code(m27q, ref, tmp_path):
    src, dst, dst2 = (str(tmp_path / n) for n in ("in.m27b", "out.m27b", "out2.m27b"))
    ents, datas = write_blob(ref, m27q, src, np.random.default_rng(7))
    err = C.create_string_buffer(256)
    assert ref.refblob_validate(src.encode(), err, 256) == 0, err.value
    m27q.retile_blob(src, dst)
    assert ref.refblob_validate(dst.encode(), err, 256) == 0, err.value
    got = read_entries(ref, dst)
    assert len(got) == len(ents)
    for e_in, e_out, d, (name, t, role, re, rc) in zip(ents, got, datas, TENSORS):
        for f in ("name", "ggml_type", "source_model", "role", "row_elems", "row_count"):
            assert e_in[f] == e_out[f]
        assert int(e_out["data_offset"]) % 256 == 0
        data = tensor_bytes(dst, ref, e_out)
        if t in (12, 13, 14, 8, 23):
            rb = re // m27q.BLOCK_ELEMS[t]
            assert e_out["reserved"] == m27q.TILED | TILED_REVISION << 16
            assert e_out["data_bytes"] == m27q.weight_bytes(t, rb, rc, m27q.TILED)
            assert np.array_equal(m27q.unpack(t, rb, rc, data), d), name
        else:
            assert e_out["reserved"] == m27q.GGUF and np.array_equal(data, d), name
    # idempotent: entries already TILED are copied
    m27q.retile_blob(dst, dst2)
    again = read_entries(ref, dst2)
    for a, b in zip(got, again):
        assert a["reserved"] == b["reserved"] and a["data_bytes"] == b["data_bytes"]
        assert np.array_equal(tensor_bytes(dst, ref, a), tensor_bytes(dst2, ref, b))
    # the header, section table and tokenizer section are carried over
    with open(src, "rb") as f1, open(dst, "rb") as f2:
        a, b = f1.read(), f2.read()
    wsec = ref.refblob_weights_offset(src.encode())
    assert a[136 + 24 * 2:wsec] == b[136 + 24 * 2:wsec]


def test_retile_blob_errors(m27q, ref, tmp_path):
    L = m27q.lib()
    p = str(tmp_path / "x.bin")
    with open(p, "wb") as f:
        f.write(b"\x00" * 1024)
    assert L.m27q_retile_blob(p.encode(), str(tmp_path / "y").encode()) == 8
    assert L.m27q_retile_blob(str(tmp_path / "missing").encode(), str(tmp_path / "y").encode()) == 8
    assert L.m27q_retile_blob(p.encode(), p.encode()) == 8
    assert L.m27q_retile_blob(None, p.encode()) == 1


def test_blob_tensors_match_the_reference_reader(m27q, ref, tmp_path):
    """m27q_blob_tensors on a re-tiled blob gives the entries the reference's
    mono27b_read_weights_section reads, with the layout from the reserved
    field, WeightView's row_blocks and absolute file offsets."""
    src, dst = str(tmp_path / "in.m27b"), str(tmp_path / "out.m27b")
    write_blob(ref, m27q, src, np.random.default_rng(9))
    m27q.retile_blob(src, dst)
    for path in (src, dst):
        want = read_entries(ref, path)
        got = m27q.blob_tensors(path)
        base = ref.refblob_weights_offset(path.encode())
        assert len(got) == len(want)
        for g, w, (name, t, role, re, rc) in zip(got, want, TENSORS):
            assert g.name == w["name"] and g.ggml_type == w["ggml_type"] and g.role == w["role"]
            assert g.source_model == w["source_model"] and g.row_elems == re and g.row_count == rc
            assert g.layout == w["reserved"] & 0xffff and g.bytes == w["data_bytes"]
            assert g.file_offset == base + int(w["data_offset"])
            assert g.row_blocks == re // m27q.BLOCK_ELEMS[t]
            assert g.bytes == m27q.weight_bytes(t, g.row_blocks, rc, g.layout)


ENTRY_OFF_RESERVED, ENTRY_OFF_DATA_OFFSET, ENTRY_OFF_DATA_BYTES = 84, 88, 96
TILED_REVISION = 2  # the TILED byte order with the Q4_K / Q5_K qs plane chunk pair first


def _patch_entry(path, ref, i, field_off, value, nbytes=8):
    base = ref.refblob_weights_offset(path.encode())
    with open(path, "r+b") as f:
        f.seek(base + 16 + i * ENTRY.itemsize + field_off)
        f.write(int(value).to_bytes(nbytes, "little"))


def test_blob_tiled_entry_of_another_revision_is_not_loadable(m27q, ref, tmp_path):
    """A TILED entry whose reserved field carries another revision of the TILED
    byte order (here the first, tag 1) is listed with row_blocks 0, which
    m27q_blob_load refuses, instead of being read in the wrong order."""
    src, dst = str(tmp_path / "in.m27b"), str(tmp_path / "out.m27b")
    write_blob(ref, m27q, src, np.random.default_rng(11))
    m27q.retile_blob(src, dst)
    ents = read_entries(ref, dst)
    i = next(k for k, e in enumerate(ents) if e["reserved"] == m27q.TILED | TILED_REVISION << 16)
    _patch_entry(dst, ref, i, ENTRY_OFF_RESERVED, m27q.TILED, nbytes=4)
    t = m27q.blob_tensors(dst)[i]
    assert t.layout == m27q.TILED and t.row_blocks == 0
    w = m27q.WeightDesc()
    assert m27q.lib().m27q_blob_load(dst.encode(), C.byref(t), 1 << 20, int(t.bytes), C.byref(w)) == 3


@pytest.mark.parametrize("field_off,value", [
    (ENTRY_OFF_DATA_OFFSET, 2 ** 64 - 8),     # offset + bytes wraps around
    (ENTRY_OFF_DATA_BYTES, 2 ** 64 - 1),      # bytes alone wraps
    (ENTRY_OFF_DATA_OFFSET, 1 << 40),         # past the section
])
def test_blob_readers_reject_out_of_range_entries(m27q, ref, tmp_path, field_off, value):
    src = str(tmp_path / "in.m27b")
    write_blob(ref, m27q, src, np.random.default_rng(10))
    _patch_entry(src, ref, 2, field_off, value)
    L = m27q.lib()
    n = C.c_int(0)
    assert L.m27q_blob_tensors(src.encode(), None, 0, C.byref(n)) == 8
    assert L.m27q_retile_blob(src.encode(), str(tmp_path / "o.m27b").encode()) == 8


def test_blob_load_checks_before_any_copy(m27q, ref, tmp_path):
    """m27q_blob_load validates the record and the destination size on the host
    and returns before any HIP call (no GPU needed for these)."""
    src = str(tmp_path / "in.m27b")
    write_blob(ref, m27q, src, np.random.default_rng(12))
    ts = m27q.blob_tensors(src)
    L = m27q.lib()
    w = m27q.WeightDesc()
    fake = 1 << 20  # never dereferenced: every case below fails its host check first
    t = m27q.BlobTensor.from_buffer_copy(ts[0])
    assert L.m27q_blob_load(src.encode(), C.byref(t), fake, int(t.bytes) - 1, C.byref(w)) == 2
    t.layout = 7
    assert L.m27q_blob_load(src.encode(), C.byref(t), fake, int(t.bytes), C.byref(w)) == 4
    t = m27q.BlobTensor.from_buffer_copy(ts[0])
    t.row_blocks = 0
    assert L.m27q_blob_load(src.encode(), C.byref(t), fake, int(t.bytes), C.byref(w)) == 3
    t = m27q.BlobTensor.from_buffer_copy(ts[0])
    t.bytes += 1
    assert L.m27q_blob_load(src.encode(), C.byref(t), fake, int(t.bytes), C.byref(w)) == 2
    assert L.m27q_blob_load(src.encode(), C.byref(ts[0]), None, 10 ** 9, C.byref(w)) == 1
