"""The bench line's contract on the CPU: the algorithmic bytes behind
roofline.achieved and the layer's GB/s, and the single-GPU refusal.

The byte counts are written out from the GGUF block sizes (Q4_K 144 B and
Q6_K 210 B per 256 weights) and the layer's shapes, so a wrong shape, block
size or term in bench.stage_bytes fails here."""
import os
import subprocess
import sys

from conftest import ROOT

sys.path.insert(0, ROOT)


def q4k(rows, k):
    return rows * (k // 256) * 144


def q6k(rows, k):
    return rows * (k // 256) * 210


def test_stage_bytes_written_out():
    import bench
    m27q = bench.load_pkg()
    want = {
        # weights + fp32 x in + fp32 y out (+ fp32 residual read)
        "qkv": q4k(6144 + 1024 + 1024, 5120) + 4 * 5120 + 4 * (6144 + 1024 + 1024),
        "o": q4k(5120, 6144) + 4 * 6144 + 4 * 5120 + 4 * 5120,
        "gate_up": 2 * q4k(17408, 5120) + 4 * 5120 + 4 * 17408,
        "down": q6k(5120, 17408) + 4 * 17408 + 4 * 5120 + 4 * 5120,
    }
    got = {n: bench.stage_bytes(m27q, n) for n in want}
    assert got == want
    assert got["gate_up"] == 100_360_192
    # the layer's weight bytes and config 1's, as the survey of the workload gives them
    assert sum(q4k(r, k) for r, k in ((6144, 5120), (1024, 5120), (1024, 5120), (5120, 6144),
                                        (17408, 5120), (17408, 5120))) + q6k(5120, 17408) == 214_671_360
    assert q4k(17408, 5120) == 50_135_040


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in (r.stdout + r.stderr)


def test_layer_bytes_and_source_stamp():
    """LAYER_BYTES (behind value and the suite's layer figures) from the block
    sizes; the source stamp that gates the profile-read kernel time is a
    stable 16-hex-digit digest."""
    import bench
    assert bench.LAYER_BYTES == 214_671_360
    h = bench.source_hash()
    assert len(h) == 16 and int(h, 16) >= 0 and h == bench.source_hash()
