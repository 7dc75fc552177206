"""Dequantization and row gather on the GPU: bit-exact against the oracle."""
import numpy as np
import pytest

from gpu_util import say, to_dev, to_host
from test_oracle import random_blocks

pytestmark = pytest.mark.gpu

TYPES = ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "IQ4_XS"]


@pytest.mark.parametrize("type_name", TYPES)
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("rb,rc", [(1, 1), (20, 13), (3, 40)])
def test_dequant_rows_bitexact(m27q, ora, dev, type_name, layout, rb, rc):
    t = getattr(m27q, type_name)
    if t == m27q.Q8_0:
        rb *= 5  # 5, 100, 15 blocks: exercises partial Q8_0 units
    blocks = random_blocks(ora, t, rb * rc, np.random.default_rng(rb * 31 + rc + layout))
    w = m27q.Weight.upload(blocks.reshape(-1), t, rb, rc, layout, dev)
    import torch
    out = torch.empty((rc, w.K), dtype=torch.float32, device=dev)
    say("dequant_rows", type_name, layout, rb, rc)
    m27q.dequant_rows(w, 0, rc, out)
    got = to_host(out)
    want = ora.dequant(t, blocks, rb, rc)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # a row window
    if rc > 3:
        out2 = torch.empty((2, w.K), dtype=torch.float32, device=dev)
        m27q.dequant_rows(w, rc - 3, 2, out2)
        assert np.array_equal(to_host(out2).view(np.uint32), want[rc - 3:rc - 1].view(np.uint32))


def test_q4k_known_answer_on_gpu(m27q, ora, dev):
    import json
    import os
    from conftest import GOLDEN
    kat = json.load(open(os.path.join(GOLDEN, "q4k_kat.json")))
    blk = np.zeros(144, np.uint8)
    blk[:32] = np.frombuffer(bytes.fromhex(kat["block_prefix_hex"]), np.uint8)
    import torch
    for layout in (0, 1):
        w = m27q.Weight.upload(blk, m27q.Q4_K, 1, 1, layout, dev)
        out = torch.empty(256, dtype=torch.float32, device=dev)
        say("q4k KAT", layout)
        m27q.embed_token(w, 0, out)
        got = to_host(out)[:16]
        assert np.array_equal(got.view(np.uint32), np.array(kat["expected_first16"], np.float32).view(np.uint32))


@pytest.mark.parametrize("type_name", TYPES)
@pytest.mark.parametrize("layout", [0, 1])
def test_embed_rows_with_bad_ids(m27q, ora, dev, type_name, layout):
    import torch
    t = getattr(m27q, type_name)
    rb, rc = (20, 300) if t != m27q.Q8_0 else (64, 300)
    blocks = random_blocks(ora, t, rb * rc, np.random.default_rng(5))
    w = m27q.Weight.upload(blocks.reshape(-1), t, rb, rc, layout, dev)
    rng = np.random.default_rng(6)
    ids = rng.integers(0, rc, 64).astype(np.int32)
    ids[[3, 17, 40]] = [-1, rc, 1 << 30]
    out = torch.full((64, w.K), 7.0, dtype=torch.float32, device=dev)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    say("embed_rows", type_name, layout)
    m27q.embed_rows(w, to_dev(ids, dev), out, bad)
    got = to_host(out)
    assert to_host(bad)[0] == 3
    want = ora.dequant(t, blocks, rb, rc)
    for i, r in enumerate(ids):
        if 0 <= r < rc:
            assert np.array_equal(got[i].view(np.uint32), want[r].view(np.uint32)), i
        else:
            assert (got[i] == 0).all()


@pytest.mark.parametrize("type_name", ["F16", "F32"])
def test_dense_rows(m27q, ora, dev, type_name):
    import torch
    t = getattr(m27q, type_name)
    K, rc = 5120, 48
    w32 = np.random.default_rng(2).standard_normal((rc, K)).astype(np.float32)
    raw = ora.quantize(t, w32)
    w = m27q.Weight.upload(raw.reshape(-1), t, K, rc, m27q.GGUF, dev)
    out = torch.empty((rc, K), dtype=torch.float32, device=dev)
    say("dense dequant", type_name)
    m27q.dequant_rows(w, 0, rc, out)
    assert np.array_equal(to_host(out).view(np.uint32), ora.dequant(t, raw, K, rc).view(np.uint32))


def test_vocab_gather_full_size(m27q, ora, dev):
    """Config-5 gather: 512 seeded ids from a 248320 x 5120 Q6_K table (random valid
    blocks built on the device); each gathered row checked bit-exactly."""
    import torch
    rb, rc = 20, 248320
    g = torch.Generator(device=dev)
    g.manual_seed(21)
    raw = torch.randint(0, 256, (rc * rb, 210), dtype=torch.uint8, device=dev, generator=g)
    raw[:, 208] = 0x1f  # d = 0x0a1f: a normal fp16 (~1.2e-4)
    raw[:, 209] = 0x0a
    w = m27q.Weight(raw.reshape(-1), m27q.Q6_K, rb, rc, m27q.GGUF)
    ids = np.random.default_rng(21).integers(0, rc, 512).astype(np.int32)
    out = torch.empty((512, 5120), dtype=torch.float32, device=dev)
    say("vocab gather 512 rows")
    m27q.embed_rows(w, to_dev(ids, dev), out)
    got = to_host(out)
    host = raw.view(rc, rb * 210)[torch.from_numpy(ids).long().to(dev)].cpu().numpy()
    want = ora.dequant(m27q.Q6_K, host, rb, 512)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
