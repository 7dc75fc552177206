"""m27q_topk_noalloc (top-k on the library's static per-device scratch) against
m27q_topk (caller scratch) through the C ABI: two calls in a row, the second
on a smaller input, each bit-identical; limits rejected on the host."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import say, to_dev, to_host


def _topk_both(m27q, dev, v, k):
    import torch
    idx = torch.empty(k, dtype=torch.int32, device=dev)
    val = torch.empty(k, dtype=torch.float32, device=dev)
    idx0 = torch.full((k,), -7, dtype=torch.int32, device=dev)
    val0 = torch.full((k,), -7.0, dtype=torch.float32, device=dev)
    lg = to_dev(v, dev)
    scratch = torch.empty(m27q.topk_scratch_bytes(v.size, k), dtype=torch.uint8, device=dev)
    m27q.topk(lg, k, idx, val, scratch)
    m27q.topk_noalloc(lg, k, idx0, val0)
    return (to_host(idx), to_host(val)), (to_host(idx0), to_host(val0))


@pytest.mark.gpu
def test_topk_noalloc_matches_topk(m27q, ora, dev):
    rng = np.random.default_rng(31)
    big = rng.standard_normal(248320).astype(np.float32)
    small = np.round(rng.standard_normal(5000) * 2).astype(np.float32)  # ties
    for v, k in ((big, 64), (small, 40), (big[:4097].copy(), 1)):
        say("topk_noalloc", v.size, k)
        (i1, v1), (i2, v2) = _topk_both(m27q, dev, v, k)
        assert np.array_equal(i1, i2) and np.array_equal(v1.view(np.uint32), v2.view(np.uint32))
        oi, ov = ora.topk(v, k)
        assert np.array_equal(i2, oi) and np.array_equal(v2.view(np.uint32), ov.view(np.uint32))


def test_topk_noalloc_limits(m27q):
    """Checked on the host before any HIP call (no GPU needed)."""
    L = m27q.lib()
    fake = 0x10000
    assert L.m27q_topk_noalloc(fake, (1 << 24) + 1, 8, fake, fake, None) == 5   # beyond the static scratch
    assert L.m27q_topk_noalloc(fake, 100, 65, fake, fake, None) == 6
    assert L.m27q_topk_noalloc(fake, 10, 11, fake, fake, None) == 6
    assert L.m27q_topk_noalloc(fake, 0, 1, fake, fake, None) == 2
    assert L.m27q_topk_noalloc(None, 10, 1, fake, fake, None) == 1
