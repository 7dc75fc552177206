"""Activation quantization on the GPU vs the oracle: bit-exact codes, scales, sums."""
import numpy as np
import pytest

from gpu_util import act_host, say, to_dev

pytestmark = pytest.mark.gpu


def edge_rows(k):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((8, k)).astype(np.float32)
    x[0, :64] = 0.0                                   # all-zero groups
    x[1, :32] = 127.0 * np.arange(32) / 31.0          # exact multiples of d
    x[1, 32:64] = np.float32(127.0)
    x[1, 33:39] = [2.5, -2.5, 0.5, -0.5, 1.5, 126.5]  # ties: round half away from zero
    x[2] *= np.float32(1e-30)                          # tiny values
    x[3] *= np.float32(1e30)                           # huge values
    x[4, ::2] = -x[4, ::2]
    x[5, :32] = -0.0
    # NaN: out of the group's amax, code 0; a group of NaNs has d = 0
    x[5, 64:72] = np.nan
    x[5, 96:128] = np.nan
    # d = 1 again: values beside the ties and beside 0.5 (the largest float
    # below 0.5 must give 0, 0.5 itself 1) and subnormal inputs
    x[6, :32] = np.float32(127.0)
    x[6, 1:16] = np.array([0.49999997, -0.49999997, 0.50000006, -0.50000006, 1.4999999, -1.4999999, 2.4999998,
                           -2.4999998, 125.49999, -125.49999, 126.50001, -0.0, 1e-40, -1e-40, 3.5],
                          dtype=np.float32)
    # subnormal scales: 1/d infinite (all codes 0), and 1/d finite (codes as usual)
    x[7, :32] = np.float32(1e-40) * np.arange(-16, 16, dtype=np.float32)
    x[7, 32:64] = np.float32(5e-37) * np.linspace(-1, 1, 32, dtype=np.float32)
    x[7, 64:96] = np.float32(1e-45)
    return x


@pytest.mark.parametrize("M,K", [(1, 5120), (4, 6144), (16, 17408), (8, 256)])
def test_quant_act_bitexact(m27q, ora, dev, M, K):
    rng = np.random.default_rng(M * 1000 + K)
    x = (rng.standard_normal((M, K)) * 10.0 ** rng.integers(-3, 4, (M, 1))).astype(np.float32)
    if M == 8:
        x = edge_rows(K)
    say("quant_act", M, K)
    act = m27q.Act(M, K, dev)
    m27q.quant_act(to_dev(x, dev), act)
    q, d, s = act_host(m27q, act)
    qo, do, so = ora.quant_act(x)
    assert np.array_equal(q, qo)
    assert np.array_equal(d.view(np.uint32), do.view(np.uint32))
    assert np.array_equal(s, so)


def gate_values(M, K, seed):
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    g[0, :8] = [0.0, -0.0, 87.0, -87.0, 90.0, -90.0, 1e4, -1e4]   # around and past the exp clamp
    g[0, 8:12] = [17.0, -17.0, 1e-30, -1e-30]
    g[0, 12:14] = np.nan   # NaN gates give NaN values (code 0), not x
    g[0, 32:64] = np.nan   # a group of them: d = 0
    return g


@pytest.mark.parametrize("M,K", [(2, 6144), (8, 256)])
def test_quant_act_gated_bitexact(m27q, ora, dev, M, K):
    """x * sigmoid(g): one exp (Cody-Waite + polynomial) on both sides, so the
    codes, scales and code sums are bit-identical."""
    x = edge_rows(K) if M == 8 else np.random.default_rng(3).standard_normal((M, K)).astype(np.float32)
    g = gate_values(M, K, 4)
    say("quant_act_gated", M, K)
    act = m27q.Act(M, K, dev)
    m27q.quant_act(to_dev(x, dev), act, gate=to_dev(g, dev))
    q, d, s = act_host(m27q, act)
    qo, do, so = ora.quant_act_gated(x, g)
    assert np.array_equal(q, qo)
    assert np.array_equal(d.view(np.uint32), do.view(np.uint32))
    assert np.array_equal(s, so)


@pytest.mark.parametrize("gated", [False, True])
def test_quant_act_unaligned_bitexact(m27q, ora, dev, gated):
    """x and gate only 4-byte aligned (one float into a buffer): the quantizer's
    scalar path, bit-identical to the oracle."""
    import torch
    M, K = 3, 5120
    rng = np.random.default_rng(17)
    x = (rng.standard_normal((M, K)) * 4).astype(np.float32)
    g = gate_values(M, K, 18)
    xb = torch.zeros(M * K + 4, dtype=torch.float32, device=dev)
    gb = torch.zeros(M * K + 4, dtype=torch.float32, device=dev)
    xb[1:1 + M * K] = to_dev(x.reshape(-1), dev)
    gb[3:3 + M * K] = to_dev(g.reshape(-1), dev)
    xv, gv = xb[1:1 + M * K], gb[3:3 + M * K]
    assert xv.data_ptr() % 16 == 4 and gv.data_ptr() % 16 == 12
    say("quant_act unaligned", gated)
    act = m27q.Act(M, K, dev)
    m27q.quant_act(xv, act, gate=gv if gated else None)
    q, d, s = act_host(m27q, act)
    qo, do, so = ora.quant_act_gated(x, g) if gated else ora.quant_act(x)
    assert np.array_equal(q, qo)
    assert np.array_equal(d.view(np.uint32), do.view(np.uint32))
    assert np.array_equal(s, so)
