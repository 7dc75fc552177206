"""Activation quantization on the GPU vs the oracle: bit-exact codes, scales, sums."""
import numpy as np
import pytest

from gpu_util import act_host, say, to_dev

pytestmark = pytest.mark.gpu


def edge_rows(k):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((7, k)).astype(np.float32)
    x[0, :64] = 0.0                                   # all-zero groups
    x[1, :32] = 127.0 * np.arange(32) / 31.0          # exact multiples of d
    x[1, 32:64] = np.float32(127.0)
    x[1, 33:39] = [2.5, -2.5, 0.5, -0.5, 1.5, 126.5]  # ties: round half away from zero
    x[2] *= np.float32(1e-30)                          # tiny values
    x[3] *= np.float32(1e30)                           # huge values
    x[4, ::2] = -x[4, ::2]
    x[5, :32] = -0.0
    # d = 1 again: values beside the ties and beside 0.5 (the largest float
    # below 0.5 must give 0, 0.5 itself 1) and subnormal inputs.  (A group
    # whose amax is below ~3.7e-37 has a subnormal d and an infinite 1/d; the
    # codes of such a group are outside the defined range of the rule.)
    x[6, :32] = np.float32(127.0)
    x[6, 1:16] = np.array([0.49999997, -0.49999997, 0.50000006, -0.50000006, 1.4999999, -1.4999999, 2.4999998,
                           -2.4999998, 125.49999, -125.49999, 126.50001, -0.0, 1e-40, -1e-40, 3.5],
                          dtype=np.float32)
    return x


@pytest.mark.parametrize("M,K", [(1, 5120), (4, 6144), (16, 17408), (7, 256)])
def test_quant_act_bitexact(m27q, ora, dev, M, K):
    rng = np.random.default_rng(M * 1000 + K)
    x = (rng.standard_normal((M, K)) * 10.0 ** rng.integers(-3, 4, (M, 1))).astype(np.float32)
    if M == 7:
        x = edge_rows(K)
    say("quant_act", M, K)
    act = m27q.Act(M, K, dev)
    m27q.quant_act(to_dev(x, dev), act)
    q, d, s = act_host(m27q, act)
    qo, do, so = ora.quant_act(x)
    assert np.array_equal(q, qo)
    assert np.array_equal(d.view(np.uint32), do.view(np.uint32))
    assert np.array_equal(s, so)


def test_quant_act_gated_close(m27q, ora, dev):
    """x * sigmoid(g): the device and host expf may differ in the last bit, so a
    code may move by one where x*sigmoid(g)/d sits at a rounding tie."""
    rng = np.random.default_rng(3)
    M, K = 2, 6144
    x = rng.standard_normal((M, K)).astype(np.float32)
    g = rng.standard_normal((M, K)).astype(np.float32) * 3
    say("quant_act_gated", M, K)
    act = m27q.Act(M, K, dev)
    m27q.quant_act(to_dev(x, dev), act, gate=to_dev(g, dev))
    q, d, s = act_host(m27q, act)
    qo, do, so = ora.quant_act_gated(x, g)
    assert np.abs(q.astype(int) - qo.astype(int)).max() <= 1
    assert (q != qo).mean() < 1e-3
    assert np.allclose(d, do, rtol=1e-6, atol=0)
