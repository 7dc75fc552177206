"""The device quantizer's two shortcuts equal the rules they replace on every input.

quant_code (m27q_device.h) rounds v = x * id as (int)(v + copysign(0.49999997f, v))
instead of (int)roundf(v), and div127 computes amax / 127 as a multiply and one
FMA correction instead of an IEEE divide.  round_rule.c checks the first over
all 2,516,582,400 floats with |v| < 2^23 (|v| <= 127.00002 in use) and the
second over all 2,139,095,040 non-negative finite floats, so the codes and
scales stay bit-identical to the oracle's."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def test_round_rule_exhaustive(tmp_path):
    exe = str(tmp_path / "round_rule")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp", "-o", exe, os.path.join(HERE, "round_rule.c"),
                    "-lm"], check=True)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout
    assert "round: 2516582400 values, 0 mismatches" in out.stdout
    assert "div127: 2139095040 values, 0 mismatches" in out.stdout
