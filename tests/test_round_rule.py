"""The device quantizer's rounding rule equals roundf on every float it can see.

quant_code (m27q_device.h) rounds v = x * id as (int)(v + copysign(0.49999997f, v))
instead of (int)roundf(v): three instructions instead of seven.  round_rule.c
checks the two against each other for all 2,516,582,400 floats with |v| < 2^23
(|v| <= 127.00002 in use), so the codes stay bit-identical to the oracle's."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def test_round_rule_exhaustive(tmp_path):
    exe = str(tmp_path / "round_rule")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, os.path.join(HERE, "round_rule.c"), "-lm"],
                   check=True)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout
    assert "2516582400 values, 0 mismatches" in out.stdout
