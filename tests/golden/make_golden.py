"""Writes tests/golden/q4k_kat.json from the reference checkout.

Input bytes: the 32-byte Q4_K block prefix held in the reference's
debug/official_dequant.c:71-74 (d = 0x04ED, dmin = 0x1039, scales[12],
qs[0..16)).  Expected values: column 11 of debug/mono_give_current.debug.tsv:2,
the first 16 fp32 values the reference's GPU embed wrote for that block
(token 44883).  Both are data held by the reference's own files; this script
only transcribes them.  Run once, in a container that has /root/reference.
"""
import json
import os
import re

REF = os.environ.get("M27Q_REFERENCE", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    src = open(os.path.join(REF, "debug", "official_dequant.c")).read()
    arr = re.search(r"uint8_t bytes\[\] = \{(.*?)\};", src, re.S).group(1)
    block = [int(v, 16) for v in re.findall(r"0x([0-9a-fA-F]{2})", arr)]
    assert len(block) == 32
    line = open(os.path.join(REF, "debug", "mono_give_current.debug.tsv")).read().splitlines()[1]
    cols = line.split("\t")
    assert cols[0] == "embed" and cols[4] == "h"
    values = [float(v) for v in cols[10].split(",")]
    assert len(values) == 16
    out = {
        "source_bytes": "debug/official_dequant.c:71-74",
        "source_values": "debug/mono_give_current.debug.tsv:2 column 11",
        "block_prefix_hex": bytes(block).hex(),
        "expected_first16": values,
    }
    with open(os.path.join(HERE, "q4k_kat.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
