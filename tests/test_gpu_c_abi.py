"""The C99 caller of include/m27q.h (tests/c_abi/abi_caller.c, linked against
libm27q.so by gcc) runs Q4_K, Q6_K and Q8_0 products on the GPU through the C
ABI: fp32 x on TILED weights, quantized x on TILED and on GGUF weights, each
within 1e-5 of sum |terms| of the library's bit-exact dequantization dotted
with the dequantized activation codes; and a token row gathered from GGUF
weights equals the row dequantized from TILED ones, bit for bit."""
import os
import subprocess

import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu

C_CALLER = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_abi", "_build", "abi_caller")


def test_c_caller_gpu():
    assert os.path.exists(C_CALLER), f"{C_CALLER} is not built (make -C tests/c_abi)"
    say("C caller --gpu")
    r = subprocess.run([C_CALLER, "--gpu"], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "abi_caller: ok (cpu and gpu checks)" in r.stdout
