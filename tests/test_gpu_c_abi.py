"""The C ABI from a plain C host (tests/c_abi/abi_consumer.c, built by
__graft_entry__.build() with gcc): upload, dequantize, QMatMul::forward on the
GEMV and GEMM paths and an error return, called the way candle's Rust FFI arm
would call include/moldq.h, with no Python or torch in the process."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "c_abi", "abi_consumer")


def test_plain_c_caller_through_the_abi():
    assert os.path.exists(BIN), "tests/c_abi/abi_consumer is not built: run __graft_entry__.build()"
    print("[c-abi] running tests/c_abi/abi_consumer", flush=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    assert "dequantize Q8_0 [192, 512] bit-exact" in r.stdout
    assert r.stdout.strip().splitlines()[-1] == "abi consumer: ok"
