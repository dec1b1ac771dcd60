"""Host C/C++ under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only).

tests/sanitize/Makefile builds, with gcc/g++ and -fsanitize=address,undefined:
  * the GGUF reader/writer of libmoldq (mold_amd/csrc/mq_gguf.cpp), which parses
    untrusted files, into gguf_driver: a valid round trip, every truncation of a
    valid file, crafted headers whose counts and string lengths claim more than
    the file holds (u8 arrays of 2^29, string arrays of 2^26 and 2^63, 2^64-1
    byte strings, arrays nested 200 deep) and 3000 seeded mutations;
  * the oracle (oracle/ggml_oracle.c) into oracle_driver: every entry point on
    random and adversarial inputs.
Any out-of-bounds access, leak or undefined behaviour fails the run.
"""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
OUT = os.path.join(ROOT, "_build", "sanitize")
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1:abort_on_error=0",
           UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
ENV.pop("LD_PRELOAD", None)


@pytest.fixture(scope="module")
def built():
    subprocess.run(["make", "-s", "-C", os.path.join(HERE, "sanitize"), f"OUT={OUT}"], check=True)
    return OUT


def _run(exe, *args):
    r = subprocess.run([exe, *args], env=ENV, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    return r.stdout


def test_gguf_reader_writer_under_asan_ubsan(built):
    out = _run(os.path.join(built, "gguf_driver"))
    assert "gguf_driver: ok" in out, out


def test_oracle_under_asan_ubsan(built):
    out = _run(os.path.join(built, "oracle_driver"))
    assert "oracle_driver: ok" in out, out


def test_sanitizer_stub_geometry_matches_library(built):
    """The driver links a host stand-in for mq_block_size / mq_type_size; it must
    agree with the built library for every id (unknown ids included)."""
    import mold_amd
    lib = mold_amd.load()
    rows = [tuple(map(int, ln.split())) for ln in _run(os.path.join(built, "gguf_driver"), "table").splitlines()]
    assert len(rows) == 17
    for dt, bs, ts in rows:
        assert (lib.mq_block_size(dt), lib.mq_type_size(dt)) == (bs, ts), dt
