"""mq_qmatmul_noalloc against mq_qmatmul, on the GPU through the C ABI.

The no-allocation entry point shares mq_qmatmul's kernels and takes its
scratch from a fixed per-GPU device array, so its outputs must be
bit-identical to mq_qmatmul's on the same inputs.  Each case makes two calls
in a row on one stream, the second with fewer rows, so the second call runs
over scratch that still holds the first call's (larger) contents.
"""
import ctypes
import sys

import numpy as np
import pytest

import mold_amd
from mold_amd import GgmlDType, QTensor, _lib
from oracle import oracle as O

pytestmark = pytest.mark.gpu

MQ_F32, MQ_BF16 = 0, 30
MQ_E_INVALID = -1


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as _t
    return _t


@pytest.fixture(scope="module")
def dev(torch):
    return mold_amd.Device(0)


def _call(fn, dev, qt, x, y, bias=None, act=0):
    torch = sys.modules["torch"]
    xt = MQ_BF16 if x.dtype == torch.bfloat16 else MQ_F32
    yt = MQ_BF16 if y.dtype == torch.bfloat16 else MQ_F32
    return fn(dev.handle, qt.handle, x.data_ptr(), xt, x.shape[0], x.stride(0), y.data_ptr(), yt, y.stride(0),
              bias.data_ptr() if bias is not None else None, act,
              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


# (type, n, k, m_first, m_second, x dtype, y dtype, act): GEMM with staged f32 x and
# split-K tail partials, GEMM reading bf16 x in place, generic GEMV with staged x,
# the Q4_K GEMV reading x in place.
CASES = [
    ("Q4_K", 1536, 3072, 1000, 300, "f32", "f32", 0),
    ("Q6_K", 1536, 4096, 2300, 700, "bf16", "bf16", 1),
    ("Q8_0", 2048, 3072, 8, 3, "bf16", "f32", 0),
    ("Q4_K", 4096, 3072, 4, 1, "f32", "f32", 0),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-n{c[1]}-k{c[2]}-m{c[3]}then{c[4]}-{c[5]}")
def test_noalloc_matches_qmatmul_two_calls(dev, torch, case):
    tname, n, k, m1, m2, xdt, ydt, act = case
    _say(f"noalloc {case}")
    lib = _lib.load()
    t = GgmlDType[tname]
    w = (np.random.default_rng(n + k).standard_normal((n, k)) * 0.02).astype(np.float32)
    qt = QTensor.from_blocks(dev, t, (n, k), O.quantize(int(t), w))
    bias = torch.from_numpy((np.random.default_rng(1).standard_normal(n) * 0.02).astype(np.float32)).cuda()
    xd = torch.float32 if xdt == "f32" else torch.bfloat16
    yd = torch.float32 if ydt == "f32" else torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(m1 + m2)
    for m in (m1, m2):
        x = torch.randn((m, k), device="cuda", generator=g).to(xd)
        y_ref = torch.full((m, n), float("nan"), device="cuda", dtype=yd)
        y = torch.full((m, n), float("nan"), device="cuda", dtype=yd)
        assert _call(lib.mq_qmatmul, dev, qt, x, y_ref, bias, act) == 0, _lib.load().mq_last_error()
        assert _call(lib.mq_qmatmul_noalloc, dev, qt, x, y, bias, act) == 0, _lib.load().mq_last_error()
        torch.cuda.synchronize()
        iv = torch.int32 if yd == torch.float32 else torch.int16
        assert torch.equal(y.view(iv), y_ref.view(iv)), (case, m)
        assert torch.isfinite(y.float()).all().item()


def test_noalloc_rejects_calls_beyond_its_scratch(dev, torch):
    """f32 x staged for the GEMM: 12000 x 3072 bf16 rows are 70 MiB > 64 MiB."""
    _say("noalloc oversize rejection")
    lib = _lib.load()
    t = GgmlDType.Q4_0
    qt = QTensor.from_blocks(dev, t, (256, 3072), O.quantize(int(t), np.zeros((256, 3072), np.float32)))
    x = torch.zeros((12000, 3072), device="cuda")
    y = torch.zeros((12000, 256), device="cuda")
    rc = _call(lib.mq_qmatmul_noalloc, dev, qt, x, y)
    assert rc == MQ_E_INVALID
    assert b"more than its fixed" in lib.mq_last_error()
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(y)) == 0          # nothing was launched
