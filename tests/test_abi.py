"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, validates arguments without touching a GPU, and parses GGUF
files (the reader is host code)."""
import ctypes
import os
import re

import numpy as np
import pytest

import mold_amd
from mold_amd import _lib
from mold_amd import gguf
from mold_amd.quantized import GgmlDType
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "moldq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_symbols()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(lib, name), name
    # the Python binding covers the whole header
    assert set(declared) == set(_lib.SIGNATURES)


def test_library_exports_nothing_but_the_c_abi():
    """The dynamic symbol table holds the header's mq_* functions and no internal
    C++ name, so two builds loaded into one process cannot bind to each other's
    internals."""
    import shutil
    import subprocess
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not on PATH")
    out = subprocess.run([nm, "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True).stdout
    names = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert names == set(_declared_symbols()), sorted(names ^ set(_declared_symbols()))[:10]

def test_version_and_type_table():
    lib = _lib.load()
    assert lib.mq_version() == 1
    for t in O.WEIGHT_TYPES:
        assert lib.mq_block_size(t) == O.block_size(t)
        assert lib.mq_type_size(t) == O.type_size(t)
    assert lib.mq_block_size(GgmlDType.F32) == 1 and lib.mq_type_size(GgmlDType.F32) == 4
    assert lib.mq_block_size(99) == 0


def test_argument_validation_without_gpu():
    lib = _lib.load()
    h = ctypes.c_void_p()
    # NULL out pointer -> invalid argument, never a crash
    assert lib.mq_ctx_create(0, None) == _lib.MQ_E_INVALID
    assert b"NULL" in lib.mq_last_error()
    assert lib.mq_qmatmul(None, None, None, 0, 1, 1, None, 0, 1, None, 0, None) == _lib.MQ_E_INVALID
    assert lib.mq_qtensor_upload(None, 12, 1, 256, None, 144, ctypes.byref(h)) == _lib.MQ_E_INVALID
    assert lib.mq_dequantize(None, None, None, 0, None) == _lib.MQ_E_INVALID
    assert lib.mq_qtensor_info(None, None, None, None, None, None) == _lib.MQ_E_INVALID
    # no device here: context creation reports a HIP error instead of aborting
    if not _gpu():
        rc = lib.mq_ctx_create(0, ctypes.byref(h))
        assert rc in (_lib.MQ_E_HIP, _lib.MQ_E_INVALID)
        assert lib.mq_last_error()


def _gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def test_gguf_roundtrip_metadata(tmp_path):
    rng = np.random.default_rng(0)
    tensors = []
    for i, t in enumerate((O.Q4_K, O.Q8_0, O.Q6_K, O.Q4_0)):
        n, k = 3 + i, 256 * (i + 1)
        blocks = O.quantize(t, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        tensors.append((f"blk.{i}.weight", GgmlDType(t), (n, k), blocks))
    tensors.append(("norm.scale", GgmlDType.F32, (7,), np.arange(7, dtype=np.float32).view(np.uint8)))
    for align in (32, 64):
        p = str(tmp_path / f"m{align}.gguf")
        gguf.write(p, tensors, metadata={"general.architecture": "flux", "some.count": 7}, alignment=align)
        c = gguf.Content.read(p)
        assert set(c.tensor_infos) == {t[0] for t in tensors}
        raw = open(p, "rb").read()
        for name, dt, shape, blocks in tensors:
            info = c.tensor_infos[name]
            assert info.dtype == dt and info.shape == tuple(shape)
            assert info.offset % align == 0
            assert raw[info.offset:info.offset + info.nbytes] == np.asarray(blocks, np.uint8).tobytes()
        c.close()


def test_gguf_rejects_garbage(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"NOTGGUF" + b"\0" * 64)
    with pytest.raises(mold_amd.MoldqError) as e:
        gguf.Content.read(str(p))
    assert e.value.code == _lib.MQ_E_IO
    # truncated after a valid header
    good = tmp_path / "t.gguf"
    gguf.write(str(good), [("w", GgmlDType.Q8_0, (2, 32), O.quantize(O.Q8_0, np.ones((2, 32), np.float32)))])
    data = good.read_bytes()
    (tmp_path / "trunc.gguf").write_bytes(data[:-60])   # past the trailing padding, into the data
    with pytest.raises(mold_amd.MoldqError):
        gguf.Content.read(str(tmp_path / "trunc.gguf"))
