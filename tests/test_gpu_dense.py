"""Dense GGUF tensors (F32 / F16 / BF16) through the C ABI: the biases, norm scales
and embeddings that mold loads onto the device with every GGUF model
(content.tensor(.., device), crates/mold-inference/src/flux/lora.rs:721-723) and
dequantizes there (crates/mold-inference/src/qwen_image/quantized_transformer.rs:83-86,
crates/mold-inference/src/flux2/quantized_transformer.rs:49-54).

Upload, device copy, GGUF load and download are byte-identical; dequantize to each
of F32 / F16 / BF16 equals torch's CPU conversion bit for bit (the same type is a
copy, widening exact, narrowing round-to-nearest-even; NaN stays NaN);
mq_quantize to a dense type is the same conversion from f32; a quantized matmul
refuses a dense weight with MQ_E_UNSUPPORTED."""
import sys

import numpy as np
import pytest

import mold_amd
from mold_amd import GgmlDType, QMatMul, QTensor, gguf
from mold_amd._lib import MQ_E_UNSUPPORTED, MoldqError

from . import gguf_ref as R

pytestmark = pytest.mark.gpu

DENSE = [GgmlDType.F32, GgmlDType.F16, GgmlDType.BF16]


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


def _tdt(torch, t):
    return {GgmlDType.F32: torch.float32, GgmlDType.F16: torch.float16, GgmlDType.BF16: torch.bfloat16}[t]


def _values(torch, n, k, seed):
    """f32 values over every range the conversions treat differently: normal, f16 and
    bf16 subnormal, overflow to inf, exact ties of both narrow types, inf, nan, +-0."""
    rng = np.random.default_rng(seed)
    v = rng.standard_normal(n * k).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 6, n * k)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65520.0, 70000.0, 1e-8, -3e-6, 2 ** -24,
                        1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 3e38, 1e-40],
                       dtype=np.float32)
    m = min(len(special), v.size)
    v[:m] = special[:m]
    return torch.from_numpy(v.reshape(n, k))


def _same_bits(torch, a, b):
    a, b = a.cpu(), b.cpu()
    assert a.dtype == b.dtype and a.shape == b.shape
    iv = torch.int32 if a.dtype == torch.float32 else torch.int16
    nan = torch.isnan(a)
    assert torch.equal(nan, torch.isnan(b))
    return torch.equal(a[~nan].view(iv), b[~nan].view(iv))


@pytest.mark.parametrize("src", DENSE, ids=lambda t: t.name)
@pytest.mark.parametrize("shape", [(1, 7), (33, 129), (64, 3072)], ids=str)
def test_dense_upload_download_and_dequantize(dev, torch, src, shape):
    n, k = shape
    _say(f"dense {src.name} {shape}")
    vals = _values(torch, n, k, seed=n * k).to(_tdt(torch, src))    # the file's values in its own type
    raw = vals.contiguous().view(torch.uint8).numpy().reshape(-1)
    qt = QTensor.from_blocks(dev, src, shape, raw)
    assert qt.dtype() == src and qt.shape == shape and qt.storage_size_in_bytes() == raw.nbytes
    assert np.array_equal(qt.data(), raw)
    for dst in DENSE:
        got = qt.dequantize(_tdt(torch, dst))
        want = vals.float().to(_tdt(torch, dst))                    # torch CPU: exact widening, RNE narrowing
        torch.cuda.synchronize()
        assert _same_bits(torch, got, want), (src.name, dst.name)
    # the same bytes already on the device
    qd = QTensor.from_device_blocks(dev, src, shape, torch.from_numpy(raw).cuda())
    assert np.array_equal(qd.data(), raw)


@pytest.mark.parametrize("dst", DENSE, ids=lambda t: t.name)
def test_dense_quantize_is_conversion(dev, torch, dst):
    """QTensor::quantize(.., F32 / F16 / BF16) (mold's F32 fallback at
    flux/pipeline.rs:223-228): the stored values are the f32 source converted,
    from a strided source too."""
    n, k = 40, 96
    _say(f"dense quantize {dst.name}")
    v = _values(torch, n, k, seed=5)
    wide = torch.zeros((n, k + 32), dtype=torch.float32, device="cuda")
    wide[:, :k] = v.cuda()
    qt = QTensor.quantize(dev, wide[:, :k], dst)
    want = v.to(_tdt(torch, dst)).contiguous().view(torch.uint8).numpy().reshape(-1)
    got = qt.data()
    if dst == GgmlDType.F32:
        assert np.array_equal(got, want)
    else:
        assert _same_bits(torch, torch.from_numpy(got.copy()).view(_tdt(torch, dst)),
                          torch.from_numpy(want.copy()).view(_tdt(torch, dst)))


def test_dense_weight_refused_by_quantized_matmul(dev, torch):
    qt = QTensor.from_blocks(dev, GgmlDType.F16, (64, 256), np.zeros(64 * 256 * 2, np.uint8))
    x = torch.zeros((4, 256), device="cuda")
    with pytest.raises(MoldqError) as e:
        QMatMul(qt).forward(x)
    assert e.value.code == MQ_E_UNSUPPORTED and "dense" in str(e.value)
    with pytest.raises(MoldqError):
        QMatMul(qt).forward(torch.zeros((300, 256), device="cuda"))


def test_dense_tensors_from_gguf_file(dev, torch, tmp_path):
    """1-, 2- and 3-D dense tensors of each type, beside a block-type one, loaded from a
    GGUF file through mq_gguf_load_tensor: [rows = product of ne[1..], ne[0]], bytes
    as stored."""
    rng = np.random.default_rng(3)
    tensors = [("bias", 0, (7,), rng.standard_normal(7).astype(np.float32).view(np.uint8)),
               ("emb", 30, (2, 5), rng.integers(0, 256, 20, dtype=np.uint8)),
               ("half", 1, (3, 1, 4), rng.integers(0, 256, 24, dtype=np.uint8)),
               ("w", 8, (2, 32), np.zeros(68, np.uint8))]
    path = str(tmp_path / "dense.gguf")
    R.write(path, [], tensors)
    c = gguf.Content.read(path)
    try:
        for name, t, shape, raw in tensors:
            qt = c.tensor(name, dev)
            rows = int(np.prod(shape[:-1])) if len(shape) > 1 else 1
            assert qt.dtype() == GgmlDType(t) and qt.shape == (rows, shape[-1]), name
            assert np.array_equal(qt.data(), raw), name
    finally:
        c.close()
