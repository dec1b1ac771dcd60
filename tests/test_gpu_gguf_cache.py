"""mold's GGUF cache producers on the GPU, through the C ABI:

* mq_quantize_fp8: FP8 E4M3 weights on the device quantized to GGUF blocks
  byte-identical to the reference quantizer applied to the exactly decoded
  values (the oracle's E4M3 decoding is pinned against torch's
  float8_e4m3fn in test_gguf_format.py);
* the writer's device tensors (add_qtensor) read back byte-identical;
* fp8_safetensors_to_gguf: the conversion of ensure_fp8_gguf_cache
  (crates/mold-inference/src/flux/pipeline.rs:180-248) on a synthetic FP8
  checkpoint with a name prefix, small and odd-shaped tensors.
"""
import ctypes
import sys

import numpy as np
import pytest

import mold_amd
from mold_amd import GgmlDType, QTensor, _lib, gguf
from oracle import oracle as O

pytestmark = pytest.mark.gpu


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


def _fp8_bytes(rng, shape):
    b = rng.integers(0, 256, shape, dtype=np.uint8)
    b[(b & 0x7F) == 0x7F] ^= 1          # no NaN codes: checkpoints hold finite weights
    return b


def _quantize_fp8(dev, torch, t, b, scale=1.0):
    n, k = b.shape
    src = torch.from_numpy(np.ascontiguousarray(b)).cuda()
    h = ctypes.c_void_p()
    rc = _lib.load().mq_quantize_fp8(dev.handle, int(t), n, k, src.data_ptr(), k, ctypes.c_float(scale), None,
                                     ctypes.byref(h))
    assert rc == 0, _lib.load().mq_last_error()
    return QTensor(dev, h)


@pytest.mark.parametrize("tname", ["Q8_0", "Q4_K", "Q6_K", "Q4_0"])
@pytest.mark.parametrize("scale", [1.0, 0.5, 0.013])
def test_quantize_fp8_matches_reference(dev, torch, tname, scale):
    t = GgmlDType[tname]
    _say(f"fp8 -> {tname} scale {scale}")
    rng = np.random.default_rng(int(t))
    b = _fp8_bytes(rng, (70, 512))
    qt = _quantize_fp8(dev, torch, t, b, scale)
    vals = (O.e4m3_to_f32(b) * np.float32(scale)).astype(np.float32)
    assert np.array_equal(qt.data(), O.quantize(int(t), vals).reshape(-1))


def test_quantize_fp8_row_stride(dev, torch):
    rng = np.random.default_rng(1)
    b = _fp8_bytes(rng, (33, 96))
    src = torch.from_numpy(b).cuda()
    h = ctypes.c_void_p()
    rc = _lib.load().mq_quantize_fp8(dev.handle, int(GgmlDType.Q8_0), 33, 64, src.data_ptr(), 96,
                                     ctypes.c_float(1.0), None, ctypes.byref(h))
    assert rc == 0, _lib.load().mq_last_error()
    qt = QTensor(dev, h)
    assert np.array_equal(qt.data(), O.quantize(O.Q8_0, O.e4m3_to_f32(b[:, :64])).reshape(-1))


def test_writer_device_tensors(dev, torch, tmp_path):
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((96, 512)) * 0.02).astype(np.float32)
    qt = QTensor.from_blocks(dev, GgmlDType.Q4_K, (96, 512), O.quantize(O.Q4_K, w))
    bias = QTensor.from_blocks(dev, GgmlDType.Q8_0, (1, 64), O.quantize(O.Q8_0, w[:1, :64]))
    p = str(tmp_path / "d.gguf")
    wr = gguf.Writer(p)
    wr.kv("general.architecture", "flux")
    wr.add_qtensor("w", qt)
    wr.add_qtensor("b", bias, shape=(64,))
    wr.finish()
    wr.close()
    c = gguf.Content.read(p)
    assert c.tensor_infos["w"].shape == (96, 512) and c.tensor_infos["b"].shape == (64,)
    assert np.array_equal(c.tensor_bytes("w"), qt.data())
    assert np.array_equal(c.tensor_bytes("b"), bias.data())
    back = c.tensor("w", dev)
    assert np.array_equal(back.data(), qt.data())
    c.close()


def test_fp8_safetensors_to_q8_gguf(dev, torch, tmp_path):
    from safetensors.torch import save_file
    _say("fp8 safetensors -> Q8_0 GGUF cache")
    rng = np.random.default_rng(3)
    pre = "model.diffusion_model."
    spec = {"img_in.weight": (96, 64), "double_blocks.0.img_attn.qkv.weight": (192, 128), "img_in.bias": (96,),
            "final_layer.norm.scale": (10,), "odd.weight": (33, 7), "tiny": (16,)}
    tensors, raw = {}, {}
    for name, shape in spec.items():
        b = _fp8_bytes(rng, shape)
        raw[name] = b
        tensors[pre + name] = torch.from_numpy(b).view(torch.float8_e4m3fn)
    tensors[pre + "f32.weight"] = torch.from_numpy((rng.standard_normal((4, 64)) * 0.1).astype(np.float32))
    src = str(tmp_path / "ckpt.safetensors")
    save_file(tensors, src)
    dst = str(tmp_path / "ckpt.q8_0.gguf")
    stored = gguf.fp8_safetensors_to_gguf(src, dst, dev)
    c = gguf.Content.read(dst)
    assert set(c.tensor_infos) == set(spec) | {"f32.weight"}            # prefix stripped
    for name, shape in spec.items():
        info = c.tensor_infos[name]
        vals = O.e4m3_to_f32(raw[name])
        k = shape[-1]
        assert info.shape == shape, name
        if int(np.prod(shape)) % 32 == 0 and k % 32 == 0:
            assert stored[name] == "Q8_0" and info.dtype == GgmlDType.Q8_0
            assert np.array_equal(c.tensor_bytes(name), O.quantize(O.Q8_0, vals.reshape(-1, k)).reshape(-1)), name
        else:
            assert stored[name] == "F32" and info.dtype == GgmlDType.F32
            assert np.array_equal(c.tensor_bytes(name).view(np.float32), vals.reshape(-1)), name
    fw = tensors[pre + "f32.weight"].numpy()
    assert np.array_equal(c.tensor_bytes("f32.weight"), O.quantize(O.Q8_0, fw).reshape(-1))
    c.close()
