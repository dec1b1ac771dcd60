"""mold's GGUF LoRA path on the GPU, through the C ABI (mq_dequantize ->
mq_lora_apply -> mq_quantize), against the oracle chain (exact dequantize,
orc_lora_apply in the same order, the reference quantizer): re-quantized blocks
byte-identical.  Reference: gguf_lora_var_builder,
crates/mold-inference/src/flux/lora.rs:661-869."""
import ctypes
import sys

import numpy as np
import pytest

import mold_amd
from mold_amd import GgmlDType, QTensor, _lib, gguf
from mold_amd import lora as L
from oracle import oracle as O

from . import gguf_ref as R

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


@pytest.mark.parametrize("rows,k,rank,ldw,scale", [(1, 1, 1, 1, 1.0), (70, 130, 16, 130, 0.5),
                                                    (200, 64, 33, 96, -1.25), (64, 3072, 128, 3072, 0.031)])
def test_lora_apply_bit_exact(torch, rows, k, rank, ldw, scale):
    _say(f"lora_apply rows={rows} k={k} rank={rank} ldw={ldw}")
    rng = np.random.default_rng(rows + k + rank)
    w = (rng.standard_normal((rows, ldw)) * 0.02).astype(np.float32)
    b = (rng.standard_normal((rows, rank)) * 0.05).astype(np.float32)
    a = (rng.standard_normal((rank, k)) * 0.05).astype(np.float32)
    wd = torch.from_numpy(w).cuda()
    L.lora_apply(wd[:, :k], torch.from_numpy(b), torch.from_numpy(a), scale)
    torch.cuda.synchronize()
    got = wd.cpu().numpy()
    want = w.copy()
    want[:, :k] = O.lora_apply(w[:, :k], b, a, scale)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_lora_apply_rejects_bad_shapes(torch):
    w = torch.zeros((4, 8), device="cuda")
    rc = _lib.load().mq_lora_apply(w.data_ptr(), 8, 4, 8, w.data_ptr(), 8, w.data_ptr(), 8, 0, ctypes.c_float(1.0),
                                   None)
    assert rc == _lib.MQ_E_INVALID


def _oracle_patch(t, blocks, n, k, patches):
    dq = O.dequantize(int(t), blocks, n, k)
    for (off, size, b, a, s) in patches:
        dq[off:off + size] = O.lora_apply(dq[off:off + size], b, a, s)
    return O.quantize(int(t), dq).reshape(-1)


@pytest.mark.parametrize("tname", ["Q8_0", "Q4_K", "Q6_K", "Q4_0"])
def test_patch_qtensor_matches_oracle_chain(dev, torch, tname):
    t = GgmlDType[tname]
    n, k, rank = 768, 512, 8
    _say(f"patch_qtensor {tname}")
    rng = np.random.default_rng(int(t))
    blocks = O.quantize(int(t), (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    pts, ref = [], []
    for comp in (0, 2):
        b = (rng.standard_normal((256, rank)) * 0.05).astype(np.float32)
        a = (rng.standard_normal((rank, k)) * 0.05).astype(np.float32)
        pts.append(L.LoraPatch(torch.from_numpy(a), torch.from_numpy(b), 0.5, L.LoraTarget("x", comp, 3)))
        ref.append((comp * 256, 256, b, a, 0.5))
    out, applied = L.patch_qtensor(qt, pts)
    assert applied == 2 and out.dtype() == t and out.shape == (n, k)
    assert np.array_equal(out.data(), _oracle_patch(t, blocks, n, k, ref))


def test_gguf_lora_var_builder(dev, torch, tmp_path):
    from safetensors.torch import save_file
    _say("gguf_lora_var_builder end to end")
    rng = np.random.default_rng(9)
    h, mlp, rank = 256, 1024, 8
    spec = {"double_blocks.0.img_attn.qkv.weight": (GgmlDType.Q8_0, 3 * h, h),
            "double_blocks.0.img_attn.proj.weight": (GgmlDType.Q4_K, h, h),
            "single_blocks.0.linear1.weight": (GgmlDType.Q6_K, 3 * h + mlp, h),
            "single_blocks.0.linear2.weight": (GgmlDType.Q4_0, h, h + mlp),
            "double_blocks.0.img_mlp.0.weight": (GgmlDType.Q4_K, 4 * h, h)}
    blocks = {nm: O.quantize(int(t), (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
              for nm, (t, n, k) in spec.items()}
    norm = rng.standard_normal(128).astype(np.float32)
    path = str(tmp_path / "flux.gguf")
    R.write(path, [], [(nm, int(spec[nm][0]), spec[nm][1:], blocks[nm]) for nm in spec] +
            [("double_blocks.0.img_attn.norm.query_norm.scale", O.F32, (128,), norm.view(np.uint8))])
    lora_layers = {"transformer.transformer_blocks.0.attn.to_q": (h, h, 4.0),
                   "transformer.transformer_blocks.0.attn.to_k": (h, h, None),
                   "transformer.transformer_blocks.0.attn.to_out.0": (h, h, 8.0),
                   "transformer.single_transformer_blocks.0.attn.to_v": (h, h, 2.0),
                   "transformer.single_transformer_blocks.0.proj_mlp": (mlp, h, 2.0),
                   "transformer.single_transformer_blocks.0.proj_out": (h, h + mlp, 2.0),
                   "transformer.not_a_layer": (h, h, None)}
    st, ab = {}, {}
    for key, (out_dim, in_dim, alpha) in lora_layers.items():
        a = (rng.standard_normal((rank, in_dim)) * 0.05).astype(np.float32)
        b = (rng.standard_normal((out_dim, rank)) * 0.05).astype(np.float32)
        st[key + ".lora_A.weight"] = torch.from_numpy(a).to(torch.bfloat16)
        st[key + ".lora_B.weight"] = torch.from_numpy(b).to(torch.bfloat16)
        if alpha is not None:
            st[key + ".alpha"] = torch.tensor(alpha)
        ab[key] = (st[key + ".lora_A.weight"].float().numpy(), st[key + ".lora_B.weight"].float().numpy(), alpha)
    lpath = str(tmp_path / "lora.safetensors")
    save_file(st, lpath)
    adapter = L.LoraAdapter.load(lpath)
    assert adapter.rank == rank
    scale = 0.8
    data, applied = L.gguf_lora_var_builder(path, adapter, scale, dev)
    assert applied == 6
    eff = {k: (scale * al / rank if al is not None else scale) for k, (_, _, al) in ab.items()}
    d0, s0 = "transformer.transformer_blocks.0.", "transformer.single_transformer_blocks.0."
    expect = {
        "double_blocks.0.img_attn.qkv.weight": [(0, h, d0 + "attn.to_q"), (h, h, d0 + "attn.to_k")],
        "double_blocks.0.img_attn.proj.weight": [(0, h, d0 + "attn.to_out.0")],
        "single_blocks.0.linear1.weight": [(2 * h, h, s0 + "attn.to_v"), (3 * h, mlp, s0 + "proj_mlp")],
        "single_blocks.0.linear2.weight": [(0, h, s0 + "proj_out")],
    }
    for nm, (t, n, k) in spec.items():
        got = data[nm]
        assert isinstance(got, QTensor) and got.dtype() == t
        if nm in expect:
            ref = _oracle_patch(t, blocks[nm], n, k, [(off, size, ab[key][1], ab[key][0], eff[key])
                                                      for off, size, key in expect[nm]])
        else:
            ref = blocks[nm].reshape(-1)
        assert np.array_equal(got.data(), ref), nm
    nrm = data["double_blocks.0.img_attn.norm.query_norm.scale"]      # a dense F32 tensor, untouched
    assert isinstance(nrm, QTensor) and nrm.dtype() == GgmlDType.F32 and nrm.shape == (1, 128)
    assert np.array_equal(nrm.data(), norm.view(np.uint8))
    assert np.array_equal(nrm.dequantize().cpu().numpy().reshape(-1), norm)
