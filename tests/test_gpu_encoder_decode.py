"""GGUF text-encoder and LLM-decode shapes through the same C ABI (the next row
of the hot-path table: new shapes behind the same boundary).

* T5-XXL encoder linears (d_model 4096, d_ff 10240, 64 heads x 64): q/k/v/o
  4096 -> 4096, GeGLU gate/up 4096 -> 10240, down 10240 -> 4096, at M = 512
  (FLUX's T5 sequence) and M = 77, for the block types T5 GGUF files ship
  (Q8_0, Q6_K, Q5_K, Q4_K).  Reference: QMatMul::from_weights for every
  attention / FF linear at crates/mold-inference/src/encoders/t5_gguf.rs:243-246,
  277-279.
* LLM prompt-expansion decode: M = 1 GEMVs at K = 4096 (N = 4096, 10240) and
  K = 10240 -> 4096 for Q8_0, Q6_K, Q5_K, Q4_K and Q4_0 weights, through
  ModelWeights::from_gguf at crates/mold-inference/src/expand.rs:200-203.

Each result is checked on sampled rows against the f64 dequantize-then-matmul
oracle (rel-L2 <= 1e-2; the generic GEMV, f32 FMA on exactly decoded weights,
to 1e-5), finite, and bit-identical on a repeat.
"""
import functools
import sys

import numpy as np
import pytest

import mold_amd
from mold_amd import GgmlDType, Linear, QTensor
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


@functools.lru_cache(maxsize=4)
def _weights(t, n, k, seed):
    w = (np.random.default_rng(seed).standard_normal((n, k)) * 0.02).astype(np.float32)
    return O.quantize(int(t), w)


T5_SHAPES = {"attn_qkvo": (4096, 4096), "ffn_gate_up": (10240, 4096), "ffn_down": (4096, 10240)}


@pytest.mark.parametrize("m", [512, 77])
@pytest.mark.parametrize("shape", list(T5_SHAPES))
@pytest.mark.parametrize("tname", ["Q8_0", "Q6_K", "Q5_K", "Q4_K"])
def test_t5_encoder_linears(dev, torch, tname, shape, m):
    n, k = T5_SHAPES[shape]
    t = GgmlDType[tname]
    _say(f"T5 {shape} {tname} m={m} {k}->{n}")
    blocks = _weights(t, n, k, seed=n + k + int(t))
    lin = Linear(QTensor.from_blocks(dev, t, (n, k), blocks))
    g = torch.Generator(device="cuda").manual_seed(m + n)
    x = torch.randn((m, k), device="cuda", generator=g)
    y = lin.forward(x)
    y2 = lin.forward(x)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32)), "not deterministic"
    assert torch.isfinite(y).all().item()
    rows = np.unique(np.concatenate([np.random.default_rng(m).choice(m, size=min(m, 12), replace=False), [m - 1]]))
    ri = torch.from_numpy(rows).cuda()
    ref = O.matmul_f64(int(t), x[ri].cpu().numpy(), blocks, n, k)
    err = O.rel_l2(y[ri].cpu().numpy(), ref)
    print(f"[case] rel-L2 {err:.2e}", flush=True)
    assert err <= 1e-2


DECODE_SHAPES = [(4096, 4096), (10240, 4096), (4096, 10240)]


@pytest.mark.parametrize("nk", DECODE_SHAPES, ids=lambda s: f"{s[1]}to{s[0]}")
@pytest.mark.parametrize("tname", ["Q8_0", "Q6_K", "Q5_K", "Q4_K", "Q4_0"])
def test_decode_gemv_m1(dev, torch, tname, nk):
    n, k = nk
    t = GgmlDType[tname]
    _say(f"decode GEMV {tname} m=1 {k}->{n}")
    blocks = _weights(t, n, k, seed=7 * n + k + int(t))
    lin = Linear(QTensor.from_blocks(dev, t, (n, k), blocks))
    g = torch.Generator(device="cuda").manual_seed(n)
    x = torch.randn((1, k), device="cuda", generator=g)
    y = lin.forward(x)
    y2 = lin.forward(x)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32)), "not deterministic"
    ref = O.matmul_f64(int(t), x.cpu().numpy(), blocks, n, k)
    err = O.rel_l2(y.cpu().numpy(), ref)
    print(f"[case] rel-L2 {err:.2e}", flush=True)
    # the generic GEMV decodes exactly and accumulates in f32; the Q4_K GEMV
    # quantizes x to Q8_K, which bounds it at the 1e-2 bar
    assert err <= (1e-2 if t == GgmlDType.Q4_K else 1e-5)
