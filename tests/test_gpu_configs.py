"""BASELINE configs 3, 4 and 5 at their full sizes on the GPU, through the C ABI.

* Config 3: the FLUX double-block MLP, fc1 3072->12288 with the GELU-tanh epilogue and
  fc2 12288->3072 on its output, at M = 4608, for Q4_K, Q4_0 and Q6_K weights.
* Config 5: the Qwen-Image low-bit GEMMs at M = 6889 (1328^2 image tokens): stacked q/k/v
  Q3_K 3072->9216 (bf16 out), MLP fc1 Q2_K 3072->12288 with GELU to bf16, MLP fc2 Q2_K
  12288->3072 and the Q4_K out-projection 3072->3072 as gated residual updates.
* Configs 4 and 5 whole steps at full size: finite, bit-identical on repeat, and every
  linear of block 0 spot-checked against the f64 oracle on sampled rows at its real M.

Each GEMM check compares sampled rows (always including the last, partial 256-row panel)
with the f64 dequantize-then-matmul of the same rows (the BASELINE bar, rel-L2 <= 1e-2),
and repeats the call to check bitwise determinism.  Weights are N(0, 0.02^2) quantized by
the oracle's reference quantizer; activations N(0, 1).  Reference call sites (under
/root/reference/crates/mold-inference/src/): flux/offload.rs:222-224 (the MLP),
qwen_image/quantized_transformer.rs:604-660 (MLP), 695-790 (attention projections).
"""
import sys

import numpy as np
import pytest

import mold_amd
from mold_amd import GgmlDType, Linear, QMatMul, QTensor
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as _t
    return _t


@pytest.fixture(scope="module")
def dev(torch):
    d = mold_amd.Device(0)
    yield d
    torch.cuda.synchronize()


def _weights(t, n, k, seed):
    w = (np.random.default_rng(seed).standard_normal((n, k)) * 0.02).astype(np.float32)
    return O.quantize(int(t), w)


def _bias(torch, n, seed):
    return torch.from_numpy((np.random.default_rng(seed).standard_normal(n) * 0.02).astype(np.float32)).cuda()


def _rows(m, seed, count=12):
    """Sampled rows: `count` random ones plus the whole last 256-row panel."""
    last = np.arange((m - 1) // 256 * 256, m)
    pick = np.random.default_rng(seed).choice(last[0], size=count, replace=False)
    return np.unique(np.concatenate([pick, last[:: max(1, len(last) // 16)], [m - 1]]))


def _gelu(v):
    return 0.5 * v * (1 + np.tanh(np.sqrt(2 / np.pi) * (v + 0.044715 * v ** 3)))


@pytest.mark.parametrize("tname", ["Q4_K", "Q4_0", "Q6_K"])
def test_config3_mlp_chain(dev, torch, tname):
    """fc1 + GELU (f32 out) then fc2 on the GPU's own fc1 output, M = 4608."""
    t = GgmlDType[tname]
    m, h, mlp = 4608, 3072, 12288
    _say(f"config 3 MLP chain {tname} m={m}")
    b1, b2 = _weights(t, mlp, h, 31), _weights(t, h, mlp, 32)
    fc1 = Linear(QTensor.from_blocks(dev, t, (mlp, h), b1), _bias(torch, mlp, 33))
    fc2 = Linear(QTensor.from_blocks(dev, t, (h, mlp), b2), _bias(torch, h, 34))
    g = torch.Generator(device="cuda").manual_seed(35)
    x = torch.randn((m, h), device="cuda", generator=g)
    hid = fc1.forward(x, act=mold_amd.ACT_GELU_TANH)
    y = fc2.forward(hid)
    y2 = fc2.forward(fc1.forward(x, act=mold_amd.ACT_GELU_TANH))
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32)), "not deterministic"
    assert torch.isfinite(y).all().item() and torch.isfinite(hid).all().item()
    rows = _rows(m, 36)
    ri = torch.from_numpy(rows).cuda()
    xs = x[ri].cpu().numpy()
    # fc1 + GELU against f64
    ref_h = _gelu(O.matmul_f64(int(t), xs, b1, mlp, h) + fc1.bias.cpu().numpy())
    got_h = hid[ri].cpu().numpy()
    e1 = O.rel_l2(got_h, ref_h)
    # fc2 against f64 on the GPU's fc1 rows (the linear alone), and the chain end to end
    ref_y = O.matmul_f64(int(t), got_h, b2, h, mlp) + fc2.bias.cpu().numpy()
    ref_chain = O.matmul_f64(int(t), ref_h.astype(np.float32), b2, h, mlp) + fc2.bias.cpu().numpy()
    got_y = y[ri].cpu().numpy()
    e2, e3 = O.rel_l2(got_y, ref_y), O.rel_l2(got_y, ref_chain)
    print(f"[case] {tname}: fc1+GELU {e1:.2e}  fc2 {e2:.2e}  chain {e3:.2e}", flush=True)
    assert e1 <= TOL and e2 <= TOL and e3 <= TOL


@pytest.mark.parametrize("shape", ["qkv_Q3_K", "fc1_Q2_K_gelu_bf16", "fc2_Q2_K_gated", "out_Q4_K_gated",
                                   "tp8_linear1_shard", "tp8_linear2_shard_gated"])
def test_config5_lowbit_gemms(dev, torch, shape):
    """Qwen-Image block linears at M = 6889 (27 row panels, the last one 233 rows), and one
    GPU's share of FLUX's single-block linears under 8-way tensor parallelism at M = 4608:
    linear1 column-split (N = 21504 / 8) and linear2's largest row share (K = 2048, 8 of its
    60 super-blocks), as timed by bench.py's tp8_shards leg."""
    m, h, mlp = 6889, 3072, 12288
    spec = {"qkv_Q3_K": ("Q3_K", 3 * h, h, "bf16"), "fc1_Q2_K_gelu_bf16": ("Q2_K", mlp, h, "gelu_bf16"),
            "fc2_Q2_K_gated": ("Q2_K", h, mlp, "gated"), "out_Q4_K_gated": ("Q4_K", h, h, "gated"),
            "tp8_linear1_shard": ("Q4_K", 21504 // 8, h, "bf16"),
            "tp8_linear2_shard_gated": ("Q4_K", h, 2048, "gated")}[shape]
    tname, n, k, mode = spec
    if shape.startswith("tp8"):
        m = 4608
    t = GgmlDType[tname]
    _say(f"config 5 {shape} m={m} n={n} k={k}")
    blocks = _weights(t, n, k, 50 + n + k)
    lin = Linear(QTensor.from_blocks(dev, t, (n, k), blocks), _bias(torch, n, 51))
    g = torch.Generator(device="cuda").manual_seed(52)
    x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)   # the step feeds bf16
    rows = _rows(m, 53)
    ri = torch.from_numpy(rows).cuda()
    ref = O.matmul_f64(int(t), x[ri].float().cpu().numpy(), blocks, n, k) + lin.bias.cpu().numpy()
    if mode == "gated":
        gate = torch.randn(n, device="cuda", generator=g)
        res0 = torch.randn((m, n), device="cuda", generator=g)
        outs = [lin.gated_add(x, gate, res0.clone()) for _ in range(2)]
        got = (outs[0] - res0)[ri].cpu().numpy()
        ref = ref * gate.cpu().numpy()
    else:
        act = mold_amd.ACT_GELU_TANH if mode == "gelu_bf16" else mold_amd.ACT_NONE
        outs = [lin.forward(x, act=act, out_dtype=torch.bfloat16) for _ in range(2)]
        got = outs[0][ri].float().cpu().numpy()
        if mode == "gelu_bf16":
            ref = _gelu(ref)
    torch.cuda.synchronize()
    a, b = outs
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)), "not deterministic"
    assert torch.isfinite(a.float()).all().item()
    err = O.rel_l2(got, ref)
    print(f"[case] {shape}: rel-L2 {err:.2e} over {len(rows)} rows", flush=True)
    assert err <= TOL


def _check_block_linears(dev, torch, lin_by_name, names, m_of, seed):
    """Every named linear of the step at its real M: sampled rows against f64."""
    for i, name in enumerate(names):
        l = lin_by_name[name]
        qt = l.matmul.w
        n, k = qt.shape
        m = m_of(name)
        g = torch.Generator(device="cuda").manual_seed(seed + i)
        x = torch.randn((m, k), device="cuda", generator=g)
        y = l.forward(x)
        rows = _rows(m, seed + i, count=6) if m > 256 else np.arange(m)
        ri = torch.from_numpy(rows).cuda()
        ref = O.matmul_f64(int(qt.dtype()), x[ri].cpu().numpy(), qt.data(), n, k)
        if l.bias is not None:
            ref = ref + l.bias.cpu().numpy()
        err = O.rel_l2(y[ri].cpu().numpy(), ref)
        assert np.isfinite(y.cpu().numpy()).all(), name
        assert err <= TOL, (name, err)


def test_config4_flux_step_full_size(dev, torch):
    """FLUX.1-dev shape at 1024^2: 19 double + 38 single blocks, Q4_K linears."""
    from mold_amd import flux as F
    cfg = F.FluxConfig.dev()
    _say("config 4 full FLUX step (1024^2, 4096 + 512 tokens)")
    params = F.FluxParams.random(cfg, dev, seed=4)
    inp = F.make_inputs(cfg, 1024, 1024, 512, device="cuda", seed=4)
    step = F.FluxStep(params)
    out = step.forward(**inp)
    out2 = step.forward(**inp)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all().item()
    assert torch.equal(out.view(torch.int32), out2.view(torch.int32)), "step is not deterministic"
    assert tuple(out.shape) == (4096, cfg.in_channels)
    names = [n_ for n_ in params.lin if n_.startswith(("double_blocks.0.", "single_blocks.0."))]
    m_of = lambda nm: 1 if "mod" in nm else (512 if ".txt_" in nm else (4608 if nm.startswith("single") else 4096))
    _check_block_linears(dev, torch, params.lin, names, m_of, seed=40)


def test_config5_qwen_step_full_size(dev, torch):
    """Qwen-Image shape at 1328^2: 60 dual-stream blocks, Q3_K q/k/v, Q2_K MLP, Q4_K rest."""
    from mold_amd import qwen_image as Q
    cfg = Q.QwenConfig.image()
    _say("config 5 full Qwen-Image step (1328^2, 6889 + 256 tokens)")
    params = Q.QwenParams.random(cfg, dev, seed=5)
    inp = Q.make_inputs(cfg, 1328, 1328, 256, device="cuda", seed=5)
    step = Q.QwenImageStep(params)
    out = step.forward(**inp)
    out2 = step.forward(**inp)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all().item()
    assert torch.equal(out.view(torch.int32), out2.view(torch.int32)), "step is not deterministic"
    names = [n_ for n_ in params.lin if n_.startswith("transformer_blocks.0.")]
    m_of = lambda nm: 1 if "_mod" in nm else (256 if ("add_" in nm or "txt_" in nm) else 6889)
    _check_block_linears(dev, torch, params.lin, names, m_of, seed=60)
