"""FLUX-shaped step built on the quantized linears (the path's caller).

The reference here is an independent f32/f64 restatement of mold's FLUX block graph
(/root/reference/crates/mold-inference/src/flux/offload.rs:21-73 helpers,
:276-325 DoubleBlock, :374-392 SingleBlock, :413-422 FinalLayer, :523-574 forward):
RoPE as a complex rotation, attention as an explicit f64 softmax, every linear as
x @ W^T + b on the dequantized weight.  The CPU test checks the host glue of
`mold_amd.flux` with dense linears; the GPU test checks the whole quantized step.
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from mold_amd import flux as F  # noqa: E402

# Whole-step rel-L2 bar (the north star's 1e-2).  bf16 GEMM inputs and bf16 attention alone give
# ~1.6e-3 on the tiny config when emulated on the CPU.
STEP_TOL = 1e-2


# ----------------------------------------------------------------- reference

def _lin(W, name, x):
    w, b = W[name]
    y = x.double() @ w.double().T
    return (y + b.double()) if b is not None else y


def _ln(x):
    mu = x.mean(-1, keepdim=True)
    var = ((x - mu) ** 2).mean(-1, keepdim=True)
    return (x - mu) / torch.sqrt(var + 1e-6)


def _rms(x, s):
    return x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6) * s.double()


def _gelu(x):
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def _silu(x):
    return x / (1.0 + torch.exp(-x))


def _rope(x, ids, axes, theta):
    """Rotate (x[2j], x[2j+1]) as a complex number by pos_axis(j) * theta^(-2j'/d_axis)."""
    ang = []
    for a, d in enumerate(axes):
        j = torch.arange(d // 2, dtype=torch.float64)
        ang.append(ids[:, a:a + 1].double() * theta ** (-2.0 * j / d)[None, :])
    ang = torch.cat(ang, dim=1)                               # [L, D/2]
    xc = torch.view_as_complex(x.double().reshape(*x.shape[:-1], -1, 2).contiguous())
    return torch.view_as_real(xc * torch.polar(torch.ones_like(ang), ang)).reshape(x.shape)


def _attn(q, k, v):
    s = (q @ k.transpose(-1, -2)) / math.sqrt(q.shape[-1])
    p = torch.softmax(s, dim=-1)
    o = p @ v                                                  # [H, L, D]
    return o.transpose(0, 1).reshape(q.shape[1], -1)


def _temb(t, dim=256):
    half = dim // 2
    f = torch.exp(-math.log(10000.0) * torch.arange(half, dtype=torch.float64) / half)
    a = t.double()[:, None] * 1000.0 * f[None]
    return torch.cat([torch.cos(a), torch.sin(a)], dim=1)


def reference_forward(cfg, W, D, inp):
    H, hd, h = cfg.num_heads, cfg.head_dim, cfg.hidden_size
    ids = torch.cat([inp["txt_ids"], inp["img_ids"]], dim=0).cpu()
    rope = lambda x: _rope(x, ids, cfg.axes_dim, cfg.theta)  # noqa: E731
    img = inp["img"].cpu().double() @ D["img_in.weight"].double().T + D["img_in.bias"].double()
    txt = _lin(W, "txt_in", inp["txt"].cpu())
    emb = lambda p, x: _lin(W, p + ".out_layer", _silu(_lin(W, p + ".in_layer", x)))  # noqa: E731
    vec = emb("time_in", _temb(inp["t"].cpu())) + emb("guidance_in", _temb(inp["guidance"].cpu())) \
        + emb("vector_in", inp["y"].cpu())
    sv = _silu(vec)

    def heads(y3, qs, ks):
        L = y3.shape[0]
        y3 = y3.reshape(L, 3, H, hd).permute(1, 2, 0, 3)      # [3, H, L, D]
        return _rms(y3[0], D[qs]), _rms(y3[1], D[ks]), y3[2]

    for i in range(cfg.depth):
        p = f"double_blocks.{i}."
        im = _lin(W, p + "img_mod.lin", sv).reshape(6, h)
        tm = _lin(W, p + "txt_mod.lin", sv).reshape(6, h)
        iq, ik, iv = heads(_lin(W, p + "img_attn.qkv", _ln(img) * (1 + im[1]) + im[0]),
                           p + "img_attn.norm.query_norm.scale", p + "img_attn.norm.key_norm.scale")
        tq, tk, tv = heads(_lin(W, p + "txt_attn.qkv", _ln(txt) * (1 + tm[1]) + tm[0]),
                           p + "txt_attn.norm.query_norm.scale", p + "txt_attn.norm.key_norm.scale")
        a = _attn(rope(torch.cat([tq, iq], 1)), rope(torch.cat([tk, ik], 1)), torch.cat([tv, iv], 1))
        lt = txt.shape[0]
        img = img + im[2] * _lin(W, p + "img_attn.proj", a[lt:])
        img = img + im[5] * _lin(W, p + "img_mlp.2", _gelu(_lin(W, p + "img_mlp.0", _ln(img) * (1 + im[4]) + im[3])))
        txt = txt + tm[2] * _lin(W, p + "txt_attn.proj", a[:lt])
        txt = txt + tm[5] * _lin(W, p + "txt_mlp.2", _gelu(_lin(W, p + "txt_mlp.0", _ln(txt) * (1 + tm[4]) + tm[3])))
    x = torch.cat([txt, img], 0)
    for i in range(cfg.depth_single_blocks):
        p = f"single_blocks.{i}."
        m = _lin(W, p + "modulation.lin", sv).reshape(3, h)
        y = _lin(W, p + "linear1", _ln(x) * (1 + m[1]) + m[0])
        q, k, v = heads(y[:, :3 * h], p + "norm.query_norm.scale", p + "norm.key_norm.scale")
        a = _attn(rope(q), rope(k), v)
        x = x + m[2] * _lin(W, p + "linear2", torch.cat([a, _gelu(y[:, 3 * h:])], 1))
    fm = _lin(W, "final_layer.adaLN_modulation.1", sv).reshape(2, h)
    x = x[txt.shape[0]:]
    return _lin(W, "final_layer.linear", _ln(x) * (1 + fm[1]) + fm[0])


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


# ----------------------------------------------------------------- CPU: glue

class _DenseLinear:
    """f32 dense linear with the `Linear.forward` calling convention (host test only)."""

    def __init__(self, w, b):
        self.w, self.b = w, b

    def forward(self, x, act=0, out_dtype=None):
        y = x.float() @ self.w.T
        if self.b is not None:
            y = y + self.b
        if act == 1:
            y = torch.nn.functional.gelu(y, approximate="tanh")
        return y.to(out_dtype or x.dtype)


def _random_dense(cfg, seed=5):
    g = torch.Generator().manual_seed(seed)
    W, lin = {}, {}
    for name, (n, k, hb) in F.linear_shapes(cfg).items():
        w = torch.randn((n, k), generator=g) * 0.02
        b = torch.randn((n,), generator=g) * 0.02 if hb else None
        W[name] = (w, b)
        lin[name] = _DenseLinear(w, b)
    D = {}
    for name, shape in F.dense_shapes(cfg).items():
        t = torch.randn(shape, generator=g) * 0.02
        D[name] = (t + 1.0) if name.endswith(".scale") else t
    return W, lin, D


def test_flux_glue_matches_reference_on_cpu():
    cfg = F.FluxConfig.tiny()
    W, lin, D = _random_dense(cfg)
    params = F.FluxParams(cfg, lin, D)
    inp = F.make_inputs(cfg, height=128, width=128, txt_len=16, device="cpu", seed=3)
    step = F.FluxStep(params, attn=F.attention_f32, gemm_dtype=torch.float32)
    out = step.forward(**inp)
    ref = reference_forward(cfg, W, D, inp)
    assert out.shape == (64, cfg.in_channels)
    assert _rel(out.numpy(), ref.numpy()) < 1e-5


def test_flux_step_flop_accounting():
    cfg = F.FluxConfig.dev()
    lin, attn = F.step_flop(cfg, 4096, 512)
    # FLUX.1-dev at 1024^2, batch 1: 5.950e13 linear FLOP (M > 1), 1.487e13 attention FLOP
    assert abs(lin / 5.950e13 - 1) < 2e-3, lin
    assert abs(attn / 1.487e13 - 1) < 2e-3, attn
    n_lin = len(F.linear_shapes(cfg))
    assert n_lin == 9 + 19 * 10 + 38 * 3


# ----------------------------------------------------------------- GPU: whole step

@pytest.mark.gpu
def test_flux_step_tiny_matches_dequantized_reference():
    import mold_amd
    from oracle import oracle as O
    cfg = F.FluxConfig.tiny()
    print(f"[flux] tiny step: hidden {cfg.hidden_size}, heads {cfg.num_heads}", flush=True)
    dev = mold_amd.Device(0)
    params = F.FluxParams.random(cfg, dev, seed=6)
    inp = F.make_inputs(cfg, height=256, width=256, txt_len=32, device="cuda", seed=6)
    step = F.FluxStep(params)
    out = step.forward(**inp)
    # the modulations as one stacked GEMV (default) or one GEMV per block: same values
    sep = F.FluxStep(params)
    sep.stack_modulations = False
    out_sep = sep.forward(**inp)
    torch.cuda.synchronize()
    assert step._mod_stack is not None and sep._mod_stack is None
    assert torch.equal(out, out_sep)
    W = {}
    for name, l in params.lin.items():
        qt = l.matmul.w
        n, k = qt.shape
        w = torch.from_numpy(O.dequantize(int(qt.dtype()), qt.data(), n, k))
        W[name] = (w, l.bias.cpu() if l.bias is not None else None)
    D = {k_: v.float().cpu() for k_, v in params.dense.items()}
    ref = reference_forward(cfg, W, D, {k_: v.cpu() for k_, v in inp.items()})
    o = out.cpu().numpy()
    assert np.isfinite(o).all()
    err = _rel(o, ref.numpy())
    print(f"[flux] rel-L2 vs f64 dequantized reference: {err:.3e}", flush=True)
    assert err <= STEP_TOL, err
    # a modulation linear replaced after the stack was built is picked up (the
    # step rebuilds its stack): stacked and per-block forwards still agree
    nm = step.modulation_names()[0]
    old = params.lin[nm]
    g = torch.Generator(device="cuda").manual_seed(99)
    w2 = torch.randn(old.matmul.w.shape, device="cuda", generator=g) * 0.02
    params.lin[nm] = mold_amd.Linear(mold_amd.QTensor.quantize(dev, w2, old.matmul.w.dtype()), old.bias)
    stack_before = step._mod_stack
    out2, out2_sep = step.forward(**inp), sep.forward(**inp)
    torch.cuda.synchronize()
    params.lin[nm] = old
    assert step._mod_stack is not stack_before
    assert torch.equal(out2, out2_sep) and not torch.equal(out2, out)


@pytest.mark.gpu
def test_flux_step_from_mold_layout_gguf(tmp_path):
    """A tiny-config FLUX GGUF in mold's layout, written by an independent
    restatement of the container (tests/gguf_ref.py): Q4_K linear weights, F32
    biases and norm scales, an F16 img_in weight (K = 64 holds no 256-wide
    super-block), candle's tensor names, GGUF ne order.  FluxParams.from_gguf loads
    it through the C ABI alone (mq_gguf_load_tensor for every tensor, dense ones
    dequantized on the device; no host read of tensor bytes), and the step
    matches the f64 restatement on the file's own values within the 1e-2 bar."""
    import mold_amd
    from oracle import oracle as O
    from . import gguf_ref as R
    cfg = F.FluxConfig.tiny()
    print("[flux] tiny step from a mold-layout GGUF", flush=True)
    rng = np.random.default_rng(12)
    tensors, W, D = [], {}, {}
    for name, (n, k, hb) in F.linear_shapes(cfg).items():
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        blocks = O.quantize(O.Q4_K, w)
        tensors.append((name + ".weight", O.Q4_K, (n, k), blocks))
        b = None
        if hb:
            b = (rng.standard_normal(n) * 0.02).astype(np.float32)
            tensors.append((name + ".bias", O.F32, (n,), b.view(np.uint8)))
        W[name] = (torch.from_numpy(O.dequantize(O.Q4_K, blocks, n, k)), None if b is None else torch.from_numpy(b))
    for name, shape in F.dense_shapes(cfg).items():
        v = rng.standard_normal(shape).astype(np.float32) * 0.02
        if name.endswith(".scale"):
            v = v + 1.0
        if name == "img_in.weight":
            h16 = v.astype(np.float16)
            tensors.append((name, O.F16, shape, h16.view(np.uint8)))
            D[name] = torch.from_numpy(h16.astype(np.float32))
        else:
            tensors.append((name, O.F32, shape, v.view(np.uint8)))
            D[name] = torch.from_numpy(v)
    path = str(tmp_path / "flux-tiny-q4_k.gguf")
    R.write(path, [("general.architecture", 8, "flux")], tensors)
    dev = mold_amd.Device(0)
    params = F.FluxParams.from_gguf(cfg, path, dev)
    # what the device holds is what the file holds (dense values converted exactly as
    # torch converts them; weights byte-identical)
    for name, (n, k, hb) in F.linear_shapes(cfg).items():
        qt = params.lin[name].matmul.w
        assert qt.dtype() == mold_amd.GgmlDType.Q4_K and qt.shape == (n, k)
        if hb:
            assert torch.equal(params.lin[name].bias.cpu(), W[name][1])
    for name, t in D.items():
        want = t if name.endswith(".bias") else t.to(torch.bfloat16)
        assert torch.equal(params.dense[name].cpu(), want), name
    inp = F.make_inputs(cfg, height=256, width=256, txt_len=32, device="cuda", seed=13)
    out = F.FluxStep(params).forward(**inp)
    torch.cuda.synchronize()
    ref = reference_forward(cfg, W, D, {k_: v.cpu() for k_, v in inp.items()})
    o = out.cpu().numpy()
    assert np.isfinite(o).all()
    err = _rel(o, ref.numpy())
    print(f"[flux] GGUF-loaded step rel-L2 vs f64 reference: {err:.3e}", flush=True)
    assert err <= STEP_TOL, err
