"""Qwen-Image-shaped step built on the quantized linears (the path's second caller).

The reference is an independent f64 restatement of mold's quantized Qwen-Image graph
(/root/reference/crates/mold-inference/src/qwen_image/quantized_transformer.rs:591-601
time embedding, :339-435 RoPE, :695-781 joint attention, :856-960 block, :977-989 output
layer): q, k, v as three separate linears on slices of the stacked weight, RoPE as a
complex rotation at closed-form positions (height/width position r - ceil(n/2), text
position max(h/2, w/2) + j), attention as an explicit f64 softmax.  The CPU test checks
`mold_amd.qwen_image`'s glue with dense linears; the GPU test checks the whole quantized
step (Q3_K / Q2_K / Q4_K linears) with the text stream overlapped on a second stream.
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

from mold_amd import qwen_image as Q  # noqa: E402
from mold_amd.flux import attention_f32  # noqa: E402

STEP_TOL = 1e-2


def _lin(W, name, x, rows=None):
    w, b = W[name]
    if rows is not None:
        w, b = w[rows], b[rows]
    return x.double() @ w.double().T + b.double()


def _ln(x):
    mu = x.mean(-1, keepdim=True)
    return (x - mu) / torch.sqrt(((x - mu) ** 2).mean(-1, keepdim=True) + 1e-6)


def _rms(x, s):
    return x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6) * s.double()


def _gelu(x):
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def _silu(x):
    return x / (1.0 + torch.exp(-x))


def _positions(gh, gw, lt):
    """[L, 3] positions (frame, height, width) for the image grid, then the text."""
    r = torch.arange(gh, dtype=torch.float64) - (gh - gh // 2)
    c = torch.arange(gw, dtype=torch.float64) - (gw - gw // 2)
    img = torch.stack([torch.zeros(gh, gw, dtype=torch.float64), r[:, None].expand(gh, gw),
                       c[None, :].expand(gh, gw)], dim=-1).reshape(-1, 3)
    tp = torch.arange(lt, dtype=torch.float64) + max(gh // 2, gw // 2)
    return img, tp[:, None].expand(lt, 3)


def _rope(x, pos, axes, theta):
    ang = []
    for a, d in enumerate(axes):
        j = torch.arange(d // 2, dtype=torch.float64)
        ang.append(pos[:, a:a + 1] * theta ** (-2.0 * j / d)[None, :])
    ang = torch.cat(ang, dim=1)
    xc = torch.view_as_complex(x.double().reshape(*x.shape[:-1], -1, 2).contiguous())
    return torch.view_as_real(xc * torch.polar(torch.ones_like(ang), ang)).reshape(x.shape)


def _attn(q, k, v):
    p = torch.softmax((q @ k.transpose(-1, -2)) / math.sqrt(q.shape[-1]), dim=-1)
    return (p @ v).transpose(0, 1).reshape(q.shape[1], -1)


def reference_forward(cfg, W, D, inp):
    H, hd, h = cfg.num_attention_heads, cfg.attention_head_dim, cfg.hidden_size
    gh, gw = inp["grid"]
    lt = inp["txt"].shape[0]
    ipos, tpos = _positions(gh, gw, lt)
    half = 128
    f = torch.exp(-math.log(10000.0) * torch.arange(half, dtype=torch.float64) / half)
    a = inp["t"].cpu().double()[:, None] * f[None]
    temb = _lin(W, "time_text_embed.timestep_embedder.linear_2",
                _silu(_lin(W, "time_text_embed.timestep_embedder.linear_1", torch.cat([a.cos(), a.sin()], 1))))
    img = inp["img"].cpu().double() @ D["img_in.weight"].double().T + D["img_in.bias"].double()
    txt = _lin(W, "txt_in", _rms(inp["txt"].cpu().double(), D["txt_norm.weight"]))
    st = _silu(temb)

    def heads(x, name, qn, kn, pos):
        L = x.shape[0]
        q, k, v = (_lin(W, name, x, slice(j * h, (j + 1) * h)).reshape(L, H, hd).transpose(0, 1)
                   for j in range(3))
        rope = lambda t: _rope(t, pos, cfg.axes_dims_rope, cfg.theta)  # noqa: E731
        return rope(_rms(q, D[qn])), rope(_rms(k, D[kn])), v

    for i in range(cfg.num_layers):
        p = f"transformer_blocks.{i}."
        im = _lin(W, p + "img_mod.1", st).reshape(6, h)
        tm = _lin(W, p + "txt_mod.1", st).reshape(6, h)
        iq, ik, iv = heads(_ln(img) * (1 + im[1]) + im[0], p + "attn.to_qkv",
                           p + "attn.norm_q.weight", p + "attn.norm_k.weight", ipos)
        tq, tk, tv = heads(_ln(txt) * (1 + tm[1]) + tm[0], p + "attn.add_qkv_proj",
                           p + "attn.norm_added_q.weight", p + "attn.norm_added_k.weight", tpos)
        att = _attn(torch.cat([tq, iq], 1), torch.cat([tk, ik], 1), torch.cat([tv, iv], 1))
        img = img + im[2] * _lin(W, p + "attn.to_out.0", att[lt:])
        txt = txt + tm[2] * _lin(W, p + "attn.to_add_out", att[:lt])
        img = img + im[5] * _lin(W, p + "img_mlp.net.2",
                                 _gelu(_lin(W, p + "img_mlp.net.0.proj", _ln(img) * (1 + im[4]) + im[3])))
        txt = txt + tm[5] * _lin(W, p + "txt_mlp.net.2",
                                 _gelu(_lin(W, p + "txt_mlp.net.0.proj", _ln(txt) * (1 + tm[4]) + tm[3])))
    om = _lin(W, "norm_out.linear", st).reshape(2, h)
    return _lin(W, "proj_out", _ln(img) * (1 + om[0]) + om[1])


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


class _DenseLinear:
    def __init__(self, w, b):
        self.w, self.b = w, b

    def forward(self, x, act=0, out_dtype=None):
        y = x.float() @ self.w.T + self.b
        if act == 1:
            y = torch.nn.functional.gelu(y, approximate="tanh")
        return y.to(out_dtype or x.dtype)


def test_qwen_glue_matches_reference_on_cpu():
    cfg = Q.QwenConfig.tiny()
    g = torch.Generator().manual_seed(9)
    W, lin = {}, {}
    for name, (n, k, _) in Q.linear_shapes(cfg).items():
        w, b = torch.randn((n, k), generator=g) * 0.02, torch.randn((n,), generator=g) * 0.02
        W[name] = (w, b)
        lin[name] = _DenseLinear(w, b)
    D = {}
    for name, shape in Q.dense_shapes(cfg).items():
        t = torch.randn(shape, generator=g) * 0.02
        D[name] = t if name.startswith("img_in") else t + 1.0
    params = Q.QwenParams(cfg, lin, D)
    inp = Q.make_inputs(cfg, height=112, width=96, txt_len=12, device="cpu", seed=3)
    out = Q.QwenImageStep(params, attn=attention_f32,
                          gemm_dtype=torch.float32).forward(**inp)
    ref = reference_forward(cfg, W, D, inp)
    assert out.shape == (7 * 6, 64)
    assert _rel(out.numpy(), ref.numpy()) < 1e-5


def test_qwen_rope_positions_follow_reference_layout():
    """Odd grid (83 x 83 at 1328^2): centred positions -42..40, text from 41."""
    cfg = Q.QwenConfig.image()
    ic, is_, tc, ts = Q.rope_tables(cfg, 1, 83, 83, 256, "cpu")
    assert ic.shape == (6889, 64) and tc.shape == (256, 64)
    ang = torch.atan2(is_, ic)
    # first image token: frame 0, height -42, width -42; width axis j=0 has frequency 1
    assert abs(ang[0, 8 + 28].item() - math.remainder(-42.0, 2 * math.pi)) < 1e-5
    assert abs(ang[0, 8].item() - math.remainder(-42.0, 2 * math.pi)) < 1e-5
    assert torch.all(ang[:, 0] == 0)
    tang = torch.atan2(ts, tc)
    assert abs(tang[0, 0].item() - math.remainder(41.0, 2 * math.pi)) < 1e-5


def test_qwen_step_flop_accounting():
    cfg = Q.QwenConfig.image()
    lin, attn = Q.step_flop(cfg, 6889, 256)
    # 60 blocks: img 2*6889*(9216+3072+2*12288)*3072 + txt 2*256*(...)*3072, plus stems
    per_tok = 2.0 * (9216 + 3072 + 2 * 12288) * 3072
    expect = 60 * (6889 + 256) * per_tok + 2.0 * 256 * 3072 * 3584 + 2.0 * 6889 * 64 * 3072
    assert abs(lin / expect - 1) < 1e-12
    assert abs(lin / 9.71e13 - 1) < 3e-3, lin
    assert abs(attn / 3.76e13 - 1) < 3e-3, attn
    assert len(Q.linear_shapes(cfg)) == 5 + 60 * 10


@pytest.mark.gpu
def test_qwen_step_tiny_matches_dequantized_reference():
    import mold_amd
    from oracle import oracle as O
    cfg = Q.QwenConfig.tiny()
    print(f"[qwen] tiny step: hidden {cfg.hidden_size}, Q3_K/Q2_K/Q4_K, overlapped text stream", flush=True)
    dev = mold_amd.Device(0)
    params = Q.QwenParams.random(cfg, dev, seed=8)
    inp = Q.make_inputs(cfg, height=272, width=240, txt_len=40, device="cuda", seed=8)
    step = Q.QwenImageStep(params)
    out = step.forward(**inp)
    out2 = step.forward(**inp)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "step is not deterministic"
    W = {}
    for name, l in params.lin.items():
        qt = l.matmul.w
        n, k = qt.shape
        W[name] = (torch.from_numpy(O.dequantize(int(qt.dtype()), qt.data(), n, k)), l.bias.cpu())
    D = {k_: v.float().cpu() for k_, v in params.dense.items()}
    ref = reference_forward(cfg, W, D, {k_: (v.cpu() if hasattr(v, "cpu") else v) for k_, v in inp.items()})
    o = out.cpu().numpy()
    assert np.isfinite(o).all()
    err = _rel(o, ref.numpy())
    print(f"[qwen] rel-L2 vs f64 dequantized reference: {err:.3e}", flush=True)
    assert err <= STEP_TOL, err
    # the serial (single-stream) order gives the same values, and so do the
    # modulations run one GEMV per block instead of one stacked GEMV
    ser = Q.QwenImageStep(params, overlap=False).forward(**inp)
    sep = Q.QwenImageStep(params)
    sep.stack_modulations = False
    out_sep = sep.forward(**inp)
    torch.cuda.synchronize()
    assert step._mod_stack is not None and sep._mod_stack is None
    assert torch.equal(out, ser)
    assert torch.equal(out, out_sep)


@pytest.mark.gpu
def test_qwen_step_from_mold_layout_gguf(tmp_path):
    """A tiny-config Qwen-Image GGUF in mold's layout, written by an independent
    restatement of the container (tests/gguf_ref.py): the config's quantized types per
    role (Q3_K attention, Q2_K MLP, Q4_K elsewhere), separate to_q / to_k / to_v and
    add_q_proj / add_k_proj / add_v_proj tensors, F32 biases and RmsNorm weights, a BF16
    img_in weight, mold's tensor names, GGUF ne order.  QwenParams.from_gguf loads it
    through the C ABI alone (one mq_gguf_load_tensors call, the q/k/v weights stacked on
    the device by mq_qtensor_concat_rows), and the step matches the f64 restatement on
    the file's own values within the 1e-2 bar."""
    import mold_amd
    from oracle import oracle as O
    from . import gguf_ref as R
    cfg = Q.QwenConfig.tiny()
    print("[qwen] tiny step from a mold-layout GGUF", flush=True)
    rng = np.random.default_rng(21)
    tensors, W, D = [], {}, {}
    for name, (n, k, role) in Q.linear_shapes(cfg).items():
        t = int(cfg.qtype(role))
        if name.endswith("attn.to_qkv") or name.endswith("attn.add_qkv_proj"):
            p = name[: name.rindex(".") + 1]
            subs = ["to_q", "to_k", "to_v"] if name.endswith("to_qkv") else ["add_q_proj", "add_k_proj", "add_v_proj"]
            names, rows = [p + s_ for s_ in subs], [n // 3] * 3
        else:
            names, rows = [name], [n]
        ws, bs = [], []
        for nm, r in zip(names, rows):
            w = (rng.standard_normal((r, k)) * 0.02).astype(np.float32)
            blocks = O.quantize(t, w)
            b = (rng.standard_normal(r) * 0.02).astype(np.float32)
            tensors.append((nm + ".weight", t, (r, k), blocks))
            tensors.append((nm + ".bias", O.F32, (r,), b.view(np.uint8)))
            ws.append(torch.from_numpy(O.dequantize(t, blocks, r, k)))
            bs.append(torch.from_numpy(b))
        W[name] = (torch.cat(ws), torch.cat(bs))
    for name, shape in Q.dense_shapes(cfg).items():
        v = rng.standard_normal(shape).astype(np.float32) * 0.02
        if name.endswith(".bias"):
            tensors.append((name, O.F32, shape, v.view(np.uint8)))
            D[name] = torch.from_numpy(v)
            continue
        if name != "img_in.weight":
            v = v + 1.0
        b16 = torch.from_numpy(v).to(torch.bfloat16)
        tensors.append((name, O.BF16, shape, b16.view(torch.int16).numpy().view(np.uint8).reshape(-1)))
        D[name] = b16.float()
    path = str(tmp_path / "qwen-tiny-mixed.gguf")
    R.write(path, [("general.architecture", 8, "qwen_image")], tensors)
    dev = mold_amd.Device(0)
    params = Q.QwenParams.from_gguf(cfg, path, dev)
    for name, (n, k, role) in Q.linear_shapes(cfg).items():
        qt = params.lin[name].matmul.w
        assert qt.dtype() == cfg.qtype(role) and qt.shape == (n, k), name
        assert torch.equal(params.lin[name].bias.cpu(), W[name][1]), name
        if qt.shape[0] == n:   # the stacked weights are the parts' blocks in order
            assert torch.equal(torch.from_numpy(O.dequantize(int(qt.dtype()), qt.data(), n, k)), W[name][0]), name
    for name, t in D.items():
        want = t if name.endswith(".bias") else t.to(torch.bfloat16)
        assert torch.equal(params.dense[name].cpu().to(want.dtype), want), name
    inp = Q.make_inputs(cfg, height=272, width=240, txt_len=40, device="cuda", seed=8)
    out = Q.QwenImageStep(params).forward(**inp)
    torch.cuda.synchronize()
    ref = reference_forward(cfg, W, {k_: v.float() for k_, v in D.items()},
                            {k_: (v.cpu() if hasattr(v, "cpu") else v) for k_, v in inp.items()})
    o = out.cpu().numpy()
    assert np.isfinite(o).all()
    err = _rel(o, ref.numpy())
    print(f"[qwen] GGUF-loaded step rel-L2 vs f64 reference: {err:.3e}", flush=True)
    assert err <= STEP_TOL, err


@pytest.mark.gpu
def test_qwen_cfg_batch2_matches_two_single_forwards():
    """Batched CFG forward (cond + uncond along dim 0, the uncond prompt shorter
    and padded, its padding masked out of attention) against two batch-1 forwards
    (the uncond one on its valid tokens only) and against the f64 restatement."""
    import mold_amd
    from oracle import oracle as O
    cfg = Q.QwenConfig.tiny()
    print("[qwen] tiny CFG batch-2 forward with a masked uncond prompt", flush=True)
    dev = mold_amd.Device(0)
    params = Q.QwenParams.random(cfg, dev, seed=11)
    inp = Q.make_inputs(cfg, height=272, width=240, txt_len=40, device="cuda", seed=11)
    g = torch.Generator(device="cuda").manual_seed(12)
    txt_u = torch.randn(inp["txt"].shape, device="cuda", generator=g)
    nv = 33
    txt_u[nv:] = 0.0                                   # the padded tail (masked)
    step = Q.QwenImageStep(params)
    img2 = torch.stack([inp["img"], inp["img"]])
    txt2 = torch.stack([inp["txt"], txt_u])
    t2 = torch.cat([inp["t"], inp["t"]])
    out = step.forward_batched(img2, txt2, t2, inp["grid"], txt_valid=[40, nv])
    out_b = step.forward_batched(img2, txt2, t2, inp["grid"], txt_valid=[40, nv])
    c0 = step.forward(inp["img"], inp["txt"], inp["t"], inp["grid"])
    u0 = step.forward(inp["img"], txt_u[:nv].contiguous(), inp["t"], inp["grid"])
    sep = Q.QwenImageStep(params)
    sep.stack_modulations = False
    out_sep = sep.forward_batched(img2, txt2, t2, inp["grid"], txt_valid=[40, nv])
    torch.cuda.synchronize()
    assert torch.equal(out, out_b), "batched forward is not deterministic"
    assert torch.equal(out, out_sep), "stacked (M = 2) and per-block modulation GEMVs differ"
    assert out.shape == (2,) + tuple(c0.shape) and torch.isfinite(out).all().item()
    e0, e1 = _rel(out[0].cpu().numpy(), c0.cpu().numpy()), _rel(out[1].cpu().numpy(), u0.cpu().numpy())
    print(f"[qwen] batched vs single: cond {e0:.2e}  uncond(masked) {e1:.2e}", flush=True)
    assert e0 <= 1e-3 and e1 <= 1e-3
    W = {}
    for name, l in params.lin.items():
        qt = l.matmul.w
        n, k = qt.shape
        W[name] = (torch.from_numpy(O.dequantize(int(qt.dtype()), qt.data(), n, k)), l.bias.cpu())
    D = {k_: v.float().cpu() for k_, v in params.dense.items()}
    ref_u = reference_forward(cfg, W, D, {"img": inp["img"].cpu(), "txt": txt_u[:nv].cpu(), "t": inp["t"].cpu(),
                                          "grid": inp["grid"]})
    err = _rel(out[1].cpu().numpy(), ref_u.numpy())
    print(f"[qwen] batched uncond vs f64 restatement on its valid tokens: {err:.2e}", flush=True)
    assert err <= STEP_TOL
