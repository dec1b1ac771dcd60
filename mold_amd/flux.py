"""FLUX.1-dev-shaped transformer step whose linears are libmoldq quantized linears.

This is the caller of the quantized-linear path that mold runs for quantized
FLUX models: every `Linear` of the transformer is a GGUF weight driven by
`QMatMul::forward` (here `mold_amd.Linear`), the glue (norms, modulation,
RoPE, attention, residuals) is ordinary tensor work.  The block graph, its op
order and constants follow mold's self-contained FLUX blocks,
/root/reference/crates/mold-inference/src/flux/offload.rs:
  timestep_embedding           :21-37   (t * 1000, 10000^(-i/half), [cos, sin])
  attention / apply_rope       :39-73   (RoPE on pairs, softmax(q k^T / sqrt(d)) v)
  LayerNorm without affine     :75-78   (eps 1e-6);  RmsNorm eps 1e-6 (:160-167)
  Modulation1 / Modulation2    :105-156 (silu(vec) -> lin -> 3 / 6 chunks)
  SelfAttention.qkv            :188-201 (reshape [L, 3, H, D], q/k RmsNorm)
  Mlp                          :222-224 (lin1 -> gelu(tanh) -> lin2)
  DoubleBlock.forward          :276-325 (txt tokens first in the joint sequence)
  SingleBlock.forward          :374-392 (linear1 -> [qkv | mlp], linear2 on [attn | gelu(mlp)])
  FinalLayer.forward           :413-422 (adaLN shift, scale; norm; linear)
  forward (stems and order)    :523-574
The position embedding is FLUX's EmbedNd (candle-transformers flux model,
called at offload.rs:534-537): per axis i of the 3-D token ids, angles
pos * theta^(-2j/d_i) for j < d_i/2, concatenated over axes, rotating each
(even, odd) pair of q and k.

Activations are f32, as in mold's quantized FLUX path
(crates/mold-inference/src/flux/pipeline.rs:1524,1639-1647).  MI355X
choices, each documented where it is made: on the GPU the modulate and the
q/k norm + RoPE + head split run as libmoldq's fused row passes
(mold_amd.fused), one HBM pass each instead of a dozen elementwise ops, and
each gated residual update x + gate * linear(h) is the GEMM's epilogue
(Linear.gated_add, updating x in place); a tensor whose only consumer is a quantized GEMM is produced directly in bf16
(the GEMM rounds its input to bf16 with round-to-nearest-even either way, so
the f32 -> bf16 staging pass disappears); attention runs in bf16 with f32
softmax accumulation (PyTorch's fused attention) rather than as three f32 ops;
and every block's adaLN modulation linear, which reads the same silu(vec),
runs in one GEMV over the stacked modulation weights (StackedLinear) at the
start of the forward, with outputs identical to the per-block linears.

Weights are synthetic (no checkpoint exists here): every linear weight is
N(0, 0.02^2) quantized on the GPU to the configured GGUF type, biases are f32
N(0, 0.02^2), RmsNorm scales are bf16 N(1, 0.02^2), and `img_in` (K = 64 is not
a multiple of a k-quant's 256-wide super-block) stays a dense bf16 weight.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Dict, Optional, Tuple

import numpy as np

from .quantized import ACT_GELU_TANH, ACT_NONE, GgmlDType, Linear, QTensor


@dataclass(frozen=True)
class FluxConfig:
    """candle-transformers `flux::model::Config::dev()` shape."""
    in_channels: int = 64
    vec_in_dim: int = 768
    context_in_dim: int = 4096
    hidden_size: int = 3072
    mlp_ratio: float = 4.0
    num_heads: int = 24
    depth: int = 19
    depth_single_blocks: int = 38
    axes_dim: Tuple[int, int, int] = (16, 56, 56)
    theta: float = 10000.0
    qkv_bias: bool = True
    guidance_embed: bool = True

    @property
    def mlp_size(self) -> int:
        return int(self.hidden_size * self.mlp_ratio)

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads

    @staticmethod
    def dev() -> "FluxConfig":
        return FluxConfig()

    @staticmethod
    def tiny() -> "FluxConfig":
        """Same graph at hidden 256 (2 heads of 128) with one block of each kind."""
        return FluxConfig(vec_in_dim=256, context_in_dim=256, hidden_size=256, num_heads=2,
                          depth=1, depth_single_blocks=1)


def linear_shapes(cfg: FluxConfig) -> Dict[str, Tuple[int, int, bool]]:
    """name -> (out_features, in_features, has_bias) for every quantized linear."""
    h, mlp = cfg.hidden_size, cfg.mlp_size
    s: Dict[str, Tuple[int, int, bool]] = {
        "txt_in": (h, cfg.context_in_dim, True),
        "time_in.in_layer": (h, 256, True), "time_in.out_layer": (h, h, True),
        "vector_in.in_layer": (h, cfg.vec_in_dim, True), "vector_in.out_layer": (h, h, True),
        "final_layer.adaLN_modulation.1": (2 * h, h, True),
        "final_layer.linear": (cfg.in_channels, h, True),
    }
    if cfg.guidance_embed:
        s["guidance_in.in_layer"] = (h, 256, True)
        s["guidance_in.out_layer"] = (h, h, True)
    for i in range(cfg.depth):
        p = f"double_blocks.{i}."
        for st in ("img", "txt"):
            s[p + f"{st}_mod.lin"] = (6 * h, h, True)
            s[p + f"{st}_attn.qkv"] = (3 * h, h, cfg.qkv_bias)
            s[p + f"{st}_attn.proj"] = (h, h, True)
            s[p + f"{st}_mlp.0"] = (mlp, h, True)
            s[p + f"{st}_mlp.2"] = (h, mlp, True)
    for i in range(cfg.depth_single_blocks):
        p = f"single_blocks.{i}."
        s[p + "modulation.lin"] = (3 * h, h, True)
        s[p + "linear1"] = (3 * h + mlp, h, True)
        s[p + "linear2"] = (h, h + mlp, True)
    return s


def dense_shapes(cfg: FluxConfig) -> Dict[str, Tuple[int, ...]]:
    """Non-quantized parameters: img_in (bf16 weight, f32 bias) and RmsNorm scales."""
    h, d = cfg.hidden_size, cfg.head_dim
    s: Dict[str, Tuple[int, ...]] = {"img_in.weight": (h, cfg.in_channels), "img_in.bias": (h,)}
    for i in range(cfg.depth):
        for st in ("img", "txt"):
            for nm in ("query_norm", "key_norm"):
                s[f"double_blocks.{i}.{st}_attn.norm.{nm}.scale"] = (d,)
    for i in range(cfg.depth_single_blocks):
        for nm in ("query_norm", "key_norm"):
            s[f"single_blocks.{i}.norm.{nm}.scale"] = (d,)
    return s


class FluxParams:
    """The transformer's parameters: `lin[name]` objects with
    `forward(x, act=ACT_NONE, out_dtype=None)` (bias applied inside), and
    `dense[name]` tensors."""

    def __init__(self, cfg: FluxConfig, lin: Dict[str, object], dense: Dict[str, object]):
        self.cfg, self.lin, self.dense = cfg, lin, dense

    @staticmethod
    def random(cfg: FluxConfig, device, qtype: GgmlDType = GgmlDType.Q4_K, seed: int = 4) -> "FluxParams":
        """Synthetic weights generated and quantized on `device` (a mold_amd.Device)."""
        import torch
        cuda = f"cuda:{device.ordinal}"
        lin, dense = {}, {}
        for idx, (name, (n, k, has_bias)) in enumerate(linear_shapes(cfg).items()):
            g = torch.Generator(device=cuda).manual_seed(seed * 1_000_003 + 2 * idx)
            w = torch.randn((n, k), device=cuda, generator=g) * 0.02
            qt = QTensor.quantize(device, w, qtype)
            del w
            bias = None
            if has_bias:
                g = torch.Generator(device=cuda).manual_seed(seed * 1_000_003 + 2 * idx + 1)
                bias = torch.randn((n,), device=cuda, generator=g) * 0.02
            lin[name] = Linear(qt, bias)
        for idx, (name, shape) in enumerate(dense_shapes(cfg).items()):
            g = torch.Generator(device=cuda).manual_seed(seed * 7_000_003 + idx)
            t = torch.randn(shape, device=cuda, generator=g) * 0.02
            if name.endswith(".scale"):
                t = (t + 1.0).to(torch.bfloat16)
            elif name == "img_in.weight":
                t = t.to(torch.bfloat16)
            dense[name] = t
        return FluxParams(cfg, lin, dense)

    @staticmethod
    def from_gguf(cfg: FluxConfig, path: str, device) -> "FluxParams":
        """The transformer's parameters from a GGUF file in mold's layout (candle's
        FLUX tensor names, `<linear>.weight` / `<linear>.bias`, norm `.scale`s,
        `img_in`), loaded the way mold's `VarBuilder::from_gguf` does
        (crates/mold-inference/src/flux/pipeline.rs:976-977): every tensor goes to
        the device through libmoldq in one pipelined call (mq_gguf_load_tensors),
        block-type weights stay quantized, and dense tensors (F32 / F16 / BF16)
        are dequantized on the device to the dtypes the step uses (f32 biases,
        bf16 norm scales and img_in weight).  No tensor byte passes through the
        host here except on the upload itself."""
        import torch
        from . import gguf
        need = {}
        for name, (n, k, has_bias) in linear_shapes(cfg).items():
            need[name + ".weight"] = (n, k)
            if has_bias:
                need[name + ".bias"] = (n,)
        need.update(dense_shapes(cfg))
        c = gguf.Content.read(path)
        try:
            for name in need:
                if name not in c.tensor_infos:
                    raise KeyError(f"{path}: tensor {name} missing")
            qts = c.tensors(need.keys(), device)
        finally:
            c.close()
        for name, shape in need.items():
            want = (int(np.prod(shape[:-1])) if len(shape) > 1 else 1, shape[-1])
            if qts[name].shape != want:
                raise ValueError(f"{name}: stored as {qts[name].shape}, the config needs {tuple(shape)}")
        lin, dense = {}, {}
        for name, (n, k, has_bias) in linear_shapes(cfg).items():
            qt = qts[name + ".weight"]
            if not qt.dtype().is_quantized:
                raise ValueError(f"{name}.weight is dense {qt.dtype().name}; the step runs quantized linears")
            bias = qts[name + ".bias"].dequantize(torch.float32).reshape(n) if has_bias else None
            lin[name] = Linear(qt, bias)
        for name, shape in dense_shapes(cfg).items():
            dt = torch.float32 if name.endswith(".bias") else torch.bfloat16
            dense[name] = qts[name].dequantize(dt).reshape(shape)
        return FluxParams(cfg, lin, dense)

    def quantized_bytes(self) -> int:
        return sum(l.matmul.w.storage_size_in_bytes() for l in self.lin.values())


# --------------------------------------------------------------------------- glue

def timestep_embedding(t, dim: int):
    """offload.rs:21-37.  t: [B] f32 -> [B, dim] f32."""
    import torch
    half = dim // 2
    freqs = torch.exp(torch.arange(half, dtype=torch.float32, device=t.device) * (-math.log(10000.0) / half))
    args = (t.float() * 1000.0)[:, None] * freqs[None, :]
    return torch.cat([torch.cos(args), torch.sin(args)], dim=-1)


def rope_angles(ids, axes_dim, theta: float):
    """EmbedNd angles: ids [L, n_axes] f32 -> [L, sum(axes_dim)/2] f32."""
    import torch
    parts = []
    for i, d in enumerate(axes_dim):
        inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float64, device=ids.device) / d))
        parts.append(ids[:, i:i + 1].double() * inv[None, :])
    return torch.cat(parts, dim=-1).float()


def apply_rope(x, cos, sin):
    """offload.rs:56-66: x [H, L, D]; pair (x[2j], x[2j+1]) rotated by angle j."""
    x2 = x.reshape(*x.shape[:-1], -1, 2)
    x0, x1 = x2[..., 0], x2[..., 1]
    out = (cos * x0 - sin * x1, sin * x0 + cos * x1)
    import torch
    return torch.stack(out, dim=-1).reshape(x.shape)


def rms_norm(x, scale):
    import torch
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * scale.float()


def layer_norm(x):
    import torch
    return torch.nn.functional.layer_norm(x, (x.shape[-1],), eps=1e-6)


def gelu_tanh(x):
    import torch
    return torch.nn.functional.gelu(x, approximate="tanh")


def silu(x):
    import torch
    return torch.nn.functional.silu(x)


_AUX: Dict[int, object] = {}


def aux_stream(device):
    """One extra stream per device (default priority) for a block's second token stream."""
    import torch
    idx = device.index if device.index is not None else torch.cuda.current_device()
    s = _AUX.get(idx)
    if s is None:
        s = torch.cuda.Stream(device=idx)
        _AUX[idx] = s
    return s


def text_stream(device, ctx):
    """aux_stream(device) for a block's text-token linears, with libmoldq's
    tail K split turned off on it for the library context `ctx` (a
    mold_amd.Device): those GEMMs run beside the image stream's, which keep
    the CUs busy, so splitting their partial last round of tiles only adds
    partial-sum traffic and reduce launches (FLUX step 0.7-0.9 % and
    Qwen-Image 1.5-3.7 % faster, same-box pairs on two boxes)."""
    s = aux_stream(device)
    done = ctx.__dict__.setdefault("_tail_split_off", set())
    if s.cuda_stream not in done:
        ctx.set_stream_tail_split(s, False)
        done.add(s.cuda_stream)
    return s


ATTENTION_BACKEND = {"name": None}


ATTN_ROWS = 256  # the fused paths pad the joint sequence to a multiple of this


def padded_len(n: int) -> int:
    return (n + ATTN_ROWS - 1) // ATTN_ROWS * ATTN_ROWS


# A padded row's share of softmax mass on its valid keys, 1 - n_pad exp(-lse),
# below which the zero-key correction is not used: dividing by a share that
# small would amplify the f32 error of lse past bf16 precision (and a share
# that cancels to zero or below gives inf or garbage), so such rows are
# recomputed over their valid keys alone.
PAD_MIN_SHARE = 2.0 ** -10


def _attention_chunked(qb, kb, vb, drop: Optional[Tuple[int, int]] = None):
    """Attention of bf16 q, k, v [H, L, D] -> [L, H*D] bf16, head-chunked, with
    scores, softmax and the value product in f32 (scores rounded to bf16 would
    err by ~0.05 at |q.k| ~ 150); the right operand of every batched product is
    made contiguous first (k^T explicitly).  Keys drop[0] .. drop[1]-1 are
    masked out (score -inf)."""
    import torch
    h, l, d = qb.shape
    out = torch.empty((l, h * d), dtype=torch.bfloat16, device=qb.device)
    scale = 1.0 / math.sqrt(d)
    step = max(1, min(h, (1 << 31) // max(1, l * l * 4)))
    for h0 in range(0, h, step):
        h1 = min(h, h0 + step)
        kt = kb[h0:h1].transpose(1, 2).float().contiguous()
        s = torch.matmul(qb[h0:h1].float(), kt) * scale
        if drop is not None and drop[1] > drop[0]:
            s[..., drop[0]:drop[1]] = float("-inf")
        p = torch.softmax(s, dim=-1)
        o = torch.matmul(p, vb[h0:h1].float().contiguous())
        out.view(l, h, d)[:, h0:h1] = o.transpose(0, 1)
    return out


def _no_fused_kernel(err: RuntimeError) -> bool:
    """True when PyTorch reports that no fused attention kernel serves the device
    or shape (as opposed to a failure such as running out of memory)."""
    msg = str(err).lower()
    if "out of memory" in msg:
        return False
    return any(s in msg for s in ("no available kernel", "not supported", "not implemented", "no kernel image",
                                  "invalid device function", "not compiled"))


def attention_bf16(q, k, v, valid: Optional[int] = None, guard=None, drop: Optional[Tuple[int, int]] = None,
                   out=None):
    """softmax(q k^T / sqrt(d)) v for q, k, v [H, L, D] -> [valid, H*D] bf16.

    Runs PyTorch's fused attention in bf16 (f32 softmax accumulation inside; on
    ROCm that is AOTriton's `attn_fwd` kernel).  `valid` < L marks rows
    valid .. L-1 as padding whose k and v rows are zero: the fused kernels run
    much faster at lengths that are multiples of 256 (1.0 vs 2.0 ms at
    24 x 7168 vs 7145 tokens on an MI355X).  Each of the n_pad zero keys adds
    exp(0) = 1 to a row's softmax denominator Z and nothing to its numerator, so
    with the log-sum-exp the kernel returns, out = out_pad / s with
    s = 1 - n_pad exp(-lse), the row's share of mass on its valid keys.  That
    division only rescales the bf16 out_pad; its error is that of s, which stays
    far below bf16 precision while s >= PAD_MIN_SHARE.  Rows under that share
    (every valid score below about -10) are recomputed exactly over the valid
    keys: with `guard` None this call finds them (one host synchronization) and
    recomputes their heads; with `guard`, a 0-dim f32 device tensor, it only
    raises guard to the largest 1 - s seen, and the caller checks it once
    (FluxStep.forward reruns the step unpadded if any row fell under the share).

    `drop` = (lo, hi) masks keys lo .. hi-1 (a text attention mask, e.g. the
    padded tail of a shorter prompt in a CFG batch): their k and v rows must be
    zero, so they are removed by the same correction (n_pad counts them too).

    `out`, a bf16 [valid, H*D] tensor whose rows may be strided (a column block
    of a wider buffer), receives the result in place of a new tensor: the
    correction pass writes it there, the unpadded path copies its [H, L, D]
    output there once.

    Where no fused kernel serves the device, it falls back to the exact
    head-chunked path on the valid rows (any other error propagates).  The
    backend used is recorded in ATTENTION_BACKEND."""
    import torch
    h, l, d = q.shape
    valid = l if valid is None else valid
    qb, kb, vb = (t.to(torch.bfloat16).contiguous() for t in (q, k, v))
    n_drop = 0 if drop is None else max(0, drop[1] - drop[0])
    if out is not None and (out.shape != (valid, h * d) or out.dtype != torch.bfloat16 or out.stride(1) != 1):
        raise ValueError(f"attention_bf16: out must be bf16 [{valid}, {h * d}] with unit column stride")
    if ATTENTION_BACKEND["name"] in (None, "fused"):
        try:
            if valid < l or n_drop:
                o_pad, lse = torch.ops.aten._scaled_dot_product_efficient_attention(qb[None], kb[None], vb[None],
                                                                                    None, True)[:2]
                if guard is not None:
                    # one fused pass (libmoldq): the share, the f32 correction, bf16, the
                    # [valid, h*d] layout and the guard
                    from .fused import attn_pad_correct
                    res = (out if out is not None
                           else torch.empty((valid, h * d), dtype=torch.bfloat16, device=q.device))
                    attn_pad_correct(o_pad, lse, _npad(q.device, (l - valid + n_drop,)), valid, guard, res)
                    ATTENTION_BACKEND["name"] = "fused"
                    return res
                pad_share = (l - valid + n_drop) * torch.exp(-lse[0, :, :valid])  # [h, valid] f32, 1 - s
                # one pass: correct in f32, round to bf16, write the [valid, h, d] layout
                res = (out.view(valid, h, d) if out is not None
                       else torch.empty((valid, h, d), dtype=torch.bfloat16, device=q.device))
                torch.mul(o_pad[0, :, :valid].transpose(0, 1), (1.0 / (1.0 - pad_share)).transpose(0, 1)[..., None],
                          out=res)
                bad = (pad_share > 1.0 - PAD_MIN_SHARE).any(dim=1)
                if bool(bad.any()):
                    heads = bad.nonzero().flatten()
                    exact = _attention_chunked(qb[heads, :valid], kb[heads, :valid], vb[heads, :valid], drop)
                    res[:, heads] = exact.view(valid, heads.numel(), d)
                ATTENTION_BACKEND["name"] = "fused"
                return out if out is not None else res.reshape(valid, h * d)
            else:
                # the memory-efficient entry: its output is laid out token-major ([L, H, D]
                # under the [H, L, D] view), so the [L, H*D] result below is a view, and it
                # runs faster than the flash entry at these shapes (24 x 4608 x 128 on an
                # MI355X: 504 vs 541 us, identical values, and flash's head-major output
                # needed a 21.5 us transposing copy)
                o = torch.ops.aten._scaled_dot_product_efficient_attention(qb[None], kb[None], vb[None], None,
                                                                           False)[0][0]
            ATTENTION_BACKEND["name"] = "fused"
            if out is not None:
                out.view(valid, h, d).copy_(o.transpose(0, 1))
                return out
            return o.transpose(0, 1).reshape(valid, h * d)
        except RuntimeError as err:
            if not _no_fused_kernel(err):
                raise
            ATTENTION_BACKEND["name"] = "chunked"
    res = _attention_chunked(qb[:, :valid], kb[:, :valid], vb[:, :valid], drop)
    if out is not None:
        out.copy_(res)
        return out
    return res


_NPAD_CACHE: dict = {}


def _npad(device, counts):
    """f32 [len(counts)] device tensor of the zero-key counts, uploaded once per
    distinct padding (not per call)."""
    import torch
    key = (device, tuple(counts))
    t = _NPAD_CACHE.get(key)
    if t is None:
        t = torch.tensor(counts, dtype=torch.float32, device=device)
        _NPAD_CACHE[key] = t
    return t


def attention_bf16_batch(q, k, v, valid: int, guard, drops):
    """attention_bf16 over a batch in one fused launch: q, k, v bf16 [B, H, L, D]
    (contiguous), rows valid .. L-1 of every element zero padding, drops[b] =
    (lo, hi) or None the masked keys of element b (zero k and v rows).  Each
    element's output is corrected by its own share s_b = 1 - n_b exp(-lse),
    n_b its padded plus dropped keys, and `guard` (required here) is raised to
    the largest 1 - s seen.  Returns [B, valid, H*D] bf16.  Without a guard, or
    where no fused kernel serves the device, each element goes through
    attention_bf16 (which recomputes ill-conditioned rows itself)."""
    import torch
    b_, h, l, d = q.shape
    per_element = lambda: torch.stack([attention_bf16(q[b], k[b], v[b], valid=valid, guard=guard, drop=drops[b])
                                       for b in range(b_)])
    if guard is None or ATTENTION_BACKEND["name"] not in (None, "fused"):
        return per_element()
    try:
        out, lse = torch.ops.aten._scaled_dot_product_efficient_attention(q, k, v, None, True)[:2]
    except RuntimeError as err:
        if not _no_fused_kernel(err):
            raise
        ATTENTION_BACKEND["name"] = "chunked"
        return per_element()
    counts = tuple(l - valid + (0 if dr is None else max(0, dr[1] - dr[0])) for dr in drops)
    from .fused import attn_pad_correct
    res = torch.empty((b_, valid, h * d), dtype=torch.bfloat16, device=q.device)
    attn_pad_correct(out, lse, _npad(q.device, counts), valid, guard, res)
    ATTENTION_BACKEND["name"] = "fused"
    return res


def attention_f32(q, k, v):
    """Same in f32 (the host-CPU leg)."""
    import torch
    h, l, d = q.shape
    o = torch.nn.functional.scaled_dot_product_attention(q[None], k[None], v[None])
    return o[0].transpose(0, 1).reshape(l, h * d)


def run_guarded(step, fwd, *args):
    """Run a step forward with padded attention under one guard: afterwards one
    host synchronization reads the largest pad share of any padded row, and if
    some row's valid-key share fell below PAD_MIN_SHARE the step reruns with
    unpadded attention buffers (exact, slower)."""
    import torch
    x = args[0]
    use = x.is_cuda and step.attn is attention_bf16 and step.pad_attention
    step._guard = torch.zeros((), dtype=torch.float32, device=x.device) if use else None
    try:
        out = fwd(*args)
        if use and float(step._guard) > 1.0 - PAD_MIN_SHARE:
            step._guard = None
            step.pad_attention = False
            try:
                out = fwd(*args)
            finally:
                step.pad_attention = True
    finally:
        step._guard = None
    return out


class FluxStep:
    """One denoising-step forward of the FLUX transformer (batch 1).

    `attn` computes attention ([H, L, D] f32 x3 -> [L, H*D]); `gemm_dtype` is the
    dtype in which tensors consumed only by a quantized linear are produced
    (bf16 on the GPU, see the module docstring)."""

    def __init__(self, params: FluxParams, attn: Callable = attention_bf16, gemm_dtype=None,
                 fused: Optional[bool] = None):
        import torch
        self.p, self.cfg = params, params.cfg
        self.attn = attn
        self.gemm_dtype = torch.bfloat16 if gemm_dtype is None else gemm_dtype
        self.fused = fused
        self.gated_epilogue = True
        # fused path: projections that feed only the fused passes (qkv, linear1) are written in bf16
        self.bf16_projections = True
        self.pad_attention = True
        self._guard = None
        # every modulation linear reads silu(vec): on the GPU they run as one
        # stacked GEMV per forward (StackedLinear, built on first use)
        self.stack_modulations = True
        self._mod_stack = None
        self._mods = None

    def _fused(self, x) -> bool:
        """Use libmoldq's fused row passes (mold_amd.fused) for the modulate and the
        q/k norm + RoPE + head split: by default on the GPU with bf16 GEMM inputs."""
        import torch
        if self.fused is not None:
            return self.fused
        return x.is_cuda and self.gemm_dtype == torch.bfloat16

    # -- pieces, each following offload.rs
    def _mod(self, name, vec, n):
        y = self._mods[name] if self._mods is not None else self.p.lin[name].forward(silu(vec))
        return y.chunk(n, dim=-1)

    def modulation_names(self):
        """The modulation linears in run order (each reads silu(vec))."""
        cfg = self.cfg
        names = []
        for i in range(cfg.depth):
            names += [f"double_blocks.{i}.img_mod.lin", f"double_blocks.{i}.txt_mod.lin"]
        names += [f"single_blocks.{i}.modulation.lin" for i in range(cfg.depth_single_blocks)]
        return names + ["final_layer.adaLN_modulation.1"]

    def _stacked_mods(self, vec):
        from .quantized import StackedLinear
        parts = [(nm, self.p.lin[nm]) for nm in self.modulation_names()]
        if self._mod_stack is None or not self._mod_stack.matches(parts):   # built once, rebuilt if a part changed
            self._mod_stack = None
            self._mod_stack = StackedLinear(parts[0][1].matmul.w.device, parts)
        return self._mod_stack.forward(silu(vec))

    def _qkv(self, prefix, x, qn, kn):
        cfg = self.cfg
        L = x.shape[0]
        qkv = self.p.lin[prefix + "qkv"].forward(x).reshape(L, 3, cfg.num_heads, cfg.head_dim)
        q = rms_norm(qkv[:, 0].transpose(0, 1), self.p.dense[qn])
        k = rms_norm(qkv[:, 1].transpose(0, 1), self.p.dense[kn])
        v = qkv[:, 2].transpose(0, 1)
        return q, k, v

    def _modulate(self, x, shift, scale):
        if self._fused(x):
            from .fused import adaln_modulate
            return adaln_modulate(x, shift, scale)
        return (layer_norm(x) * (1.0 + scale) + shift).to(self.gemm_dtype)

    def _gated(self, name, h, gate, res):
        """res + gate * lin(h): on the fused path with `gated_epilogue` the GEMM's
        epilogue updates res in place (Linear.gated_add); otherwise a new tensor."""
        import torch
        if self._fused(res) and self.gated_epilogue:
            return self.p.lin[name].gated_add(h, gate, res)
        return res + gate * self.p.lin[name].forward(h, out_dtype=torch.float32)

    def _attn_padded(self, q, k, v, valid, out=None):
        """Attention over the fused path's padded joint buffers (rows >= valid zero),
        written into `out` ([valid, H*D], rows may be strided) when given."""
        if self.attn is attention_bf16:
            return attention_bf16(q, k, v, valid, guard=self._guard, out=out)
        a = self.attn(q[:, :valid], k[:, :valid], v[:, :valid])
        if out is not None:
            out.copy_(a)
            return out
        return a

    def _joint_len(self, total: int) -> int:
        """Rows of the joint attention buffers: padded to a multiple of 256 unless
        a rerun for ill-conditioned padded rows turned padding off."""
        return padded_len(total) if self.pad_attention else total

    def _heads_fused(self, segments, cos, sin):
        """q, k, v bf16 [H, L, D] of the joint sequence from (qkv f32 [L_seg, >= 3h],
        query-norm name, key-norm name) segments in sequence order."""
        from .fused import new_heads, qk_norm_rope
        total = sum(y.shape[0] for y, _, _ in segments)
        q, k, v = new_heads(self.cfg.num_heads, self._joint_len(total), segments[0][0].device, valid=total)
        off = 0
        for y, qn, kn in segments:
            n = y.shape[0]
            qk_norm_rope(y, self.cfg.num_heads, self.p.dense[qn], self.p.dense[kn], cos[off:off + n],
                         sin[off:off + n], q, k, v, off)
            off += n
        return q, k, v

    def double_block(self, i, img, txt, vec, cos, sin):
        p = f"double_blocks.{i}."
        i_s1, i_c1, i_g1, i_s2, i_c2, i_g2 = self._mod(p + "img_mod.lin", vec, 6)
        t_s1, t_c1, t_g1, t_s2, t_c2, t_g2 = self._mod(p + "txt_mod.lin", vec, 6)
        import torch
        if self._fused(img):
            return self._double_block_fused(p, img, txt, cos, sin, (i_s1, i_c1, i_g1, i_s2, i_c2, i_g2),
                                            (t_s1, t_c1, t_g1, t_s2, t_c2, t_g2))
        iq, ik, iv = self._qkv(p + "img_attn.", self._modulate(img, i_s1, i_c1),
                               p + "img_attn.norm.query_norm.scale", p + "img_attn.norm.key_norm.scale")
        tq, tk, tv = self._qkv(p + "txt_attn.", self._modulate(txt, t_s1, t_c1),
                               p + "txt_attn.norm.query_norm.scale", p + "txt_attn.norm.key_norm.scale")
        q = apply_rope(torch.cat([tq, iq], dim=1), cos, sin)
        k = apply_rope(torch.cat([tk, ik], dim=1), cos, sin)
        v = torch.cat([tv, iv], dim=1)
        a = self.attn(q, k, v)
        lt = txt.shape[0]
        t_att, i_att = a[:lt], a[lt:]
        img = self._gated(p + "img_attn.proj", i_att, i_g1, img)
        h = self.p.lin[p + "img_mlp.0"].forward(self._modulate(img, i_s2, i_c2), act=ACT_GELU_TANH,
                                               out_dtype=self.gemm_dtype)
        img = self._gated(p + "img_mlp.2", h, i_g2, img)
        txt = self._gated(p + "txt_attn.proj", t_att, t_g1, txt)
        h = self.p.lin[p + "txt_mlp.0"].forward(self._modulate(txt, t_s2, t_c2), act=ACT_GELU_TANH,
                                               out_dtype=self.gemm_dtype)
        txt = self._gated(p + "txt_mlp.2", h, t_g2, txt)
        return img, txt

    def _double_block_fused(self, p, img, txt, cos, sin, im, tm):
        """The double block on the GPU: the text stream's linears (M = 512) run on a
        second HIP stream while the image stream's (M = 4096) fill the rest of the
        chip, joined before attention and at the end.  Tensors made on one stream and
        read on the other are recorded on the reader (caching-allocator safety).  The
        text-side linears take bf16 activations read in place, so they use none of the
        library context's shared staging scratch."""
        import torch
        from .fused import new_heads, qk_norm_rope
        bf16 = torch.bfloat16 if self.bf16_projections else torch.float32  # qkv feeds only the fused pass
        lt, H = txt.shape[0], self.cfg.num_heads
        total = lt + img.shape[0]
        q, k, v = new_heads(H, self._joint_len(total), img.device, valid=total)
        main = torch.cuda.current_stream(img.device)
        aux = text_stream(img.device, self.p.lin[p + "txt_attn.qkv"].matmul.w.device)
        aux.wait_stream(main)
        with torch.cuda.stream(aux):
            ty = self.p.lin[p + "txt_attn.qkv"].forward(self._modulate(txt, tm[0], tm[1]), out_dtype=bf16)
            qk_norm_rope(ty, H, self.p.dense[p + "txt_attn.norm.query_norm.scale"],
                         self.p.dense[p + "txt_attn.norm.key_norm.scale"], cos[:lt], sin[:lt], q, k, v, 0)
        for t in (txt, tm[0], q, k, v, cos, sin):
            t.record_stream(aux)
        iy = self.p.lin[p + "img_attn.qkv"].forward(self._modulate(img, im[0], im[1]), out_dtype=bf16)
        qk_norm_rope(iy, H, self.p.dense[p + "img_attn.norm.query_norm.scale"],
                     self.p.dense[p + "img_attn.norm.key_norm.scale"], cos[lt:], sin[lt:], q, k, v, lt)
        main.wait_stream(aux)
        a = self._attn_padded(q, k, v, total)
        t_att, i_att = a[:lt], a[lt:]
        aux.wait_stream(main)
        with torch.cuda.stream(aux):
            txt = self._gated(p + "txt_attn.proj", t_att, tm[2], txt)
            h = self.p.lin[p + "txt_mlp.0"].forward(self._modulate(txt, tm[3], tm[4]), act=ACT_GELU_TANH,
                                                   out_dtype=self.gemm_dtype)
            txt = self._gated(p + "txt_mlp.2", h, tm[5], txt)
        a.record_stream(aux)
        img = self._gated(p + "img_attn.proj", i_att, im[2], img)
        h = self.p.lin[p + "img_mlp.0"].forward(self._modulate(img, im[3], im[4]), act=ACT_GELU_TANH,
                                               out_dtype=self.gemm_dtype)
        img = self._gated(p + "img_mlp.2", h, im[5], img)
        main.wait_stream(aux)
        return img, txt

    def single_block(self, i, x, vec, cos, sin):
        import torch
        cfg = self.cfg
        p = f"single_blocks.{i}."
        shift, scale, gate = self._mod(p + "modulation.lin", vec, 3)
        L, h = x.shape[0], cfg.hidden_size
        if self._fused(x) and self.bf16_projections and self.gemm_dtype == torch.bfloat16:
            # linear1 in bf16 with GELU on its MLP columns only (mq_qmatmul_act_from): y =
            # [q | k | v | gelu(mlp)].  The norm/RoPE pass copies q, k, v into the joint
            # buffers, after which attention writes its rows over the v columns, so that
            # y[:, 2h:] = [attention | gelu(mlp)] is linear2's input as it stands (no GELU
            # pass, no concatenation buffer)
            y = self.p.lin[p + "linear1"].forward(self._modulate(x, shift, scale), out_dtype=torch.bfloat16,
                                                  act=ACT_GELU_TANH, act_from=3 * h)
            heads = self._heads_fused([(y, p + "norm.query_norm.scale", p + "norm.key_norm.scale")], cos, sin)
            self._attn_padded(*heads, L, out=y[:, 2 * h:3 * h])
            return self._gated(p + "linear2", y[:, 2 * h:], gate, x)
        # on the fused path linear1's output feeds only the norm/RoPE and GELU passes: bf16
        y_dtype = torch.bfloat16 if self._fused(x) and self.bf16_projections else torch.float32
        y = self.p.lin[p + "linear1"].forward(self._modulate(x, shift, scale), out_dtype=y_dtype)
        cat = torch.empty((L, h + cfg.mlp_size), dtype=self.gemm_dtype, device=x.device)
        if self._fused(x):
            # attention writes its rows straight into linear2's concatenated input
            self._attn_padded(*self._heads_fused([(y, p + "norm.query_norm.scale", p + "norm.key_norm.scale")],
                                                 cos, sin), L, out=cat[:, :h])
            from .fused import gelu_tanh_bf16
            gelu_tanh_bf16(y[:, 3 * h:], cat[:, h:])
        else:
            qkv = y[:, :3 * h].reshape(L, 3, cfg.num_heads, cfg.head_dim)
            q = rms_norm(qkv[:, 0].transpose(0, 1), self.p.dense[p + "norm.query_norm.scale"])
            k = rms_norm(qkv[:, 1].transpose(0, 1), self.p.dense[p + "norm.key_norm.scale"])
            v = qkv[:, 2].transpose(0, 1)
            cat[:, :h] = self.attn(apply_rope(q, cos, sin), apply_rope(k, cos, sin), v)
            cat[:, h:] = gelu_tanh(y[:, 3 * h:])
        return self._gated(p + "linear2", cat, gate, x)

    def stems(self, img, txt, t, guidance, y):
        import torch
        P = self.p
        txt_h = P.lin["txt_in"].forward(txt.to(self.gemm_dtype), out_dtype=torch.float32)
        img_h = torch.nn.functional.linear(img, P.dense["img_in.weight"].float(), P.dense["img_in.bias"])

        def mlp_embed(prefix, x):
            return P.lin[prefix + ".out_layer"].forward(silu(P.lin[prefix + ".in_layer"].forward(x)))
        vec = mlp_embed("time_in", timestep_embedding(t, 256))
        if self.cfg.guidance_embed:
            vec = vec + mlp_embed("guidance_in", timestep_embedding(guidance, 256))
        vec = vec + mlp_embed("vector_in", y)
        return img_h, txt_h, vec

    def final_layer(self, x, vec):
        shift, scale = self._mod("final_layer.adaLN_modulation.1", vec, 2)
        import torch
        return self.p.lin["final_layer.linear"].forward(self._modulate(x, shift, scale), out_dtype=torch.float32)

    def rope(self, img_ids, txt_ids):
        import torch
        ang = rope_angles(torch.cat([txt_ids, img_ids], dim=0), self.cfg.axes_dim, self.cfg.theta)
        return torch.cos(ang), torch.sin(ang)

    def forward(self, img, img_ids, txt, txt_ids, t, y, guidance=None, blocks: Optional[Tuple[int, int]] = None):
        """img [L_img, in_channels], txt [L_txt, context_in_dim], y [1, vec_in_dim],
        t and guidance [1]; ids [L, 3] f32.  Returns [L_img, in_channels] f32.
        `blocks` = (double, single) limits the number of blocks run (host leg)."""
        return run_guarded(self, self._forward, img, img_ids, txt, txt_ids, t, y, guidance, blocks)

    def _forward(self, img, img_ids, txt, txt_ids, t, y, guidance, blocks):
        import torch
        nd = self.cfg.depth if blocks is None else blocks[0]
        ns = self.cfg.depth_single_blocks if blocks is None else blocks[1]
        cos, sin = self.rope(img_ids, txt_ids)
        img_h, txt_h, vec = self.stems(img, txt, t, guidance, y)
        stacked = self.stack_modulations and vec.is_cuda and blocks is None
        self._mods = self._stacked_mods(vec) if stacked else None
        try:
            for i in range(nd):
                img_h, txt_h = self.double_block(i, img_h, txt_h, vec, cos, sin)
            x = torch.cat([txt_h, img_h], dim=0)
            for i in range(ns):
                x = self.single_block(i, x, vec, cos, sin)
            return self.final_layer(x[txt_h.shape[0]:], vec)
        finally:
            self._mods = None


def make_inputs(cfg: FluxConfig, height: int = 1024, width: int = 1024, txt_len: int = 512,
                device="cuda", seed: int = 4):
    """Packed latents [(h/16)*(w/16), 64], ids, T5 states [txt_len, 4096], pooled
    CLIP [1, 768], timestep 0.5, guidance 3.5, all N(0, 1) from `seed`."""
    import torch
    g = torch.Generator(device=device).manual_seed(seed)
    gh, gw = height // 16, width // 16
    img = torch.randn((gh * gw, cfg.in_channels), device=device, generator=g)
    txt = torch.randn((txt_len, cfg.context_in_dim), device=device, generator=g)
    y = torch.randn((1, cfg.vec_in_dim), device=device, generator=g)
    rows = torch.arange(gh, device=device, dtype=torch.float32)[:, None].expand(gh, gw)
    cols = torch.arange(gw, device=device, dtype=torch.float32)[None, :].expand(gh, gw)
    img_ids = torch.stack([torch.zeros_like(rows), rows, cols], dim=-1).reshape(-1, 3)
    txt_ids = torch.zeros((txt_len, 3), device=device)
    t = torch.full((1,), 0.5, device=device)
    guidance = torch.full((1,), 3.5, device=device)
    return dict(img=img, img_ids=img_ids, txt=txt, txt_ids=txt_ids, t=t, y=y, guidance=guidance)


def step_flop(cfg: FluxConfig, l_img: int, l_txt: int) -> Tuple[float, float]:
    """(linear FLOP with M > 1, attention FLOP) of one forward."""
    L = l_img + l_txt
    lin = 0.0
    for name, (n, k, _) in linear_shapes(cfg).items():
        if name.startswith("double_blocks"):
            m = l_img if ".img_" in name else l_txt
            m = 1 if name.endswith("_mod.lin") else m
        elif name.startswith("single_blocks"):
            m = 1 if name.endswith("modulation.lin") else L
        elif name == "txt_in":
            m = l_txt
        elif name == "final_layer.linear":
            m = l_img
        else:
            m = 1
        if m > 1:
            lin += 2.0 * m * n * k
    blocks = cfg.depth + cfg.depth_single_blocks
    attn = blocks * 2 * (2.0 * cfg.num_heads * L * L * cfg.head_dim)
    return lin, attn
