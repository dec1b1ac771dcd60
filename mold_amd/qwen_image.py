"""Qwen-Image-shaped MMDiT step whose linears are libmoldq quantized linears.

This is the second caller of the quantized-linear path: mold's quantized
Qwen-Image transformer, /root/reference/crates/mold-inference/src/qwen_image/
quantized_transformer.rs.  On CUDA mold runs each GGUF linear as a full
dequantize to bf16 plus a dense matmul on every forward (`QwenLinear::Dequant`,
:44-77); here every linear is `QMatMul::forward` on the resident GGUF blocks
(the fused dequant GEMM), which is the replacement that file's Metal arm
already uses (`QwenLinear::QMatMul`, :86-88).  Op order and constants follow:
  TimestepProjEmbeddings.forward   :591-601 (10000^(-i/half), [cos, sin], lin1 -> silu -> lin2)
  LayerNormNoParams                :126-158 (eps 1e-6, no affine)
  DynamicRmsNorm                   :97-112  (x / sqrt(mean(x^2) + eps) * w)
  QwenRopeEmbedder.forward         :339-435 (frame axis from 0, height/width axes centred
                                             (-ceil(n/2) .. floor(n/2)-1), text from max(h/2, w/2))
  JointAttention.forward           :695-781 (img: to_q/k/v, norm_q/k; txt: add_*_proj,
                                             norm_added_q/k; RoPE; joint [txt, img]; to_out.0 and
                                             to_add_out)
  FeedForward                      :604-641 (net.0.proj -> gelu(tanh) -> net.2)
  QwenImageTransformerBlock.forward:856-960 (silu(temb) -> img_mod.1 / txt_mod.1, 6 chunks
                                             shift, scale, gate (msa), shift, scale, gate (mlp))
  OutputLayer.forward              :977-989 (chunks scale, shift; norm; proj_out)
  forward                          :1048-1139 (time embed, img_in, txt_norm -> txt_in, blocks)
RoPE rotates interleaved pairs (x[2j], x[2j+1]) by angle j, candle's
`z_image::transformer::apply_rotary_emb` (called at :742-745).

Layout choices made here (the graph's values are unchanged by them):
  * q, k and v of each stream are one weight: the rows of to_q, to_k, to_v
    (or add_q_proj, add_k_proj, add_v_proj) stacked [3h, h].  GGUF rows are
    independent, so the stacked blocks are the three tensors' blocks
    concatenated, and y[:, :h], y[:, h:2h], y[:, 2h:] are the three outputs.
    One GEMM with N = 9216 fills the chip where three with N = 3072 leave it
    partly idle.
  * The text stream's linears (M = 256 at 1328^2) run on a second HIP stream,
    concurrently with the image stream's (M = 6889), joined by events before
    the joint attention and at the end of each block.
  * The residual streams stay f32; a tensor whose only consumer is a quantized
    GEMM is produced in bf16 (the GEMM rounds its input to bf16 either way).
  * On the GPU the modulate and the q/k norm + RoPE + head split run as
    libmoldq's fused row passes (mold_amd.fused), writing q, k, v straight
    into the joint [heads, L, 128] bf16 buffers attention reads, and each
    gated residual update x + gate * linear(h) is the GEMM's epilogue
    (Linear.gated_add, updating x in place).
  * Every block's img_mod.1 / txt_mod.1 and the output layer's norm_out.linear
    read the same silu(temb): on the GPU they run as one GEMV (one GEMM row
    per batch element) over their weights stacked by rows (StackedLinear) at
    the start of the forward, with outputs identical to the separate linears.
  * The text attention mask is all ones for an unpadded prompt, which makes the
    mask a no-op (:813-815 add 0 to every score), so none is applied.

Weights are synthetic: every linear is N(0, 0.02^2) quantized on the GPU to the
type `QwenConfig.qtypes` assigns (config 5: attention q/k/v Q3_K, MLP Q2_K,
output projections and modulation Q4_K; stems and the output layer Q4_K),
biases f32 N(0, 0.02^2), RmsNorm weights bf16 N(1, 0.02^2), `img_in` (K = 64,
not a multiple of 256) a dense bf16 weight.
"""
from __future__ import annotations

import contextlib
import math
from dataclasses import dataclass, field
from typing import Callable, Dict, Optional, Tuple

import numpy as np

from .flux import apply_rope, attention_bf16, attention_bf16_batch, gelu_tanh, layer_norm, padded_len, run_guarded, silu, text_stream
from .quantized import ACT_GELU_TANH, GgmlDType, Linear, QTensor

MAX_PERIOD = 10000.0


@dataclass(frozen=True)
class QwenConfig:
    """Qwen-Image transformer shape (qwen_image/transformer.rs QwenImageConfig defaults)."""
    in_channels: int = 64             # 16 latent channels x 2 x 2 patch
    out_channels: int = 16
    patch_size: int = 2
    num_layers: int = 60
    attention_head_dim: int = 128
    num_attention_heads: int = 24
    joint_attention_dim: int = 3584
    mlp_hidden: int = 12288
    axes_dims_rope: Tuple[int, int, int] = (16, 56, 56)
    norm_eps: float = 1e-6
    theta: float = 10000.0
    # GGUF type per linear role (BASELINE config 5's mixed low-bit mapping)
    qtypes: Tuple[Tuple[str, GgmlDType], ...] = field(default_factory=lambda: (
        ("qkv", GgmlDType.Q3_K), ("mlp", GgmlDType.Q2_K), ("out", GgmlDType.Q4_K),
        ("mod", GgmlDType.Q4_K), ("stem", GgmlDType.Q4_K)))

    @property
    def hidden_size(self) -> int:
        return self.num_attention_heads * self.attention_head_dim

    def qtype(self, role: str) -> GgmlDType:
        return dict(self.qtypes)[role]

    @staticmethod
    def image() -> "QwenConfig":
        return QwenConfig()

    @staticmethod
    def tiny() -> "QwenConfig":
        """Same graph at hidden 256 (2 heads of 128), one block, small text dim."""
        return QwenConfig(num_layers=1, num_attention_heads=2, joint_attention_dim=512, mlp_hidden=1024)


def linear_shapes(cfg: QwenConfig) -> Dict[str, Tuple[int, int, str]]:
    """name -> (out_features, in_features, role) for every quantized linear.
    `attn.to_qkv` / `attn.add_qkv_proj` are the stacked q, k, v weights."""
    h, mlp = cfg.hidden_size, cfg.mlp_hidden
    s: Dict[str, Tuple[int, int, str]] = {
        "time_text_embed.timestep_embedder.linear_1": (h, 256, "stem"),
        "time_text_embed.timestep_embedder.linear_2": (h, h, "stem"),
        "txt_in": (h, cfg.joint_attention_dim, "stem"),
        "norm_out.linear": (2 * h, h, "stem"),
        "proj_out": (cfg.patch_size ** 2 * cfg.out_channels, h, "stem"),
    }
    for i in range(cfg.num_layers):
        p = f"transformer_blocks.{i}."
        s[p + "img_mod.1"] = (6 * h, h, "mod")
        s[p + "txt_mod.1"] = (6 * h, h, "mod")
        s[p + "attn.to_qkv"] = (3 * h, h, "qkv")
        s[p + "attn.add_qkv_proj"] = (3 * h, h, "qkv")
        s[p + "attn.to_out.0"] = (h, h, "out")
        s[p + "attn.to_add_out"] = (h, h, "out")
        for st in ("img_mlp", "txt_mlp"):
            s[p + f"{st}.net.0.proj"] = (mlp, h, "mlp")
            s[p + f"{st}.net.2"] = (h, mlp, "mlp")
    return s


def dense_shapes(cfg: QwenConfig) -> Dict[str, Tuple[int, ...]]:
    """Non-quantized parameters: img_in (bf16 weight, f32 bias) and RmsNorm weights."""
    h, d = cfg.hidden_size, cfg.attention_head_dim
    s: Dict[str, Tuple[int, ...]] = {"img_in.weight": (h, cfg.in_channels), "img_in.bias": (h,),
                                     "txt_norm.weight": (cfg.joint_attention_dim,)}
    for i in range(cfg.num_layers):
        for nm in ("norm_q", "norm_k", "norm_added_q", "norm_added_k"):
            s[f"transformer_blocks.{i}.attn.{nm}.weight"] = (d,)
    return s


class QwenParams:
    """`lin[name]` objects with `forward(x, act=0, out_dtype=None)` (bias inside)
    and `dense[name]` tensors."""

    def __init__(self, cfg: QwenConfig, lin: Dict[str, object], dense: Dict[str, object]):
        self.cfg, self.lin, self.dense = cfg, lin, dense

    @staticmethod
    def random(cfg: QwenConfig, device, seed: int = 5) -> "QwenParams":
        """Synthetic weights generated and quantized on `device` (a mold_amd.Device)."""
        import torch
        cuda = f"cuda:{device.ordinal}"
        lin, dense = {}, {}
        for idx, (name, (n, k, role)) in enumerate(linear_shapes(cfg).items()):
            g = torch.Generator(device=cuda).manual_seed(seed * 1_000_003 + 2 * idx)
            w = torch.randn((n, k), device=cuda, generator=g) * 0.02
            qt = QTensor.quantize(device, w, cfg.qtype(role))
            del w
            g = torch.Generator(device=cuda).manual_seed(seed * 1_000_003 + 2 * idx + 1)
            lin[name] = Linear(qt, torch.randn((n,), device=cuda, generator=g) * 0.02)
        for idx, (name, shape) in enumerate(dense_shapes(cfg).items()):
            g = torch.Generator(device=cuda).manual_seed(seed * 7_000_003 + idx)
            t = torch.randn(shape, device=cuda, generator=g) * 0.02
            if name.endswith("norm_q.weight") or name.endswith("norm_k.weight") or "norm_added" in name \
                    or name == "txt_norm.weight":
                t = (t + 1.0).to(torch.bfloat16)
            elif name == "img_in.weight":
                t = t.to(torch.bfloat16)
            dense[name] = t
        return QwenParams(cfg, lin, dense)

    @staticmethod
    def from_gguf(cfg: QwenConfig, path: str, device) -> "QwenParams":
        """The transformer's parameters from a GGUF file in mold's layout (the names
        `qlinear` reads, qwen_image/quantized_transformer.rs:79-93, 584-611, 631-632,
        679-687, 847-851, 972-973, 1011-1016: `<linear>.weight` / `.bias`, separate
        `attn.to_q` / `to_k` / `to_v` and `add_q_proj` / `add_k_proj` / `add_v_proj`,
        RmsNorm `.weight`s), read the way `VarBuilder::from_gguf` does
        (qwen_image/pipeline.rs:936): every tensor to the device in one pipelined
        call (mq_gguf_load_tensors).  The step's stacked q/k/v weights are the three
        tensors concatenated by rows on the device (mq_qtensor_concat_rows; they must
        share one type), biases dequantized to f32, img_in's weight (stored in any
        type: its K = in_channels holds no 256-wide block) and the norm weights
        dequantized to bf16.  No tensor byte passes through the host."""
        import torch
        from . import gguf
        parts: Dict[str, Tuple[str, ...]] = {}
        for name in linear_shapes(cfg):
            if name.endswith("attn.to_qkv"):
                p = name[:-len("to_qkv")]
                parts[name] = (p + "to_q", p + "to_k", p + "to_v")
            elif name.endswith("attn.add_qkv_proj"):
                p = name[:-len("add_qkv_proj")]
                parts[name] = (p + "add_q_proj", p + "add_k_proj", p + "add_v_proj")
            else:
                parts[name] = (name,)
        need = [q + sfx for ps in parts.values() for q in ps for sfx in (".weight", ".bias")] + list(dense_shapes(cfg))
        c = gguf.Content.read(path)
        try:
            missing = [nm for nm in need if nm not in c.tensor_infos]
            if missing:
                raise KeyError(f"{path}: tensors missing: {missing[:4]}")
            qts = c.tensors(need, device)
        finally:
            c.close()
        lin, dense = {}, {}
        for name, (n, k, _) in linear_shapes(cfg).items():
            ws = [qts[q + ".weight"] for q in parts[name]]
            if any(w.shape[1] != k for w in ws) or sum(w.shape[0] for w in ws) != n:
                raise ValueError(f"{name}: stored as {[w.shape for w in ws]}, the config needs ({n}, {k})")
            if len({w.dtype() for w in ws}) != 1:
                raise ValueError(f"{name}: {parts[name]} are stored as {[w.dtype().name for w in ws]}; "
                                 "the stacked projection needs one type")
            if not ws[0].dtype().is_quantized:
                raise ValueError(f"{name} is dense {ws[0].dtype().name}; the step runs quantized linears")
            w = ws[0] if len(ws) == 1 else QTensor.concat_rows(device, ws)
            bias = torch.cat([qts[q + ".bias"].dequantize(torch.float32).reshape(-1) for q in parts[name]])
            lin[name] = Linear(w, bias.contiguous())
        for name, shape in dense_shapes(cfg).items():
            t = qts[name]
            want = (int(np.prod(shape[:-1])) if len(shape) > 1 else 1, shape[-1])
            if t.shape != want:
                raise ValueError(f"{name}: stored as {t.shape}, the config needs {tuple(shape)}")
            dt = torch.float32 if name.endswith(".bias") else torch.bfloat16
            dense[name] = t.dequantize(dt).reshape(shape)
        return QwenParams(cfg, lin, dense)

    def quantized_bytes(self) -> int:
        return sum(l.matmul.w.storage_size_in_bytes() for l in self.lin.values())


# --------------------------------------------------------------------------- glue

def timestep_embedding(t, dim: int = 256):
    """quantized_transformer.rs:591-599 (no 1000x scale: t is the scheduler timestep)."""
    import torch
    half = dim // 2
    freqs = torch.exp(torch.arange(half, dtype=torch.float32, device=t.device) * (-math.log(MAX_PERIOD) / half))
    args = t.float()[:, None] * freqs[None, :]
    return torch.cat([torch.cos(args), torch.sin(args)], dim=-1)


def rms_norm(x, w, eps: float = 1e-6):
    import torch
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w.float()


def _axis_angles(pos, dim: int, theta: float):
    """angles[p, j] = pos[p] * theta^(-2j/dim), j < dim/2."""
    import torch
    inv = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64, device=pos.device) / dim))
    return pos.double()[:, None] * inv[None, :]


def rope_tables(cfg: QwenConfig, frames: int, height: int, width: int, txt_len: int, device):
    """QwenRopeEmbedder.forward (:339-435): (img_cos, img_sin, txt_cos, txt_sin),
    each [L, head_dim / 2] f32."""
    import torch
    fd, hd, wd = cfg.axes_dims_rope

    def centred(n):
        # negative half first: -(n - n//2) .. -1, then 0 .. n//2 - 1
        return torch.cat([torch.arange(-(n - n // 2), 0, device=device),
                          torch.arange(0, n // 2, device=device)]).double()

    fa = _axis_angles(torch.arange(frames, device=device).double(), fd, cfg.theta)
    ha = _axis_angles(centred(height), hd, cfg.theta)
    wa = _axis_angles(centred(width), wd, cfg.theta)
    img = torch.cat([fa[:, None, None, :].expand(frames, height, width, fd // 2),
                     ha[None, :, None, :].expand(frames, height, width, hd // 2),
                     wa[None, None, :, :].expand(frames, height, width, wd // 2)], dim=-1)
    img = img.reshape(frames * height * width, -1)
    start = max(height // 2, width // 2)
    tp = torch.arange(start, start + txt_len, device=device).double()
    txt = torch.cat([_axis_angles(tp, d, cfg.theta) for d in (fd, hd, wd)], dim=-1)
    return (torch.cos(img).float(), torch.sin(img).float(), torch.cos(txt).float(), torch.sin(txt).float())


class QwenImageStep:
    """One denoising-step forward of the Qwen-Image transformer (batch 1).

    `attn` computes attention ([H, L, D] f32 x3 -> [L, H*D]); `gemm_dtype` is the
    dtype of tensors consumed only by a quantized linear; `overlap` runs the text
    stream's work on a second HIP stream (GPU only)."""

    def __init__(self, params: QwenParams, attn: Callable = attention_bf16, gemm_dtype=None,
                 overlap: Optional[bool] = None):
        import torch
        self.p, self.cfg = params, params.cfg
        self.attn = attn
        self.gemm_dtype = torch.bfloat16 if gemm_dtype is None else gemm_dtype
        self.overlap = overlap
        self.gated_epilogue = True
        # fused path: the qkv projections, which feed only the fused pass, are written in bf16
        self.bf16_projections = True
        self.pad_attention = True
        self._guard = None
        self.stack_modulations = True
        self._mod_stack = None
        self._mods = None

    def modulation_names(self):
        """The linears that read silu(temb), in run order."""
        names = []
        for i in range(self.cfg.num_layers):
            names += [f"transformer_blocks.{i}.img_mod.1", f"transformer_blocks.{i}.txt_mod.1"]
        return names + ["norm_out.linear"]

    def _start_mods(self, ts, blocks):
        """Run the stacked modulation GEMV for this forward (GPU, all blocks)."""
        from .quantized import StackedLinear
        self._mods = None
        if not (self.stack_modulations and ts.is_cuda and blocks is None):
            return
        parts = [(nm, self.p.lin[nm]) for nm in self.modulation_names()]
        if self._mod_stack is None or not self._mod_stack.matches(parts):   # built once, rebuilt if a part changed
            self._mod_stack = None
            self._mod_stack = StackedLinear(parts[0][1].matmul.w.device, parts)
        self._mods = self._mod_stack.forward(ts)

    def _modf(self, name, ts):
        """Output of modulation linear `name` on ts = silu(temb)."""
        return self._mods[name] if self._mods is not None else self.p.lin[name].forward(ts)

    def _fused(self, x) -> bool:
        """Use libmoldq's fused row passes (mold_amd.fused): on the GPU with bf16 GEMM inputs."""
        import torch
        return x.is_cuda and self.gemm_dtype == torch.bfloat16

    def _modulate(self, x, shift, scale):
        if self._fused(x):
            from .fused import adaln_modulate
            return adaln_modulate(x, shift, scale)
        return (layer_norm(x) * (1.0 + scale) + shift).to(self.gemm_dtype)

    def _heads(self, y, qn, kn):
        """[L, 3h] -> q, k (RmsNormed), v as [H, L, D] f32."""
        cfg = self.cfg
        L = y.shape[0]
        y = y.reshape(L, 3, cfg.num_attention_heads, cfg.attention_head_dim)
        q = rms_norm(y[:, 0].transpose(0, 1), self.p.dense[qn], cfg.norm_eps)
        k = rms_norm(y[:, 1].transpose(0, 1), self.p.dense[kn], cfg.norm_eps)
        return q, k, y[:, 2].transpose(0, 1).float()

    def _txt_qkv(self, p, txt, mods, cos, sin, heads=None):
        """The text stream's q, k, v: [H, L_txt, D] f32, or written into the joint
        bf16 buffers `heads` = (q, k, v) at rows 0 .. L_txt - 1 (fused path)."""
        t_s1, t_c1 = mods[0], mods[1]
        import torch
        y_dtype = torch.bfloat16 if heads is not None and self.bf16_projections else torch.float32
        y = self.p.lin[p + "attn.add_qkv_proj"].forward(self._modulate(txt, t_s1, t_c1), out_dtype=y_dtype)
        if heads is not None:
            from .fused import qk_norm_rope
            qk_norm_rope(y, self.cfg.num_attention_heads, self.p.dense[p + "attn.norm_added_q.weight"],
                         self.p.dense[p + "attn.norm_added_k.weight"], cos, sin, *heads, 0, self.cfg.norm_eps)
            return None
        q, k, v = self._heads(y, p + "attn.norm_added_q.weight", p + "attn.norm_added_k.weight")
        return apply_rope(q, cos, sin), apply_rope(k, cos, sin), v

    def _gated(self, name, h, gate, res):
        """res + gate * lin(h): on the fused path with `gated_epilogue` the GEMM's
        epilogue updates res in place (Linear.gated_add); otherwise a new tensor."""
        import torch
        if self._fused(res) and self.gated_epilogue:
            return self.p.lin[name].gated_add(h, gate, res)
        return res + gate * self.p.lin[name].forward(h, out_dtype=torch.float32)

    def _txt_tail(self, p, txt, t_att, mods):
        _, _, t_g1, t_s2, t_c2, t_g2 = mods
        txt = self._gated(p + "attn.to_add_out", t_att, t_g1, txt)
        h = self.p.lin[p + "txt_mlp.net.0.proj"].forward(self._modulate(txt, t_s2, t_c2), act=ACT_GELU_TANH,
                                                        out_dtype=self.gemm_dtype)
        return self._gated(p + "txt_mlp.net.2", h, t_g2, txt)

    def block(self, i, img, txt, temb_silu, rope):
        """QwenImageTransformerBlock.forward (:856-960)."""
        import torch
        p = f"transformer_blocks.{i}."
        img_cos, img_sin, txt_cos, txt_sin = rope
        i_mod_all = self._modf(p + "img_mod.1", temb_silu)
        t_mod_all = self._modf(p + "txt_mod.1", temb_silu)
        i_mod, t_mod = i_mod_all.chunk(6, dim=-1), t_mod_all.chunk(6, dim=-1)
        aux = self._aux(img)
        lt = txt.shape[0]
        fused = self._fused(img)
        heads = None
        total = lt + img.shape[0]
        if fused:
            from .fused import new_heads
            heads = new_heads(self.cfg.num_attention_heads, padded_len(total) if self.pad_attention else total,
                              img.device, valid=total)
        if aux is None:
            tqkv = self._txt_qkv(p, txt, t_mod, txt_cos, txt_sin, heads)
        else:
            # text stream on `aux`: tensors made on one stream and read on the
            # other are recorded on the reader, so the caching allocator does
            # not hand their memory out again while the reader may still run.
            main = torch.cuda.current_stream(img.device)
            aux.wait_stream(main)
            with torch.cuda.stream(aux):
                tqkv = self._txt_qkv(p, txt, t_mod, txt_cos, txt_sin, heads)
            for t in (txt, t_mod_all) + (heads if heads is not None else ()):
                t.record_stream(aux)
            for t in (tqkv if tqkv is not None else ()):
                t.record_stream(main)
        y = self.p.lin[p + "attn.to_qkv"].forward(self._modulate(img, i_mod[0], i_mod[1]),
                                                 out_dtype=torch.bfloat16 if fused and self.bf16_projections
                                                 else torch.float32)
        if fused:
            from .fused import qk_norm_rope
            qk_norm_rope(y, self.cfg.num_attention_heads, self.p.dense[p + "attn.norm_q.weight"],
                         self.p.dense[p + "attn.norm_k.weight"], img_cos, img_sin, *heads, lt, self.cfg.norm_eps)
        else:
            iq, ik, iv = self._heads(y, p + "attn.norm_q.weight", p + "attn.norm_k.weight")
            iq, ik = apply_rope(iq, img_cos, img_sin), apply_rope(ik, img_cos, img_sin)
        if aux is not None:
            main.wait_stream(aux)
        if fused and self.attn is attention_bf16:
            a = attention_bf16(*heads, valid=total, guard=self._guard)
        elif fused:
            a = self.attn(*(t[:, :total] for t in heads))
        else:
            tq, tk, tv = tqkv
            a = self.attn(torch.cat([tq, iq], dim=1), torch.cat([tk, ik], dim=1), torch.cat([tv, iv], dim=1))
        t_att, i_att = a[:lt], a[lt:]
        if aux is None:
            txt = self._txt_tail(p, txt, t_att, t_mod)
        else:
            aux.wait_stream(main)
            with torch.cuda.stream(aux):
                txt_new = self._txt_tail(p, txt, t_att, t_mod)
            for t in (txt, a, t_mod_all):
                t.record_stream(aux)
            txt = txt_new
        _, _, i_g1, i_s2, i_c2, i_g2 = i_mod
        img = self._gated(p + "attn.to_out.0", i_att, i_g1, img)
        h = self.p.lin[p + "img_mlp.net.0.proj"].forward(self._modulate(img, i_s2, i_c2), act=ACT_GELU_TANH,
                                                        out_dtype=self.gemm_dtype)
        img = self._gated(p + "img_mlp.net.2", h, i_g2, img)
        if aux is not None:
            main.wait_stream(aux)
            txt.record_stream(main)
        return img, txt

    def _aux(self, x):
        """The text stream's HIP stream, or None to run everything in order.
        Only with bf16 GEMM inputs: the linears then read their activations in
        place and use none of the library context's shared staging scratch."""
        import torch
        use = self.overlap if self.overlap is not None else x.is_cuda
        if not use or not x.is_cuda or self.gemm_dtype != torch.bfloat16:
            return None
        return text_stream(x.device, self.p.lin["txt_in"].matmul.w.device)

    def stems(self, img, txt, t):
        import torch
        P, cfg = self.p, self.cfg
        e = timestep_embedding(t, 256)
        temb = P.lin["time_text_embed.timestep_embedder.linear_2"].forward(
            silu(P.lin["time_text_embed.timestep_embedder.linear_1"].forward(e)))
        img_h = torch.nn.functional.linear(img, P.dense["img_in.weight"].float(), P.dense["img_in.bias"])
        txt_n = rms_norm(txt, P.dense["txt_norm.weight"], cfg.norm_eps).to(self.gemm_dtype)
        txt_h = P.lin["txt_in"].forward(txt_n, out_dtype=torch.float32)
        return img_h, txt_h, temb

    def output_layer(self, x, temb):
        """OutputLayer.forward (:977-989): chunk 0 is scale, chunk 1 shift."""
        import torch
        scale, shift = self._modf("norm_out.linear", silu(temb)).chunk(2, dim=-1)
        return self.p.lin["proj_out"].forward(self._modulate(x, shift, scale), out_dtype=torch.float32)

    def forward(self, img, txt, t, grid: Tuple[int, int], blocks: Optional[int] = None):
        """img [H/2*W/2, 64] packed latents, txt [L_txt, joint_attention_dim], t [1];
        grid = (H/2, W/2) in patches.  Returns [L_img, 64] f32.  `blocks` limits the
        number of blocks run (host leg)."""
        return run_guarded(self, self._forward, img, txt, t, grid, blocks)

    # ------------------------------------------------------------ batch (CFG)
    def forward_batched(self, img, txt, t, grid: Tuple[int, int], txt_valid=None, blocks: Optional[int] = None):
        """The batched forward mold runs for classifier-free guidance
        (pipeline.rs:1866-1899 batches cond and uncond along dim 0 when
        supports_cfg_batching(), quantized_transformer.rs:1044-1046; the forward
        is :1048-1139 with batch B): img [B, L, 64], txt [B, L_txt, 3584], t [B],
        `txt_valid` the number of valid (mask = 1) leading text tokens per element
        (the encoder_attention_mask of a padded prompt; default all).  Masked text
        keys are excluded from attention (:764-768, :804-823); masked text rows
        still run through the text stream, as in mold.  Every linear runs once
        over all B elements' rows (the image GEMMs at M = B*L); modulation,
        gating and attention are per element.  GPU fused path only.  Returns
        [B, L, 64] f32."""
        import torch
        B, L, _ = img.shape
        lt = txt.shape[1]
        if not self._fused(img.reshape(B * L, -1)):
            raise ValueError("forward_batched runs on the GPU with bf16 GEMM inputs")
        valid = [lt] * B if txt_valid is None else [int(v) for v in txt_valid]
        if len(valid) != B or any(v < 1 or v > lt for v in valid):
            raise ValueError("txt_valid needs one count in 1 .. L_txt per batch element")
        return run_guarded(self, self._forward_batched, img, txt, t, grid, valid, blocks)

    def _mod_rows(self, x, mods, j0, j1, B):
        """Per-element modulate of x [B*Lx, h] with chunks j0 (shift), j1 (scale)
        of each element's modulation, into one bf16 [B*Lx, h] buffer."""
        import torch
        from .fused import adaln_modulate
        lx = x.shape[0] // B
        out = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
        for b in range(B):
            adaln_modulate(x[b * lx:(b + 1) * lx], mods[b][j0], mods[b][j1], out=out[b * lx:(b + 1) * lx])
        return out

    def _gated_rows(self, name, h, mods, j, res, B):
        """res[b rows] += gate_b * lin(h_b) per element (GEMM epilogue), h_b
        element b's rows of h, or h[b] when h is a list of per-element inputs."""
        lx = res.shape[0] // B
        for b in range(B):
            hb = h[b] if isinstance(h, (list, tuple)) else h[b * lx:(b + 1) * lx]
            self.p.lin[name].gated_add(hb, mods[b][j], res[b * lx:(b + 1) * lx])
        return res

    def block_batched(self, i, img, txt, ts, rope, B, valid):
        import torch
        from .fused import new_heads, qk_norm_rope
        cfg, P = self.cfg, self.p
        p = f"transformer_blocks.{i}."
        img_cos, img_sin, txt_cos, txt_sin = rope
        L, lt = img.shape[0] // B, txt.shape[0] // B
        H = cfg.num_attention_heads
        im = [r.chunk(6, dim=-1) for r in self._modf(p + "img_mod.1", ts)]      # M = B GEMV
        t_mod_all = self._modf(p + "txt_mod.1", ts)
        tm = [r.chunk(6, dim=-1) for r in t_mod_all]
        total = lt + L
        # q, k, v of all elements in one [B, H, L, D] buffer each (one batched
        # attention launch); heads_b[b] are element b's [H, L, D] views
        hq, hk, hv = new_heads(H, padded_len(total) if self.pad_attention else total, img.device, valid=total,
                               batch=B)
        heads_b = [(hq[b], hk[b], hv[b]) for b in range(B)]
        # text stream on `aux` as in block(): its modulate, qkv projection and
        # q/k norm overlap the image qkv projection, its tail overlaps the image
        # out-projection and MLP; tensors shared across the streams are recorded
        # on the reader
        aux = self._aux(img)
        main = torch.cuda.current_stream(img.device) if aux is not None else None
        on_aux = (lambda: torch.cuda.stream(aux)) if aux is not None else contextlib.nullcontext
        if aux is not None:
            aux.wait_stream(main)
        with on_aux():
            ty = P.lin[p + "attn.add_qkv_proj"].forward(self._mod_rows(txt, tm, 0, 1, B), out_dtype=torch.bfloat16)
            for b in range(B):
                qk_norm_rope(ty[b * lt:(b + 1) * lt], H, P.dense[p + "attn.norm_added_q.weight"],
                             P.dense[p + "attn.norm_added_k.weight"], txt_cos, txt_sin, *heads_b[b], 0, cfg.norm_eps)
        if aux is not None:
            for t in (txt, t_mod_all, hq, hk, hv):
                t.record_stream(aux)
        y = P.lin[p + "attn.to_qkv"].forward(self._mod_rows(img, im, 0, 1, B), out_dtype=torch.bfloat16)
        for b in range(B):
            qk_norm_rope(y[b * L:(b + 1) * L], H, P.dense[p + "attn.norm_q.weight"], P.dense[p + "attn.norm_k.weight"],
                         img_cos, img_sin, *heads_b[b], lt, cfg.norm_eps)
        if aux is not None:
            main.wait_stream(aux)
        drops = []
        for b in range(B):
            drops.append((valid[b], lt) if valid[b] < lt else None)
            if valid[b] < lt:
                heads_b[b][1][:, valid[b]:lt].zero_()
                heads_b[b][2][:, valid[b]:lt].zero_()
        if self.pad_attention:
            a = attention_bf16_batch(hq, hk, hv, valid=total, guard=self._guard, drops=drops)
        else:   # the guarded rerun: exact attention over the kept keys
            from .flux import _attention_chunked
            a = [_attention_chunked(*(t[:, :total] for t in heads_b[b]), drops[b]) for b in range(B)]
        # each element's text and image rows of the attention output feed its
        # out-projections in place (strided rows, no copy)
        t_att = [a[b][:lt] for b in range(B)]
        i_att = [a[b][lt:] for b in range(B)]
        if aux is not None:
            aux.wait_stream(main)
        with on_aux():
            txt = self._gated_rows(p + "attn.to_add_out", t_att, tm, 2, txt, B)
            ht = P.lin[p + "txt_mlp.net.0.proj"].forward(self._mod_rows(txt, tm, 3, 4, B), act=ACT_GELU_TANH,
                                                         out_dtype=torch.bfloat16)
            txt = self._gated_rows(p + "txt_mlp.net.2", ht, tm, 5, txt, B)
        if aux is not None:
            for t in (a if isinstance(a, list) else [a]):
                t.record_stream(aux)
        img = self._gated_rows(p + "attn.to_out.0", i_att, im, 2, img, B)
        h = P.lin[p + "img_mlp.net.0.proj"].forward(self._mod_rows(img, im, 3, 4, B), act=ACT_GELU_TANH,
                                                    out_dtype=torch.bfloat16)
        img = self._gated_rows(p + "img_mlp.net.2", h, im, 5, img, B)
        if aux is not None:
            main.wait_stream(aux)
        return img, txt

    def _forward_batched(self, img, txt, t, grid, valid, blocks):
        import torch
        cfg = self.cfg
        B, L, c = img.shape
        lt = txt.shape[1]
        nb = cfg.num_layers if blocks is None else blocks
        rope = rope_tables(cfg, 1, grid[0], grid[1], lt, img.device)
        img_h, txt_h, temb = self.stems(img.reshape(B * L, c), txt.reshape(B * lt, -1), t)
        ts = silu(temb)                                   # [B, h]
        self._start_mods(ts, blocks)
        try:
            for i in range(nb):
                img_h, txt_h = self.block_batched(i, img_h, txt_h, ts, rope, B, valid)
            om = [r.chunk(2, dim=-1) for r in self._modf("norm_out.linear", ts)]   # (scale, shift)
        finally:
            self._mods = None
        x = self._mod_rows(img_h, [(o[1], o[0]) for o in om], 0, 1, B)
        return self.p.lin["proj_out"].forward(x, out_dtype=torch.float32).reshape(B, L, -1)

    def _forward(self, img, txt, t, grid, blocks):
        cfg = self.cfg
        nb = cfg.num_layers if blocks is None else blocks
        rope = rope_tables(cfg, 1, grid[0], grid[1], txt.shape[0], img.device)
        img_h, txt_h, temb = self.stems(img, txt, t)
        ts = silu(temb)
        self._start_mods(ts, blocks)
        try:
            for i in range(nb):
                img_h, txt_h = self.block(i, img_h, txt_h, ts, rope)
            return self.output_layer(img_h, temb)
        finally:
            self._mods = None


def make_inputs(cfg: QwenConfig, height: int = 1328, width: int = 1328, txt_len: int = 256,
                device="cuda", seed: int = 5):
    """Packed latents [(h/16)*(w/16), 64] and text states [txt_len, 3584], N(0, 1);
    timestep 500 (sigma 0.5 on the 0..1000 scale)."""
    import torch
    g = torch.Generator(device=device).manual_seed(seed)
    gh, gw = height // 16, width // 16
    img = torch.randn((gh * gw, cfg.in_channels), device=device, generator=g)
    txt = torch.randn((txt_len, cfg.joint_attention_dim), device=device, generator=g)
    t = torch.full((1,), 500.0, device=device)
    return dict(img=img, txt=txt, t=t, grid=(gh, gw))


def step_flop(cfg: QwenConfig, l_img: int, l_txt: int) -> Tuple[float, float]:
    """(linear FLOP with M > 1, attention FLOP) of one forward."""
    L = l_img + l_txt
    lin = 0.0
    for name, (n, k, _) in linear_shapes(cfg).items():
        if name.startswith("transformer_blocks"):
            if name.endswith("_mod.1"):
                continue
            m = l_txt if (".add_" in name or "txt_mlp" in name or "to_add_out" in name) else l_img
        elif name == "txt_in":
            m = l_txt
        elif name == "proj_out":
            m = l_img
        else:
            continue
        lin += 2.0 * m * n * k
    attn = cfg.num_layers * 2 * (2.0 * cfg.num_attention_heads * L * L * cfg.attention_head_dim)
    return lin, attn
