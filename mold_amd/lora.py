"""mold's GGUF LoRA path on the device (crates/mold-inference/src/flux/lora.rs).

mold patches a GGUF FLUX transformer with a diffusers-format LoRA by loading
every tensor, then for each targeted tensor: dequantize to f32 on the CPU, add
delta = (B . A) * effective_scale on the whole tensor or a row slice of a fused
tensor, and re-quantize to the original GGML type with quantize_onto
(gguf_lora_var_builder, lora.rs:661-869).  Here the tensor never leaves HBM:
mq_dequantize -> mq_lora_apply (per patch, on the target rows) -> mq_quantize.

Restated from the reference (same names, same rules): the adapter file format
(LoraAdapter::load, lora.rs:63-97), the diffusers -> candle key mapping
(map_lora_key, :117-235), the fused-slice rows (fused_slice_range, :237-261)
and the effective scale scale * alpha / rank (:689-692).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

from . import _lib
from ._lib import check
from .quantized import Device, GgmlDType, QTensor, _stream_ptr


@dataclass
class LoraTarget:
    """Direct (num_components is None) or a fused row slice of candle_key."""
    candle_key: str
    component: Optional[int] = None
    num_components: Optional[int] = None

    @property
    def fused(self) -> bool:
        return self.component is not None


_DOUBLE_FUSED = {
    "attn.to_q": ("img_attn.qkv.weight", 0), "attn.to_k": ("img_attn.qkv.weight", 1),
    "attn.to_v": ("img_attn.qkv.weight", 2), "attn.add_q_proj": ("txt_attn.qkv.weight", 0),
    "attn.add_k_proj": ("txt_attn.qkv.weight", 1), "attn.add_v_proj": ("txt_attn.qkv.weight", 2),
}
_DOUBLE_DIRECT = {
    "attn.to_out.0": "img_attn.proj.weight", "attn.to_add_out": "txt_attn.proj.weight",
    "ff.net.0.proj": "img_mlp.0.weight", "ff.net.2": "img_mlp.2.weight",
    "ff_context.net.0.proj": "txt_mlp.0.weight", "ff_context.net.2": "txt_mlp.2.weight",
    "norm1.linear": "img_mod.lin.weight", "norm1_context.linear": "txt_mod.lin.weight",
}
_SINGLE_FUSED = {"attn.to_q": 0, "attn.to_k": 1, "attn.to_v": 2, "proj_mlp": 3}
_SINGLE_DIRECT = {"proj_out": "linear2.weight", "norm.linear": "modulation.lin.weight"}


def map_lora_key(diffusers_key: str) -> Optional[LoraTarget]:
    """map_lora_key (lora.rs:117-235): None for keys mold does not recognize."""
    key = diffusers_key[len("transformer."):] if diffusers_key.startswith("transformer.") else diffusers_key
    for prefix, block_fmt, fused, direct, ncomp in (
            ("transformer_blocks.", "double_blocks.{}", _DOUBLE_FUSED, _DOUBLE_DIRECT, 3),
            ("single_transformer_blocks.", "single_blocks.{}", None, _SINGLE_DIRECT, 0)):
        if not key.startswith(prefix):
            continue
        rest = key[len(prefix):]
        if "." not in rest:
            return None
        idx, layer = rest.split(".", 1)
        if not idx.isdigit():
            return None
        block = block_fmt.format(idx)
        if fused is not None and layer in fused:
            name, comp = fused[layer]
            return LoraTarget(f"{block}.{name}", comp, ncomp)
        if fused is None and layer in _SINGLE_FUSED:
            return LoraTarget(f"{block}.linear1.weight", _SINGLE_FUSED[layer], 0)   # 0: single-block rule
        if layer in direct:
            return LoraTarget(f"{block}.{direct[layer]}")
        return None
    return None


def fused_slice_range(base_rows: int, lora_out_dim: int, component: int, num_components: int) -> Tuple[int, int]:
    """fused_slice_range (lora.rs:237-261): (row offset, rows) of a component.
    num_components > 0: equal split; 0: single-block linear1 [Q, K, V, MLP]."""
    if num_components > 0:
        size = base_rows // num_components
        return component * size, size
    if component < 3:
        return component * lora_out_dim, lora_out_dim
    qkv_dim = (base_rows - lora_out_dim) // 3
    return 3 * qkv_dim, lora_out_dim


@dataclass
class LoraLayer:
    a: object          # torch tensor [rank, in]
    b: object          # torch tensor [out, rank]
    alpha: Optional[float]


class LoraAdapter:
    """LoraAdapter::load (lora.rs:63-97): `<layer>.lora_A.weight`,
    `<layer>.lora_B.weight` and optional `<layer>.alpha` from a safetensors file."""

    def __init__(self, layers: Dict[str, LoraLayer], rank: int):
        self.layers = layers
        self.rank = rank

    @classmethod
    def load(cls, path: str) -> "LoraAdapter":
        import torch
        from safetensors.torch import load_file
        tensors = load_file(path, device="cpu")
        a_t, b_t, alpha = {}, {}, {}
        rank = 0
        for name, t in tensors.items():
            if name.endswith(".lora_A.weight"):
                layer = name[:-len(".lora_A.weight")]
                rank = max(rank, t.shape[0])
                a_t[layer] = t
            elif name.endswith(".lora_B.weight"):
                b_t[name[:-len(".lora_B.weight")]] = t
            elif name.endswith(".alpha"):
                # mold keeps alpha only when `tensor.to_scalar::<f32>()` succeeds
                # (lora.rs:77-79): a rank-0 F32 tensor.  Any other alpha (bf16 / f16,
                # or shape [1]) is dropped there, so the effective scale is `scale`.
                if t.dim() == 0 and t.dtype == torch.float32:
                    alpha[name[:-len(".alpha")]] = float(t.item())
        layers = {k: LoraLayer(a, b_t[k], alpha.get(k)) for k, a in a_t.items() if k in b_t}
        if not layers:
            raise ValueError(f"no LoRA A/B pairs found in {path}")
        return cls(layers, rank)


@dataclass
class LoraPatch:
    a: object
    b: object
    effective_scale: float
    target: LoraTarget


def build_patches(adapter: LoraAdapter, scale: float) -> Tuple[Dict[str, List[LoraPatch]], int]:
    """The patch index of gguf_lora_var_builder (lora.rs:681-707): per candle key,
    its patches with effective_scale = scale * alpha / rank (or scale without
    alpha); returns (patches, skipped).  Patches keep the adapter's key order."""
    patches: Dict[str, List[LoraPatch]] = {}
    skipped = 0
    for key, layer in adapter.layers.items():
        target = map_lora_key(key)
        if target is None:
            skipped += 1
            continue
        rank = layer.a.shape[0]
        eff = scale * layer.alpha / rank if layer.alpha is not None else scale
        patches.setdefault(target.candle_key, []).append(LoraPatch(layer.a, layer.b, eff, target))
    return patches, skipped


def lora_apply(w, b, a, scale: float, stream=None) -> None:
    """w[rows, k] += (b . a) * scale in place on device f32 tensors (mq_lora_apply)."""
    import torch
    assert w.dtype == torch.float32 and w.dim() == 2 and w.stride(1) == 1
    b = b.to(device=w.device, dtype=torch.float32).contiguous()
    a = a.to(device=w.device, dtype=torch.float32).contiguous()
    rows, k = w.shape
    rank = a.shape[0]
    if b.shape != (rows, rank) or a.shape != (rank, k):
        raise ValueError(f"LoRA shapes b {tuple(b.shape)} a {tuple(a.shape)} do not fit rows {rows} x k {k}")
    check(_lib.load().mq_lora_apply(w.data_ptr(), w.stride(0), rows, k, b.data_ptr(), rank, a.data_ptr(), k, rank,
                                    ctypes.c_float(scale), _stream_ptr(stream)))


def patch_qtensor(qt: QTensor, patches: List[LoraPatch]) -> Tuple[QTensor, int]:
    """One targeted tensor (lora.rs:748-849) on the device: dequantize to f32,
    apply each patch (whole tensor, or its fused row slice; an out-of-range
    slice is skipped as mold does), re-quantize to the original type.
    Returns (new tensor, patches applied)."""
    t = qt.dequantize()
    base_rows = t.shape[0]
    applied = 0
    for p in patches:
        if p.target.fused:
            off, size = fused_slice_range(base_rows, p.b.shape[0], p.target.component, p.target.num_components)
            if off + size > base_rows:
                continue
            lora_apply(t[off:off + size], p.b, p.a, p.effective_scale)
        else:
            lora_apply(t, p.b, p.a, p.effective_scale)
        applied += 1
    out = QTensor.quantize(qt.device, t, qt.dtype())
    return out, applied


def gguf_lora_var_builder(transformer_path: str, adapter: LoraAdapter, scale: float, device: Device):
    """gguf_lora_var_builder (lora.rs:661-869) with the patching on the GPU.
    Every tensor of the file is loaded to the device as a QTensor
    (content.tensor(.., device), lora.rs:721-723), dense F32 / F16 / BF16 ones
    included; each targeted tensor is dequantized to f32, patched and
    re-quantized to its own type (quantize_onto, :849), as mold does.
    Returns ({name: QTensor}, applied patch count): the tensor set that mold
    hands to VarBuilder::from_qtensors (:868)."""
    from . import gguf
    patches, _ = build_patches(adapter, scale)
    c = gguf.Content.read(transformer_path)
    data: Dict[str, QTensor] = {}
    try:
        for name in c.tensor_infos:
            data[name] = c.tensor(name, device)
    finally:
        c.close()
    applied = 0
    for key, plist in patches.items():
        if key in data:
            data[key], n = patch_qtensor(data[key], plist)
            applied += n
    return data, applied
