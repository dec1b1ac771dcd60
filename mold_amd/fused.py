"""Fused block glue on the device: libmoldq's row passes between the quantized
linears (mq_adaln_modulate, mq_gelu_tanh_bf16, mq_qk_norm_rope and
mq_attn_pad_correct in include/moldq.h).

All run on torch's current stream and allocate only their outputs.  They need
the HIP library (no fallback); the host-CPU path of the block graphs keeps the
equivalent torch ops.
"""
from __future__ import annotations

from . import _lib
from ._lib import check
from .quantized import _stream_ptr

HEAD_DIM = 128


def adaln_modulate(x, shift, scale, eps: float = 1e-6, out=None):
    """bf16(LayerNorm_eps(x) * (1 + scale) + shift) for x f32 [rows, cols] (row
    stride x.stride(0)), shift and scale f32 with cols elements."""
    import torch
    if x.dtype != torch.float32 or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("adaln_modulate: x must be a 2-D f32 tensor with unit column stride")
    rows, cols = x.shape
    shift = shift.reshape(-1)
    scale = scale.reshape(-1)
    for t in (shift, scale):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != cols:
            raise ValueError("adaln_modulate: shift and scale must be contiguous f32 with cols elements")
    if out is None:
        out = torch.empty((rows, cols), dtype=torch.bfloat16, device=x.device)
    check(_lib.load().mq_adaln_modulate(x.data_ptr(), rows, cols, x.stride(0), shift.data_ptr(), scale.data_ptr(),
                                        float(eps), out.data_ptr(), out.stride(0), _stream_ptr()))
    return out


def gelu_tanh_bf16(src, out):
    """out[:] = bf16(gelu_tanh(src)) for src f32 or bf16 [rows, cols] and out bf16 [rows, cols],
    both with unit column stride (row strides free, multiples of 4)."""
    import torch
    from .quantized import _dtype_code
    if src.dtype not in (torch.float32, torch.bfloat16) or out.dtype != torch.bfloat16 or src.dim() != 2 \
            or tuple(out.shape) != tuple(src.shape) or src.stride(1) != 1 or out.stride(1) != 1:
        raise ValueError("gelu_tanh_bf16: src f32/bf16 and out bf16 of one 2-D shape with unit column stride")
    rows, cols = src.shape
    check(_lib.load().mq_gelu_tanh_bf16(src.data_ptr(), _dtype_code(src.dtype), rows, cols, src.stride(0),
                                        out.data_ptr(), out.stride(0), _stream_ptr()))
    return out


def new_heads(heads: int, l_total: int, device, valid=None, batch=None):
    """bf16 q, k, v buffers [heads, l_total, 128] for qk_norm_rope ([batch, heads,
    l_total, 128] with `batch`).  Rows from `valid` on (padding of the joint
    sequence) are zero, rows before it are left for qk_norm_rope to fill."""
    import torch
    shape = (heads, l_total, HEAD_DIM) if batch is None else (batch, heads, l_total, HEAD_DIM)
    # one allocation, so that the padding rows of all three clear in one launch
    qkv = torch.empty((3,) + shape, dtype=torch.bfloat16, device=device)
    if valid is not None and valid < l_total:
        qkv[..., valid:, :].zero_()
    return qkv[0], qkv[1], qkv[2]


def attn_pad_correct(o, lse, npad, rows: int, guard, out):
    """Rows 0 .. rows-1 of an attention computed over zero-padded keys, corrected
    to the softmax over the real keys: out[b, r, h*128 + j] = bf16(o[b, h, r, j]
    / (1 - npad[b] exp(-lse[b, h, r]))), and guard (0-dim f32) raised to the
    largest npad exp(-lse) (mq_attn_pad_correct).  o bf16 [B, H, >= rows, 128]
    with unit stride along the head dim; lse f32 [B, H, >= rows] with unit
    stride along rows; npad f32 [B] (contiguous); out bf16 [B, rows, H*128] or,
    for B = 1, [rows, H*128], unit column stride."""
    import torch
    if o.dtype != torch.bfloat16 or o.dim() != 4 or o.shape[3] != HEAD_DIM or o.stride(3) != 1 or o.shape[2] < rows:
        raise ValueError("attn_pad_correct: o must be bf16 [B, H, >= rows, 128] with unit stride along the head dim")
    b_, h = o.shape[0], o.shape[1]
    if lse.dtype != torch.float32 or lse.dim() != 3 or tuple(lse.shape[:2]) != (b_, h) or lse.shape[2] < rows \
            or lse.stride(2) != 1:
        raise ValueError("attn_pad_correct: lse must be f32 [B, H, >= rows] with unit stride along rows")
    if npad.dtype != torch.float32 or not npad.is_contiguous() or npad.numel() != b_:
        raise ValueError("attn_pad_correct: npad must be contiguous f32 [B]")
    if guard.dtype != torch.float32 or guard.numel() != 1:
        raise ValueError("attn_pad_correct: guard must be a one-element f32 tensor")
    o3 = out if out.dim() == 3 else out.unsqueeze(0)
    if out.dtype != torch.bfloat16 or tuple(o3.shape) != (b_, rows, h * HEAD_DIM) or o3.stride(2) != 1:
        raise ValueError("attn_pad_correct: out must be bf16 [B, rows, H*128] with unit column stride")
    for t in (o, lse, npad, guard, out):
        if t.device != o.device:
            raise ValueError("attn_pad_correct: every tensor must be on o's device")
    check(_lib.load().mq_attn_pad_correct(o.data_ptr(), b_, h, rows, o.stride(0), o.stride(1), o.stride(2),
                                          lse.data_ptr(), lse.stride(0), lse.stride(1), npad.data_ptr(),
                                          out.data_ptr(), o3.stride(0), o3.stride(1), guard.data_ptr(),
                                          _stream_ptr()))
    return out


def qk_norm_rope(qkv, heads: int, q_weight, k_weight, cos, sin, q_out, k_out, v_out, row_off: int,
                 eps: float = 1e-6):
    """RmsNorm(q), RmsNorm(k), RoPE and the head split of one segment's projection
    output qkv f32 or bf16 [rows, >= 3*heads*128] (q | k | v column blocks) into bf16
    [heads, l_total, 128] at rows row_off ..; cos / sin f32 [rows, 64] for the
    segment's tokens; q_weight / k_weight bf16 [128]."""
    import torch
    from .quantized import _dtype_code
    if qkv.dtype not in (torch.float32, torch.bfloat16) or qkv.dim() != 2 or qkv.stride(1) != 1:
        raise ValueError("qk_norm_rope: qkv must be a 2-D f32 or bf16 tensor with unit column stride")
    rows = qkv.shape[0]
    for t in (cos, sin):
        if t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != (rows, HEAD_DIM // 2):
            raise ValueError("qk_norm_rope: cos / sin must be contiguous f32 [rows, 64]")
    for t in (q_weight, k_weight):
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.numel() != HEAD_DIM:
            raise ValueError("qk_norm_rope: norm weights must be contiguous bf16 [128]")
    l_total = q_out.shape[1]
    for t in (q_out, k_out, v_out):
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or tuple(t.shape) != (heads, l_total, HEAD_DIM):
            raise ValueError("qk_norm_rope: outputs must be contiguous bf16 [heads, l_total, 128]")
    check(_lib.load().mq_qk_norm_rope(qkv.data_ptr(), _dtype_code(qkv.dtype), qkv.stride(0), rows, heads, HEAD_DIM,
                                      q_weight.data_ptr(),
                                      k_weight.data_ptr(), float(eps), cos.data_ptr(), sin.data_ptr(),
                                      q_out.data_ptr(), k_out.data_ptr(), v_out.data_ptr(), row_off, l_total,
                                      _stream_ptr()))
