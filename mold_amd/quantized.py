"""Host-side mirror of candle's quantized API, backed by libmoldq's HIP kernels.

Names, argument meaning and error behaviour follow candle-core-mold 0.9.10's
`quantized` module and candle-transformers-mold's `quantized_nn` (pinned at
/root/reference/Cargo.lock:507-597), as mold calls them:

  GgmlDType.block_size()          flux/pipeline.rs:198
  QTensor.dtype() / dequantize()  flux/lora.rs:759,765; qwen_image/quantized_transformer.rs:62-66
  QMatMul.forward(x)              flux2/quantized_transformer.rs:40-45 (via Linear)
  Linear(weight, bias)            qwen_image/quantized_transformer.rs:89 (Linear::from_arc)
  Device(ordinal)                 device.rs:165 (Device::new_cuda)

(paths under /root/reference/crates/mold-inference/src).  torch tensors are
only the carrier for device memory and streams; every computation is a
libmoldq call.  Errors raise MoldqError (candle returns Err(..)).
"""
from __future__ import annotations

import ctypes
import enum
from typing import Dict, Optional, Sequence, Tuple

import numpy as np

from . import _lib
from ._lib import check


class GgmlDType(enum.IntEnum):
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    BF16 = 30

    def block_size(self) -> int:
        return _lib.load().mq_block_size(int(self))

    def type_size(self) -> int:
        return _lib.load().mq_type_size(int(self))

    @property
    def is_quantized(self) -> bool:
        return self.block_size() > 1


QUANT_TYPES = [GgmlDType.Q4_0, GgmlDType.Q4_1, GgmlDType.Q5_0, GgmlDType.Q5_1, GgmlDType.Q8_0,
               GgmlDType.Q2_K, GgmlDType.Q3_K, GgmlDType.Q4_K, GgmlDType.Q5_K, GgmlDType.Q6_K]


def _torch():
    import torch
    return torch


def _stream_ptr(stream=None) -> int:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


class Device:
    """One GPU (libmoldq context).  candle: Device::new_cuda(ordinal)."""

    def __init__(self, ordinal: int = 0):
        lib = _lib.load()
        h = ctypes.c_void_p()
        check(lib.mq_ctx_create(ordinal, ctypes.byref(h)))
        self._h = h
        self.ordinal = ordinal

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def reserve_arena(self, nbytes: int) -> None:
        check(_lib.load().mq_ctx_reserve_arena(self._h, nbytes))

    def reserve_scratch(self, nbytes: int) -> None:
        """Minimum size of every stream's workspace (staging + split-K partials)."""
        check(_lib.load().mq_ctx_reserve_scratch(self._h, nbytes))

    def reserve_stream_scratch(self, nbytes: int, stream=None) -> None:
        """Grow one stream's workspace now (e.g. before capturing it in a graph)."""
        check(_lib.load().mq_ctx_reserve_stream_scratch(self._h, _stream_ptr(stream), nbytes))

    def set_stream_tail_split(self, stream, enabled: bool) -> None:
        """mq_ctx_set_stream_tail_split: whether GEMMs on `stream` may split K
        over a partial last round of tiles (off for a stream whose GEMMs run
        beside another stream's)."""
        check(_lib.load().mq_ctx_set_stream_tail_split(self._h, _stream_ptr(stream), int(bool(enabled))))

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.load().mq_ctx_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _dtype_code(dt) -> int:
    torch = _torch()
    if dt in (torch.float32, "f32", GgmlDType.F32):
        return int(GgmlDType.F32)
    if dt in (torch.bfloat16, "bf16", GgmlDType.BF16):
        return int(GgmlDType.BF16)
    if dt in (torch.float16, "f16", GgmlDType.F16):
        return int(GgmlDType.F16)
    raise ValueError(f"unsupported dtype {dt}")


class QTensor:
    """A device-resident GGUF weight [n, k] (rows = output features)."""

    def __init__(self, device: Device, handle: ctypes.c_void_p):
        self.device = device
        self._h = handle
        lib = _lib.load()
        dt, n, k = ctypes.c_int(), ctypes.c_int64(), ctypes.c_int64()
        gb, db = ctypes.c_size_t(), ctypes.c_size_t()
        check(lib.mq_qtensor_info(handle, ctypes.byref(dt), ctypes.byref(n), ctypes.byref(k),
                                  ctypes.byref(gb), ctypes.byref(db)))
        self._dtype = GgmlDType(dt.value)
        self.shape = (n.value, k.value)
        self._gguf_bytes = gb.value
        self.device_bytes = db.value

    # candle: a QTensor from GGUF blocks already in host memory (the upload
    # path); QTensor::quantize_onto is `quantize` below, on the GPU.
    @classmethod
    def from_blocks(cls, device: Device, dtype: GgmlDType, shape: Sequence[int], blocks) -> "QTensor":
        """Upload GGUF blocks from host memory (bytes / numpy uint8)."""
        n, k = int(shape[0]), int(shape[1])
        buf = np.ascontiguousarray(np.frombuffer(blocks, dtype=np.uint8) if isinstance(blocks, (bytes, bytearray))
                                   else np.asarray(blocks, dtype=np.uint8)).reshape(-1)
        h = ctypes.c_void_p()
        check(_lib.load().mq_qtensor_upload(device.handle, int(dtype), n, k, buf.ctypes.data, buf.nbytes,
                                            ctypes.byref(h)))
        return cls(device, h)

    @classmethod
    def quantize(cls, device: Device, src, dtype: GgmlDType, stream=None) -> "QTensor":
        """candle QTensor::quantize_onto: f32 [n, k] device tensor -> GGUF blocks
        quantized on the GPU (ggml reference quantizer, byte-identical)."""
        torch = _torch()
        if src.dtype != torch.float32 or src.dim() != 2 or src.stride(1) != 1:
            raise ValueError("QTensor.quantize needs a 2-D f32 device tensor with unit column stride")
        n, k = src.shape
        h = ctypes.c_void_p()
        check(_lib.load().mq_quantize(device.handle, int(dtype), n, k, src.data_ptr(), src.stride(0),
                                      _stream_ptr(stream), ctypes.byref(h)))
        return cls(device, h)

    @classmethod
    def from_device_blocks(cls, device: Device, dtype: GgmlDType, shape: Sequence[int], blocks_tensor,
                           stream=None) -> "QTensor":
        """Build from GGUF blocks already in device memory (a uint8 torch tensor)."""
        n, k = int(shape[0]), int(shape[1])
        h = ctypes.c_void_p()
        check(_lib.load().mq_qtensor_from_device(device.handle, int(dtype), n, k, blocks_tensor.data_ptr(),
                                                 blocks_tensor.numel() * blocks_tensor.element_size(),
                                                 _stream_ptr(stream), ctypes.byref(h)))
        return cls(device, h)

    @classmethod
    def concat_rows(cls, device: Device, parts: Sequence["QTensor"]) -> "QTensor":
        """Stack tensors of one type and k by rows, on the device (mq_qtensor_concat_rows)."""
        parts = list(parts)
        arr = (ctypes.c_void_p * max(1, len(parts)))(*[p.handle.value for p in parts])
        h = ctypes.c_void_p()
        check(_lib.load().mq_qtensor_concat_rows(device.handle, arr, len(parts), ctypes.byref(h)))
        return cls(device, h)

    def dtype(self) -> GgmlDType:
        return self._dtype

    def storage_size_in_bytes(self) -> int:
        return self._gguf_bytes

    def data(self) -> np.ndarray:
        """GGUF blocks read back from the device (byte-identical to the upload)."""
        out = np.empty(self._gguf_bytes, dtype=np.uint8)
        check(_lib.load().mq_qtensor_download(self.device.handle, self._h, out.ctypes.data, out.nbytes))
        return out

    def dequantize(self, dtype=None, out=None, stream=None):
        """Dense [n, k] torch tensor on the device (f32 by default, or f16/bf16)."""
        torch = _torch()
        dtype = torch.float32 if dtype is None else dtype
        if out is None:
            out = torch.empty(self.shape, dtype=dtype, device=f"cuda:{self.device.ordinal}")
        assert out.is_contiguous() and tuple(out.shape) == self.shape and out.dtype == dtype
        check(_lib.load().mq_dequantize(self.device.handle, self._h, out.data_ptr(), _dtype_code(dtype),
                                        _stream_ptr(stream)))
        return out

    def free(self) -> None:
        if getattr(self, "_h", None):
            _lib.load().mq_qtensor_free(self._h)
            self._h = None

    @property
    def handle(self):
        return self._h

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


ACT_NONE, ACT_GELU_TANH = 0, 1


class QMatMul:
    """candle QMatMul: y = x . W^T with W a QTensor; x [..., k] on the device."""

    def __init__(self, w: QTensor):
        self.w = w

    @classmethod
    def from_qtensor(cls, w: QTensor) -> "QMatMul":
        return cls(w)

    def workspace_bytes(self, m: int, x_dtype=None, gated: bool = False) -> int:
        """Stream workspace a call with `m` rows needs (the bound over x placements)."""
        torch = _torch()
        out = ctypes.c_size_t()
        check(_lib.load().mq_qmatmul_workspace_size(self.w.device.handle, self.w.handle,
                                                    _dtype_code(x_dtype or torch.float32), int(m), int(gated),
                                                    ctypes.byref(out)))
        return out.value

    def forward(self, x, bias=None, act: int = ACT_NONE, out_dtype=None, out=None, stream=None, act_from: int = 0):
        """y = act(x . W^T + bias); with act_from > 0 the activation applies to output
        columns act_from .. n-1 only (mq_qmatmul_act_from)."""
        torch = _torch()
        n, k = self.w.shape
        if not 0 <= act_from <= n:
            raise ValueError(f"QMatMul: act_from {act_from} outside 0 .. {n}")

        def call(xp, xt, m, ldx, y, yt, ldy, b):
            lib = _lib.load()
            if act_from:
                return lib.mq_qmatmul_act_from(self.w.device.handle, self.w.handle, xp, xt, m, ldx, y, yt, ldy, b,
                                               int(act), int(act_from), _stream_ptr(stream))
            return lib.mq_qmatmul(self.w.device.handle, self.w.handle, xp, xt, m, ldx, y, yt, ldy, b, int(act),
                                  _stream_ptr(stream))
        if isinstance(x, Q8KActivations):
            if x.k != k:
                raise ValueError(f"QMatMul: x k {x.k} != weight k {k}")
            out_dtype = out_dtype or (out.dtype if out is not None else torch.float32)
            if out is None:
                out = torch.empty((x.m, n), dtype=out_dtype, device=x.data.device)
            assert out.dtype == out_dtype and tuple(out.shape) == (x.m, n)
            if bias is not None:
                assert bias.dtype == torch.float32 and bias.is_contiguous() and bias.numel() == n
            check(call(x.data.data_ptr(), _lib.MQ_X_Q8K, x.m, k, out.data_ptr(), _dtype_code(out_dtype), out.stride(0),
                       bias.data_ptr() if bias is not None else None))
            return out.reshape(*x.lead, n)
        if x.shape[-1] != k:
            raise ValueError(f"QMatMul: x last dim {x.shape[-1]} != weight k {k}")
        lead = x.shape[:-1]
        x2 = x.reshape(-1, k)
        if x2.stride(1) != 1:
            x2 = x2.contiguous()
        m = x2.shape[0]
        if out_dtype is None:
            out_dtype = out.dtype if out is not None else x.dtype
        if out is None:
            out = torch.empty((m, n), dtype=out_dtype, device=x.device)
        else:
            assert out.dtype == out_dtype and tuple(out.shape) == (m, n)
        if bias is not None:
            assert bias.dtype == torch.float32 and bias.is_contiguous() and bias.numel() == n
        check(call(x2.data_ptr(), _dtype_code(x2.dtype), m, x2.stride(0), out.data_ptr(), _dtype_code(out_dtype),
                   out.stride(0), bias.data_ptr() if bias is not None else None))
        return out.reshape(*lead, n)

    __call__ = forward


class Q8KActivations:
    """Activations quantized once (mq_quantize_x_q8k) for several Q4_K GEMVs
    (m <= 8): QMatMul.forward on them equals QMatMul.forward on the f32 / bf16 x
    they came from, bit for bit, without re-quantizing x in every call.  Every
    adaLN modulation linear of a DiT step reads the same silu(vec)
    (crates/mold-inference/src/flux/offload.rs:143-156)."""

    def __init__(self, device: Device, x, stream=None):
        torch = _torch()
        x2 = x.reshape(-1, x.shape[-1])
        if x2.stride(1) != 1 or (x2.data_ptr() % 16) or (x2.stride(0) * x2.element_size()) % 16:
            x2 = x2.contiguous()
        self.m, self.k = int(x2.shape[0]), int(x2.shape[1])
        self.lead = tuple(x.shape[:-1])
        self.data = torch.empty((self.m, (self.k // 256) * _lib.MQ_X_Q8K_BLOCK_BYTES), dtype=torch.uint8,
                                device=x.device)
        check(_lib.load().mq_quantize_x_q8k(device.handle, x2.data_ptr(), _dtype_code(x2.dtype), self.m, self.k,
                                            x2.stride(0), self.data.data_ptr(), _stream_ptr(stream)))


class Linear:
    """candle-transformers quantized_nn::Linear: QMatMul plus optional f32 bias."""

    def __init__(self, weight: QTensor, bias=None):
        self.matmul = QMatMul(weight)
        self.bias = bias

    @classmethod
    def from_arc(cls, weight: QTensor, bias=None) -> "Linear":
        return cls(weight, bias)

    def forward(self, x, act: int = ACT_NONE, out_dtype=None, stream=None, act_from: int = 0):
        return self.matmul.forward(x, bias=self.bias, act=act, out_dtype=out_dtype, stream=stream, act_from=act_from)

    def gated_add(self, x, gate, residual, stream=None):
        """residual += gate * forward(x), in place, fused into the GEMM epilogue
        (mq_qmatmul_gated_add); residual f32 [m, n] with unit column stride,
        gate f32 with n elements.  Returns residual."""
        torch = _torch()
        qt = self.matmul.w
        n, k = qt.shape
        x2 = x.reshape(-1, k)
        if x2.stride(1) != 1:
            x2 = x2.contiguous()
        g = gate.reshape(-1)
        if residual.dtype != torch.float32 or residual.dim() != 2 or residual.stride(1) != 1 \
                or tuple(residual.shape) != (x2.shape[0], n):
            raise ValueError("gated_add: residual must be f32 [m, n] with unit column stride")
        if g.dtype != torch.float32 or not g.is_contiguous() or g.numel() != n:
            raise ValueError("gated_add: gate must be contiguous f32 with n elements")
        b = self.bias
        check(_lib.load().mq_qmatmul_gated_add(qt.device.handle, qt.handle, x2.data_ptr(), _dtype_code(x2.dtype),
                                               x2.shape[0], x2.stride(0), residual.data_ptr(), residual.stride(0),
                                               b.data_ptr() if b is not None else None, g.data_ptr(),
                                               _stream_ptr(stream)))
        return residual

    __call__ = forward


class StackedLinear:
    """Quantized linears that read the same input, stacked by rows into one
    resident weight so that one GEMV / GEMM computes all of them.

    mold's DiT blocks each project the same conditioning vector (FLUX's
    `vec`, Qwen-Image's `temb`) through their own adaLN modulation linear
    (flux/offload.rs:143-156 and :282-283, qwen_image/quantized_transformer.rs:869-881);
    stacked, a step's modulations are one launch streaming every modulation
    weight once.  At GEMV sizes (m <= 8) each output row is computed by the
    same per-row arithmetic as in the part's own forward, so the outputs are
    identical; a larger m runs the GEMM, which may split K differently for the
    tiles of a partial last round (same values within f32 rounding).  The stacked
    weight is a byte copy of the parts' GGUF blocks (same type and k), made on
    the device when the stack is built (a second resident copy: 1.83 GB for
    FLUX.1-dev's 77 modulations, 3.85 GB for Qwen-Image's 121); the parts stay
    usable on their own, and a part replaced afterwards is seen by `matches`
    (callers rebuild the stack, again without a host round trip)."""

    def __init__(self, device: Device, parts: Sequence[Tuple[str, Linear]]):
        torch = _torch()
        if not parts:
            raise ValueError("StackedLinear needs at least one part")
        w0 = parts[0][1].matmul.w
        dtype, k = w0.dtype(), w0.shape[1]
        self.names, self.offsets = [], {}
        self._ids = [(name, id(lin), id(lin.matmul.w), id(lin.bias)) for name, lin in parts]
        # the objects behind the ids stay alive (so no id is reused) while the stack lives
        self._keep = [(lin, lin.matmul.w, lin.bias) for _, lin in parts]
        ws, biases, row = [], [], 0
        for name, lin in parts:
            w = lin.matmul.w
            if w.dtype() != dtype or w.shape[1] != k:
                raise ValueError(f"StackedLinear: {name} is {w.dtype().name} [{w.shape[0]}, {w.shape[1]}], "
                                 f"the stack {dtype.name} with k = {k}")
            n = w.shape[0]
            ws.append(w)
            biases.append(lin.bias if lin.bias is not None
                          else torch.zeros((n,), dtype=torch.float32, device=f"cuda:{device.ordinal}"))
            self.names.append(name)
            self.offsets[name] = (row, n)
            row += n
        qt = QTensor.concat_rows(device, ws)     # the parts' GGUF blocks in order, built on the device
        self.linear = Linear(qt, torch.cat([b.reshape(-1).float() for b in biases]).contiguous())

    def matches(self, parts: Sequence[Tuple[str, Linear]]) -> bool:
        """True when `parts` are the very Linear objects (weights and biases) stacked."""
        return [(name, id(lin), id(lin.matmul.w), id(lin.bias)) for name, lin in parts] == self._ids

    def forward(self, x, out_dtype=None, stream=None) -> Dict[str, object]:
        """{part name: its output [..., n_part]} (column views of one result)."""
        y = self.linear.forward(x, out_dtype=out_dtype, stream=stream)
        return {name: y[..., r0:r0 + n] for name, (r0, n) in self.offsets.items()}

    __call__ = forward
