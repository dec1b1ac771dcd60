"""GGUF files through libmoldq: the reader (candle gguf_file::Content::read,
used by mold at /root/reference/crates/mold-inference/src/flux/pipeline.rs:286-287
and through VarBuilder::from_gguf at :976), its metadata, the writer (candle
gguf_file::write, pipeline.rs:240 and :541), and mold's two GGUF cache
producers built on them:

* fp8_safetensors_to_gguf: the conversion step of ensure_fp8_gguf_cache
  (pipeline.rs:120-252): every FP8 E4M3 tensor of a safetensors checkpoint is
  quantized to Q8_0 on the GPU (mq_quantize_fp8), the small or odd-shaped ones
  are stored as F32, the checkpoint's name prefix is stripped;
* patch_embeddings: the patch step of ensure_gguf_embeddings (pipeline.rs:
  431-547): a city96-format GGUF that ships only the diffusion blocks gets the
  FLUX input embedding tensors copied from a complete reference GGUF.

The cache-path naming, cleanup of older cache names and the search for a
downloaded reference model stay with the caller (they are file management,
not formats).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, Iterable, List, Optional, Sequence, Tuple, Union

import numpy as np

from . import _lib
from ._lib import check
from .quantized import Device, GgmlDType, QTensor, _stream_ptr

# GGUF metadata value types
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_NP = {T_U8: np.uint8, T_I8: np.int8, T_U16: np.uint16, T_I16: np.int16, T_U32: np.uint32, T_I32: np.int32,
       T_F32: np.float32, T_BOOL: np.uint8, T_U64: np.uint64, T_I64: np.int64, T_F64: np.float64}


@dataclass
class TensorInfo:
    name: str
    dtype: GgmlDType
    dims: List[int]      # GGUF order: dims[0] = ne[0] (contiguous axis)
    offset: int
    nbytes: int

    @property
    def shape(self) -> Tuple[int, ...]:
        """candle shape (reversed GGUF dims)."""
        return tuple(reversed(self.dims))


class Content:
    """candle gguf_file::Content: tensor table and metadata of a GGUF file."""

    def __init__(self, path: str):
        lib = _lib.load()
        h = ctypes.c_void_p()
        check(lib.mq_gguf_open(path.encode(), ctypes.byref(h)))
        self._h = h
        self.path = path
        self.version = lib.mq_gguf_version(h)
        self.tensor_infos: Dict[str, TensorInfo] = {}
        self._index: Dict[str, int] = {}
        for i in range(lib.mq_gguf_tensor_count(h)):
            name = ctypes.c_char_p()
            dt, nd = ctypes.c_int(), ctypes.c_int()
            dims = (ctypes.c_int64 * 4)()
            off, nb = ctypes.c_uint64(), ctypes.c_size_t()
            check(lib.mq_gguf_tensor_info(h, i, ctypes.byref(name), ctypes.byref(dt), ctypes.byref(nd), dims,
                                          ctypes.byref(off), ctypes.byref(nb)))
            nm = name.value.decode()
            self.tensor_infos[nm] = TensorInfo(nm, GgmlDType(dt.value), [dims[j] for j in range(nd.value)],
                                               off.value, nb.value)
            self._index[nm] = i
        self.metadata: Dict[str, object] = {}
        self.metadata_types: Dict[str, Tuple[int, int]] = {}
        for i in range(lib.mq_gguf_kv_count(h)):
            key = ctypes.c_char_p()
            ty, et, cnt = ctypes.c_int(), ctypes.c_int(), ctypes.c_uint64()
            check(lib.mq_gguf_kv_info(h, i, ctypes.byref(key), ctypes.byref(ty), ctypes.byref(et),
                                      ctypes.byref(cnt)))
            k = key.value.decode()
            self.metadata_types[k] = (ty.value, et.value)
            vals = [self._kv_elem(i, et.value, j) for j in range(cnt.value)] if et.value != T_ARR else None
            self.metadata[k] = vals if ty.value == T_ARR else vals[0]

    def _kv_elem(self, i: int, et: int, j: int):
        lib = _lib.load()
        if et == T_STR:
            p, n = ctypes.c_void_p(), ctypes.c_uint64()
            check(lib.mq_gguf_kv_str(self._h, i, j, ctypes.byref(p), ctypes.byref(n)))
            return ctypes.string_at(p.value, n.value).decode("utf-8", errors="surrogateescape")
        if et in (T_F32, T_F64):
            v = ctypes.c_double()
            check(lib.mq_gguf_kv_float(self._h, i, j, ctypes.byref(v)))
            return v.value
        v = ctypes.c_int64()
        check(lib.mq_gguf_kv_int(self._h, i, j, ctypes.byref(v)))
        return bool(v.value) if et == T_BOOL else (v.value if et != T_U64 else v.value & ((1 << 64) - 1))

    @classmethod
    def read(cls, path: str) -> "Content":
        return cls(path)

    def tensor(self, name: str, device: Device) -> QTensor:
        """Upload one quantized tensor (candle content.tensor(reader, name, device))."""
        if name not in self._index:
            raise KeyError(name)
        h = ctypes.c_void_p()
        check(_lib.load().mq_gguf_load_tensor(device.handle, self._h, self._index[name], ctypes.byref(h)))
        return QTensor(device, h)

    def tensors(self, names, device: Device) -> Dict[str, QTensor]:
        """Upload several tensors in one pipelined call (candle's quantized
        VarBuilder::from_gguf(path, device), crates/mold-inference/src/flux/
        pipeline.rs:976, which loads every tensor of the file): {name: QTensor},
        in the order given."""
        names = list(names)
        for n in names:
            if n not in self._index:
                raise KeyError(n)
        idx = (ctypes.c_int64 * max(1, len(names)))(*[self._index[n] for n in names])
        outs = (ctypes.c_void_p * max(1, len(names)))()
        check(_lib.load().mq_gguf_load_tensors(device.handle, self._h, idx, len(names), outs))
        return {n: QTensor(device, ctypes.c_void_p(outs[i])) for i, n in enumerate(names)}

    def var_builder(self, device: Device) -> Dict[str, QTensor]:
        """Every tensor of the file on the device, by name (VarBuilder::from_gguf)."""
        return self.tensors(self.tensor_infos.keys(), device)

    def tensor_bytes(self, name: str) -> np.ndarray:
        """The tensor's stored bytes (any type), as uint8."""
        if name not in self._index:
            raise KeyError(name)
        out = np.empty(self.tensor_infos[name].nbytes, dtype=np.uint8)
        check(_lib.load().mq_gguf_read_tensor(self._h, self._index[name], out.ctypes.data, out.nbytes))
        return out

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.load().mq_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _dims(shape: Sequence[int]) -> Tuple[int, ctypes.Array]:
    """candle shape -> (n_dims, GGUF-ordered int64 dims)."""
    dims = [int(s) for s in reversed(tuple(shape))]
    return len(dims), (ctypes.c_int64 * len(dims))(*dims)


class Writer:
    """candle gguf_file::write through libmoldq's writer: metadata and tensors in
    the order added; finish() writes the file (atomically, via a temp name)."""

    def __init__(self, path: str, alignment: int = 32):
        h = ctypes.c_void_p()
        check(_lib.load().mq_gguf_writer_create(path.encode(), alignment, ctypes.byref(h)))
        self._h = h
        self.path = path
        self._keep: List[object] = []   # device tensors referenced until finish

    def kv(self, key: str, value, type: Optional[int] = None) -> None:
        """One metadata value: str, bool, int (u32 by default, u64 if larger),
        float (f32), or a list of one of those (an array); `type` forces the
        GGUF value type (the element type for lists)."""
        lib = _lib.load()
        k = key.encode()
        if isinstance(value, (list, tuple)):
            if all(isinstance(v, str) for v in value) and value:
                arr = (ctypes.c_char_p * len(value))(*[v.encode() for v in value])
                check(lib.mq_gguf_writer_kv_str_array(self._h, k, arr, len(value)))
                return
            et = type if type is not None else _auto_type(value)
            a = np.ascontiguousarray(np.asarray(value, dtype=_NP[et]))
            check(lib.mq_gguf_writer_kv_array(self._h, k, et, a.ctypes.data, a.size))
            return
        if isinstance(value, str):
            check(lib.mq_gguf_writer_kv_str(self._h, k, value.encode()))
            return
        t = type if type is not None else _auto_type([value])
        a = np.asarray([value], dtype=_NP[t])
        check(lib.mq_gguf_writer_kv_scalar(self._h, k, t, a.ctypes.data))

    def add_tensor(self, name: str, dtype: GgmlDType, shape: Sequence[int], data) -> None:
        """Raw stored bytes (numpy array or bytes) of a tensor of candle `shape`."""
        buf = np.ascontiguousarray(np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray))
                                   else np.asarray(data).view(np.uint8)).reshape(-1)
        nd, dims = _dims(shape)
        check(_lib.load().mq_gguf_writer_add_tensor(self._h, name.encode(), int(dtype), nd, dims,
                                                    buf.ctypes.data, buf.nbytes))

    def add_qtensor(self, name: str, qt: QTensor, shape: Optional[Sequence[int]] = None) -> None:
        """A device-resident weight (read back at finish); `shape` (candle order,
        same element count, last dim = k) overrides its stored [n, k]."""
        if shape is None:
            nd, dims = 0, None
        else:
            nd, dims = _dims(shape)
        check(_lib.load().mq_gguf_writer_add_qtensor(self._h, qt.device.handle, name.encode(), qt.handle, nd, dims))
        self._keep.append(qt)

    def finish(self) -> None:
        check(_lib.load().mq_gguf_writer_finish(self._h))
        self._keep.clear()

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.load().mq_gguf_writer_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _auto_type(values: Sequence) -> int:
    if all(isinstance(v, bool) for v in values):
        return T_BOOL
    if all(isinstance(v, (int, np.integer)) and not isinstance(v, bool) for v in values):
        if all(0 <= int(v) < 2 ** 32 for v in values):
            return T_U32
        if all(-2 ** 63 <= int(v) < 0 or 0 <= int(v) < 2 ** 63 for v in values):
            return T_I64 if any(int(v) < 0 for v in values) else T_U64
        return T_U64
    return T_F32


def write(path: str, tensors: Sequence[Tuple[str, GgmlDType, Sequence[int], np.ndarray]],
          metadata: Dict[str, object] = None, alignment: int = 32) -> None:
    """Write a GGUF v3 file (candle gguf_file::write): `tensors` holds (name,
    dtype, candle shape, stored bytes)."""
    w = Writer(path, alignment)
    try:
        for k, v in (metadata or {}).items():
            w.kv(k, v)
        for name, dt, shape, raw in tensors:
            w.add_tensor(name, dt, shape, raw)
        w.finish()
    finally:
        w.close()


# ------------------------------------------------- mold's GGUF cache producers

def _strip_prefix(names: Iterable[str]) -> str:
    """The checkpoint prefix mold strips (pipeline.rs:183-192)."""
    names = set(names)
    for p in ("", "model.diffusion_model.", "diffusion_model."):
        if p + "img_in.weight" in names:
            return p
    return ""


def fp8_safetensors_to_gguf(src: str, dst: str, device: Device, dtype: GgmlDType = GgmlDType.Q8_0) -> Dict[str, str]:
    """The conversion of mold's ensure_fp8_gguf_cache (pipeline.rs:180-248).

    Every tensor of the safetensors file `src` is read; a tensor whose element
    count is a non-zero multiple of the block size and whose last dimension is
    a multiple of it (candle's quantizer blocks rows) is quantized to `dtype`
    on the GPU (FP8 E4M3 tensors through mq_quantize_fp8, other float dtypes
    through mq_quantize from f32); the rest are stored as F32.  Names lose the
    checkpoint prefix.  Returns {name: stored type name}."""
    import torch
    from safetensors import safe_open

    bs = {GgmlDType.Q8_0: 32, GgmlDType.Q4_0: 32, GgmlDType.Q4_1: 32, GgmlDType.Q5_0: 32,
          GgmlDType.Q5_1: 32}.get(dtype, 256)
    stored: Dict[str, str] = {}
    w = Writer(dst)
    try:
        with safe_open(src, framework="pt", device="cpu") as f:
            names = list(f.keys())
            prefix = _strip_prefix(names)
            for name in names:
                t = f.get_tensor(name)
                out_name = name[len(prefix):] if prefix and name.startswith(prefix) else name
                numel = t.numel()
                k = t.shape[-1] if t.dim() > 0 else 1
                shape = tuple(t.shape) if t.dim() > 0 else (1,)
                if numel >= bs and numel % bs == 0 and k % bs == 0:
                    n = numel // k
                    if t.dtype == torch.float8_e4m3fn:
                        src_dev = t.contiguous().view(torch.uint8).reshape(n, k).to(f"cuda:{device.ordinal}")
                        h = ctypes.c_void_p()
                        check(_lib.load().mq_quantize_fp8(device.handle, int(dtype), n, k, src_dev.data_ptr(), k,
                                                          1.0, _stream_ptr(None), ctypes.byref(h)))
                        qt = QTensor(device, h)
                    else:
                        qt = QTensor.quantize(device, t.float().reshape(n, k).to(f"cuda:{device.ordinal}"), dtype)
                    w.add_qtensor(out_name, qt, shape)
                    stored[out_name] = dtype.name
                else:
                    w.add_tensor(out_name, GgmlDType.F32, shape, t.float().contiguous().numpy())
                    stored[out_name] = "F32"
        w.finish()
    finally:
        w.close()
    return stored


FLUX_EMBEDDING_TENSORS = [
    "img_in.weight", "img_in.bias",
    "time_in.in_layer.weight", "time_in.in_layer.bias", "time_in.out_layer.weight", "time_in.out_layer.bias",
    "vector_in.in_layer.weight", "vector_in.in_layer.bias", "vector_in.out_layer.weight",
    "vector_in.out_layer.bias",
]
FLUX_GUIDANCE_EMBEDDING_TENSORS = [
    "guidance_in.in_layer.weight", "guidance_in.in_layer.bias", "guidance_in.out_layer.weight",
    "guidance_in.out_layer.bias",
]


def has_embeddings(path: str) -> bool:
    """gguf_has_embeddings (pipeline.rs:284-288): header-only check for img_in."""
    c = Content(path)
    try:
        return "img_in.weight" in c.tensor_infos
    finally:
        c.close()


def has_guidance(path: str) -> bool:
    """gguf_has_guidance (pipeline.rs:292-299)."""
    c = Content(path)
    try:
        return "guidance_in.in_layer.weight" in c.tensor_infos
    finally:
        c.close()


def patch_embeddings(src: str, reference: str, dst: str, is_schnell: bool) -> int:
    """The patch of ensure_gguf_embeddings (pipeline.rs:488-547): every tensor of
    `src` in its order, then each needed embedding tensor that `src` lacks,
    copied byte for byte from `reference`; written to `dst` with no metadata
    (as mold does).  Returns the number of tensors patched; raises ValueError
    (mold's message) when the reference lacks one."""
    needed = FLUX_EMBEDDING_TENSORS + ([] if is_schnell else FLUX_GUIDANCE_EMBEDDING_TENSORS)
    s, r = Content(src), Content(reference)
    w = Writer(dst)
    try:
        for name, info in s.tensor_infos.items():
            w.add_tensor(name, info.dtype, info.shape, s.tensor_bytes(name))
        patched = 0
        for name in needed:
            if name in s.tensor_infos:
                continue
            if name not in r.tensor_infos:
                raise ValueError(f"the only downloaded reference is also missing '{name}'. This model needs a "
                                 f"complete flux-dev GGUF")
            info = r.tensor_infos[name]
            w.add_tensor(name, info.dtype, info.shape, r.tensor_bytes(name))
            patched += 1
        w.finish()
        return patched
    finally:
        w.close()
        s.close()
        r.close()
