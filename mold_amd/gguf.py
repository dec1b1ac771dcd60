"""GGUF files: a writer (mirrors candle gguf_file::write, used by mold at
/root/reference/crates/mold-inference/src/flux/pipeline.rs:240) and the reader
exposed by libmoldq (candle gguf_file::Content::read, pipeline.rs:286-287,
and VarBuilder::from_gguf, pipeline.rs:976).
"""
from __future__ import annotations

import ctypes
import struct
from dataclasses import dataclass
from typing import Dict, List, Sequence, Tuple, Union

import numpy as np

from . import _lib
from ._lib import check
from .quantized import Device, GgmlDType, QTensor

GGUF_MAGIC = 0x46554747
_T_U32, _T_STR, _T_F32, _T_U64 = 4, 8, 6, 10


def _gstr(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def write(path: str, tensors: Sequence[Tuple[str, GgmlDType, Sequence[int], np.ndarray]],
          metadata: Dict[str, Union[int, float, str]] = None, alignment: int = 32, version: int = 3) -> None:
    """Write a GGUF v3 file.  `tensors` holds (name, dtype, shape, raw bytes);
    shape is given candle-style [rows, cols] and stored reversed (ne[0] = cols)."""
    metadata = dict(metadata or {})
    if alignment != 32:
        metadata["general.alignment"] = int(alignment)
    out = bytearray()
    out += struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(metadata))
    for key, val in metadata.items():
        out += _gstr(key)
        if isinstance(val, str):
            out += struct.pack("<I", _T_STR) + _gstr(val)
        elif isinstance(val, float):
            out += struct.pack("<If", _T_F32, val)
        elif key == "general.alignment":
            out += struct.pack("<II", _T_U32, val)
        else:
            out += struct.pack("<IQ", _T_U64, val)
    offsets = []
    off = 0
    for name, dt, shape, raw in tensors:
        raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
        offsets.append(off)
        off += raw.nbytes
        off = (off + alignment - 1) // alignment * alignment
        ne = list(reversed([int(s) for s in shape]))
        out += _gstr(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne)
        out += struct.pack("<IQ", int(dt), offsets[-1])
    pad = (-len(out)) % alignment
    out += b"\0" * pad
    data_start = len(out)
    for (name, dt, shape, raw), o in zip(tensors, offsets):
        raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
        cur = len(out) - data_start
        out += b"\0" * (o - cur)
        out += raw.tobytes()
    with open(path, "wb") as f:
        f.write(out)


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
    """candle gguf_file::Content: tensor table of a GGUF file (via libmoldq)."""

    def __init__(self, path: str):
        lib = _lib.load()
        h = ctypes.c_void_p()
        check(lib.mq_gguf_open(path.encode(), ctypes.byref(h)))
        self._h = h
        self.path = path
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

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.load().mq_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
