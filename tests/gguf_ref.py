"""An independent restatement of the GGUF v3 byte layout, for tests only: the
library's writer must produce exactly these bytes, and its reader must parse
what this writes (nested arrays included, which the library cannot write).

Layout (the published GGUF spec that candle's gguf_file implements): u32 magic
"GGUF", u32 version, u64 n_tensors, u64 n_kv, the metadata (u64-length key,
u32 type, value; arrays are u32 element type, u64 count, elements), the tensor
infos (name, u32 n_dims, u64 ne[n_dims], u32 ggml type, u64 offset from the
data start), zero padding to the alignment, then the data, each tensor at an
aligned offset.
"""
import struct

import numpy as np

MAGIC = 0x46554747
FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}


def gstr(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def value(vtype: int, v, elem_type: int = None) -> bytes:
    """Encoded value of GGUF type `vtype` (for arrays: list `v` of `elem_type`)."""
    if vtype == 8:
        return gstr(v)
    if vtype == 9:
        out = struct.pack("<IQ", elem_type, len(v))
        for e in v:
            if elem_type == 9:
                et2, vals = e
                out += value(9, vals, et2)
            else:
                out += value(elem_type, e)
        return out
    return struct.pack(FMT[vtype], int(v) if vtype == 7 else v)


def write(path, metadata, tensors, alignment=32):
    """metadata: list of (key, type, value[, elem_type]); tensors: list of
    (name, ggml type, candle shape, bytes)."""
    out = bytearray(struct.pack("<IIQQ", MAGIC, 3, len(tensors), len(metadata)))
    for kv in metadata:
        key, vt, v = kv[0], kv[1], kv[2]
        out += gstr(key) + struct.pack("<I", vt) + value(vt, v, kv[3] if len(kv) > 3 else None)
    off = 0
    offsets = []
    for name, dt, shape, raw in tensors:
        raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
        ne = [int(s) for s in reversed(shape)]
        out += gstr(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne)
        out += struct.pack("<IQ", int(dt), off)
        offsets.append(off)
        off = (off + raw.nbytes + alignment - 1) // alignment * alignment
    out += b"\0" * ((-len(out)) % alignment)
    start = len(out)
    for (name, dt, shape, raw), o in zip(tensors, offsets):
        raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
        out += b"\0" * (start + o - len(out))
        out += raw.tobytes()
    out += b"\0" * ((start - len(out)) % alignment)
    with open(path, "wb") as f:
        f.write(bytes(out))
