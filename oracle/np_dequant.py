"""Second, independent restatement of the GGUF dequantize formulas in numpy.

TEST INFRASTRUCTURE ONLY (same rules as ``oracle.py``).

Written vectorised from the ggml block specification (ggml-common.h layouts,
ggml-quants.c ``dequantize_row_*``), with a different evaluation structure from
the scalar C oracle: every type is decoded by building the full integer code
and scale planes as arrays and then applying one f32 expression.  The two are
compared bit-for-bit in tests/test_oracle.py, so a slip in either one (a wrong
nibble, shift, sub-block index or sign) shows up as a mismatch.

Each function takes ``blocks`` (uint8, shape [nblocks, type_size]) and returns
float32 of shape [nblocks, block_size].
"""
from __future__ import annotations

import numpy as np


def _h(b: np.ndarray, off: int) -> np.ndarray:
    """Little-endian f16 field at byte offset ``off`` of every block -> f32 column."""
    return b[:, off:off + 2].copy().view(np.float16).astype(np.float32)


def _f32(*xs):
    return [np.asarray(x, dtype=np.float32) for x in xs]


def q4_0(b):
    d = _h(b, 0)
    qs = b[:, 2:18]
    q = np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(np.int32) - 8
    return (q.astype(np.float32) * d).astype(np.float32)


def q4_1(b):
    d, m = _h(b, 0), _h(b, 2)
    qs = b[:, 4:20]
    q = np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(np.float32)
    return (q * d + m).astype(np.float32)


def _qh_bits(b, off):
    qh = b[:, off:off + 4].copy().view("<u4")[:, 0].astype(np.uint64)
    bits = (qh[:, None] >> np.arange(32, dtype=np.uint64)[None, :]) & 1
    return bits.astype(np.int32)  # [nb, 32], bit j -> element j


def q5_0(b):
    d = _h(b, 0)
    hb = _qh_bits(b, 2)
    qs = b[:, 6:22]
    lo = np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(np.int32)
    q = lo + 16 * hb - 16
    return (q.astype(np.float32) * d).astype(np.float32)


def q5_1(b):
    d, m = _h(b, 0), _h(b, 2)
    hb = _qh_bits(b, 4)
    qs = b[:, 8:24]
    lo = np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(np.int32)
    q = (lo + 16 * hb).astype(np.float32)
    return (q * d + m).astype(np.float32)


def q8_0(b):
    d = _h(b, 0)
    q = b[:, 2:34].view(np.int8).astype(np.float32)
    return (q * d).astype(np.float32)


def _crumbs(qs32):
    """[nb, 32] bytes -> [nb, 128] 2-bit codes; element 32*s + l is bits 2s..2s+1 of byte l."""
    return np.concatenate([(qs32 >> (2 * s)) & 3 for s in range(4)], axis=1).astype(np.int32)


def q2_K(b):
    sc = b[:, 0:16].astype(np.int32)
    qs = b[:, 16:80]
    d, dmin = _h(b, 80), _h(b, 82)
    q = np.concatenate([_crumbs(qs[:, 0:32]), _crumbs(qs[:, 32:64])], axis=1)  # [nb, 256]
    grp = np.arange(256) // 16
    dl = d * (sc[:, grp] & 0xF).astype(np.float32)
    ml = dmin * (sc[:, grp] >> 4).astype(np.float32)
    return (dl * q.astype(np.float32) - ml).astype(np.float32)


def _q3_scales(s12):
    """12 packed bytes -> 16 six-bit scales (unsigned, still offset by 32)."""
    s12 = s12.astype(np.int32)
    j = np.arange(16)
    low = np.where(j < 8, s12[:, j % 8] & 0xF, s12[:, j % 8] >> 4)
    high = (s12[:, 8 + (j % 4)] >> (2 * (j // 4))) & 3
    return low | (high << 4)


def q3_K(b):
    hmask = b[:, 0:32]
    qs = b[:, 32:96]
    sc = _q3_scales(b[:, 96:108]) - 32
    d = _h(b, 108)
    q2 = np.concatenate([_crumbs(qs[:, 0:32]), _crumbs(qs[:, 32:64])], axis=1)
    e = np.arange(256)
    hbit = (hmask[:, e % 32].astype(np.int32) >> (e // 32)) & 1
    q = q2 - np.where(hbit == 1, 0, 4)
    dl = d * sc[:, e // 16].astype(np.float32)
    return (dl * q.astype(np.float32)).astype(np.float32)


def _k4_scale_min(s12):
    """12 packed bytes -> (8 six-bit scales, 8 six-bit mins)."""
    s = s12.astype(np.int32)
    j = np.arange(8)
    lo = j < 4
    jj = np.where(lo, j, 0)
    sc = np.where(lo, s[:, jj] & 63, (s[:, np.minimum(j + 4, 11)] & 0xF) | ((s[:, np.maximum(j - 4, 0)] >> 6) << 4))
    mn = np.where(lo, s[:, jj + 4] & 63, (s[:, np.minimum(j + 4, 11)] >> 4) | ((s[:, j] >> 6) << 4))
    return sc, mn


def _nibbles_k(qs128):
    """[nb,128] bytes -> [nb,256] nibbles: group g (64 elems) = low then high nibbles of bytes 32g..32g+31."""
    parts = []
    for g in range(4):
        seg = qs128[:, 32 * g:32 * g + 32]
        parts += [seg & 0xF, seg >> 4]
    return np.concatenate(parts, axis=1).astype(np.int32)


def q4_K(b):
    d, dmin = _h(b, 0), _h(b, 2)
    sc, mn = _k4_scale_min(b[:, 4:16])
    q = _nibbles_k(b[:, 16:144])
    sub = np.arange(256) // 32
    d1 = d * sc[:, sub].astype(np.float32)
    m1 = dmin * mn[:, sub].astype(np.float32)
    return (d1 * q.astype(np.float32) - m1).astype(np.float32)


def q5_K(b):
    d, dmin = _h(b, 0), _h(b, 2)
    sc, mn = _k4_scale_min(b[:, 4:16])
    qh = b[:, 16:48]
    q = _nibbles_k(b[:, 48:176])
    e = np.arange(256)
    hbit = (qh[:, e % 32].astype(np.int32) >> (e // 32)) & 1
    q = q + 16 * hbit
    sub = e // 32
    d1 = d * sc[:, sub].astype(np.float32)
    m1 = dmin * mn[:, sub].astype(np.float32)
    return (d1 * q.astype(np.float32) - m1).astype(np.float32)


def q6_K(b):
    ql = b[:, 0:128].astype(np.int32)
    qh = b[:, 128:192].astype(np.int32)
    sc = b[:, 192:208].view(np.int8).astype(np.float32)
    d = _h(b, 208)
    e = np.arange(256)
    half = e // 128           # which 128-element half
    r = e % 128
    part = r // 32            # 0..3 inside the half
    l = r % 32
    ql_idx = 64 * half + l + 32 * (part % 2)
    low = np.where(part < 2, ql[:, ql_idx] & 0xF, ql[:, ql_idx] >> 4)
    high = (qh[:, 32 * half + l] >> (2 * part)) & 3
    q = (low | (high << 4)) - 32
    s = sc[:, 8 * half + 2 * part + l // 16]
    return ((d * s) * q.astype(np.float32)).astype(np.float32)


DEQUANT = {2: q4_0, 3: q4_1, 6: q5_0, 7: q5_1, 8: q8_0, 10: q2_K, 11: q3_K, 12: q4_K, 13: q5_K, 14: q6_K}
BLOCK = {2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
         10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


def dequantize(t: int, blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    bs, ts = BLOCK[t]
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, ts)
    with np.errstate(invalid="ignore", over="ignore"):
        out = DEQUANT[t](b)
    return out.reshape(n, k)
