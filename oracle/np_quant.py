"""Second, independent restatement of ggml's reference quantizers in numpy.

TEST INFRASTRUCTURE ONLY (same rules as ``oracle.py``): only tests/ import it,
as a checker of the C oracle's quantizers (``oracle/ggml_oracle.c``).

Restated from ggml's published ``quantize_row_*_ref`` and its helpers
``make_qx_quants`` / ``make_q3_quants`` / ``make_qkx2_quants`` and
``nearest_int`` (ggml-quants.c, MIT; the algorithms candle's QTensor::quantize
ports, reached from crates/mold-inference/src/flux/pipeline.rs:219-229 and
crates/mold-inference/src/flux/lora.rs:849).  The evaluation structure differs
from the scalar C oracle on purpose, so that a slip in either one shows up as a
byte mismatch in tests/test_oracle.py:

  * every block (and every 16- / 32-element sub-block) of the input is
    processed at once as a numpy column: the loops run over the elements of a
    sub-block and over the search steps, never over blocks;
  * rounding is numpy's (``np.rint``: half to even, ggml's ``nearest_int``
    magic add for |v| < 2^22; ``trunc`` for the C casts; half away from zero
    for ``roundf``, evaluated in float64 where float32 ``floor(|v| + 0.5)``
    could round);
  * the block bytes are assembled from field arrays with numpy views, not by
    writing a packed struct.

The IEEE operations themselves (float32 products, sums in element order, one
division, f16 round-to-nearest-even of the stored scales) must be the same
ones ggml performs, because the bytes depend on every rounding: every
expression below keeps ggml's operand order, and every intermediate is a
float32 array (no fused multiply-add, no pairwise summation).

Each public function takes x (float32, shape [nblocks * block_size]) and
returns uint8 blocks of shape [nblocks, type_size].
"""
from __future__ import annotations

import numpy as np

F = np.float32
GROUP_MAX_EPS = F(1e-15)


def _f(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32)


def _nearest(v: np.ndarray) -> np.ndarray:
    """ggml nearest_int: for |v| <= 2^22 its magic add (v + 1.5 * 2^23 in float32,
    low 23 bits minus 2^22) is round half to even, taken here from np.rint.  Past
    that range ggml returns whatever the low mantissa bits hold (a search step can
    divide by a near-zero sum), and so does this function, bit for bit."""
    v = _f(v)
    with np.errstate(invalid="ignore", over="ignore"):
        inside = np.abs(v) <= F(2 ** 22)
        r = np.rint(np.where(inside, v, F(0))).astype(np.int64)
        bits = _f(v + F(12582912.0)).view(np.int32).astype(np.int64)
    return np.where(inside, r, (bits & 0x7FFFFF) - 0x400000)


def _trunc(v: np.ndarray) -> np.ndarray:
    """C float -> integer conversion (toward zero)."""
    return np.trunc(_f(v).astype(np.float64)).astype(np.int64)


def _round_away(v: np.ndarray) -> np.ndarray:
    """C roundf: half away from zero (exact in float64 for float32 inputs)."""
    v = _f(v).astype(np.float64)
    return (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int64)


def _half_bits(v: np.ndarray) -> np.ndarray:
    """f32 -> IEEE binary16 bits, round to nearest even (GGML_FP32_TO_FP16)."""
    with np.errstate(over="ignore"):
        return _f(v).astype(np.float16).view(np.uint16)


def _half_val(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def _first_absmax(x: np.ndarray):
    """(amax, max): the largest |x| over the last axis and the signed value of its
    first occurrence (ggml's `if (amax < |x|)` / `if (|x| > amax)` scans)."""
    a = np.abs(x)
    idx = np.argmax(a, axis=-1)
    amax = np.take_along_axis(a, idx[..., None], axis=-1)[..., 0]
    mx = np.take_along_axis(x, idx[..., None], axis=-1)[..., 0]
    # no element beats the initial 0: max stays +0.0 (its sign reaches f16(d))
    mx = np.where(amax == 0, F(0), mx)
    return _f(amax), _f(mx)


def _scan_min_max(x: np.ndarray):
    """min / max over the last axis by ggml's sequential `v < min` / `v > max`
    scan (the first of equal values wins, which fixes the sign of a zero)."""
    mn = x[..., 0].copy()
    mx = x[..., 0].copy()
    for i in range(1, x.shape[-1]):
        mn = np.where(x[..., i] < mn, x[..., i], mn)
        mx = np.where(x[..., i] > mx, x[..., i], mx)
    return _f(mn), _f(mx)


def _pack_bytes(*fields) -> np.ndarray:
    """Concatenate per-block byte fields (each [nb, bytes]) into blocks."""
    return np.ascontiguousarray(np.concatenate([np.asarray(f, np.uint8) for f in fields], axis=1))


def _u16_bytes(bits: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(bits, np.uint16).reshape(-1, 1)).view(np.uint8).reshape(-1, 2)


def _u32_bytes(v: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(v, np.uint32).reshape(-1, 1)).view(np.uint8).reshape(-1, 4)


# ------------------------------------------------------------ 32-element types

def _sym_scale(xb: np.ndarray, div: float):
    """d = (first largest-magnitude value) / div, id = 1/d (0 when d = 0)."""
    _, mx = _first_absmax(xb)
    d = _f(mx / F(div))
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, _f(F(1.0) / d), F(0.0))
    return d, _f(idv)


def q4_0(x):
    xb = _f(x).reshape(-1, 32)
    d, idv = _sym_scale(xb, -8.0)
    x0 = _f(xb[:, :16] * idv[:, None])
    x1 = _f(xb[:, 16:] * idv[:, None])
    q0 = np.minimum(15, _trunc(_f(x0 + F(8.5))))
    q1 = np.minimum(15, _trunc(_f(x1 + F(8.5))))
    qs = (q0 | (q1 << 4)).astype(np.uint8)
    return _pack_bytes(_u16_bytes(_half_bits(d)), qs)


def _min_max_scale(xb: np.ndarray, levels: int):
    mn, mxv = _scan_min_max(xb)
    d = _f(_f(mxv - mn) / F(levels))
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, _f(F(1.0) / d), F(0.0))
    return d, _f(idv), mn


def q4_1(x):
    xb = _f(x).reshape(-1, 32)
    d, idv, mn = _min_max_scale(xb, 15)
    x0 = _f(_f(xb[:, :16] - mn[:, None]) * idv[:, None])
    x1 = _f(_f(xb[:, 16:] - mn[:, None]) * idv[:, None])
    q0 = np.minimum(15, _trunc(_f(x0 + F(0.5))))
    q1 = np.minimum(15, _trunc(_f(x1 + F(0.5))))
    qs = (q0 | (q1 << 4)).astype(np.uint8)
    return _pack_bytes(_u16_bytes(_half_bits(d)), _u16_bytes(_half_bits(mn)), qs)


def _high_bits(q0: np.ndarray, q1: np.ndarray) -> np.ndarray:
    """qh word: bit j = bit 4 of element j (j < 16 from q0, 16.. from q1)."""
    bits = np.concatenate([(q0 >> 4) & 1, (q1 >> 4) & 1], axis=1).astype(np.uint64)
    return (bits << np.arange(32, dtype=np.uint64)[None, :]).sum(axis=1).astype(np.uint32)


def q5_0(x):
    xb = _f(x).reshape(-1, 32)
    d, idv = _sym_scale(xb, -16.0)
    x0 = _f(xb[:, :16] * idv[:, None])
    x1 = _f(xb[:, 16:] * idv[:, None])
    q0 = np.minimum(31, _trunc(_f(x0 + F(16.5))))
    q1 = np.minimum(31, _trunc(_f(x1 + F(16.5))))
    qs = ((q0 & 15) | ((q1 & 15) << 4)).astype(np.uint8)
    return _pack_bytes(_u16_bytes(_half_bits(d)), _u32_bytes(_high_bits(q0, q1)), qs)


def q5_1(x):
    xb = _f(x).reshape(-1, 32)
    d, idv, mn = _min_max_scale(xb, 31)
    x0 = _f(_f(xb[:, :16] - mn[:, None]) * idv[:, None])
    x1 = _f(_f(xb[:, 16:] - mn[:, None]) * idv[:, None])
    q0 = _trunc(_f(x0 + F(0.5))) & 0xFF          # (uint8_t) cast, no clamp in ggml
    q1 = _trunc(_f(x1 + F(0.5))) & 0xFF
    qs = ((q0 & 15) | ((q1 & 15) << 4)).astype(np.uint8)
    return _pack_bytes(_u16_bytes(_half_bits(d)), _u16_bytes(_half_bits(mn)), _u32_bytes(_high_bits(q0, q1)), qs)


def q8_0(x):
    xb = _f(x).reshape(-1, 32)
    amax = _f(np.abs(xb).max(axis=1))
    d = _f(amax / F(127))
    with np.errstate(divide="ignore"):
        idv = _f(np.where(d != 0, _f(F(1.0) / d), F(0.0)))
    q = _round_away(_f(xb * idv[:, None]))
    return _pack_bytes(_u16_bytes(_half_bits(d)), q.astype(np.int8).view(np.uint8))


# ------------------------------------------------ activation quantizers

def q8_1(x):
    """The Q8_1 activation block {f16 d, f16 s, i8 qs[32]} with s = f16(f16(sum q) * d)."""
    xb = _f(x).reshape(-1, 32)
    amax = _f(np.abs(xb).max(axis=1))
    d = _f(amax / F(127))
    with np.errstate(divide="ignore"):
        idv = _f(np.where(d != 0, _f(F(1.0) / d), F(0.0)))
    q = _round_away(_f(xb * idv[:, None]))
    dbits = _half_bits(d)
    s = _f(_half_val(_half_bits(_f(q.sum(axis=1)))) * _half_val(dbits))
    return _pack_bytes(_u16_bytes(dbits), _u16_bytes(_half_bits(s)), q.astype(np.int8).view(np.uint8))


def q8_K(x):
    """The Q8_K activation block {f32 d, i8 qs[256], i16 bsums[16]}: iscale = -128 /
    (the first element of largest magnitude), q = min(round_half_away(iscale x), 127),
    d = 1 / iscale; an all-zero block is all zeros.  (This is the convention the
    oracle states for candle's CPU path; it is not ggml's quantize_row_q8_K_ref,
    which uses -127 / max and half-to-even.)"""
    xb = _f(x).reshape(-1, 256)
    amax, mx = _first_absmax(xb)
    nz = amax != 0
    with np.errstate(divide="ignore", invalid="ignore"):
        iscale = _f(np.where(nz, _f(F(-128.0) / mx), F(0.0)))
        v = _round_away(_f(iscale[:, None] * xb))
    q = np.where(nz[:, None], np.minimum(v, 127), 0)
    bsums = q.reshape(-1, 16, 16).sum(axis=2)
    with np.errstate(divide="ignore"):
        d = _f(np.where(nz, _f(F(1.0) / np.where(nz, iscale, F(1.0))), F(0.0)))
    return _pack_bytes(np.ascontiguousarray(d.reshape(-1, 1)).view(np.uint8).reshape(-1, 4),
                       q.astype(np.int8).view(np.uint8),
                       np.ascontiguousarray(bsums.astype(np.int16)).view(np.uint8).reshape(-1, 32))


# ---------------------------------------------------------- k-quant helpers

def make_qkx2(x: np.ndarray, w: np.ndarray, nmax: int, rmin: float, rdelta: float, nstep: int, use_mad: bool):
    """ggml make_qkx2_quants over every row of x [rows, n] with weights w:
    (codes [rows, n], scale [rows], the_min [rows] = -min)."""
    x, w = _f(x), _f(w)
    rows, n = x.shape
    mn, mx = _scan_min_max(x)
    sum_w = w[:, 0].copy()
    sum_x = _f(sum_w * x[:, 0])
    for i in range(1, n):
        sum_w = _f(sum_w + w[:, i])
        sum_x = _f(sum_x + _f(w[:, i] * x[:, i]))
    mn = np.where(mn > 0, F(0), mn).astype(np.float32)
    flat = mx == mn
    rng = _f(mx - mn)
    safe = np.where(flat, F(1), rng).astype(np.float32)
    iscale = _f(F(nmax) / safe)
    scale = _f(F(1) / iscale)
    L = np.clip(_nearest(_f(iscale[:, None] * _f(x - mn[:, None]))), 0, nmax)
    Lf = L.astype(np.float32)
    best = np.zeros(rows, np.float32)
    for i in range(n):
        diff = _f(_f(_f(scale * Lf[:, i]) + mn) - x[:, i])
        diff = np.abs(diff) if use_mad else _f(diff * diff)
        best = _f(best + _f(w[:, i] * diff))
    for step in range(nstep + 1):
        # ggml reads `min` here as the search left it: a step that improved
        # the fit moved min to its this_min, which then shifts both the
        # range (max - min) and the codes of every later step
        span = np.where(flat, F(1), _f(mx - mn)).astype(np.float32)
        isc = _f(_f(_f(F(rmin) + _f(F(rdelta) * F(step))) + F(nmax)) / span)
        la = np.clip(_nearest(_f(isc[:, None] * _f(x - mn[:, None]))), 0, nmax)
        laf = la.astype(np.float32)
        sl = np.zeros(rows, np.float32)
        sl2 = np.zeros(rows, np.float32)
        sxl = np.zeros(rows, np.float32)
        for i in range(n):
            wl = _f(w[:, i] * laf[:, i])
            sl = _f(sl + wl)
            sl2 = _f(sl2 + _f(wl * laf[:, i]))
            sxl = _f(sxl + _f(wl * x[:, i]))
        D = _f(_f(sum_w * sl2) - _f(sl * sl))
        ok = D > 0
        Ds = np.where(ok, D, F(1)).astype(np.float32)
        ts = _f(_f(_f(sum_w * sxl) - _f(sum_x * sl)) / Ds)
        tm = _f(_f(_f(sl2 * sum_x) - _f(sl * sxl)) / Ds)
        pos = tm > 0
        with np.errstate(divide="ignore", invalid="ignore"):
            ts = np.where(pos, _f(sxl / sl2), ts).astype(np.float32)
        tm = np.where(pos, F(0), tm).astype(np.float32)
        mad = np.zeros(rows, np.float32)
        for i in range(n):
            diff = _f(_f(_f(ts * laf[:, i]) + tm) - x[:, i])
            diff = np.abs(diff) if use_mad else _f(diff * diff)
            mad = _f(mad + _f(w[:, i] * diff))
        take = ok & (mad < best) & ~flat
        L = np.where(take[:, None], la, L)
        Lf = L.astype(np.float32)
        best = np.where(take, mad, best).astype(np.float32)
        scale = np.where(take, ts, scale).astype(np.float32)
        mn = np.where(take, tm, mn).astype(np.float32)
    L = np.where(flat[:, None], 0, L)
    scale = np.where(flat, F(0), scale).astype(np.float32)
    return L, scale, _f(-mn)


def make_q3(x: np.ndarray, nmax: int):
    """ggml make_q3_quants(n, nmax, x, L, do_rmse = true) over every row:
    (codes + nmax [rows, n], scale [rows])."""
    x = _f(x)
    rows, n = x.shape
    amax, mx = _first_absmax(x)
    zero = amax < GROUP_MAX_EPS
    safe = np.where(zero, F(1), mx).astype(np.float32)
    iscale = _f(F(-nmax) / safe)
    L = np.clip(_nearest(_f(iscale[:, None] * x)), -nmax, nmax - 1)
    w = _f(x * x)
    sumlx = np.zeros(rows, np.float32)
    suml2 = np.zeros(rows, np.float32)
    for i in range(n):
        li = L[:, i].astype(np.float32)
        sumlx = _f(sumlx + _f(_f(w[:, i] * x[:, i]) * li))
        suml2 = _f(suml2 + _f(_f(w[:, i] * li) * li))
    # Coordinate passes.  A pass that changes nothing leaves the state as it
    # was, so running all five passes on every row equals ggml's early exit.
    for _ in range(5):
        for i in range(n):
            li = L[:, i].astype(np.float32)
            wx = _f(w[:, i] * x[:, i])
            slx = _f(sumlx - _f(wx * li))
            act = slx > 0
            sl2 = _f(suml2 - _f(_f(w[:, i] * li) * li))
            with np.errstate(divide="ignore", invalid="ignore"):
                nl = np.clip(_nearest(np.where(act, _f(_f(x[:, i] * sl2) / slx), F(0))), -nmax, nmax - 1)
            act &= nl != L[:, i]
            nlf = nl.astype(np.float32)
            slx2 = _f(slx + _f(wx * nlf))
            sl22 = _f(sl2 + _f(_f(w[:, i] * nlf) * nlf))
            better = act & (sl22 > 0) & (_f(_f(slx2 * slx2) * suml2) > _f(_f(sumlx * sumlx) * sl22))
            L[:, i] = np.where(better, nl, L[:, i])
            sumlx = np.where(better, slx2, sumlx).astype(np.float32)
            suml2 = np.where(better, sl22, suml2).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = _f(sumlx / np.where(zero, F(1), suml2))
    L = np.where(zero[:, None], 0, L + nmax)
    scale = np.where(zero, F(0), scale).astype(np.float32)
    return L, scale


def make_qx(x: np.ndarray, nmax: int):
    """ggml make_qx_quants(n, nmax, x, L, rmse_type = 1, NULL) over every row:
    (codes + nmax [rows, n], scale [rows])."""
    x = _f(x)
    rows, n = x.shape
    amax, mx = _first_absmax(x)
    zero = amax < GROUP_MAX_EPS
    safe = np.where(zero, F(1), mx).astype(np.float32)
    w = _f(x * x)

    def sums(isc):
        l = np.clip(_nearest(_f(isc[:, None] * x)), -nmax, nmax - 1)
        sx = np.zeros(rows, np.float32)
        s2 = np.zeros(rows, np.float32)
        for i in range(n):
            li = l[:, i].astype(np.float32)
            sx = _f(sx + _f(_f(w[:, i] * x[:, i]) * li))
            s2 = _f(s2 + _f(_f(w[:, i] * li) * li))
        return l, sx, s2

    L, sumlx, suml2 = sums(_f(F(-nmax) / safe))
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.where(suml2 != 0, _f(sumlx / suml2), F(0)).astype(np.float32)
    best = _f(scale * sumlx)
    for step in list(range(-9, 0)) + list(range(1, 10)):
        isc = _f(_f(-_f(F(nmax) + _f(F(0.1) * F(step)))) / safe)
        l, sx, s2 = sums(isc)
        with np.errstate(divide="ignore", invalid="ignore"):
            take = (s2 > 0) & (_f(sx * sx) > _f(best * s2))
            ns = _f(sx / np.where(take, s2, F(1)))
        L = np.where(take[:, None], l, L)
        scale = np.where(take, ns, scale).astype(np.float32)
        best = np.where(take, _f(ns * sx), best).astype(np.float32)
    L = np.where(zero[:, None], 0, L + nmax)
    scale = np.where(zero, F(0), scale).astype(np.float32)
    return L, scale


def _crumb_pack(L: np.ndarray) -> np.ndarray:
    """[nb, 256] 2-bit codes -> [nb, 64] bytes: byte 32 h + l holds elements
    128 h + l + 32 s at bits 2 s (s = 0..3)."""
    Lb = L.reshape(-1, 2, 4, 32).astype(np.uint8)
    return (Lb[:, :, 0] | (Lb[:, :, 1] << 2) | (Lb[:, :, 2] << 4) | (Lb[:, :, 3] << 6)).reshape(-1, 64)


def _nibble_pack(L: np.ndarray) -> np.ndarray:
    """[nb, 256] 4-bit codes -> [nb, 128] bytes: byte 32 g + l holds element 64 g + l
    (low nibble) and 64 g + 32 + l (high nibble)."""
    Lb = L.reshape(-1, 4, 2, 32).astype(np.uint8)
    return (Lb[:, :, 0] | (Lb[:, :, 1] << 4)).reshape(-1, 128)


def _requant(x: np.ndarray, d: np.ndarray, dm, lo: int, hi: int, L: np.ndarray, offset: int) -> np.ndarray:
    """Second pass of the k-quant quantizers: where d != 0, L = clamp(nearest((x + dm) / d))
    + offset; elsewhere the search's codes stay."""
    with np.errstate(divide="ignore", invalid="ignore"):
        num = _f(x + dm) if dm is not None else x
        v = _f(num / np.where(d != 0, d, F(1)))
    nl = np.clip(_nearest(v), lo, hi) + offset
    return np.where(d != 0, nl, L)


def q2_K(x):
    xs = _f(x).reshape(-1, 16, 16)                      # [nb, sub-block, 16]
    nb = xs.shape[0]
    L, sc, mins = make_qkx2(xs.reshape(-1, 16), np.abs(xs).reshape(-1, 16), 3, -0.5, 0.1, 15, True)
    L = L.reshape(nb, 16, 16)
    sc, mins = sc.reshape(nb, 16), mins.reshape(nb, 16)
    max_scale = np.maximum(sc.max(axis=1), F(0)).astype(np.float32)
    max_min = np.maximum(mins.max(axis=1), F(0)).astype(np.float32)
    pos_s, pos_m = max_scale > 0, max_min > 0
    with np.errstate(divide="ignore"):
        is_s = _f(F(15) / np.where(pos_s, max_scale, F(1)))
        is_m = _f(F(15) / np.where(pos_m, max_min, F(1)))
    lsc = np.where(pos_s[:, None], _nearest(_f(is_s[:, None] * sc)), 0)
    lmn = np.where(pos_m[:, None], _nearest(_f(is_m[:, None] * mins)), 0)
    scales = (lsc | (lmn << 4)) & 0xFF
    dbits = np.where(pos_s, _half_bits(_f(max_scale / F(15))), _half_bits(F(0))).astype(np.uint16)
    mbits = np.where(pos_m, _half_bits(_f(max_min / F(15))), _half_bits(F(0))).astype(np.uint16)
    d = _f(_half_val(dbits)[:, None] * _f(scales & 15))
    dm = _f(_half_val(mbits)[:, None] * _f(scales >> 4))
    L = _requant(xs, d[:, :, None], dm[:, :, None], 0, 3, L, 0).reshape(nb, 256)
    return _pack_bytes(scales.astype(np.uint8), _crumb_pack(L), _u16_bytes(dbits), _u16_bytes(mbits))


def q3_K(x):
    xs = _f(x).reshape(-1, 16, 16)
    nb = xs.shape[0]
    L, sc = make_q3(xs.reshape(-1, 16), 4)
    L, sc = L.reshape(nb, 16, 16), sc.reshape(nb, 16)
    _, max_scale = _first_absmax(sc)
    has = max_scale != 0
    with np.errstate(divide="ignore"):
        iscale = _f(F(-32) / np.where(has, max_scale, F(1)))
    l6 = np.clip(_nearest(_f(iscale[:, None] * sc)), -32, 31) + 32
    l6 = np.where(has[:, None], l6, 0)
    packed = np.zeros((nb, 12), np.int64)
    packed[:, 0:8] = (l6[:, 0:8] & 15) | ((l6[:, 8:16] & 15) << 4)
    hi = l6 >> 4                                           # [nb, 16], 0..3
    packed[:, 8:12] = hi[:, 0:4] | (hi[:, 4:8] << 2) | (hi[:, 8:12] << 4) | (hi[:, 12:16] << 6)
    dbits = np.where(has, _half_bits(_f(F(1) / iscale)), _half_bits(F(0))).astype(np.uint16)
    d = _f(_half_val(dbits)[:, None] * _f(l6 - 32))         # the stored scale, read back
    L = _requant(xs, d[:, :, None], None, -4, 3, L, 4).reshape(nb, 256)
    hmask = ((L.reshape(nb, 8, 32) > 3).astype(np.int64) << np.arange(8)[None, :, None]).sum(axis=1)
    L = np.where(L > 3, L - 4, L)
    return _pack_bytes(hmask.astype(np.uint8), _crumb_pack(L), packed.astype(np.uint8), _u16_bytes(dbits))


def _k45(x, five: bool):
    xs = _f(x).reshape(-1, 8, 32)
    nb = xs.shape[0]
    sq = np.zeros((nb, 8), np.float32)
    for l in range(32):
        sq = _f(sq + _f(xs[:, :, l] * xs[:, :, l]))
    av = np.sqrt(_f(sq / F(32))).astype(np.float32)
    wts = _f(av[:, :, None] + np.abs(xs))
    nmax = 31 if five else 15
    rmin, nstep = (-0.5, 15) if five else (-1.0, 20)
    L, sc, mins = make_qkx2(xs.reshape(-1, 32), wts.reshape(-1, 32), nmax, rmin, 0.1, nstep, False)
    L, sc, mins = L.reshape(nb, 8, 32), sc.reshape(nb, 8), mins.reshape(nb, 8)
    max_scale = np.maximum(sc.max(axis=1), F(0)).astype(np.float32)
    max_min = np.maximum(mins.max(axis=1), F(0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv_s = np.where(max_scale > 0, _f(F(63) / np.where(max_scale > 0, max_scale, F(1))), F(0))
        inv_m = np.where(max_min > 0, _f(F(63) / np.where(max_min > 0, max_min, F(1))), F(0))
    ls = np.minimum(63, _nearest(_f(_f(inv_s)[:, None] * sc)) & 0xFF)      # (uint8_t) cast, then MIN
    lm = np.minimum(63, _nearest(_f(_f(inv_m)[:, None] * mins)) & 0xFF)
    packed = np.zeros((nb, 12), np.int64)
    packed[:, 0:4] = ls[:, 0:4] | ((ls[:, 4:8] >> 4) << 6)
    packed[:, 4:8] = lm[:, 0:4] | ((lm[:, 4:8] >> 4) << 6)
    packed[:, 8:12] = (ls[:, 4:8] & 15) | ((lm[:, 4:8] & 15) << 4)
    dbits = _half_bits(_f(max_scale / F(63)))
    mbits = _half_bits(_f(max_min / F(63)))
    d = _f(_half_val(dbits)[:, None] * _f(ls))
    dm = _f(_half_val(mbits)[:, None] * _f(lm))
    L = _requant(xs, d[:, :, None], dm[:, :, None], 0, nmax, L, 0).reshape(nb, 256)
    dmb = np.stack([_u16_bytes(dbits), _u16_bytes(mbits)], axis=1).reshape(nb, 4)
    if not five:
        return _pack_bytes(dmb, packed.astype(np.uint8), _nibble_pack(L))
    qh = ((L.reshape(nb, 8, 32) >> 4) << np.arange(8)[None, :, None]).sum(axis=1)
    return _pack_bytes(dmb, packed.astype(np.uint8), qh.astype(np.uint8), _nibble_pack(L & 15))


def q4_K(x):
    return _k45(x, False)


def q5_K(x):
    return _k45(x, True)


def q6_K(x):
    xs = _f(x).reshape(-1, 16, 16)
    nb = xs.shape[0]
    L, sc = make_qx(xs.reshape(-1, 16), 32)
    L, sc = L.reshape(nb, 16, 16), sc.reshape(nb, 16)
    amax, max_scale = _first_absmax(sc)
    zero = amax < GROUP_MAX_EPS
    with np.errstate(divide="ignore"):
        iscale = _f(F(-128) / np.where(zero, F(1), max_scale))
    dbits = np.where(zero, _half_bits(F(0)), _half_bits(_f(F(1) / iscale))).astype(np.uint16)
    sc8 = np.minimum(127, _nearest(_f(iscale[:, None] * sc)))
    sc8 = np.where(zero[:, None], 0, sc8)
    d = _f(_half_val(dbits)[:, None] * _f(sc8))
    L = _requant(xs, d[:, :, None], None, -32, 31, L, 32).reshape(nb, 256)
    L = np.where(zero[:, None], 0, L)                     # an all-zero super-block is zero bytes
    Lq = L.reshape(nb, 2, 4, 32)
    ql = np.concatenate([(Lq[:, :, 0] & 15) | ((Lq[:, :, 2] & 15) << 4),
                         (Lq[:, :, 1] & 15) | ((Lq[:, :, 3] & 15) << 4)], axis=2).reshape(nb, 128)
    qh = ((Lq[:, :, 0] >> 4) | ((Lq[:, :, 1] >> 4) << 2) | ((Lq[:, :, 2] >> 4) << 4)
          | ((Lq[:, :, 3] >> 4) << 6)).reshape(nb, 64)
    return _pack_bytes(ql.astype(np.uint8), qh.astype(np.uint8), sc8.astype(np.int8).view(np.uint8),
                       _u16_bytes(dbits))


# ggml type id -> quantizer
QUANT = {2: q4_0, 3: q4_1, 6: q5_0, 7: q5_1, 8: q8_0, 10: q2_K, 11: q3_K, 12: q4_K, 13: q5_K, 14: q6_K}
ACT = {8: q8_0, 9: q8_1, 15: q8_K}


def quantize(t: int, x: np.ndarray) -> np.ndarray:
    """[n, k] f32 -> [n, row_bytes] uint8 (every row's blocks in order)."""
    x = _f(x)
    if x.ndim == 1:
        x = x[None, :]
    n = x.shape[0]
    return QUANT[t](x.reshape(-1)).reshape(n, -1)
