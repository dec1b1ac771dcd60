"""Pins for the CPU oracle (oracle/ggml_oracle.c, oracle/np_dequant.py).

The reference's arithmetic for this path lives in candle-core-mold 0.9.10 /
candle-kernels 0.9.2 (crates.io, /root/reference/Cargo.lock:507-543), whose
source is not in the container, and the reference holds no golden vector for
any quantized type.  The oracle is therefore pinned by:
  * independent implementations: numpy's IEEE half conversion, torch's bf16
    rounding, numpy float64 BLAS for the matmul reference, and a second,
    vectorised restatement of every dequantize formula (np_dequant.py);
  * llama.cpp's published known-answer test (tests/test-quantize-fns.cpp):
    synthetic data 0.1 + 2cos(i + offset), 4096 values, round-trip error
    bounds and a vec_dot-vs-float bound;
  * hand-built blocks whose expected values are worked out from the GGUF
    block specification in the comments;
  * mathematical facts: the f32 dequant equals the once-rounded exact value;
    linearity; zero blocks give zeros;
  * the reference's own GGUF file sizes (crates/mold-core/src/manifest.rs),
    which fix the bytes per weight of Q8_0, Q4_1 and Q6_K;
  * for the reference quantizers: hand-worked known-answer rows of the legacy
    types (ties, the signed-max choice, all-zero and constant blocks, f16
    rounding of d), a second numpy restatement (oracle/np_quant.py) compared
    byte for byte on random and adversarial rows, and exact round trips on
    each format's grid;
  * for candle's CPU algorithm: known-answer activation rows (Q8_0 / Q8_1 /
    Q8_K), vec_dot against the exact product to f32 rounding, and the matmul
    as quantized rows times vec_dot.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O
from oracle import np_dequant as N


@pytest.fixture(scope="module", autouse=True)
def _built():
    O.lib()


# ----------------------------------------------------------------- type table

# ggml type_traits (blck_size, type_size) as published in ggml.c.
GGML_TRAITS = {
    O.Q4_0: (32, 18), O.Q4_1: (32, 20), O.Q5_0: (32, 22), O.Q5_1: (32, 24),
    O.Q8_0: (32, 34), O.Q8_1: (32, 36), O.Q2_K: (256, 84), O.Q3_K: (256, 110),
    O.Q4_K: (256, 144), O.Q5_K: (256, 176), O.Q6_K: (256, 210), O.Q8_K: (256, 292),
    O.F32: (1, 4), O.F16: (1, 2), O.BF16: (1, 2),
}


def test_type_table_matches_ggml():
    for t, (bs, ts) in GGML_TRAITS.items():
        assert O.block_size(t) == bs, O.NAMES[t]
        assert O.type_size(t) == ts, O.NAMES[t]


def test_reference_gguf_file_sizes_fix_bytes_per_weight():
    # FLUX.1-dev GGUF files in the reference manifest (same tensor set, three
    # encodings): crates/mold-core/src/manifest.rs:487-490 (Q8_0),
    # :518-521 (Q4_1), :549-552 (Q6_K).
    q8_0, q4_1, q6_k = 12_708_281_504, 7_530_806_432, 9_857_000_736

    def bpw(t):
        return O.type_size(t) / O.block_size(t)

    n_a = (q8_0 - q4_1) / (bpw(O.Q8_0) - bpw(O.Q4_1))
    n_b = (q6_k - q4_1) / (bpw(O.Q6_K) - bpw(O.Q4_1))
    # Both differences must imply the same quantized-weight count (FLUX.1-dev
    # is ~11.9e9 parameters); the few tensors K-quants cannot hold (K not a
    # multiple of 256) leave a <1% gap.
    assert 11.5e9 < n_a < 12.2e9
    assert abs(n_a - n_b) / n_a < 0.01
    # A Q6_K block two bytes shorter or a Q8_0 block two bytes longer would
    # break the agreement by >3%: the check can fail.
    n_bad = (q6_k - q4_1) / (208 / 256 - bpw(O.Q4_1))
    assert abs(n_a - n_bad) / n_a > 0.03
    n_bad = (q8_0 - q4_1) / (36 / 32 - bpw(O.Q4_1))
    assert abs(n_bad - n_b) / n_b > 0.03


# --------------------------------------------------------------------- halves

def test_fp16_to_fp32_exhaustive_against_numpy():
    L = O.lib()
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([L.orc_fp16_to_fp32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_fp32_to_fp16_round_to_nearest_even_against_numpy():
    L = O.lib()
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2 ** -24, 2 ** -25, 2 ** -25 * 1.0001,
                  2 ** -14, 2 ** -14 * (1 - 2 ** -11), 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, np.inf, -np.inf],
                 dtype=np.float32),
        # exact ties in the normal and subnormal ranges
        (np.arange(1, 2000, dtype=np.float32) * 2 + 1) * np.float32(2 ** -12),
        (np.arange(1, 500, dtype=np.float32) * 2 + 1) * np.float32(2 ** -25),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([L.orc_fp32_to_fp16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_fp32_to_bf16_against_torch():
    torch = pytest.importorskip("torch")
    L = O.lib()
    rng = np.random.default_rng(2)
    vals = np.concatenate([rng.standard_normal(5000).astype(np.float32) * 1000,
                           np.array([0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, np.inf, 3e38], np.float32)])
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([L.orc_fp32_to_bf16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


# ----------------------------------------------------------------- dequantize

def _bitwise_equal(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    same = (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))
    return bool(same.all())


@pytest.mark.parametrize("t", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
def test_dequant_c_equals_numpy_restatement_on_random_bytes(t):
    # Every byte pattern is a valid block, including Inf/NaN/subnormal halves.
    bs, ts = N.BLOCK[t]
    rng = np.random.default_rng(100 + t)
    nb = 1500
    blocks = rng.integers(0, 256, size=(nb, ts), dtype=np.uint8)
    a = O.dequantize(t, blocks, 1, nb * bs)
    b = N.dequantize(t, blocks, 1, nb * bs)
    assert _bitwise_equal(a, b)


@pytest.mark.parametrize("t", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
def test_dequant_is_once_rounded_exact_value(t):
    # Each dequantized value is (f16 scale x small integer) +- (f16 min x small
    # integer): the products are exact in f32 and f64, so the f32 result must
    # equal the f64 evaluation rounded once to f32, whatever the order of
    # evaluation.  Finite halves only.
    bs, ts = N.BLOCK[t]
    rng = np.random.default_rng(200 + t)
    w = rng.standard_normal((64, 4 * bs)).astype(np.float32) * 0.02
    blocks = O.quantize(t, w)
    got = O.dequantize(t, blocks, 64, 4 * bs)
    b = blocks.reshape(-1, ts)
    with np.errstate(all="ignore"):
        # f64 re-evaluation of the same formulas through the numpy module with
        # float64 arithmetic: cast inputs up by evaluating on a float64 view.
        ref64 = _dequant_f64(t, b).reshape(64, 4 * bs)
    assert np.array_equal(got, ref64.astype(np.float32))


def _dequant_f64(t, b):
    """Dequant in float64 (exact for every GGUF type) for the once-rounding check."""
    h = lambda off: b[:, off:off + 2].copy().view(np.float16).astype(np.float64)
    if t in (O.Q4_0, O.Q4_1, O.Q5_0, O.Q5_1, O.Q8_0):
        q = N.DEQUANT[t]  # integer codes are recovered by dequantizing with d=1, m=0
        bb = b.copy()
        one = np.array([1.0], np.float16).view(np.uint8)
        zero = np.array([0.0], np.float16).view(np.uint8)
        bb[:, 0:2] = one
        if t in (O.Q4_1, O.Q5_1):
            bb[:, 2:4] = zero
        codes = q(bb).astype(np.float64)
        d = h(0)
        out = codes * d
        if t in (O.Q4_1, O.Q5_1):
            out = out + h(2)
        return out
    if t == O.Q2_K:
        sc = b[:, 0:16].astype(np.int64)
        codes = np.concatenate([N._crumbs(b[:, 16:48]), N._crumbs(b[:, 48:80])], axis=1).astype(np.float64)
        g = np.arange(256) // 16
        return h(80) * (sc[:, g] & 15) * codes - h(82) * (sc[:, g] >> 4)
    if t == O.Q3_K:
        bb = b.copy()
        bb[:, 108:110] = np.array([1.0], np.float16).view(np.uint8)
        return N.q3_K(bb).astype(np.float64) * h(108)
    if t in (O.Q4_K, O.Q5_K):
        sc, mn = N._k4_scale_min(b[:, 4:16])
        if t == O.Q4_K:
            codes = N._nibbles_k(b[:, 16:144]).astype(np.float64)
        else:
            e = np.arange(256)
            codes = (N._nibbles_k(b[:, 48:176]) + 16 * ((b[:, 16:48][:, e % 32].astype(np.int64) >> (e // 32)) & 1)).astype(np.float64)
        sub = np.arange(256) // 32
        return h(0) * sc[:, sub] * codes - h(2) * mn[:, sub]
    if t == O.Q6_K:
        bb = b.copy()
        bb[:, 208:210] = np.array([1.0], np.float16).view(np.uint8)
        return N.q6_K(bb).astype(np.float64) * h(208)
    raise AssertionError(t)


def _half(v):
    return np.array([v], np.float16).view(np.uint8)


def test_kat_q4_0_nibble_order():
    # block_q4_0 {f16 d; u8 qs[16]}: low nibble of qs[j] -> element j,
    # high nibble -> element j+16; value (q - 8) * d.
    blk = np.zeros(18, np.uint8)
    blk[0:2] = _half(0.5)
    for j in range(16):
        blk[2 + j] = j | ((15 - j) << 4)
    y = O.dequantize(O.Q4_0, blk, 1, 32)[0]
    exp = [(j - 8) * 0.5 for j in range(16)] + [(7 - j) * 0.5 for j in range(16)]
    assert y.tolist() == exp


def test_kat_q8_0_and_q4_1_and_q5_0():
    blk = np.zeros(34, np.uint8)
    blk[0:2] = _half(0.25)
    blk[2:34] = np.arange(-128, 128, 8, dtype=np.int8).view(np.uint8)
    y = O.dequantize(O.Q8_0, blk, 1, 32)[0]
    assert y.tolist() == [v * 0.25 for v in range(-128, 128, 8)]

    blk = np.zeros(20, np.uint8)                        # {d, m, qs[16]}: q*d + m
    blk[0:2] = _half(2.0)
    blk[2:4] = _half(-1.0)
    blk[4:20] = 0x51                                     # low 1, high 5
    y = O.dequantize(O.Q4_1, blk, 1, 32)[0]
    assert y.tolist() == [1.0] * 16 + [9.0] * 16

    blk = np.zeros(22, np.uint8)                        # {d, qh[4], qs[16]}
    blk[0:2] = _half(1.0)
    blk[2:6] = np.array([0x01, 0x00, 0x01, 0x80], np.uint8)  # qh bits 0, 16, 31
    y = O.dequantize(O.Q5_0, blk, 1, 32)[0]
    exp = [-16.0] * 32
    exp[0] = 0.0      # bit 0 -> element 0 gets +16
    exp[16] = 0.0     # bit 16 -> element 16
    exp[31] = 0.0     # bit 31 -> element 31
    assert y.tolist() == exp


def test_kat_q4_k_scale_packing_and_nibbles():
    # block_q4_K {f16 d, dmin; u8 scales[12]; u8 qs[128]}.  Sub-block j (32
    # elements) has 6-bit scale sc_j and min m_j: j<4 -> scales[j] & 63,
    # scales[j+4] & 63; j>=4 -> low 4 bits in scales[j+4] (sc low nibble,
    # m high nibble) and the top 2 bits in bits 6..7 of scales[j-4] (sc) and
    # scales[j] (m).  Elements 64g..64g+31 are the low nibbles of qs[32g..],
    # elements 64g+32.. the high nibbles.  value = d*sc_j*q - dmin*m_j.
    sc = [1, 2, 3, 63, 17, 33, 48, 60]
    mn = [5, 0, 7, 9, 62, 16, 1, 35]
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = sc[j] & 63
        s[j + 4] = mn[j] & 63
    for j in range(4, 8):
        s[j + 4] = (sc[j] & 15) | ((mn[j] & 15) << 4)
        s[j - 4] |= (sc[j] >> 4) << 6
        s[j] |= (mn[j] >> 4) << 6
    blk = np.zeros(144, np.uint8)
    blk[0:2] = _half(0.5)
    blk[2:4] = _half(0.25)
    blk[4:16] = s
    qs = np.zeros(128, np.uint8)
    qs[0] = 0x3A          # element 0 <- 10, element 32 <- 3
    qs[31] = 0xF1         # element 31 <- 1, element 63 <- 15
    qs[32 * 3 + 5] = 0x72  # element 197 <- 2, element 229 <- 7
    blk[16:144] = qs
    y = O.dequantize(O.Q4_K, blk, 1, 256)[0]
    assert y[0] == 0.5 * 1 * 10 - 0.25 * 5
    assert y[32] == 0.5 * 2 * 3 - 0.25 * 0
    assert y[31] == 0.5 * 1 * 1 - 0.25 * 5
    assert y[63] == 0.5 * 2 * 15 - 0.25 * 0
    assert y[197] == 0.5 * 48 * 2 - 0.25 * 1        # sub-block 6
    assert y[229] == 0.5 * 60 * 7 - 0.25 * 35       # sub-block 7
    # element 100 = 64*1 + 36 -> high nibble of qs[36] (zero), sub-block 3
    assert y[100] == 0.5 * 63 * 0 - 0.25 * 9


def test_kat_q4_k_subblock_of_each_element():
    # Give every sub-block a distinct min and zero codes: element e must read
    # back -dmin * m_{e // 32}.
    mn = [3, 5, 7, 11, 13, 17, 19, 23]
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j + 4] = mn[j]
    for j in range(4, 8):
        s[j + 4] = (mn[j] & 15) << 4
        s[j] |= (mn[j] >> 4) << 6
    blk = np.zeros(144, np.uint8)
    blk[0:2] = _half(1.0)
    blk[2:4] = _half(1.0)
    blk[4:16] = s
    y = O.dequantize(O.Q4_K, blk, 1, 256)[0]
    assert y.tolist() == [-float(mn[e // 32]) for e in range(256)]


def test_kat_q6_k_layout():
    # block_q6_K {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d}.  Within each
    # 128-element half h, element 32p + l (p = 0..3) takes its low 4 bits from
    # ql[64h + l + 32*(p%2)] (low nibble for p<2, high for p>=2) and its top 2
    # bits from qh[32h + l] >> 2p; code - 32; scale scales[8h + 2p + l//16].
    blk = np.zeros(210, np.uint8)
    blk[208:210] = _half(1.0)
    blk[192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8)   # scale j = j+1
    blk[0:128] = 0x00
    blk[128:192] = 0xAA        # every 2-bit field = 2 -> code 32 -> value 0
    y = O.dequantize(O.Q6_K, blk, 1, 256)[0]
    assert np.all(y == 0.0)
    blk[128 + 32 + 3] = 0x00    # half 1, l = 3: all four parts get high bits 0
    blk[64 + 3] = 0x5F           # ql[64+3]: low 15 (p=0), high 5 (p=2)
    blk[64 + 32 + 3] = 0x9C      # ql[64+32+3]: low 12 (p=1), high 9 (p=3)
    y = O.dequantize(O.Q6_K, blk, 1, 256)[0]
    assert y[128 + 0 + 3] == (15 - 32) * 9     # scale index 8+0+0 -> 9
    assert y[128 + 32 + 3] == (12 - 32) * 11   # scale 8+2 -> 11
    assert y[128 + 64 + 3] == (5 - 32) * 13    # scale 8+4 -> 13
    assert y[128 + 96 + 3] == (9 - 32) * 15    # scale 8+6 -> 15
    assert np.count_nonzero(y) == 4


def test_kat_q3_k_and_q2_k_layout():
    # Q3_K: scale j (16 of them, 6 bits, offset 32): low 4 bits from scales[j]
    # (j<8) or scales[j-8]>>4, high 2 bits from scales[8 + j%4] >> 2*(j//4).
    # Element e: 2 low bits (qs[32*(e//128) + e%32] >> 2*((e%128)//32)) & 3,
    # minus 4 unless hmask[e%32] bit (e//32) is set.
    blk = np.zeros(110, np.uint8)
    blk[108:110] = _half(1.0)
    sc = np.zeros(12, np.uint8)
    sc[0:8] = 0x0 | (0x1 << 4)      # j<8 low 0, j>=8 low 1
    sc[8:12] = 0b10_10_10_10        # high bits 2 for every j -> sc = 32 + low
    blk[96:108] = sc
    blk[0:32] = 0xFF                # all high bits set -> no -4
    blk[32:96] = 0x00
    blk[32 + 32 + 7] = 0b01_00_00_00  # e = 128 + 96 + 7 -> code 1
    y = O.dequantize(O.Q3_K, blk, 1, 256)[0]
    e = 128 + 96 + 7
    assert y[e] == 1.0 * (33 - 32) * 1   # scale index e//16 = 14 >= 8 -> low nibble 1 -> 33
    assert np.count_nonzero(y) == 1
    blk[0 + 7] &= ~np.uint8(1 << (e // 32))   # clear that element's high bit
    y = O.dequantize(O.Q3_K, blk, 1, 256)[0]
    assert y[e] == (1 - 4) * 1.0
    # Q2_K {scales[16]; qs[64]; f16 d, dmin}: scales[j] low nibble * d, high
    # nibble * dmin, per 16 elements; codes as Q3_K's low bits.
    blk = np.zeros(84, np.uint8)
    blk[80:82] = _half(2.0)
    blk[82:84] = _half(0.5)
    blk[0:16] = np.array([(j % 16) | ((15 - j) << 4) for j in range(16)], np.uint8)
    blk[16 + 5] = 0b11_00_10_01       # e=5 -> 1, e=37 -> 2, e=69 -> 0, e=101 -> 3
    y = O.dequantize(O.Q2_K, blk, 1, 256)[0]
    for e_, code in ((5, 1), (37, 2), (69, 0), (101, 3)):
        j = e_ // 16
        assert y[e_] == 2.0 * (j % 16) * code - 0.5 * (15 - j)


def test_kat_q5_k_high_bit():
    # Q5_K: element 64g + l (l<32) adds 16 when qh[l] bit 2g is set; element
    # 64g + 32 + l when bit 2g+1 is set.
    blk = np.zeros(176, np.uint8)
    blk[0:2] = _half(1.0)
    blk[2:4] = _half(0.0)
    s = np.zeros(12, np.uint8)
    s[0:4] = 1
    s[8:12] = 1          # sub-blocks 4..7 scale low nibble 1
    blk[4:16] = s
    blk[16 + 9] = 0b0100_0010   # qh[9]: bit 1 (e = 32+9) and bit 6 (e = 192+9)
    y = O.dequantize(O.Q5_K, blk, 1, 256)[0]
    assert y[41] == 16.0 and y[201] == 16.0
    assert np.count_nonzero(y) == 2


# -------------------------------------------- llama.cpp test-quantize-fns

def _llama_data(offset, n=32 * 128):
    return (0.1 + 2 * np.cos(np.arange(n, dtype=np.float32) + np.float32(offset))).astype(np.float32)


# thresholds from llama.cpp tests/test-quantize-fns.cpp
MAX_TOTAL = 0.002
MAX_TOTAL_2BITS = 0.0075
MAX_TOTAL_3BITS = 0.0040
MAX_DOT = 0.02
MAX_DOT_LOWBIT = 0.04


@pytest.mark.parametrize("t", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
def test_llama_quantize_fns_known_answer(t):
    n = 32 * 128
    x = _llama_data(0.0)
    blocks = O.quantize(t, x)
    y = O.dequantize(t, blocks, 1, n)[0]
    # array_rmse() in that test is sqrt(sum d^2) / n
    err = math.sqrt(float(np.sum((y.astype(np.float64) - x) ** 2))) / n
    bound = MAX_TOTAL_2BITS if t == O.Q2_K else MAX_TOTAL_3BITS if t == O.Q3_K else MAX_TOTAL
    assert err < bound, (O.NAMES[t], err)
    x2 = _llama_data(1.0)
    dot = O.vec_dot(t, n, blocks, O.quantize_act(t, x2))
    ref = float(np.dot(x.astype(np.float64), x2.astype(np.float64)))
    bound = MAX_DOT_LOWBIT if t == O.Q2_K else MAX_DOT
    assert abs(dot - ref) / n < bound, (O.NAMES[t], dot, ref)


@pytest.mark.parametrize("t", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
def test_vec_dot_consistent_with_dequantized_activations(t):
    # The integer vec_dot must equal float dot(dequant(W), dequant(act)) to f32
    # accumulation accuracy: a wrong sub-block scale or min index in either
    # vec_dot or dequant breaks this by far more than rounding.
    n = 1024
    rng = np.random.default_rng(300 + t)
    w = rng.standard_normal(n).astype(np.float32) * 0.02
    a = rng.standard_normal(n).astype(np.float32)
    wb = O.quantize(t, w)
    ab = O.quantize_act(t, a)
    vdt = O.lib().orc_vec_dot_type(t)
    wd = O.dequantize(t, wb, 1, n)[0].astype(np.float64)
    if vdt == O.Q8_K:
        blk = ab.reshape(-1, 292)
        d = blk[:, 0:4].copy().view(np.float32).astype(np.float64)
        ad = (blk[:, 4:260].view(np.int8).astype(np.float64) * d).ravel()
    else:
        ts = 34 if vdt == O.Q8_0 else 36
        blk = ab.reshape(-1, ts)
        d = blk[:, 0:2].copy().view(np.float16).astype(np.float64)
        ad = (blk[:, ts - 32:].view(np.int8).astype(np.float64) * d).ravel()
    ref = float(wd @ ad)
    got = O.vec_dot(t, n, wb, ab)
    scale = float(np.abs(wd).sum() * np.abs(ad).max())
    assert abs(got - ref) <= 2e-3 * scale + 1e-6, (got, ref)


# ---------------------------------------------------------------------- matmul

@pytest.mark.parametrize("t", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
def test_matmul_f64_equals_numpy_blas(t):
    rng = np.random.default_rng(400 + t)
    m, n, k = 7, 33, 512
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    wb = O.quantize(t, w)
    y = O.matmul_f64(t, x, wb, n, k)
    ref = x.astype(np.float64) @ O.dequantize(t, wb, n, k).astype(np.float64).T
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("t", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
def test_candle_cpu_matmul_within_bar_of_f64(t):
    rng = np.random.default_rng(500 + t)
    m, n, k = 5, 64, 768
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    wb = O.quantize(t, w)
    y = O.matmul_candle(t, x, wb, n, k, nthreads=4)
    ref = O.matmul_f64(t, x, wb, n, k)
    assert O.rel_l2(y, ref) < 1e-2
    # threads only split columns: results are identical for any thread count
    assert np.array_equal(y, O.matmul_candle(t, x, wb, n, k, nthreads=1))


def test_matmul_linearity_and_zero_blocks():
    rng = np.random.default_rng(7)
    t, m, n, k = O.Q4_K, 3, 16, 512
    wb = O.quantize(t, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    # quarter-integers: 2*x1 + x2 is exact in f32, so linearity holds to f64 rounding
    x1 = (rng.integers(-8, 8, (m, k)) / 4).astype(np.float32)
    x2 = (rng.integers(-8, 8, (m, k)) / 4).astype(np.float32)
    y = O.matmul_f64(t, (2 * x1 + x2).astype(np.float32), wb, n, k)
    assert np.allclose(y, 2 * O.matmul_f64(t, x1, wb, n, k) + O.matmul_f64(t, x2, wb, n, k), rtol=1e-9, atol=1e-9)
    zero = np.zeros_like(wb)
    assert np.all(O.matmul_f64(t, x1, zero, n, k) == 0)
    assert np.all(O.matmul_candle(t, x1, zero, n, k) == 0)


# ------------------------------------------- reference quantizers: second restatement

def _adversarial_rows(k, rng):
    """Rows that reach every branch of the quantizers: zero, constant, one-signed,
    tiny (scales underflow f16), huge, sparse, on small integer grids (ties in the
    rounding and in the search), +-1, signed zeros, heavy tails."""
    rows = [rng.standard_normal(k) * 0.02, np.zeros(k), np.full(k, 1.25), np.abs(rng.standard_normal(k)),
            -np.abs(rng.standard_normal(k)) * 3, rng.standard_normal(k) * 1e-30, rng.standard_normal(k) * 1e4,
            np.where(np.arange(k) % 17 == 0, rng.standard_normal(k), 0), rng.integers(-8, 8, k) / 4,
            rng.integers(-3, 4, k) * 1.0, np.where(rng.random(k) < 0.5, 1.0, -1.0), rng.standard_normal(k) * 1e-6,
            np.full(k, -0.0), rng.standard_normal(k) ** 3, rng.standard_cauchy(k),
            np.where(rng.random(k) < 0.5, 0.0, -0.0), rng.standard_normal(k) * 2e-7,
            rng.integers(-2, 3, k) * 0.1, np.repeat(rng.standard_normal(k // 16), 16)]
    return np.array(rows, dtype=np.float32)


@pytest.mark.parametrize("t", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
def test_reference_quantizer_equals_numpy_restatement(t):
    """The C oracle's quantizers against oracle/np_quant.py, a second restatement of
    ggml's quantize_row_*_ref / make_qkx2_quants / make_q3_quants / make_qx_quants
    with a different evaluation structure (all blocks at once, numpy rounding):
    byte for byte on N(0, 0.02^2) weight rows and on adversarial rows.  A slip in
    either one (a wrong rdelta / nstep / rmin, weight choice, search update, tie
    rule, clamp or bit packing) changes bytes here."""
    from oracle import np_quant as NQ
    rng = np.random.default_rng(600 + t)
    k = 1024
    x = np.concatenate([_adversarial_rows(k, rng), (rng.standard_normal((48, k)) * 0.02).astype(np.float32)])
    a = O.quantize(t, x)
    with np.errstate(over="ignore"):
        b = NQ.quantize(t, x)
    bad = [i for i in range(x.shape[0]) if not np.array_equal(a[i], b[i])]
    assert not bad, f"{O.NAMES[t]}: rows {bad} differ"


def test_activation_quantizers_equal_numpy_restatement():
    from oracle import np_quant as NQ
    rng = np.random.default_rng(610)
    k = 4096
    L = O.lib()
    for vdt, fn in ((O.Q8_0, L.orc_quantize_row_q8_0), (O.Q8_1, L.orc_quantize_row_q8_1),
                    (O.Q8_K, L.orc_quantize_row_q8_K)):
        for x in _adversarial_rows(k, rng):
            out = np.zeros(O.row_bytes(vdt, k), np.uint8)
            fn(x.ctypes.data, out.ctypes.data, k)
            assert np.array_equal(out, NQ.ACT[vdt](x).reshape(-1)), O.NAMES[vdt]


# ------------------------------------------- legacy quantizers: known answers

def _row(n, items):
    x = np.zeros(n, np.float32)
    for i, v in items.items():
        x[i] = v
    return x


def _codes4(blk, off):
    qs = blk[off:off + 16]
    return [int(b) & 15 for b in qs] + [int(b) >> 4 for b in qs]


def _halfbits(blk, off):
    return int(blk[off]) | (int(blk[off + 1]) << 8)


def test_kat_quantize_q4_0():
    # ggml quantize_row_q4_0_ref: d = (first value of largest |x|) / -8, id = 1/d,
    # code = min(15, trunc(x * id + 8.5)).
    # (a) max is x[3] = -4 (x[10] = +4 comes later): d = 0.5, id = 2.
    x = _row(32, {0: 1.0, 3: -4.0, 10: 4.0, 11: 0.25, 12: -0.25, 13: 0.75, 14: -0.75, 15: 0.2, 16: 3.74})
    blk = O.quantize(O.Q4_0, x)[0]
    assert _halfbits(blk, 0) == 0x3800                      # f16(0.5)
    exp = [8] * 32
    exp[0] = 10       # 2 + 8.5 = 10.5 -> 10
    exp[3] = 0        # -8 + 8.5 = 0.5 -> 0
    exp[10] = 15      # 8 + 8.5 = 16.5 -> 16 -> clamped to 15
    exp[11] = 9       # 0.5 + 8.5 = 9.0: a tie goes up
    exp[12] = 8       # -0.5 + 8.5 = 8.0
    exp[13] = 10      # 1.5 + 8.5 = 10.0
    exp[14] = 7       # -1.5 + 8.5 = 7.0
    exp[15] = 8       # 0.4 + 8.5 = 8.9 -> 8
    exp[16] = 15      # 7.48 + 8.5 = 15.98 -> 15
    assert _codes4(blk, 2) == exp
    # (b) the positive +4 comes first: d = -0.5, id = -2, so -4 -> 16.5 -> 15
    x = _row(32, {2: 4.0, 5: -4.0, 6: 1.0})
    blk = O.quantize(O.Q4_0, x)[0]
    assert _halfbits(blk, 0) == 0xB800                      # f16(-0.5)
    c = _codes4(blk, 2)
    assert (c[2], c[5], c[6], c[0]) == (0, 15, 6, 8)        # 1 * -2 + 8.5 = 6.5 -> 6
    # (c) all zero: d = +0 / -8 = -0, stored as the f16 -0 bits; id = 0, codes 8
    blk = O.quantize(O.Q4_0, np.zeros(32, np.float32))[0]
    assert _halfbits(blk, 0) == 0x8000 and _codes4(blk, 2) == [8] * 32
    # (d) d rounds to f16: max -1.0001 -> d = 0.1250125 -> f16 0.125 (0x3000), while
    # the codes use the unrounded id = 1 / 0.1250125
    x = _row(32, {0: -1.0001, 1: 0.5})
    blk = O.quantize(O.Q4_0, x)[0]
    assert _halfbits(blk, 0) == 0x3000
    assert _codes4(blk, 2)[:2] == [0, 12]                   # 0.5 * 7.9992 + 8.5 = 12.4996 -> 12


def test_kat_quantize_q8_0():
    # ggml quantize_row_q8_0_ref: d = max|x| / 127, q = roundf(x / d) (half away from zero).
    x = _row(32, {0: 127.0, 1: 2.5, 2: -2.5, 3: 0.5, 4: -0.5, 5: 1.5, 6: -126.5, 7: 126.4, 8: 0.49})
    blk = O.quantize(O.Q8_0, x)[0]
    assert _halfbits(blk, 0) == 0x3C00                      # d = 1
    q = blk[2:34].view(np.int8).tolist()
    assert q[:9] == [127, 3, -3, 1, -1, 2, -127, 126, 0] and q[9:] == [0] * 23
    # d = 254 / 127 = 2 (the sign of the largest value does not matter), id = 0.5
    x = _row(32, {7: -254.0, 0: 5.0, 1: -1.0, 2: 3.0})
    blk = O.quantize(O.Q8_0, x)[0]
    assert _halfbits(blk, 0) == 0x4000
    assert blk[2:34].view(np.int8).tolist()[:8] == [3, -1, 2, 0, 0, 0, 0, -127]
    # d = 1.0001 is stored as f16 1.0 while the codes use 1 / 1.0001
    x = _row(32, {0: 127.0127, 1: 64.0})
    blk = O.quantize(O.Q8_0, x)[0]
    assert _halfbits(blk, 0) == 0x3C00
    assert blk[2:4].view(np.int8).tolist() == [127, 64]     # 64 / 1.0001 = 63.994 -> 64
    blk = O.quantize(O.Q8_0, np.zeros(32, np.float32))[0]
    assert not blk.any()                                   # d = +0, all codes 0


def test_kat_quantize_q4_1_and_q5_1():
    # ggml quantize_row_q4_1_ref: d = (max - min) / 15, m = min,
    # code = min(15, trunc((x - min) / d + 0.5)).  min = -1, max = 14: d = 1.
    x = np.zeros(32, np.float32)
    x[4], x[9], x[0], x[1], x[2], x[3] = -1.0, 14.0, -0.5, 0.4, 13.5, 2.5
    blk = O.quantize(O.Q4_1, x)[0]
    assert (_halfbits(blk, 0), _halfbits(blk, 2)) == (0x3C00, 0xBC00)   # d = 1, m = -1
    exp = [1] * 32                  # x = 0: 1 + 0.5 -> 1
    exp[4], exp[9] = 0, 15
    exp[0] = 1                      # 0.5 + 0.5 = 1.0: the tie goes up
    exp[1] = 1                      # 1.4 + 0.5 = 1.9 -> 1
    exp[2] = 15                     # 14.5 + 0.5 = 15
    exp[3] = 4                      # 3.5 + 0.5 = 4
    assert _codes4(blk, 4) == exp
    # a constant block: d = 0 (so id = 0, every code 0) and m holds the value
    blk = O.quantize(O.Q4_1, np.full(32, 3.0, np.float32))[0]
    assert (_halfbits(blk, 0), _halfbits(blk, 2)) == (0x0000, 0x4200) and not blk[4:].any()
    # Q5_1: the same with 31 levels and no clamp; the fifth bits go to qh
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2], x[3] = -1.0, 30.0, 15.0, -0.5
    blk = O.quantize(O.Q5_1, x)[0]
    assert (_halfbits(blk, 0), _halfbits(blk, 2)) == (0x3C00, 0xBC00)
    qh = int.from_bytes(bytes(blk[4:8]), "little")
    codes = [c | (((qh >> j) & 1) << 4) for j, c in enumerate(_codes4(blk, 8))]
    assert codes[:4] == [0, 31, 16, 1] and codes[4:] == [1] * 28


def test_kat_quantize_q5_0():
    # ggml quantize_row_q5_0_ref: d = (first largest |x|) / -16,
    # code = min(31, trunc(x / d + 16.5)); bit 4 of code j is qh bit j.
    x = _row(32, {1: -8.0, 20: 8.0, 2: 0.25, 3: -0.25})
    blk = O.quantize(O.Q5_0, x)[0]
    assert _halfbits(blk, 0) == 0x3800                      # d = -8 / -16 = 0.5
    qh = int.from_bytes(bytes(blk[2:6]), "little")
    codes = [c | (((qh >> j) & 1) << 4) for j, c in enumerate(_codes4(blk, 6))]
    exp = [16] * 32                  # 0 + 16.5 -> 16
    exp[1] = 0                       # -16 + 16.5 = 0.5 -> 0
    exp[20] = 31                     # 16 + 16.5 = 32.5 -> 32 -> clamped to 31
    exp[2] = 17                      # 0.5 + 16.5 = 17.0
    exp[3] = 16                      # -0.5 + 16.5 = 16.0
    assert codes == exp


def test_kat_activation_quantizers():
    """Q8_0 / Q8_1 / Q8_K activation blocks (candle's CPU vec-dot inputs) on
    hand-worked rows.  Q8_K follows the convention this oracle states for candle
    (iscale = -128 / the first value of largest magnitude, roundf, clamp at +127);
    the rows separate it from ggml's quantize_row_q8_K_ref (-127 / max, ties to
    even), which would give other codes here.  Whether candle rounds this way is
    not pinnable without its source (parity unpinned); the GPU GEMV is held to a
    bound that holds for either convention."""
    L = O.lib()
    # Q8_K (a): max is x[10] = -128: iscale = 1, d = 1
    x = np.zeros(256, np.float32)
    x[10], x[0], x[1], x[2], x[3], x[4] = -128.0, 2.5, -2.5, 127.5, 0.5, -127.5
    out = np.zeros(292, np.uint8)
    L.orc_quantize_row_q8_K(x.ctypes.data, out.ctypes.data, 256)
    assert out[0:4].view(np.float32)[0] == 1.0
    q = out[4:260].view(np.int8)
    assert q[:5].tolist() == [3, -3, 127, 1, -128] and q[10] == -128 and np.count_nonzero(q) == 6
    assert out[260:292].view(np.int16).tolist() == [3 - 3 + 127 + 1 - 128 - 128] + [0] * 15
    # Q8_K (b): +64 first: iscale = -2, d = -0.5; -64 -> 128 -> clamped to 127; 1.25 -> -2.5 -> -3
    x = np.zeros(256, np.float32)
    x[0], x[1], x[300 - 256] = 64.0, -64.0, 1.25
    L.orc_quantize_row_q8_K(x.ctypes.data, out.ctypes.data, 256)
    assert out[0:4].view(np.float32)[0] == -0.5
    q = out[4:260].view(np.int8)
    assert q[:2].tolist() == [-128, 127] and q[44] == -3 and np.count_nonzero(q) == 3
    # Q8_K (c): an all-zero block is all zero bytes
    z = np.zeros(256, np.float32)
    L.orc_quantize_row_q8_K(z.ctypes.data, out.ctypes.data, 256)
    assert not out.any()
    # Q8_1: d = 127 / 127 = 1, q = roundf(x), s = f16(f16(sum q) * d)
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2], x[3] = 127.0, 2.5, -0.5, 100.0
    o1 = np.zeros(36, np.uint8)
    L.orc_quantize_row_q8_1(x.ctypes.data, o1.ctypes.data, 32)
    assert (_halfbits(o1, 0), _halfbits(o1, 2)) == (0x3C00, int(np.float16(229.0).view(np.uint16)))
    assert o1[4:8].view(np.int8).tolist() == [127, 3, -1, 100]
    # sum 16 * 127 + 17 = 2049 is not an f16 (spacing 2 there; the tie goes to even
    # 2048), so s = 2048, not 2049
    x = np.zeros(32, np.float32)
    x[:16] = 127.0
    x[16] = 17.0
    L.orc_quantize_row_q8_1(x.ctypes.data, o1.ctypes.data, 32)
    assert _halfbits(o1, 2) == int(np.float16(2048.0).view(np.uint16))


# ------------------------------------------- reference quantizers: the exact grid

def _h16(v):
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def _f16_scale(rng, n, lo=-9, hi=-1, signed=False):
    """n f16-representable scales m * 2^e with a 5-bit mantissa (so every product
    the formats form with them is exact), optionally of random sign."""
    v = rng.integers(16, 32, n) * np.exp2(rng.integers(lo, hi, n).astype(np.float64) - 4)
    if signed:
        v = v * rng.choice([-1.0, 1.0], n)
    return v.astype(np.float32)


def _codes_with(rng, shape, lo, hi, must):
    """Random integer codes in [lo, hi] where every row (last axis) holds each value
    of `must` at a random position."""
    c = rng.integers(lo, hi + 1, shape)
    flat = c.reshape(-1, shape[-1])
    for row in flat:
        pos = rng.choice(shape[-1], len(must), replace=False)
        row[pos] = must
    return flat.reshape(shape)


def _grid_blocks(t, nb, rng):
    """GGUF blocks on which the reference quantizer is exact: each block's (sub-)block
    scales include the extreme stored value, every (sub-)block holds its extreme
    codes, and the f16 scales are short enough that every dequantized value, range
    and ratio the quantizer forms is exact (or within a few f32 ulps of it)."""
    if t in (O.Q4_0, O.Q5_0):
        top = 15 if t == O.Q4_0 else 31
        q = _codes_with(rng, (nb, 32), 0, top, [0])          # code 0: the unique largest |value|
        d = _f16_scale(rng, nb, signed=True)
        qs = (q[:, :16] & 15) | ((q[:, 16:] & 15) << 4)
        out = [_h16(d).reshape(-1, 1).view(np.uint8)]
        if t == O.Q5_0:
            qh = ((q >> 4).astype(np.uint64) << np.arange(32, dtype=np.uint64)).sum(axis=1).astype(np.uint32)
            out.append(qh.reshape(-1, 1).view(np.uint8))
        return np.concatenate(out + [qs.astype(np.uint8)], axis=1)
    if t in (O.Q4_1, O.Q5_1):
        top = 15 if t == O.Q4_1 else 31
        q = _codes_with(rng, (nb, 32), 0, top, [0, top])
        d = (rng.integers(1, 64, nb) * 2.0 ** -8).astype(np.float32)
        m = (rng.integers(-64, 65, nb) * 2.0 ** -6).astype(np.float32)
        qs = (q[:, :16] & 15) | ((q[:, 16:] & 15) << 4)
        out = [_h16(d).reshape(-1, 1).view(np.uint8), _h16(m).reshape(-1, 1).view(np.uint8)]
        if t == O.Q5_1:
            qh = ((q >> 4).astype(np.uint64) << np.arange(32, dtype=np.uint64)).sum(axis=1).astype(np.uint32)
            out.append(qh.reshape(-1, 1).view(np.uint8))
        return np.concatenate(out + [qs.astype(np.uint8)], axis=1)
    if t == O.Q8_0:
        q = _codes_with(rng, (nb, 32), -127, 127, [127])
        q = q * rng.choice([-1, 1], (nb, 1))
        d = _f16_scale(rng, nb)
        return np.concatenate([_h16(d).reshape(-1, 1).view(np.uint8), q.astype(np.int8).view(np.uint8)], axis=1)
    if t == O.Q2_K:
        lo = _codes_with(rng, (nb, 16), 1, 15, [15])
        hi = _codes_with(rng, (nb, 16), 0, 15, [15])
        q = _codes_with(rng, (nb, 16, 16), 0, 3, [0, 3]).reshape(nb, 2, 4, 32)
        qs = (q[:, :, 0] | (q[:, :, 1] << 2) | (q[:, :, 2] << 4) | (q[:, :, 3] << 6)).reshape(nb, 64)
        return np.concatenate([(lo | (hi << 4)).astype(np.uint8), qs.astype(np.uint8),
                               _h16(_f16_scale(rng, nb)).reshape(-1, 1).view(np.uint8),
                               _h16(_f16_scale(rng, nb)).reshape(-1, 1).view(np.uint8)], axis=1)
    if t == O.Q3_K:
        s = _codes_with(rng, (nb, 16), -31, 31, [-32])       # stored scale - 32; none zero
        s = np.where(s == 0, 5, s) + 32
        packed = np.zeros((nb, 12), np.int64)
        packed[:, 0:8] = (s[:, 0:8] & 15) | ((s[:, 8:16] & 15) << 4)
        h = s >> 4
        packed[:, 8:12] = h[:, 0:4] | (h[:, 4:8] << 2) | (h[:, 8:12] << 4) | (h[:, 12:16] << 6)
        l = _codes_with(rng, (nb, 16, 16), -4, 3, [-4]).reshape(nb, 256) + 4     # 0..7
        hmask = (((l >> 2) & 1).reshape(nb, 8, 32) << np.arange(8)[None, :, None]).sum(axis=1)
        c = (l & 3).reshape(nb, 2, 4, 32)
        qs = (c[:, :, 0] | (c[:, :, 1] << 2) | (c[:, :, 2] << 4) | (c[:, :, 3] << 6)).reshape(nb, 64)
        return np.concatenate([hmask.astype(np.uint8), qs.astype(np.uint8), packed.astype(np.uint8),
                               _h16(_f16_scale(rng, nb, signed=True)).reshape(-1, 1).view(np.uint8)], axis=1)
    if t in (O.Q4_K, O.Q5_K):
        top = 15 if t == O.Q4_K else 31
        ls = _codes_with(rng, (nb, 8), 1, 63, [63])
        lm = _codes_with(rng, (nb, 8), 0, 63, [63])
        packed = np.zeros((nb, 12), np.int64)
        packed[:, 0:4] = ls[:, 0:4] | ((ls[:, 4:8] >> 4) << 6)
        packed[:, 4:8] = lm[:, 0:4] | ((lm[:, 4:8] >> 4) << 6)
        packed[:, 8:12] = (ls[:, 4:8] & 15) | ((lm[:, 4:8] & 15) << 4)
        q = _codes_with(rng, (nb, 8, 32), 0, top, [0, top])
        nib = (q & 15).reshape(nb, 4, 2, 32)
        qs = (nib[:, :, 0] | (nib[:, :, 1] << 4)).reshape(nb, 128)
        dm = np.concatenate([_h16(_f16_scale(rng, nb, -12, -6)).reshape(-1, 1).view(np.uint8),
                             _h16(_f16_scale(rng, nb, -12, -6)).reshape(-1, 1).view(np.uint8)], axis=1)
        parts = [dm, packed.astype(np.uint8)]
        if t == O.Q5_K:
            parts.append(((q.reshape(nb, 8, 32) >> 4) << np.arange(8)[None, :, None]).sum(axis=1).astype(np.uint8))
        return np.concatenate(parts + [qs.astype(np.uint8)], axis=1)
    if t == O.Q6_K:
        sc = _codes_with(rng, (nb, 16), -127, 127, [-128])
        sc = np.where(sc == 0, 7, sc)
        L = _codes_with(rng, (nb, 16, 16), 0, 63, [0]).reshape(nb, 2, 4, 32)    # code 0: value -32 d sc
        ql = np.concatenate([(L[:, :, 0] & 15) | ((L[:, :, 2] & 15) << 4),
                             (L[:, :, 1] & 15) | ((L[:, :, 3] & 15) << 4)], axis=2).reshape(nb, 128)
        qh = ((L[:, :, 0] >> 4) | ((L[:, :, 1] >> 4) << 2) | ((L[:, :, 2] >> 4) << 4)
              | ((L[:, :, 3] >> 4) << 6)).reshape(nb, 64)
        return np.concatenate([ql.astype(np.uint8), qh.astype(np.uint8), sc.astype(np.int8).view(np.uint8),
                               _h16(_f16_scale(rng, nb, -14, -8, signed=True)).reshape(-1, 1).view(np.uint8)],
                              axis=1)
    raise AssertionError(t)


@pytest.mark.parametrize("t", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
def test_reference_quantizer_is_exact_on_its_grid(t):
    """What the mathematics fixes for every quantizer: weights that some block of
    the format represents exactly, with every extreme the search starts from present
    (the extreme code in each (sub-)block, the extreme stored scale and min in each
    super-block), come back as that very block: quantize(dequantize(B)) == B.  A
    wrong nmax, offset, sign rule, clamp, scale packing or code packing breaks the
    round trip."""
    bs, ts = O.block_size(t), O.type_size(t)
    rng = np.random.default_rng(700 + t)
    nb = 256
    blocks = _grid_blocks(t, nb, rng)
    assert blocks.shape == (nb, ts)
    x = O.dequantize(t, blocks, 1, nb * bs)
    again = O.quantize(t, x).reshape(nb, ts)
    bad = [i for i in range(nb) if not np.array_equal(again[i], blocks[i])]
    assert not bad, f"{O.NAMES[t]}: {len(bad)} of {nb} blocks changed, first {bad[:5]}"


# ------------------------------------------- candle's CPU algorithm: vec_dot, matmul

def _act_values(vdt, ab, k):
    """Exact values of a quantized activation row (Q8_0 / Q8_1: d * q with f16 d;
    Q8_K: d * q with f32 d), in float64."""
    if vdt == O.Q8_K:
        blk = ab.reshape(-1, 292)
        d = blk[:, 0:4].copy().view(np.float32).astype(np.float64)
        return (blk[:, 4:260].view(np.int8).astype(np.float64) * d).ravel()
    ts = 34 if vdt == O.Q8_0 else 36
    blk = ab.reshape(-1, ts)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64)
    return (blk[:, ts - 32:].view(np.int8).astype(np.float64) * d).ravel()


# byte offsets of the f16 scale whose zeroing leaves only the min / offset part of
# every dequantized value (types with an additive term)
_SCALE_OFF = {O.Q4_1: 0, O.Q5_1: 0, O.Q2_K: 80, O.Q4_K: 0, O.Q5_K: 0}


@pytest.mark.parametrize("t", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
def test_vec_dot_equals_exact_product_to_f32_rounding(t):
    """candle's integer vec_dot of a weight row and a quantized activation row is the
    exact sum of (dequantized weight) x (dequantized activation) up to the float32
    roundings of its per-block scale products and running sum: |vd - exact| <=
    (blocks + 4) 2^-23 (sum |scale part x a| + sum |min part x a|), plus, for Q4_1 /
    Q5_1 (whose Q8_1 partner stores s = f16(f16(sum q) d)), 2^-10 of the min mass.
    A dropped or doubled min term, a wrong sub-block scale or a misplaced element
    moves the result by orders of magnitude more."""
    rng = np.random.default_rng(900 + t)
    k = 2048
    nblk = k // O.block_size(t)
    vdt = O.lib().orc_vec_dot_type(t)
    for trial in range(12):
        w = (rng.standard_normal(k) * (0.02 if trial % 3 else 1.0)).astype(np.float32)
        a = rng.standard_normal(k).astype(np.float32) * np.float32(10.0 ** rng.integers(-3, 3))
        if trial == 5:
            a[:300] = 0.0
        wb = O.quantize(t, w)
        ab = O.quantize_act(t, a)
        wd = O.dequantize(t, wb, 1, k)[0].astype(np.float64)
        ad = _act_values(vdt, ab, k)
        exact = float(wd @ ad)
        if t in _SCALE_OFF:
            z = wb.reshape(nblk, -1).copy()
            z[:, _SCALE_OFF[t]:_SCALE_OFF[t] + 2] = 0
            minpart = O.dequantize(t, z, 1, k)[0].astype(np.float64)
        else:
            minpart = np.zeros(k)
        mass_min = float(np.abs(minpart * ad).sum())
        mass = float(np.abs((wd - minpart) * ad).sum()) + mass_min
        bound = (nblk + 4) * 2.0 ** -23 * mass + (2.0 ** -10 * mass_min if vdt == O.Q8_1 else 0.0) + 1e-30
        got = O.vec_dot(t, k, wb, ab)
        assert abs(got - exact) <= bound, (O.NAMES[t], trial, got, exact, bound)


@pytest.mark.parametrize("t", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
def test_matmul_candle_is_quantized_rows_times_vec_dot(t):
    """candle's CPU QMatMul (quantized/mod.rs matmul_t): each activation row is
    quantized once to the vec-dot type, then every output is one vec_dot.  The
    threaded oracle matmul equals that composition bit for bit, for any thread
    count."""
    rng = np.random.default_rng(950 + t)
    m, n, k = 3, 9, 512
    wb = O.quantize(t, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = O.matmul_candle(t, x, wb, n, k, nthreads=3)
    for r in range(m):
        ab = O.quantize_act(t, x[r])
        for c in range(n):
            assert y[r, c] == np.float32(O.vec_dot(t, k, wb[c], ab)), (r, c)
