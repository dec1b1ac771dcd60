"""GPU parity of libmoldq (HIP, gfx950) against the CPU oracle, through the C ABI.

Bars:
  * dequantized weights bit-exact with the GGUF formulas (oracle/ggml_oracle.c
    restates ggml's dequantize_row_*; candle's QTensor::dequantize evaluates
    the same formulas, called at crates/mold-inference/src/qwen_image/
    quantized_transformer.rs:62-66);
  * QMatMul::forward output within rel-L2 1e-2 of an f64-accumulated
    dequantize-then-matmul (the GEMV is held to 1e-5 against the algorithm it
    runs: candle's Q8_K integer-dot path for Q4_K, f32 accumulation of exact
    weights for the other types);
  * no NaN for finite inputs (the reference scrubs NaN from candle's CUDA
    QMatMul, crates/mold-inference/src/flux2/quantized_transformer.rs:40-45);
  * identical outputs on repeated calls (no races in the LDS pipeline).
Full BASELINE shapes are checked on sampled rows plus size-independent
properties (linearity, determinism, NaN-freedom).
"""
import ctypes
import sys

import numpy as np
import pytest

import mold_amd
from mold_amd import GgmlDType, QMatMul, QTensor
from mold_amd._lib import MoldqError
from oracle import oracle as O

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-2   # BASELINE: rel-L2 <= 1e-2 vs f32 dequantize-then-matmul
GEMV_TOL = 1e-5   # exact weights (or exact Q8_K products) summed in f32


def _q8k_row_bound(x, blocks, t, n, k):
    """Per-output bound on |y_gpu - y_exact| for a GEMV that quantizes x to Q8_K.

    Whatever Q8_K's rounding convention (scale -128/max or -127/max, ties to even or
    away from zero, the +max clamp to 127), every quantized element is within one
    step d_x = max|x_sb| / 127 of x, so |sum_i w_i (x_i - q_i d_x)| <= sum_sb d_x
    sum_{i in sb} |w_i|.  The f32 combine adds at most ~K ulps of sum |w x|.  The bound
    therefore holds for any correct Q8_K GEMV and fails on a wrong scale, a dropped
    term or a misplaced super-block (errors of order |y|)."""
    w = O.dequantize(t, blocks, n, k).astype(np.float64)
    xa = np.abs(x.astype(np.float64)).reshape(x.shape[0], k // 256, 256)
    dx = xa.max(axis=2) / 127.0                                   # [m, sb]
    wa = np.abs(w).reshape(n, k // 256, 256).sum(axis=2)           # [n, sb]
    quant = dx @ wa.T                                              # [m, n]
    f32 = 4 * k * 2.0 ** -24 * (np.abs(x.astype(np.float64)) @ np.abs(w).T)
    return quant + f32 + 1e-30


def _gemv_check(t, x, y, blocks, n, k, extra=None):
    """GEMV parity on pinned references only.

    * Every type: rel-L2 <= 1e-2 against the f64 dequantize-then-matmul (the BASELINE
      bar) and finite outputs.
    * Q4_K (the kernel quantizes x to Q8_K, candle's k-quant algorithm): every output
      within _q8k_row_bound of the exact product.
    * Other types (exact weights times f32 x, summed in f32): rel-L2 <= 1e-5 against f64.
    Agreement with the oracle's restatement of candle's CPU QMatMul is printed, not
    asserted: that restatement's Q8_K conventions come from candle's source, which is
    not in this container (parity unpinned)."""
    ref_exact = O.matmul_f64(int(t), x, blocks, n, k)
    if extra is not None:
        ref_exact = extra(ref_exact)
    assert np.isfinite(y).all()
    assert O.rel_l2(y, ref_exact) <= GEMM_TOL
    if int(t) == O.Q4_K:
        if extra is None:
            bound = _q8k_row_bound(x, blocks, int(t), n, k)
            err = np.abs(y.astype(np.float64) - ref_exact)
            assert (err <= bound).all(), float((err / bound).max())
        cand = O.matmul_candle(int(t), x, blocks, n, k).astype(np.float64)
        if extra is not None:
            cand = extra(cand)
        print(f"[report] Q4_K GEMV vs candle CPU restatement: rel-L2 {O.rel_l2(y, cand):.2e}", flush=True)
    else:
        assert O.rel_l2(y, ref_exact) <= GEMV_TOL


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as _t
    return _t


@pytest.fixture(scope="module")
def dev(torch):
    d = mold_amd.Device(0)
    yield d
    torch.cuda.synchronize()


def _weights(t, n, k, seed, scale=0.02):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * scale).astype(np.float32)
    return O.quantize(t, w)


def _random_blocks(t, n, k, seed):
    """Arbitrary bytes: every byte pattern is a valid GGUF block (f16 scales may be
    subnormal, Inf or NaN)."""
    rng = np.random.default_rng(seed)
    return rng.integers(0, 256, size=(n, O.row_bytes(t, k)), dtype=np.uint8)


def _bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    return np.array_equal(a.view(np.uint32)[~na], b.view(np.uint32)[~nb])


TYPES = [GgmlDType(t) for t in O.WEIGHT_TYPES]
IDS = [t.name for t in TYPES]


# ------------------------------------------------------------- upload / dequant

@pytest.mark.parametrize("t", TYPES, ids=IDS)
def test_upload_download_byte_identical(dev, t):
    n, k = 131, 2 * 256
    _say(f"upload/download {t.name} [{n},{k}]")
    blocks = _random_blocks(int(t), n, k, 1)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    assert qt.dtype() == t and qt.shape == (n, k)
    assert qt.storage_size_in_bytes() == blocks.nbytes
    assert np.array_equal(qt.data(), blocks.reshape(-1))


@pytest.mark.parametrize("t", TYPES, ids=IDS)
@pytest.mark.parametrize("shape", [(1, 256), (64, 512), (130, 768), (257, 256)], ids=str)
def test_dequantize_bit_exact_quantized_weights(dev, torch, t, shape):
    n, k = shape
    _say(f"dequant {t.name} {shape}")
    blocks = _weights(int(t), n, k, seed=n + k)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    got = qt.dequantize().cpu().numpy()
    torch.cuda.synchronize()
    assert _bits_equal(got, O.dequantize(int(t), blocks, n, k))


@pytest.mark.parametrize("t", TYPES, ids=IDS)
def test_dequantize_bit_exact_random_bytes(dev, torch, t):
    n, k = 67, 512
    _say(f"dequant random bytes {t.name}")
    blocks = _random_blocks(int(t), n, k, 7)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    got = qt.dequantize().cpu().numpy()
    assert _bits_equal(got, O.dequantize(int(t), blocks, n, k))


@pytest.mark.parametrize("t", [GgmlDType.Q4_K, GgmlDType.Q8_0, GgmlDType.Q6_K, GgmlDType.Q3_K], ids=lambda t: t.name)
def test_dequantize_half_outputs_round_nearest_even(dev, torch, t):
    n, k = 96, 512
    _say(f"dequant f16/bf16 {t.name}")
    blocks = _weights(int(t), n, k, seed=3, scale=1.0)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    exact = torch.from_numpy(O.dequantize(int(t), blocks, n, k))
    for dt in (torch.bfloat16, torch.float16):
        got = qt.dequantize(dtype=dt).cpu()
        assert torch.equal(got.view(torch.int16), exact.to(dt).view(torch.int16)), dt
    # arbitrary blocks: scales of every magnitude (double rounding would show here)
    blocks = _random_blocks(int(t), n, k, 8)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    exact = torch.from_numpy(O.dequantize(int(t), blocks, n, k))
    nan = torch.isnan(exact)
    for dt in (torch.bfloat16, torch.float16):
        got = qt.dequantize(dtype=dt).cpu()
        assert torch.equal(torch.isnan(got), nan), dt
        assert torch.equal(got[~nan].view(torch.int16), exact[~nan].to(dt).view(torch.int16)), dt


# --------------------------------------------------------------------- GEMV

@pytest.mark.parametrize("t", TYPES, ids=IDS)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 8])
def test_gemv_matches_f64_oracle(dev, torch, t, m):
    n, k = 200, 1024
    _say(f"gemv {t.name} m={m}")
    blocks = _weights(int(t), n, k, seed=m)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    rng = np.random.default_rng(100 + m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = QMatMul(qt).forward(torch.from_numpy(x).cuda()).cpu().numpy()
    _gemv_check(t, x, y, blocks, n, k)


def test_gemv_bias_gelu_strides_bf16(dev, torch):
    t, n, k, m = GgmlDType.Q4_K, 300, 768, 2
    _say("gemv bias/gelu/strides/bf16")
    blocks = _weights(int(t), n, k, seed=11)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    rng = np.random.default_rng(12)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal(n) * 0.1).astype(np.float32)
    def gelu_of(r):
        r = r + b
        return 0.5 * r * (1 + np.tanh(np.sqrt(2 / np.pi) * (r + 0.044715 * r ** 3)))
    bias = torch.from_numpy(b).cuda()
    # strided x: view into a wider buffer
    xw = torch.zeros((m, k + 64), dtype=torch.float32, device="cuda")
    xw[:, :k] = torch.from_numpy(x).cuda()
    lin = mold_amd.Linear(qt, bias)
    y = lin.forward(xw[:, :k], act=mold_amd.ACT_GELU_TANH).cpu().numpy()
    _gemv_check(t, x, y, blocks, n, k, extra=gelu_of)
    # bf16 in / bf16 out
    xb = torch.from_numpy(x).cuda().to(torch.bfloat16)
    ref_b = O.matmul_f64(int(t), xb.float().cpu().numpy(), blocks, n, k) + b
    yb = lin.forward(xb).float().cpu().numpy()
    assert O.rel_l2(yb, ref_b) <= 1e-2


@pytest.mark.parametrize("n,k,m", [(3072, 256, 1), (3072, 256, 3), (640, 768, 1), (9216, 256, 1)])
def test_gemv_q4k_bf16_x_odd_item_count(dev, torch, n, k, m):
    """bf16 x staged two items (row of x over one super-block) per direct load: with an
    odd item count (k = 256 at m = 1: FLUX's time_in / guidance_in linear_1 [3072, 256])
    the last load must fill only its item.  The result meets the Q8_K bound of the exact
    product, and repeats bit for bit."""
    t = GgmlDType.Q4_K
    _say(f"gemv bf16 x odd items n={n} k={k} m={m}")
    blocks = _weights(int(t), n, k, seed=n + k + m)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    xb = torch.from_numpy(np.random.default_rng(k * m).standard_normal((m, k)).astype(np.float32)).cuda()
    xb = xb.to(torch.bfloat16)
    mm = QMatMul(qt)
    y1 = mm.forward(xb, out_dtype=torch.float32).clone()
    y2 = mm.forward(xb, out_dtype=torch.float32).clone()
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int32), y2.view(torch.int32))
    x = xb.float().cpu().numpy()
    y = y1.cpu().numpy()
    ref = O.matmul_f64(int(t), x, blocks, n, k)
    assert np.isfinite(y).all()
    assert (np.abs(y.astype(np.float64) - ref) <= _q8k_row_bound(x, blocks, int(t), n, k)).all()


def test_gemv_q8k_activation_edge_cases(dev, torch):
    """Q8_K staging of the Q4_K GEMV on awkward activations: ties in |x| with opposite
    signs, all-zero super-blocks (d = 0), a lone non-zero element, a constant block (every
    q at the clamp), a tiny scale.  Each row must stay inside the convention-independent
    Q8_K error bound of the exact product, and rows of zeros must give exact zeros."""
    t, n, k = GgmlDType.Q4_K, 128, 1024
    _say("gemv Q8_K activation edge cases")
    blocks = _weights(int(t), n, k, seed=77)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    rng = np.random.default_rng(78)
    x = rng.standard_normal((5, k)).astype(np.float32)
    x[0, 3], x[0, 200] = -2.5, 2.5           # tie: element 3 (negative) comes first
    x[0, 300], x[0, 301] = 3.0, -3.0         # second super-block: + first
    x[1, :256] = 0.0                         # zero super-block
    x[1, 256:512] = 0.0
    x[1, 400] = 1.5                          # lone element
    x[2, 512:768] = 1.0                      # constant block: every q = -128
    x[3, 768:] *= 1e-30                      # tiny scale
    x[4] = 0.0                               # all zero
    y = QMatMul(qt).forward(torch.from_numpy(x).cuda()).cpu().numpy()
    assert np.isfinite(y).all()
    assert not y[4].any()
    ref = O.matmul_f64(int(t), x, blocks, n, k)
    err = np.abs(y.astype(np.float64) - ref)
    assert (err <= _q8k_row_bound(x, blocks, int(t), n, k)).all()
    cand = O.matmul_candle(int(t), x, blocks, n, k)
    print(f"[report] edge cases vs candle CPU restatement: rel-L2 {O.rel_l2(y, cand):.2e}", flush=True)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("n,k", [(18432, 3072), (9216, 3072), (1000, 256), (4096, 4096)], ids=str)
def test_gemv_q4k_pre_quantized_x_bit_identical(dev, torch, m, n, k):
    """mq_quantize_x_q8k + mq_qmatmul(x_dtype = MQ_X_Q8K) equals mq_qmatmul on the f32 /
    bf16 x itself bit for bit (both quantize x by the same code), with bias, GELU and a
    bf16 output; reusing one quantized x for two weights is the same as two calls.  Where
    the Q4_K GEMV does not run (m = 8 at K = 3072: its LDS would not hold x as f32) the
    pre-quantized form is refused."""
    from mold_amd._lib import MQ_E_UNSUPPORTED, MQ_X_Q8K
    _say(f"gemv pre-quantized x m={m} [{n},{k}]")
    g = torch.Generator(device="cuda").manual_seed(n + k + m)
    qt = QTensor.quantize(dev, torch.randn((n, k), device="cuda", generator=g) * 0.02, GgmlDType.Q4_K)
    size = ctypes.c_size_t()
    if mold_amd._lib.load().mq_qmatmul_workspace_size(dev.handle, qt.handle, MQ_X_Q8K, m, 0,
                                                       ctypes.byref(size)) == MQ_E_UNSUPPORTED:
        assert m >= 4, (m, n, k)
        with pytest.raises(MoldqError) as e:
            QMatMul(qt).forward(mold_amd.Q8KActivations(dev, torch.randn((m, k), device="cuda")))
        assert e.value.code == MQ_E_UNSUPPORTED
        return
    qt2 = QTensor.quantize(dev, torch.randn((n, k), device="cuda", generator=g) * 0.02, GgmlDType.Q4_K)
    bias = torch.randn(n, device="cuda", generator=g)
    for xdt in (torch.float32, torch.bfloat16):
        x = (torch.randn((m, k), device="cuda", generator=g) * 3).to(xdt)
        xq = mold_amd.Q8KActivations(dev, x)
        for w in (qt, qt2):
            mm = QMatMul(w)
            assert torch.equal(mm.forward(xq, out_dtype=torch.float32), mm.forward(x, out_dtype=torch.float32))
            a = mm.forward(xq, bias=bias, act=mold_amd.ACT_GELU_TANH, out_dtype=torch.bfloat16)
            b = mm.forward(x, bias=bias, act=mold_amd.ACT_GELU_TANH, out_dtype=torch.bfloat16)
            assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    torch.cuda.synchronize()


def test_quantize_x_q8k_blocks_match_the_oracle(dev, torch):
    """The blocks' quants and scale are the oracle's Q8_K (candle's BlockQ8K convention as
    restated there), the sums are its per-16 sums added in pairs, the pad bytes zero;
    an all-zero item gives d = 0 and zero quants."""
    from mold_amd._lib import MQ_X_Q8K_BLOCK_BYTES as B
    m, k = 3, 1024
    x = np.random.default_rng(12).standard_normal((m, k)).astype(np.float32) * 5
    x[1, 256:512] = 0.0
    x[2, 3] = -x[2, :256].__abs__().max() * 1.5       # a negative first maximum
    xq = mold_amd.Q8KActivations(dev, torch.from_numpy(x).cuda())
    got = xq.data.cpu().numpy().reshape(m, k // 256, B)
    for r in range(m):
        ref = O.quantize_act(O.Q4_K, x[r]).reshape(k // 256, 292)
        for sb in range(k // 256):
            d_ref = ref[sb, :4].view(np.float32)[0]
            qs_ref = ref[sb, 4:260]
            bs_ref = ref[sb, 260:292].view(np.int16).astype(np.int32)
            assert np.array_equal(got[r, sb, :256], qs_ref), (r, sb)
            assert np.array_equal(got[r, sb, 256:288].view(np.int32), bs_ref[0::2] + bs_ref[1::2]), (r, sb)
            assert got[r, sb, 288:292].view(np.float32)[0].tobytes() == np.float32(d_ref).tobytes(), (r, sb)
            assert not got[r, sb, 292:].any()
    assert not got[1, 1, :288].any()


def test_pre_quantized_x_refused_outside_the_q4k_gemv(dev, torch):
    from mold_amd._lib import MQ_E_UNSUPPORTED, MQ_E_INVALID
    g = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn((2, 512), device="cuda", generator=g)
    xq = mold_amd.Q8KActivations(dev, x)
    q8 = QTensor.quantize(dev, torch.randn((64, 512), device="cuda", generator=g), GgmlDType.Q8_0)
    with pytest.raises(MoldqError) as e:
        QMatMul(q8).forward(xq)
    assert e.value.code == MQ_E_UNSUPPORTED
    q4 = QTensor.quantize(dev, torch.randn((64, 512), device="cuda", generator=g), GgmlDType.Q4_K)
    lib = mold_amd._lib.load()
    res, gate = torch.zeros((2, 64), device="cuda"), torch.zeros(64, device="cuda")
    assert lib.mq_qmatmul_gated_add(dev.handle, q4.handle, xq.data.data_ptr(), mold_amd._lib.MQ_X_Q8K, 2, 512,
                                    res.data_ptr(), 64, None, gate.data_ptr(), None) == MQ_E_UNSUPPORTED
    y = torch.empty((2, 64), device="cuda")
    assert lib.mq_qmatmul(dev.handle, q4.handle, xq.data.data_ptr(), mold_amd._lib.MQ_X_Q8K, 2, 1024,
                          y.data_ptr(), 0, 64, None, 0, None) == MQ_E_INVALID          # ldx != k
    assert lib.mq_quantize_x_q8k(dev.handle, x.data_ptr(), 0, 2, 500, 512, xq.data.data_ptr(), None) == MQ_E_INVALID


@pytest.mark.parametrize("m", [1, 3, 8])
def test_gemv_q4k_exact_on_q8k_grid(dev, torch, m):
    """Activations already on a Q8_K grid: per super-block x = c * q with integer q in
    [-127, 127] and one element at -128 c (the unique element of largest magnitude, so the
    scale -128 / max reproduces c exactly and every q is representable).  Quantization is
    then lossless, so the GEMV's integer dots and its d_w * d_x, dmin_w * d_x combine must
    equal the exact product up to f32 summation (1e-5).  A wrong activation scale (e.g.
    -127 / max), a wrong sub-block sum or a misplaced nibble fails this by orders of
    magnitude; the rounding tie rule is not exercised (no ties)."""
    t, n, k = GgmlDType.Q4_K, 448, 2048
    _say(f"gemv Q4_K exact on the Q8_K grid m={m}")
    blocks = _weights(int(t), n, k, seed=90 + m)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    rng = np.random.default_rng(91 + m)
    q = rng.integers(-127, 128, size=(m, k // 256, 256))
    q[:, :, 17] = -128
    c = np.ldexp(1.0, rng.integers(-12, -4, size=(m, k // 256, 1)))   # powers of two: c * q exact in f32
    x = (q * c).reshape(m, k).astype(np.float32)
    y = QMatMul(qt).forward(torch.from_numpy(x).cuda()).cpu().numpy()
    ref = O.matmul_f64(int(t), x, blocks, n, k)
    assert np.isfinite(y).all()
    assert O.rel_l2(y, ref) <= GEMV_TOL, O.rel_l2(y, ref)


@pytest.mark.parametrize("n,k,m", [(64 * 37, 3072, 1), (64 * 37, 3072, 3), (320, 4096, 2), (200, 2048, 8),
                                   (64 * 300, 8192, 1), (64 * 300, 8192, 2)])
def test_gemv_q4k_odd_tile_counts_repeat_bit_identical(dev, torch, n, k, m):
    """Q4_K GEMV at tile counts that are not a multiple of 8 (uneven spread over XCDs)
    and K up to 8192 (at 19200 x 8192 a workgroup owns 75 rows x 32 super-blocks =
    2400 (row, super-block) pairs: the first 512 issued at once, the next 512 spread
    over the waves once those landed, the rest loaded one by one): repeated calls,
    with another shape in between, are bit-identical and match candle's algorithm."""
    t = GgmlDType.Q4_K
    _say(f"gemv odd tiles n={n} k={k} m={m}")
    blocks = _weights(int(t), n, k, seed=n + m)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    x = np.random.default_rng(k + m).standard_normal((m, k)).astype(np.float32)
    xt = torch.from_numpy(x).cuda()
    mm = QMatMul(qt)
    y1 = mm.forward(xt).clone()
    other = QMatMul(QTensor.from_blocks(dev, t, (128, k), _weights(int(t), 128, k, seed=3)))
    other.forward(xt[:1])
    y2 = mm.forward(xt).clone()
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int32), y2.view(torch.int32))
    _gemv_check(t, x, y1.cpu().numpy(), blocks, n, k)


FRAG_TYPES = [GgmlDType.Q8_0, GgmlDType.Q4_0, GgmlDType.Q4_1, GgmlDType.Q5_0, GgmlDType.Q5_K, GgmlDType.Q6_K,
              GgmlDType.Q2_K, GgmlDType.Q3_K]


@pytest.mark.parametrize("t", FRAG_TYPES, ids=lambda t: t.name)
@pytest.mark.parametrize("m", [1, 2, 3])
def test_gemv_long_k_offset_x(dev, torch, t, m):
    """The f32 GEMV at K = 10240 (x, and at m = 1 its sums over runs of 8, fill
    most of the workgroup's LDS) on x with a common offset, x = 4 + N(0, 1): at
    m = 1 each fragment's dot is a * (u . x) + b * sum(x), and the offset makes
    the b * sum(x) term the large part of every partial.  Held to f64 like every
    other GEMV (1e-5 for these types)."""
    n, k = 96, 10240
    _say(f"gemv long K offset x {t.name} m={m}")
    blocks = _weights(int(t), n, k, seed=17 + m)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    x = (4.0 + np.random.default_rng(300 + m).standard_normal((m, k))).astype(np.float32)
    y = QMatMul(qt).forward(torch.from_numpy(x).cuda()).cpu().numpy()
    _gemv_check(t, x, y, blocks, n, k)


def test_gemv_ksplit_large_k(dev, torch):
    # few row tiles, long K: the launcher splits K across workgroups
    t, n, k, m = GgmlDType.Q4_K, 64, 256 * 48, 4
    _say("gemv k-split")
    blocks = _weights(int(t), n, k, seed=5)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    x = np.random.default_rng(6).standard_normal((m, k)).astype(np.float32)
    y = QMatMul(qt).forward(torch.from_numpy(x).cuda()).cpu().numpy()
    _gemv_check(t, x, y, blocks, n, k)


@pytest.mark.parametrize("t", TYPES, ids=IDS)
def test_tiny_shapes_brute_force(dev, torch, t):
    """Every combination of small shapes: m in {1, 3, 9, 33} (both sides of the
    GEMV / GEMM switch at m = 8), n in {1, 33, 65} (a single row in a padded
    64-row tile, and one row past a tile), and k of one and three blocks plus,
    for the 32-element types, one 256-element unit and a block (K below or off
    the fast kernels' unit: the generic kernels).  Every output finite and
    bit-identical on a repeat.  A single output's relative error says little
    (one dot can be near zero), so for each k the outputs of all (m, n) pairs of
    a path are pooled and held to that path's rel-L2 bar against the f64
    dequantize-then-matmul (GEMV 1e-5 on exact weights, the Q4_K Q8_K GEMV and
    the GEMM 1e-2), and every Q4_K GEMV output also to its Q8_K error bound."""
    bs = O.block_size(int(t))
    ks = [bs, 3 * bs] + ([256 + bs] if bs == 32 else [])
    for k in ks:
        pooled = {"gemv": ([], []), "gemm": ([], [])}
        for n in (1, 33, 65):
            blocks = _weights(int(t), n, k, seed=7 * n + k)
            qt = QTensor.from_blocks(dev, t, (n, k), blocks)
            mm = QMatMul(qt)
            for m in (1, 3, 9, 33):
                _say(f"tiny {t.name} m={m} n={n} k={k}")
                x = np.random.default_rng(m + n + k).standard_normal((m, k)).astype(np.float32)
                xt = torch.from_numpy(x).cuda()
                y = mm.forward(xt)
                y2 = mm.forward(xt)
                torch.cuda.synchronize()
                assert torch.equal(y.view(torch.int32), y2.view(torch.int32)), (m, n, k)
                yn = y.cpu().numpy()
                assert np.isfinite(yn).all(), (m, n, k)
                ref = O.matmul_f64(int(t), x, blocks, n, k)
                path = "gemv" if m <= 8 else "gemm"
                pooled[path][0].append(yn.ravel())
                pooled[path][1].append(ref.ravel())
                if path == "gemv" and int(t) == O.Q4_K:
                    err = np.abs(yn.astype(np.float64) - ref)
                    bound = _q8k_row_bound(x, blocks, int(t), n, k)
                    assert (err <= bound).all(), (m, n, k, float((err / bound).max()))
        for path, (ys, refs) in pooled.items():
            err = O.rel_l2(np.concatenate(ys), np.concatenate(refs))
            tol = GEMV_TOL if path == "gemv" and int(t) != O.Q4_K else GEMM_TOL
            print(f"[case] {t.name} k={k} {path} pooled rel-L2 {err:.2e}", flush=True)
            assert err <= tol, (path, k, err)


# --------------------------------------------------------------------- GEMM

@pytest.mark.parametrize("t", TYPES, ids=IDS)
@pytest.mark.parametrize("mnk", [(9, 64, 256), (300, 200, 512), (513, 320, 768)], ids=str)
def test_gemm_matches_f64_oracle(dev, torch, t, mnk):
    m, n, k = mnk
    _say(f"gemm {t.name} {mnk}")
    blocks = _weights(int(t), n, k, seed=m + n)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    y = QMatMul(qt).forward(torch.from_numpy(x).cuda()).cpu().numpy()
    ref = O.matmul_f64(int(t), x, blocks, n, k)
    err = O.rel_l2(y, ref)
    assert err <= GEMM_TOL, err
    assert np.isfinite(y).all()


@pytest.mark.parametrize("t", TYPES, ids=IDS)
@pytest.mark.parametrize("m", [9, 63, 64, 65, 77, 128, 129, 256, 257, 512, 768, 2048])
def test_gemm_row_tiles_64_128_256(dev, torch, t, m):
    """The fast GEMM's 64-, 128- and 256-row block tiles, chosen by m (64 or 128 up to 128
    rows, 128 up to 256, above that 256, or 128 for a launch of one partial round of
    256-row tiles: few tiles at short K (m = 257, 512, 768 here), or a K split that
    128-row tiles avoid (m = 2048)), at and around each boundary: rel-L2 to f64, rows
    past m untouched (the output is a view into a larger buffer), bf16 output, and the
    gated epilogue; n = 4096 at k = 1024 leaves few tiles, so the partial last round
    also takes the K split."""
    n, k = 4096, 1024
    _say(f"gemm row tiles {t.name} m={m}")
    blocks = _weights(int(t), n, k, seed=3 * m + 1)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    x = np.random.default_rng(m + 7).standard_normal((m, k)).astype(np.float32)
    xt = torch.from_numpy(x).cuda()
    ref = O.matmul_f64(int(t), x, blocks, n, k)
    buf = torch.full((m + 5, n), 7.0, device="cuda")
    y = QMatMul(qt).forward(xt, out=buf[:m])
    torch.cuda.synchronize()
    assert O.rel_l2(y.cpu().numpy(), ref) <= GEMM_TOL
    assert torch.all(buf[m:] == 7.0)
    yb = QMatMul(qt).forward(xt.to(torch.bfloat16), out_dtype=torch.bfloat16).float().cpu().numpy()
    refb = O.matmul_f64(int(t), xt.to(torch.bfloat16).float().cpu().numpy(), blocks, n, k)
    assert O.rel_l2(yb, refb) <= GEMM_TOL
    res = torch.from_numpy(np.random.default_rng(m).standard_normal((m, n)).astype(np.float32)).cuda()
    gate = torch.from_numpy(np.random.default_rng(m + 1).standard_normal(n).astype(np.float32)).cuda()
    want = res.double().cpu().numpy() + gate.double().cpu().numpy() * ref
    mold_amd.Linear(qt).gated_add(xt, gate, res)
    assert O.rel_l2(res.cpu().numpy(), want) <= GEMM_TOL


@pytest.mark.parametrize("t", [GgmlDType.Q4_0, GgmlDType.Q8_0, GgmlDType.Q5_1], ids=lambda t: t.name)
def test_gemm_k_not_multiple_of_64(dev, torch, t):
    # 32-element blocks allow k = 32 * odd: the last K step is half padding
    m, n, k = 100, 96, 32 * 13
    _say(f"gemm ragged k {t.name}")
    blocks = _weights(int(t), n, k, seed=2)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    x = np.random.default_rng(4).standard_normal((m, k)).astype(np.float32)
    for xdt in (torch.float32, torch.bfloat16):
        xt = torch.from_numpy(x).cuda().to(xdt)
        y = QMatMul(qt).forward(xt).float().cpu().numpy()
        ref = O.matmul_f64(int(t), xt.float().cpu().numpy(), blocks, n, k)
        assert O.rel_l2(y, ref) <= GEMM_TOL


def test_gemm_bias_gelu_bf16_and_strides(dev, torch):
    t, m, n, k = GgmlDType.Q4_K, 260, 384, 1024
    _say("gemm bias/gelu/bf16/strides")
    blocks = _weights(int(t), n, k, seed=21)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    rng = np.random.default_rng(22)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal(n) * 0.1).astype(np.float32)
    ref = O.matmul_f64(int(t), x, blocks, n, k) + b
    gelu = 0.5 * ref * (1 + np.tanh(np.sqrt(2 / np.pi) * (ref + 0.044715 * ref ** 3)))
    lin = mold_amd.Linear(qt, torch.from_numpy(b).cuda())
    xw = torch.zeros((m, k + 128), dtype=torch.float32, device="cuda")
    xw[:, :k] = torch.from_numpy(x).cuda()
    y = lin.forward(xw[:, :k], act=mold_amd.ACT_GELU_TANH).cpu().numpy()
    assert O.rel_l2(y, gelu) <= GEMM_TOL
    # bf16 activations read in place (k % 64 == 0, aligned rows), bf16 output
    xb = torch.from_numpy(x).cuda().to(torch.bfloat16)
    yb = lin.forward(xb, out_dtype=torch.bfloat16)
    assert yb.dtype == torch.bfloat16
    ref_b = O.matmul_f64(int(t), xb.float().cpu().numpy(), blocks, n, k) + b
    assert O.rel_l2(yb.float().cpu().numpy(), ref_b) <= GEMM_TOL
    # output with a row stride: write into a slice of a wider buffer
    out = torch.full((m, n + 32), 7.0, dtype=torch.float32, device="cuda")
    ys = lin.matmul.forward(torch.from_numpy(x).cuda(), bias=lin.bias, out=out[:, :n])
    assert O.rel_l2(ys.cpu().numpy(), ref) <= GEMM_TOL
    assert torch.all(out[:, n:] == 7.0)


@pytest.mark.parametrize("m,n,k,tname,xbf16", [(300, 200, 512, "Q4_K", False), (4, 128, 256, "Q8_0", True),
                                                (513, 320, 768, "Q6_K", False), (256, 3072, 3072, "Q2_K", True)])
def test_qmatmul_gated_add(dev, torch, m, n, k, tname, xbf16):
    """mq_qmatmul_gated_add: residual += gate * (x . W^T + bias) in the GEMM epilogue,
    on a strided residual; the update must meet the GEMM bar against the f64 oracle and
    leave the columns past n untouched."""
    t = GgmlDType[tname]
    _say(f"gated add {tname} m={m} n={n} k={k} bf16={xbf16}")
    blocks = _weights(int(t), n, k, seed=m + n)
    lin = mold_amd.Linear(QTensor.from_blocks(dev, t, (n, k), blocks),
                          torch.from_numpy((np.random.default_rng(1).standard_normal(n) * 0.1).astype(np.float32)).cuda())
    rng = np.random.default_rng(m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    xt = torch.from_numpy(x).cuda()
    if xbf16:
        xt = xt.to(torch.bfloat16)
        x = xt.float().cpu().numpy()
    gate = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
    res0 = torch.from_numpy(rng.standard_normal((m, n + 16)).astype(np.float32)).cuda()
    res = res0.clone()
    out = lin.gated_add(xt, gate, res[:, :n])
    torch.cuda.synchronize()
    assert out.data_ptr() == res.data_ptr()
    ref = (O.matmul_f64(int(t), x, blocks, n, k) + lin.bias.cpu().numpy()) * gate.cpu().numpy()
    delta = (res[:, :n] - res0[:, :n]).cpu().numpy()
    assert np.isfinite(delta).all()
    assert O.rel_l2(delta, ref) <= GEMM_TOL
    assert torch.equal(res[:, n:], res0[:, n:])


def test_gemm_and_gemv_deterministic(dev, torch):
    t, n, k = GgmlDType.Q4_K, 512, 1536
    _say("determinism")
    qt = QTensor.from_blocks(dev, t, (n, k), _weights(int(t), n, k, seed=31))
    mm = QMatMul(qt)
    for m in (1, 4, 700):
        x = torch.randn((m, k), generator=torch.Generator().manual_seed(m)).cuda()
        a = mm.forward(x).clone()
        b = mm.forward(x).clone()
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), m


def test_gpu_and_candle_cpu_algorithm_within_bar(dev, torch):
    """candle's CPU QMatMul quantizes x to Q8_0/Q8_1/Q8_K first.  Both the GPU path and the
    oracle's restatement of candle's CPU algorithm must sit inside the 1e-2 envelope of the
    exact f64 product (the pinned bar); their mutual distance is reported."""
    _say("gpu vs candle cpu algorithm")
    m, n, k = 64, 256, 1024
    x = np.random.default_rng(41).standard_normal((m, k)).astype(np.float32)
    for t in TYPES:
        blocks = _weights(int(t), n, k, seed=42)
        qt = QTensor.from_blocks(dev, t, (n, k), blocks)
        y = QMatMul(qt).forward(torch.from_numpy(x).cuda()).cpu().numpy()
        exact = O.matmul_f64(int(t), x, blocks, n, k)
        cand = O.matmul_candle(int(t), x, blocks, n, k)
        assert O.rel_l2(y, exact) <= GEMM_TOL, t.name
        assert O.rel_l2(cand, exact) <= GEMM_TOL, t.name
        print(f"[report] {t.name}: GPU vs candle CPU restatement rel-L2 {O.rel_l2(y, cand):.2e}", flush=True)


# --------------------------------------------------------- errors and edges

def test_errors_are_reported_not_raised_as_crashes(dev, torch):
    _say("error paths")
    lib = mold_amd.load()
    h = ctypes.c_void_p()
    blocks = _weights(int(GgmlDType.Q4_K), 4, 256, seed=1)
    # k not a multiple of the block size
    assert lib.mq_qtensor_upload(dev.handle, int(GgmlDType.Q4_K), 4, 255, blocks.ctypes.data, blocks.nbytes,
                                 ctypes.byref(h)) == mold_amd._lib.MQ_E_INVALID
    # byte count mismatch
    assert lib.mq_qtensor_upload(dev.handle, int(GgmlDType.Q4_K), 4, 256, blocks.ctypes.data, blocks.nbytes - 1,
                                 ctypes.byref(h)) == mold_amd._lib.MQ_E_INVALID
    qt = QTensor.from_blocks(dev, GgmlDType.Q4_K, (4, 256), blocks)
    with pytest.raises(ValueError):
        QMatMul(qt).forward(torch.zeros((3, 128), device="cuda"))
    with pytest.raises(MoldqError):
        QMatMul(qt).forward(torch.zeros((3, 256), device="cuda", dtype=torch.float16))
    # m = 0 is a no-op
    y = QMatMul(qt).forward(torch.zeros((0, 256), device="cuda"))
    assert tuple(y.shape) == (0, 4)


def test_zero_weights_and_single_block(dev, torch):
    _say("zero / single-block weights")
    t, n, k = GgmlDType.Q4_K, 70, 512
    blocks = np.zeros((n, O.row_bytes(int(t), k)), np.uint8)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    x = torch.randn((300, k), generator=torch.Generator().manual_seed(0)).cuda()
    assert torch.count_nonzero(QMatMul(qt).forward(x)) == 0
    assert torch.count_nonzero(QMatMul(qt).forward(x[:2])) == 0
    # one non-zero row: output column equals x . row
    w = np.zeros((n, k), np.float32)
    w[5] = np.random.default_rng(1).standard_normal(k) * 0.02
    blocks = O.quantize(int(t), w)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    y = QMatMul(qt).forward(x).cpu().numpy()
    ref = O.matmul_f64(int(t), x.cpu().numpy(), blocks, n, k)
    assert np.count_nonzero(y[:, np.arange(n) != 5]) == 0
    assert O.rel_l2(y[:, 5], ref[:, 5]) <= GEMM_TOL


def test_gguf_file_to_device(dev, torch, tmp_path):
    _say("gguf load")
    from mold_amd import gguf
    tensors = []
    for i, t in enumerate((GgmlDType.Q4_K, GgmlDType.Q8_0, GgmlDType.Q2_K)):
        n, k = 65 + i, 512
        tensors.append((f"double_blocks.{i}.img_mlp.0.weight", t, (n, k), _weights(int(t), n, k, seed=i)))
    p = str(tmp_path / "w.gguf")
    gguf.write(p, tensors)
    c = gguf.Content.read(p)
    for name, t, (n, k), blocks in tensors:
        qt = c.tensor(name, dev)
        assert qt.dtype() == t and qt.shape == (n, k)
        assert np.array_equal(qt.data(), blocks.reshape(-1))
        assert _bits_equal(qt.dequantize().cpu().numpy(), O.dequantize(int(t), blocks, n, k))
    c.close()


def test_gguf_batched_load_equals_one_by_one(dev, torch, tmp_path):
    """mq_gguf_load_tensors (VarBuilder::from_gguf): every type, sizes from one block
    to several chunks per upload thread (a 37 MB Q4_K), dense tensors between them,
    a tensor named twice, any order; the same bytes as a load of each tensor alone
    and as the file holds.  A bad index fails the whole call and leaves no tensor."""
    _say("gguf batched load")
    from mold_amd import gguf
    from mold_amd._lib import MQ_E_INVALID
    rng = np.random.default_rng(11)
    tensors = [("big", GgmlDType.Q4_K, (21504, 3072), _random_blocks(int(GgmlDType.Q4_K), 21504, 3072, 2))]
    for i, t in enumerate(TYPES):
        n, k = (1, 256) if i % 3 == 0 else (257 + 64 * i, 1024 + 512 * (i % 2))
        tensors.append((f"w{i}", t, (n, k), _random_blocks(int(t), n, k, 20 + i)))
        tensors.append((f"d{i}", GgmlDType.F32, (1, 7 + i), rng.integers(0, 256, 4 * (7 + i), dtype=np.uint8)))
    tensors.append(("bf", GgmlDType.BF16, (3072, 1000), rng.integers(0, 256, 3072 * 2000, dtype=np.uint8)))
    p = str(tmp_path / "many.gguf")
    gguf.write(p, [(nm, t, shape, b) for nm, t, shape, b in tensors])
    c = gguf.Content.read(p)
    try:
        names = [nm for nm, *_ in tensors]
        order = [names[j] for j in rng.permutation(len(names))] + ["w3"]
        got = c.tensors(order, dev)
        assert list(got) == list(dict.fromkeys(order))
        for nm, t, shape, b in tensors:
            qt = got[nm]
            assert qt.dtype() == t and qt.shape == shape, nm
            assert np.array_equal(qt.data(), b.reshape(-1)), nm
            one = c.tensor(nm, dev)
            assert np.array_equal(one.data(), qt.data()), nm
            one.free()
        allt = c.var_builder(dev)
        assert set(allt) == set(names)
        assert np.array_equal(allt["big"].data(), tensors[0][3].reshape(-1))
        del got, allt
        lib = mold_amd._lib.load()
        idx = (ctypes.c_int64 * 3)(0, 1, len(names))
        outs = (ctypes.c_void_p * 3)(1, 2, 3)
        assert lib.mq_gguf_load_tensors(dev.handle, c._h, idx, 3, outs) == MQ_E_INVALID
        assert all(o is None for o in outs)
        assert lib.mq_gguf_load_tensors(dev.handle, c._h, idx, 0, outs) == 0
    finally:
        c.close()


@pytest.mark.parametrize("t", TYPES, ids=IDS)
def test_from_device_blocks_at_any_alignment(dev, torch, t):
    """mq_qtensor_from_device on GGUF blocks that start 0, 1, 2, 6 and 16 bytes into
    a device buffer: the repack reads byte by byte where the start is not 16-byte
    aligned; the tensor equals the host upload's, and downloads its own bytes."""
    n, k = 130, 2 * O.block_size(int(t))
    blocks = _random_blocks(int(t), n, k, 31).reshape(-1)
    ref = QTensor.from_blocks(dev, t, (n, k), blocks)
    buf = torch.zeros(blocks.size + 64, dtype=torch.uint8, device="cuda")
    for shift in (0, 1, 2, 6, 16):
        _say(f"from_device {t.name} shift {shift}")
        buf[shift:shift + blocks.size] = torch.from_numpy(blocks).cuda()
        qt = QTensor.from_device_blocks(dev, t, (n, k), buf[shift:shift + blocks.size])
        torch.cuda.synchronize()
        assert np.array_equal(qt.data(), blocks), shift
        assert _bits_equal(qt.dequantize().cpu().numpy(), ref.dequantize().cpu().numpy()), shift


@pytest.mark.parametrize("t", TYPES + [GgmlDType.F32, GgmlDType.BF16], ids=IDS + ["F32", "BF16"])
def test_concat_rows_is_the_row_concatenation(dev, torch, t):
    """mq_qtensor_concat_rows: the parts' GGUF bytes in order (row counts that end
    inside a 64-row tile and a part below one tile), dequantizing to the stacked
    dequantized parts; parts of another type or k are refused."""
    from mold_amd._lib import MQ_E_INVALID
    bs = O.block_size(int(t)) if int(t) in O.WEIGHT_TYPES else 32
    k = 2 * max(bs, 32)
    rows = [65, 3, 128, 1]
    _say(f"concat_rows {t.name} {rows} x {k}")
    rng = np.random.default_rng(17)
    blocks, parts = [], []
    for i, n in enumerate(rows):
        if int(t) in O.WEIGHT_TYPES:
            b = _random_blocks(int(t), n, k, 40 + i).reshape(-1)
        else:
            b = rng.standard_normal(n * k).astype(np.float32)
            b = (b if t == GgmlDType.F32 else torch.from_numpy(b).to(torch.bfloat16).view(torch.uint8).numpy())
            b = np.ascontiguousarray(b).view(np.uint8).reshape(-1)
        blocks.append(b)
        parts.append(QTensor.from_blocks(dev, t, (n, k), b))
    st = QTensor.concat_rows(dev, parts)
    assert st.dtype() == t and st.shape == (sum(rows), k)
    assert np.array_equal(st.data(), np.concatenate(blocks))
    dq = torch.cat([p.dequantize() for p in parts])
    assert _bits_equal(st.dequantize().cpu().numpy(), dq.cpu().numpy())
    other = GgmlDType.Q8_0 if t != GgmlDType.Q8_0 else GgmlDType.Q4_0
    odd = QTensor.from_blocks(dev, other, (1, k), np.zeros(O.row_bytes(int(other), k), np.uint8))
    with pytest.raises(MoldqError) as e:
        QTensor.concat_rows(dev, [parts[0], odd])
    assert e.value.code == MQ_E_INVALID


@pytest.mark.parametrize("t", [GgmlDType.Q4_K, GgmlDType.Q8_0], ids=lambda t: t.name)
def test_large_host_upload_through_the_pipeline(dev, t):
    """Weights above one pinned chunk go through the threaded upload pipeline:
    byte-identical, including a size that is not a multiple of the chunk."""
    n, k = 20001, 4096
    _say(f"large host upload {t.name} [{n},{k}]")
    blocks = _random_blocks(int(t), n, k, 9)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    assert np.array_equal(qt.data(), blocks.reshape(-1))


def test_arena_residency(torch):
    _say("arena")
    d = mold_amd.Device(0)
    d.reserve_arena(64 << 20)
    ws = []
    for i, t in enumerate(TYPES):
        blocks = _weights(int(t), 128, 512, seed=i)
        ws.append((t, blocks, QTensor.from_blocks(d, t, (128, 512), blocks)))
    for t, blocks, qt in ws:
        assert np.array_equal(qt.data(), blocks.reshape(-1)), t.name
    del ws
    d.close()


# ----------------------------------------------------- BASELINE full shapes

def _sampled_rows_check(dev, torch, t, m, n, k, seed, rows=24):
    blocks = _weights(int(t), n, k, seed=seed)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn((m, k), device="cuda", generator=g)
    mm = QMatMul(qt)
    y = mm.forward(x)
    assert not torch.isnan(y).any().item()
    idx = np.sort(np.random.default_rng(seed).choice(m, size=rows, replace=False))
    idx[-1] = m - 1
    xs = x[torch.from_numpy(idx).cuda()].cpu().numpy()
    ref = O.matmul_f64(int(t), xs, blocks, n, k)
    err = O.rel_l2(y[torch.from_numpy(idx).cuda()].cpu().numpy(), ref)
    assert err <= GEMM_TOL, err
    # linearity: W(x1 + x2) = W x1 + W x2 (within bf16 staging error)
    x2 = torch.randn((m, k), device="cuda", generator=g)
    lin = (mm.forward(x + x2) - y - mm.forward(x2)).norm() / y.norm()
    assert lin.item() <= 2 * GEMM_TOL
    return err


@pytest.mark.parametrize("m,tname,mode", [(2304, "Q4_K", "plain"), (2300, "Q3_K", "gated"),
                                          (2300, "Q2_K", "gelu_bf16")])
def test_gemm_tail_tiles_split_k(dev, torch, m, tname, mode):
    """270 tiles of 256 x 256 on 256 CUs: one full round plus 14 tail tiles, which the GEMM
    splits over K into parts that a second kernel adds in order and passes through the
    epilogue (plain f32, gated residual update, or GELU-tanh to bf16).  Every row of the tail
    (the last 256-row panel, including a partial one) is checked against f64, as are
    sampled rows of the full round; repeated calls are bit-identical."""
    t = GgmlDType[tname]
    n, k = 7680, 1024
    gated = mode == "gated"
    _say(f"gemm tail split-K {tname} m={m} {mode}")
    blocks = _weights(int(t), n, k, seed=m)
    lin = mold_amd.Linear(QTensor.from_blocks(dev, t, (n, k), blocks),
                          torch.from_numpy((np.random.default_rng(2).standard_normal(n) * 0.1).astype(np.float32)).cuda())
    g = torch.Generator(device="cuda").manual_seed(m)
    x = torch.randn((m, k), device="cuda", generator=g)
    if gated:
        gate = torch.randn(n, device="cuda", generator=g)
        res0 = torch.randn((m, n), device="cuda", generator=g)
        outs = [lin.gated_add(x, gate, res0.clone()) for _ in range(2)]
        y = outs[0] - res0
    elif mode == "gelu_bf16":
        outs = [lin.forward(x, act=mold_amd.ACT_GELU_TANH, out_dtype=torch.bfloat16) for _ in range(2)]
        y = outs[0].float()
    else:
        outs = [lin.forward(x) for _ in range(2)]
        y = outs[0]
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    rows = np.concatenate([np.arange(2048, m), np.random.default_rng(m).choice(2048, size=16, replace=False)])
    ref = O.matmul_f64(int(t), x[torch.from_numpy(rows).cuda()].cpu().numpy(), blocks, n, k) + lin.bias.cpu().numpy()
    if gated:
        ref = ref * gate.cpu().numpy()
    if mode == "gelu_bf16":
        ref = 0.5 * ref * (1 + np.tanh(np.sqrt(2 / np.pi) * (ref + 0.044715 * ref ** 3)))
    got = y[torch.from_numpy(rows).cuda()].cpu().numpy()
    assert np.isfinite(got).all()
    assert O.rel_l2(got, ref) <= GEMM_TOL


@pytest.mark.parametrize("m,n,k,tname,out_bf16", [
    (600, 1024, 512, "Q4_K", True),    # 256 x 256 tiles
    (2304, 7680, 1024, "Q2_K", False), # a full round plus tail tiles split over K
    (77, 1024, 1024, "Q8_0", True),    # small-m tiles with the tail split
    (1, 768, 512, "Q4_K", False),      # Q4_K GEMV
    (3, 640, 512, "Q6_K", True),       # frag GEMV
    (6, 640, 512, "Q3_K", False),      # generic GEMV
    (300, 200, 96, "Q4_0", True),      # generic GEMM (k not a whole unit), edge tiles
])
def test_qmatmul_act_from_splits_the_epilogue(dev, torch, m, n, k, tname, out_bf16):
    """mq_qmatmul_act_from: output columns before act_col0 equal mq_qmatmul without the
    activation, columns from act_col0 on equal mq_qmatmul with GELU, bit for bit, on the GEMM
    (whole tiles, tail split, small-m tiles), the generic GEMM and every GEMV kernel; act_col0
    at a tile boundary, inside a wave's 32 columns, and at 0 and n."""
    t = GgmlDType[tname]
    _say(f"act_from {tname} m={m} n={n} k={k} bf16={out_bf16}")
    blocks = _weights(int(t), n, k, seed=n + m)
    b = torch.from_numpy((np.random.default_rng(5).standard_normal(n) * 0.1).astype(np.float32)).cuda()
    mm = mold_amd.QMatMul(QTensor.from_blocks(dev, t, (n, k), blocks))
    x = torch.randn((m, k), device="cuda", generator=torch.Generator(device="cuda").manual_seed(m))
    od = torch.bfloat16 if out_bf16 else torch.float32
    plain = mm.forward(x, bias=b, out_dtype=od)
    gelu = mm.forward(x, bias=b, act=mold_amd.ACT_GELU_TANH, out_dtype=od)
    for c0 in sorted({min(256, n), 100, 0, n}):
        y = mm.forward(x, bias=b, act=mold_amd.ACT_GELU_TANH, out_dtype=od, act_from=c0)
        torch.cuda.synchronize()
        assert torch.equal(y[:, :c0], plain[:, :c0]), c0
        assert torch.equal(y[:, c0:], gelu[:, c0:]), c0
    lib = mold_amd.load()
    y = torch.empty((m, n), device="cuda")
    rc = lib.mq_qmatmul_act_from(dev.handle, mm.w.handle, x.data_ptr(), 0, m, k, y.data_ptr(), 0, n, None, 1, n + 1,
                                 None)
    assert rc == -1 and b"act_col0" in lib.mq_last_error()


def test_full_flux_single_block_linear1_q4k(dev, torch):
    _say("full shape Q4_K 4608x3072->21504")
    _sampled_rows_check(dev, torch, GgmlDType.Q4_K, 4608, 21504, 3072, seed=4)


def test_full_config1_q8_0_out_proj(dev, torch):
    _say("full shape Q8_0 4608x3072->3072")
    _sampled_rows_check(dev, torch, GgmlDType.Q8_0, 4608, 3072, 3072, seed=1)


@pytest.mark.parametrize("t", [GgmlDType.Q4_K, GgmlDType.Q4_0, GgmlDType.Q6_K], ids=lambda t: t.name)
def test_full_config3_mlp_fc2(dev, torch, t):
    _say(f"full shape {t.name} 4608x12288->3072")
    _sampled_rows_check(dev, torch, t, 4608, 3072, 12288, seed=3)


@pytest.mark.parametrize("n", [18432, 9216])
@pytest.mark.parametrize("m", [1, 2, 4])
def test_full_config2_modulation_gemv(dev, torch, n, m):
    _say(f"full shape Q4_K GEMV m={m} 3072->{n}")
    t, k = GgmlDType.Q4_K, 3072
    blocks = _weights(int(t), n, k, seed=2)
    qt = QTensor.from_blocks(dev, t, (n, k), blocks)
    x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    y = QMatMul(qt).forward(torch.from_numpy(x).cuda()).cpu().numpy()
    _gemv_check(t, x, y, blocks, n, k)


@pytest.mark.parametrize("t", [GgmlDType.Q4_K, GgmlDType.Q8_0], ids=lambda t: t.name)
@pytest.mark.parametrize("m", [1, 2])
def test_stacked_linear_matches_separate_linears(dev, torch, t, m):
    """A step's modulation linears stacked by rows (FLUX's double-block, single-block
    and final-layer shapes): every part's columns of the one stacked GEMV equal
    that part's own forward bit for bit, including when the stack is long enough
    for a workgroup to hold more than two (row, super-block) pairs per thread."""
    from mold_amd.quantized import Linear, StackedLinear
    _say(f"stacked modulation GEMV {t.name} m={m}")
    k = 3072
    g = torch.Generator(device="cuda").manual_seed(31)
    parts = []
    for i, n in enumerate((18432, 18432, 9216, 6144)):
        w = torch.randn((n, k), device="cuda", generator=g) * 0.02
        bias = torch.randn((n,), device="cuda", generator=g) * 0.02 if i != 2 else None
        parts.append((f"part{i}", Linear(QTensor.quantize(dev, w, t), bias)))
        del w
    stack = StackedLinear(dev, parts)
    assert stack.linear.matmul.w.shape == (52224, k)
    x = torch.randn((m, k), device="cuda", generator=g)
    ys = stack.forward(x)
    for name, lin in parts:
        ref = lin.forward(x)
        assert torch.equal(ys[name], ref), name
    # one part anchored to the f64 product (bias-free part)
    qt = parts[2][1].matmul.w
    n2 = qt.shape[0]
    _gemv_check(t, x.cpu().numpy(), ys["part2"].cpu().numpy(), qt.data(), n2, k)
    with pytest.raises(ValueError):
        StackedLinear(dev, [parts[0], ("other_k", Linear(QTensor.quantize(
            dev, torch.zeros((64, 256), device="cuda"), t)))])


# ------------------------------------------------------------- quantizer

def _quant_inputs(k, seed):
    rng = np.random.default_rng(seed)
    rows = [
        rng.standard_normal(k) * 0.02,                      # BASELINE weight law
        rng.standard_normal(k),
        np.zeros(k),                                        # all-zero blocks
        np.full(k, 0.37),                                   # constant (max == min)
        np.where(rng.random(k) < 0.1, rng.standard_normal(k) * 50, rng.standard_normal(k) * 1e-3),  # outliers
        rng.standard_normal(k) * 1e-20,                     # below GROUP_MAX_EPS
        np.abs(rng.standard_normal(k)),                     # one-signed (min > 0)
        -np.abs(rng.standard_normal(k)) * 3,
    ]
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("t", TYPES, ids=IDS)
def test_gpu_quantizer_byte_identical_to_reference(dev, torch, t):
    _say(f"quantize {t.name}")
    k = 512
    x = _quant_inputs(k, seed=int(t))
    xt = torch.from_numpy(x).cuda()
    qt = QTensor.quantize(dev, xt, t)
    got = qt.data().reshape(x.shape[0], -1)
    ref = O.quantize(int(t), x)
    bad = [i for i in range(x.shape[0]) if not np.array_equal(got[i], ref[i])]
    assert not bad, f"rows differ: {bad}"
    # strided source (row stride > k) gives the same blocks
    wide = torch.zeros((x.shape[0], k + 64), device="cuda")
    wide[:, :k] = xt
    qs = QTensor.quantize(dev, wide[:, :k], t)
    assert np.array_equal(qs.data(), ref.reshape(-1))
