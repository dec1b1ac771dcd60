"""ctypes front-end of the C oracle (``oracle/ggml_oracle.c``).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker or the reported CPU baseline.  The product (``mold_amd``) never imports
it and fails loudly when its own HIP library is missing.

The restated algorithms (ggml block formats and reference quantizers, candle's
CPU QMatMul) and the reference call sites they stand for are listed in the
header of ``ggml_oracle.c``.

Pins of every function here (tests/test_oracle.py unless noted):
  block_size / type_size ..... ggml's type table and the reference's GGUF file sizes
  quantize ................... known-answer rows (legacy types), byte identity with
                               oracle/np_quant.py, exact round trips on each grid
  dequantize ................. known-answer blocks, oracle/np_dequant.py, the
                               once-rounded exact value
  quantize_act ............... known-answer rows, byte identity with np_quant
  vec_dot .................... the exact product to f32 rounding
  matmul_candle .............. quantized rows x vec_dot, bit for bit; 1e-2 of f64
  matmul_f64 ................. numpy float64 BLAS, linearity, zero blocks
  e4m3_to_f32 ................ every byte against torch.float8_e4m3fn
                               (tests/test_gguf_format.py)
  lora_apply ................. exact cases and an f64 bound (tests/test_lora.py)
Parity unpinned: candle's own Q8_K / Q8_1 rounding convention (``quantize_act``
follows the stated one; no assertion on the GPU depends on it).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

# ggml type ids (GGML_TYPE_*), identical to GGUF's tensor type ids.
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1 = 0, 1, 2, 3, 6, 7, 8, 9
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K, BF16 = 10, 11, 12, 13, 14, 15, 30

NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q4_1: "Q4_1", Q5_0: "Q5_0", Q5_1: "Q5_1",
         Q8_0: "Q8_0", Q8_1: "Q8_1", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K",
         Q5_K: "Q5_K", Q6_K: "Q6_K", Q8_K: "Q8_K", BF16: "BF16"}
BY_NAME = {v: k for k, v in NAMES.items()}
WEIGHT_TYPES = [Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K]

_lib = None


def build() -> str:
    """Compile liboracle.so with the committed Makefile (gcc, no GPU)."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run `make -C oracle`)")
        _lib = _bind(ctypes.CDLL(_LIB_PATH))
    return _lib


def _bind(L: ctypes.CDLL) -> ctypes.CDLL:
    """Declare the C signatures on a loaded oracle library."""
    vp, i64, c_int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    L.orc_fp32_to_fp16.restype = ctypes.c_uint16
    L.orc_fp32_to_fp16.argtypes = [ctypes.c_float]
    L.orc_fp16_to_fp32.restype = ctypes.c_float
    L.orc_fp16_to_fp32.argtypes = [ctypes.c_uint16]
    L.orc_fp32_to_bf16.restype = ctypes.c_uint16
    L.orc_fp32_to_bf16.argtypes = [ctypes.c_float]
    L.orc_block_size.restype = c_int
    L.orc_block_size.argtypes = [c_int]
    L.orc_type_size.restype = c_int
    L.orc_type_size.argtypes = [c_int]
    L.orc_dequantize_row.restype = c_int
    L.orc_dequantize_row.argtypes = [c_int, vp, vp, i64]
    L.orc_quantize_row.restype = c_int
    L.orc_quantize_row.argtypes = [c_int, vp, vp, i64]
    for nm in ("orc_quantize_row_q8_0", "orc_quantize_row_q8_1", "orc_quantize_row_q8_K"):
        getattr(L, nm).restype = None
        getattr(L, nm).argtypes = [vp, vp, i64]
    L.orc_vec_dot_type.restype = c_int
    L.orc_vec_dot_type.argtypes = [c_int]
    L.orc_vec_dot.restype = ctypes.c_float
    L.orc_vec_dot.argtypes = [c_int, i64, vp, vp]
    L.orc_matmul_candle.restype = c_int
    L.orc_matmul_candle.argtypes = [c_int, i64, i64, i64, vp, vp, vp, c_int]
    L.orc_matmul_f64.restype = c_int
    L.orc_matmul_f64.argtypes = [c_int, i64, i64, i64, vp, vp, vp]
    L.orc_lora_apply.restype = None
    L.orc_lora_apply.argtypes = [vp, i64, i64, i64, vp, i64, vp, i64, c_int, ctypes.c_float]
    return L


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def block_size(t: int) -> int:
    return lib().orc_block_size(t)


def type_size(t: int) -> int:
    return lib().orc_type_size(t)


def row_bytes(t: int, k: int) -> int:
    bs = block_size(t)
    assert k % bs == 0, (t, k)
    return k // bs * type_size(t)


def quantize(t: int, x: np.ndarray) -> np.ndarray:
    """ggml reference quantizer: f32 [n, k] -> uint8 [n, row_bytes]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    n, k = x.shape
    out = np.zeros((n, row_bytes(t, k)), dtype=np.uint8)
    rc = lib().orc_quantize_row(t, _ptr(x), _ptr(out), n * k)
    if rc != 0:
        raise ValueError(f"quantize failed for type {t}")
    return out


def dequantize(t: int, blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    """Closed-form ggml dequantize: blocks -> f32 [n, k]."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    assert blocks.size == n * row_bytes(t, k)
    out = np.empty((n, k), dtype=np.float32)
    rc = lib().orc_dequantize_row(t, _ptr(blocks), _ptr(out), n * k)
    if rc != 0:
        raise ValueError(f"dequantize failed for type {t}")
    return out


def quantize_act(t: int, x: np.ndarray) -> np.ndarray:
    """Activation quantizer that candle's CPU vec_dot uses for weight type t."""
    vdt = lib().orc_vec_dot_type(t)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.zeros(row_bytes(vdt, x.size), dtype=np.uint8)
    fn = {Q8_0: lib().orc_quantize_row_q8_0, Q8_1: lib().orc_quantize_row_q8_1,
          Q8_K: lib().orc_quantize_row_q8_K}[vdt]
    fn(_ptr(x), _ptr(out), x.size)
    return out


def vec_dot(t: int, k: int, w_row: np.ndarray, act_row: np.ndarray) -> float:
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    act_row = np.ascontiguousarray(act_row, dtype=np.uint8)
    return float(lib().orc_vec_dot(t, k, _ptr(w_row), _ptr(act_row)))


def matmul_candle(t: int, x: np.ndarray, w_blocks: np.ndarray, n: int, k: int, nthreads: int = 0) -> np.ndarray:
    """candle CPU QMatMul: quantized activations x integer block dots."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.shape[0]
    assert x.shape == (m, k)
    w_blocks = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    y = np.empty((m, n), dtype=np.float32)
    rc = lib().orc_matmul_candle(t, m, n, k, _ptr(x), _ptr(w_blocks), _ptr(y), nthreads)
    if rc != 0:
        raise ValueError(f"matmul_candle failed rc={rc}")
    return y


def matmul_f64(t: int, x: np.ndarray, w_blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    """f64-accumulated x . dequant(W)^T, dequant bit-exact in f32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.shape[0]
    assert x.shape == (m, k)
    w_blocks = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    y = np.empty((m, n), dtype=np.float64)
    rc = lib().orc_matmul_f64(t, m, n, k, _ptr(x), _ptr(w_blocks), _ptr(y))
    if rc != 0:
        raise ValueError(f"matmul_f64 failed rc={rc}")
    return y


def rel_l2(a: np.ndarray, ref: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref.ravel())
    return float(np.linalg.norm((a - ref).ravel()) / (den if den > 0 else 1.0))


def e4m3_to_f32(b: np.ndarray) -> np.ndarray:
    """FP8 E4M3 ("fn": bias 7, no infinities, S.1111.111 NaN) bytes -> f32,
    exact (the OCP 8-bit float spec; safetensors F8_E4M3).  Normal:
    (-1)^s 2^(e-7) (1 + m/8); subnormal (e = 0): (-1)^s 2^-6 m/8."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int64)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    out = (s * mag).astype(np.float32)
    out[(e == 0xF) & (m == 7)] = np.nan
    return out


def lora_apply(w: np.ndarray, b: np.ndarray, a: np.ndarray, scale: float) -> np.ndarray:
    """w + (b . a) * scale in the device kernel's order (see orc_lora_apply);
    w [rows, k], b [rows, rank], a [rank, k], all f32.  Returns a new array."""
    w = np.array(w, dtype=np.float32, order="C", copy=True)
    b = np.ascontiguousarray(b, dtype=np.float32)
    a = np.ascontiguousarray(a, dtype=np.float32)
    rows, k = w.shape
    rank = b.shape[1]
    assert b.shape == (rows, rank) and a.shape == (rank, k)
    lib().orc_lora_apply(_ptr(w), k, rows, k, _ptr(b), rank, _ptr(a), k, rank, float(scale))
    return w
