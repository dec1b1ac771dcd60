"""Writes tests/golden/golden.npz: small fixed vectors of the quantized-linear path.

Per weight type (Q4_0 .. Q6_K): a seeded N(0, 0.02^2) weight [4, 512] quantized by
the oracle's restatement of ggml's reference quantizers (the GGUF blocks), the
bit-exact f32 dequantization of those blocks, and x [3, 512] with y = x . W^T
computed in f64 on the dequantized weight.  Plus one Q4_K GEMV case whose x lies on
a Q8_K grid (lossless activation quantization).

These are regression pins for the oracle and the GPU path: the blocks are inputs,
the dequantized values and products are expected outputs.  The reference holds no
golden vector for any quantized type, so the expected values come from the
restatements pinned in tests/test_oracle.py (closed forms, known-answer blocks, a
second numpy restatement).  Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402


def main():
    out = {}
    k, n, m = 512, 4, 3
    for t in O.WEIGHT_TYPES:
        rng = np.random.default_rng(1000 + t)
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        blocks = O.quantize(t, w)
        x = rng.standard_normal((m, k)).astype(np.float32)
        name = O.NAMES[t]
        out[f"{name}_w"] = w
        out[f"{name}_blocks"] = blocks
        out[f"{name}_deq"] = O.dequantize(t, blocks, n, k)
        out[f"{name}_x"] = x
        out[f"{name}_y"] = O.matmul_f64(t, x, blocks, n, k)
    # Q4_K GEMV on a Q8_K grid: x = c * q, integer q in [-127, 127], one -128 per
    # super-block, c a power of two
    rng = np.random.default_rng(77)
    kk, nn = 1024, 64
    w = (rng.standard_normal((nn, kk)) * 0.02).astype(np.float32)
    blocks = O.quantize(O.Q4_K, w)
    q = rng.integers(-127, 128, size=(2, kk // 256, 256))
    q[:, :, 5] = -128
    c = np.ldexp(1.0, rng.integers(-10, -5, size=(2, kk // 256, 1)))
    x = (q * c).reshape(2, kk).astype(np.float32)
    out["grid_blocks"] = blocks
    out["grid_x"] = x
    out["grid_y"] = O.matmul_f64(O.Q4_K, x, blocks, nn, kk)
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **out)
    print(f"wrote {len(out)} arrays to {os.path.join(HERE, 'golden.npz')}")


if __name__ == "__main__":
    main()
