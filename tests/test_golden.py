"""Golden vectors of the quantized-linear path (tests/golden/golden.npz, written by
tests/golden/make_golden.py).

CPU: the oracle reproduces every fixture (quantizer bytes, bit-exact dequantization,
the f64 product), so a change to a restatement shows up as a failed pin.
GPU (marked `gpu`): libmoldq, through the C ABI, dequantizes the fixture blocks bit for
bit, meets the 1e-2 bar on the fixture products, and reproduces the Q8_K-grid GEMV to
f32 precision.
"""
import os

import numpy as np
import pytest

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "golden.npz"))   # arrays only (allow_pickle=False)
K, N = 512, 4


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("t", O.WEIGHT_TYPES, ids=[O.NAMES[t] for t in O.WEIGHT_TYPES])
def test_oracle_reproduces_golden(t):
    nm = O.NAMES[t]
    blocks = G[f"{nm}_blocks"]
    assert np.array_equal(O.quantize(t, G[f"{nm}_w"]), blocks)
    assert np.array_equal(_bits(O.dequantize(t, blocks, N, K)), _bits(G[f"{nm}_deq"]))
    assert np.array_equal(O.matmul_f64(t, G[f"{nm}_x"], blocks, N, K), G[f"{nm}_y"])


def test_oracle_reproduces_grid_case():
    y = O.matmul_f64(O.Q4_K, G["grid_x"], G["grid_blocks"], 64, 1024)
    assert np.array_equal(y, G["grid_y"])


@pytest.mark.gpu
@pytest.mark.parametrize("t", O.WEIGHT_TYPES, ids=[O.NAMES[t] for t in O.WEIGHT_TYPES])
def test_gpu_matches_golden(t):
    import torch
    import mold_amd
    from mold_amd import GgmlDType, QMatMul, QTensor
    nm = O.NAMES[t]
    dev = mold_amd.Device(0)
    qt = QTensor.from_blocks(dev, GgmlDType(t), (N, K), G[f"{nm}_blocks"])
    assert np.array_equal(_bits(qt.dequantize().cpu().numpy()), _bits(G[f"{nm}_deq"]))
    x = torch.from_numpy(G[f"{nm}_x"]).cuda()
    y = QMatMul(qt).forward(x).cpu().numpy()                          # m = 3: the GEMV
    assert O.rel_l2(y, G[f"{nm}_y"]) <= 1e-2
    xs = torch.cat([x] * 100)                                         # m = 300: the GEMM
    ys = QMatMul(qt).forward(xs).cpu().numpy()
    assert O.rel_l2(ys, np.concatenate([G[f"{nm}_y"]] * 100)) <= 1e-2


@pytest.mark.gpu
def test_gpu_matches_golden_grid_gemv():
    import torch
    import mold_amd
    from mold_amd import GgmlDType, QMatMul, QTensor
    dev = mold_amd.Device(0)
    qt = QTensor.from_blocks(dev, GgmlDType.Q4_K, (64, 1024), G["grid_blocks"])
    y = QMatMul(qt).forward(torch.from_numpy(G["grid_x"]).cuda()).cpu().numpy()
    assert O.rel_l2(y, G["grid_y"]) <= 1e-5
