"""Per-stream workspaces of the quantized matmul, on the GPU through the C ABI.

* Two streams run f32-input GEMMs concurrently (both stage their activations
  as bf16 in their own stream's workspace): each result is bit-identical to
  the same call run alone on the null stream.
* A stream's workspace grows while earlier work on that stream is still
  queued (no synchronization in between): the earlier result is unchanged.
* A HIP graph captured after the workspace is sized replays bit-identically to
  the eager call, with eager work and synchronizations between replays; a call
  that would have to grow a capturing stream's workspace is refused with a
  clear error instead of allocating.
* A stream with the tail K split turned off runs a partial-round GEMM unsplit
  (same values up to the K summation order) and split again once turned on.
* A GGUF file is loaded through the pinned, double-buffered upload (tensors
  larger than one 16 MiB chunk) and reads back byte-identical.
"""
import sys

import numpy as np
import pytest

import mold_amd
from mold_amd import GgmlDType, QMatMul, QTensor
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as _t
    return _t


def _qt(dev, tname, n, k, seed):
    w = (np.random.default_rng(seed).standard_normal((n, k)) * 0.02).astype(np.float32)
    t = GgmlDType[tname]
    return QTensor.from_blocks(dev, t, (n, k), O.quantize(int(t), w))


def test_two_streams_f32_input_gemms(torch):
    dev = mold_amd.Device(0)
    _say("two streams: Q4_K m=1000 k=3072 n=3072 and Q6_K m=2300 k=3072 n=1536, f32 x")
    wa, wb = QMatMul(_qt(dev, "Q4_K", 3072, 3072, 1)), QMatMul(_qt(dev, "Q6_K", 1536, 3072, 2))
    g = torch.Generator(device="cuda").manual_seed(3)
    xa = torch.randn((1000, 3072), device="cuda", generator=g)
    xb = torch.randn((2300, 3072), device="cuda", generator=g)
    ref_a, ref_b = wa.forward(xa), wb.forward(xb)          # null-stream (current) results
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for rep in range(3):
        with torch.cuda.stream(s1):
            ya = wa.forward(xa)
        with torch.cuda.stream(s2):
            yb = wb.forward(xb)
        with torch.cuda.stream(s1):
            ya2 = wa.forward(xa)
        outs.append((ya, yb, ya2))
    torch.cuda.synchronize()
    for ya, yb, ya2 in outs:
        assert torch.equal(ya.view(torch.int32), ref_a.view(torch.int32))
        assert torch.equal(ya2.view(torch.int32), ref_a.view(torch.int32))
        assert torch.equal(yb.view(torch.int32), ref_b.view(torch.int32))
    rows = np.array([0, 517, 999])
    blocks = wa.w.data()
    ref = O.matmul_f64(int(GgmlDType.Q4_K), xa[torch.from_numpy(rows).cuda()].cpu().numpy(), blocks, 3072, 3072)
    assert O.rel_l2(ref_a[torch.from_numpy(rows).cuda()].cpu().numpy(), ref) <= 1e-2


def test_stream_without_tail_split(torch):
    """mq_ctx_set_stream_tail_split: a GEMM whose last round of tiles is partial
    (m=512: 2 x 24 tiles, split 8 ways by default) runs unsplit on a stream with
    the split turned off, with the same values up to the order of the K sum, and
    split again once it is turned back on (bit-identical to the default)."""
    dev = mold_amd.Device(0)
    _say("tail split off on one stream: Q4_K m=512 k=3072 n=3072, bf16 x")
    w = QMatMul(_qt(dev, "Q4_K", 3072, 3072, 4))
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn((512, 3072), device="cuda", generator=g).to(torch.bfloat16)
    ref = w.forward(x, out_dtype=torch.float32)          # current stream: split
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    dev.set_stream_tail_split(s, False)
    with torch.cuda.stream(s):
        y_off = w.forward(x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    dev.set_stream_tail_split(s, True)
    with torch.cuda.stream(s):
        y_on = w.forward(x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y_on.view(torch.int32), ref.view(torch.int32))
    assert not torch.equal(y_off.view(torch.int32), ref.view(torch.int32)), "the split setting had no effect"
    assert torch.allclose(y_off, ref, rtol=1e-5, atol=1e-5)
    rows = np.array([0, 255, 511])
    ri = torch.from_numpy(rows).cuda()
    exact = O.matmul_f64(int(GgmlDType.Q4_K), x[ri].float().cpu().numpy(), w.w.data(), 3072, 3072)
    assert O.rel_l2(y_off[ri].cpu().numpy(), exact) <= 1e-2
    # the gated residual update (the blocks' out-projections) on the unsplit stream
    lin = mold_amd.Linear(w.w, torch.randn(3072, device="cuda", generator=g) * 0.02)
    gate = torch.randn(3072, device="cuda", generator=g)
    res0 = torch.randn((512, 3072), device="cuda", generator=g)
    r_split, r_off = res0.clone(), res0.clone()
    lin.gated_add(x, gate, r_split)
    torch.cuda.synchronize()
    dev.set_stream_tail_split(s, False)
    with torch.cuda.stream(s):
        lin.gated_add(x, gate, r_off)
    torch.cuda.synchronize()
    assert torch.allclose(r_off, r_split, rtol=1e-5, atol=1e-5)
    assert torch.allclose(r_off - res0, gate * (ref + lin.bias), rtol=1e-3, atol=1e-4)


def test_workspace_growth_keeps_queued_work(torch):
    dev = mold_amd.Device(0)
    _say("workspace growth behind queued work: Q4_K k=4096 n=2048, m=300 then m=5000, f32 x")
    w = QMatMul(_qt(dev, "Q4_K", 2048, 4096, 4))
    g = torch.Generator(device="cuda").manual_seed(5)
    x_small = torch.randn((300, 4096), device="cuda", generator=g)
    x_big = torch.randn((5000, 4096), device="cuda", generator=g)
    ref_small = w.forward(x_small)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    dev2 = mold_amd.Device(0)                                 # a context whose workspaces start empty
    w2 = QMatMul(QTensor.from_blocks(dev2, GgmlDType.Q4_K, (2048, 4096), w.w.data()))
    with torch.cuda.stream(s):
        y_small = w2.forward(x_small)                         # sizes the workspace for m=300
        y_big = w2.forward(x_big)                             # grows it while y_small may still run
        y_small2 = w2.forward(x_small)
    torch.cuda.synchronize()
    assert torch.equal(y_small.view(torch.int32), ref_small.view(torch.int32))
    assert torch.equal(y_small2.view(torch.int32), ref_small.view(torch.int32))
    assert torch.equal(y_big.view(torch.int32), w.forward(x_big).view(torch.int32))


def test_graph_replay_matches_eager(torch):
    dev = mold_amd.Device(0)
    _say("graph capture: Q4_K k=3072 n=3072 m=700 f32 x (staged) + GEMV m=1")
    w = QMatMul(_qt(dev, "Q4_K", 3072, 3072, 6))
    wv = QMatMul(_qt(dev, "Q6_K", 3072, 3072, 7))
    g = torch.Generator(device="cuda").manual_seed(8)
    x = torch.randn((700, 3072), device="cuda", generator=g)
    xv = torch.randn((1, 3072), device="cuda", generator=g)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        eager = w.forward(x)
        eager_v = wv.forward(xv)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    y = torch.empty_like(eager)
    yv = torch.empty_like(eager_v)
    with torch.cuda.graph(graph, stream=s):
        w.forward(x, out=y)
        wv.forward(xv, out=yv)
    for rep in range(4):
        y.zero_()
        yv.zero_()
        z = w.forward(x)                                      # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), eager.view(torch.int32)), rep
        assert torch.equal(yv.view(torch.int32), eager_v.view(torch.int32)), rep
        assert torch.equal(z.view(torch.int32), eager.view(torch.int32)), rep


def test_capture_refuses_workspace_growth(torch):
    dev = mold_amd.Device(0)
    _say("capture without a sized workspace is refused")
    w = QMatMul(_qt(dev, "Q4_K", 1024, 2048, 9))
    x = torch.randn((600, 2048), device="cuda")
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(mold_amd._lib.MoldqError, match="being captured"):
        with torch.cuda.graph(graph, stream=s):
            w.forward(x)
    torch.cuda.synchronize()
    # after reserving the stream's workspace the same capture works
    need = w.workspace_bytes(600, torch.float32)
    assert need >= 600 * 2048 * 2
    dev.reserve_stream_scratch(need, stream=s)
    y = torch.empty((600, 1024), device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        w.forward(x, out=y)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), w.forward(x).view(torch.int32))


def test_gguf_pinned_upload_multi_chunk(torch, tmp_path):
    """Tensors of 1.1, 2.6 and 0.01 upload chunks through the double-buffered file upload."""
    from mold_amd import gguf
    dev = mold_amd.Device(0)
    specs = [("a", "Q4_K", 4096, 7424), ("b", "Q8_0", 9216, 4864), ("c", "Q6_K", 64, 4096)]
    tensors = []
    for i, (name, tname, n, k) in enumerate(specs):
        t = GgmlDType[tname]
        nbytes = n * O.row_bytes(int(t), k)
        tensors.append((name, t, (n, k), np.random.default_rng(20 + i).integers(0, 256, nbytes, dtype=np.uint8)))
    p = str(tmp_path / "w.gguf")
    gguf.write(p, tensors)
    _say(f"gguf pinned upload, {sum(r.nbytes for *_, r in tensors) / 2**20:.1f} MiB")
    c = gguf.Content.read(p)
    for name, t, (n, k), raw in tensors:
        qt = c.tensor(name, dev)
        assert qt.dtype() == t and qt.shape == (n, k)
        assert np.array_equal(qt.data(), raw), name
    c.close()
