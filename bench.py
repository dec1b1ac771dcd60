"""Benchmark of the GGUF quantized-linear hot path on one MI355X.

Headline (the `value`): the fused dequant -> bf16-MFMA GEMM of a Q4_K weight
at FLUX single-block linear1 shape, x [4608, 3072] . W[21504, 3072]^T ->
y f32 [4608, 21504] (the shape the north star's
>= 50 % of bf16 MFMA peak target names).  x is bf16 and resident in HBM: that
is what the FLUX step feeds linear1 (its adaLN modulation writes bf16).  One
step = one QMatMul::forward call = exactly one GEMM kernel launch, so the
HIP-event time over the timed launches (roofline.kernel_ms, on the launch
stream) is that kernel's average duration, and ms_per_step is the host wall
clock around the same launches.  `value` = 2*M*N*K / ms_per_step in TFLOP/s.
Before the W warmup steps the GEMM runs for one second untimed, so that the
timed steps see the chip's steady, power-limited clock rather than its ramp.

Also on the same JSON line:
  * "roofline": that kernel against the 2.5 PFLOP/s dense bf16 MFMA peak;
    `traffic` (HBM bytes per launch) comes from the committed counter summary
    profiles/gemm_q4k_linear1_traffic.md only when the kernel sources' digest
    recorded there matches the sources of this build (else null);
  * "f32_input": the same call with f32 x (candle's QMatMul input dtype):
    staging to bf16 plus the GEMM;
  * "config1_q8_0": BASELINE config 1, the Q8_0 3072x3072 out-projection at
    M=4608 with f32 x and y;
  * "config3_mlp": BASELINE config 3, the MLP chain fc1 (3072->12288, GELU-tanh
    epilogue, bf16 out) then fc2 (12288->3072, f32 out) on f32 x [4608, 3072],
    for Q4_K, Q4_0 and Q6_K weights;
  * "flux_single_block": FLUX's single-block linear1 and linear2 as the step runs
    them: linear1 with bf16 output and GELU on its MLP columns only
    (mq_qmatmul_act_from), linear2 as the gated residual update reading
    linear1's output columns 6144.. in place (row stride 21504);
  * "tp8_shards": one GPU's share of FLUX's linear1 (column split, N/8) and linear2
    (row split, largest whole-super-block share, gated) under 8-way tensor
    parallelism, at the real shapes (no collective is run);
  * "dequant": QTensor::dequantize of a Q4_K 18432x3072 weight to f32 and to
    bf16, in GB/s of algorithmic bytes (GGUF blocks read + dense out written);
  * "gemv": the skinny-M Q4_K modulation GEMVs (config 2, M in {1, 2, 4},
    N in {18432, 9216}), rotating through > 256 MB of distinct weight copies
    so reads miss the Infinity Cache, in GB/s of algorithmic bytes against
    the 8 TB/s HBM peak.  The rotation is captured once in a HIP graph and
    replayed, so the figure is the kernels' own rate, not Python's launch
    rate.  Beside it, "read_ceiling": the fastest of three single-launch
    streaming-read shapes over the same weight bytes (libmoldq_probe.so),
    cold, in the same run;
  * "dense_bf16_ceiling": torch's bf16 linear (hipBLASLt) at the headline shape
    with a dense bf16 weight, the achievable-MFMA reference;
  * "encoder_decode": T5-XXL encoder linears at M=512 and LLM-decode M=1
    GEMVs at K=4096 / N=10240 (the text-encoder and prompt-expansion shapes);
  * "lora_merge": device LoRA merge (dequantize -> rank-32 patches ->
    re-quantize) of a single-block linear1, with the host chain on a sample;
  * "upload": GGUF file -> HBM rate of mq_gguf_load_tensor per tensor and of
    one batched mq_gguf_load_tensors call (threaded pinned pipeline) over a
    1.2 GB file just written (so read from the page cache: PCIe and the
    pipeline, not the disk), of the host-buffer upload, and the pinned
    host -> device copy rate of the same process;
  * "flux_step": one FLUX.1-dev-shaped denoising-step forward at 1024^2
    (19 double + 38 single blocks, hidden 3072,
    4096 image + 512 text tokens, every linear Q4_K except the bf16 img_in),
    built by mold_amd.flux on these quantized linears, in ms per step, with
    its own host-CPU baseline (stems, one double block, one single block and
    the final layer on the CPU, extrapolated x19 / x38 and labelled so); its
    "modulation_stack" is the step's 77 adaLN modulation linears (one
    StackedLinear, 1,056,768 x 3072 Q4_K) as the one GEMV the step runs, timed
    alone, in GB/s against the HBM peak; its "graphed" is the same forward
    captured into a HIP graph and replayed (mold_amd.graphs.GraphedStep), in ms
    per step, and whether a replay equals the eager output bit for bit (the
    same for "qwen_step");
  * "qwen_step": one Qwen-Image-shaped denoising-step forward at 1328^2
    (60 dual-stream blocks, 6889 image + 256 text
    tokens, q/k/v Q3_K, MLP Q2_K, out-projections and modulation Q4_K), built
    by mold_amd.qwen_image, in ms per step, with a host-CPU baseline (stems,
    block 0 and the output layer on the CPU, extrapolated x60), and the
    batch-2 classifier-free-guidance forward (cond + a shorter, masked uncond
    prompt) in ms ("cfg_batch2_ms", captured and replayed as a graph in
    "cfg_batch2_graphed"), and its 121 modulation linears' stacked
    GEMV (2,217,984 x 3072 Q4_K) at M = 1 and 2 ("modulation_stack");
  * "cpu_baseline": candle's CPU QMatMul algorithm (quantize x to Q8_K,
    integer block dots, threads over output columns), restated as scalar C
    under oracle/ (gcc -O3, portable x86-64-v2 build), timed on a bounded row
    sample of the headline workload on the host cores this process may use
    (`nproc`, up to the 16-core share of one GPU), with the CPU model named.

Weights are N(0, 0.02^2) quantized to GGUF blocks on the GPU by libmoldq's
quantizer; activations are N(0, 1) from torch's seeded generator.
Everything is resident in HBM before each timed region.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-gemv] [--no-flux] [--no-qwen]
       python bench.py --pmc-pass     (few launches of each kernel, for counters)
       python bench.py --flux-only    (the FLUX step alone, for kernel traces)
       python bench.py --qwen-only    (the Qwen-Image step alone)
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import re
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
GEMM_KERNEL = "mq::gemm_fast_kernel<12, float, false>"   # Q4_K weights, f32 output, no gated epilogue
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemm_q4k_linear1_traffic.md")
GEMM_SOURCES = ["mq_gemm.hip", "mq_bfrag.h", "mq_kernels.h", "mq_common.h"]


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemm_source_digest() -> str:
    """sha256 (first 16 hex digits) over the GEMM kernel's source files."""
    h = hashlib.sha256()
    for name in GEMM_SOURCES:
        with open(os.path.join(ROOT, "mold_amd", "csrc", name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def make_weight(dev, dtype, n, k, seed):
    """N(0, 0.02^2) f32 on the device, quantized to GGUF blocks there."""
    import torch
    import mold_amd
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn((n, k), device="cuda", generator=g) * 0.02
    qt = mold_amd.QTensor.quantize(dev, w, dtype)
    del w
    return qt


def timed(fn, steps, warmup=0, prewarm_s=0.0):
    """Run fn `prewarm_s` seconds and `warmup` times untimed, then `steps` times
    between two synchronizations: returns (wall ms per step, HIP-event ms per
    step on the current stream over the same launches)."""
    import torch
    if prewarm_s > 0:
        t_end = time.perf_counter() + prewarm_s
        while time.perf_counter() < t_end:
            for _ in range(20):
                fn()
            torch.cuda.synchronize()
    for _ in range(warmup):
        fn()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return wall, s.elapsed_time(e) / steps


def bench_gemm(dev, args):
    import torch
    import mold_amd
    from mold_amd import GgmlDType
    m, n, k = 4608, 21504, 3072
    log(f"GEMM Q4_K {m}x{k}->{n}: quantizing weight")
    qt = make_weight(dev, GgmlDType.Q4_K, n, k, seed=4)
    mm = mold_amd.QMatMul(qt)
    g = torch.Generator(device="cuda").manual_seed(40)
    x = torch.randn((m, k), device="cuda", generator=g)
    xb = x.to(torch.bfloat16)
    y = torch.empty((m, n), device="cuda", dtype=torch.float32)
    flop = 2.0 * m * n * k
    log(f"pre-warm 1 s, warmup {args.warmup}, timing {args.steps} steps")
    wall_ms, kern_ms = timed(lambda: mm.forward(xb, out=y), args.steps, args.warmup, prewarm_s=1.0)
    assert torch.isfinite(y).all().item(), "non-finite GEMM output"
    f32_wall, f32_ev = timed(lambda: mm.forward(x, out=y), max(20, args.steps // 4), 3, prewarm_s=1.0)
    res = {
        "ms_per_step": wall_ms,
        "tflops": flop / (wall_ms * 1e-3) / 1e12,
        "kernel_ms": kern_ms,
        "kernel_tflops": flop / (kern_ms * 1e-3) / 1e12,
        "flop": flop,
        "f32_input": {"ms": round(f32_ev, 4), "tflops": round(flop / (f32_ev * 1e-3) / 1e12, 1),
                      "frac": round(flop / (f32_ev * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                      "what": "QMatMul::forward with f32 x [4608,3072]: f32->bf16 staging kernel + the GEMM"},
    }
    blocks = qt.data() if not args.no_cpu else None
    return res, blocks, x


def bench_config1(dev, args):
    """Q8_0 3072x3072 at M=4608, f32 x and y."""
    import torch
    import mold_amd
    from mold_amd import GgmlDType
    m, n, k = 4608, 3072, 3072
    log("config 1: Q8_0 3072x3072, M=4608")
    mm = mold_amd.QMatMul(make_weight(dev, GgmlDType.Q8_0, n, k, seed=1))
    g = torch.Generator(device="cuda").manual_seed(10)
    x = torch.randn((m, k), device="cuda", generator=g)
    xb = x.to(torch.bfloat16)
    y = torch.empty((m, n), device="cuda")
    flop = 2.0 * m * n * k
    steps = max(50, args.steps)
    _, ms = timed(lambda: mm.forward(x, out=y), steps, 5, prewarm_s=0.2)
    _, kms = timed(lambda: mm.forward(xb, out=y), steps, 5)
    return {"m": m, "n": n, "k": k, "ms": round(ms, 4), "tflops": round(flop / (ms * 1e-3) / 1e12, 1),
            "frac": round(flop / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "gemm_kernel_ms": round(kms, 4),
            "gemm_kernel_frac": round(flop / (kms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "what": "f32 x staged to bf16 + fused Q8_0 GEMM (ms, tflops, frac); the GEMM alone on bf16 x "
                    "(gemm_kernel_*)"}


def bench_single_block(dev, args):
    """FLUX's single-block linears at full size, as FluxStep runs them on its fused path:
    linear1 Q4_K 3072 -> 21504 on bf16 x with bf16 output and GELU on columns 9216.. only
    (mq_qmatmul_act_from), then linear2 Q4_K 15360 -> 3072 as the gated residual update whose x
    is linear1's output columns 6144.. (attention rows over the dead v columns, then the GELU'd
    MLP half), read in place with row stride 21504."""
    import torch
    import mold_amd
    from mold_amd import GgmlDType
    from mold_amd.quantized import Linear
    m, h, mlp = 4608, 3072, 12288
    log("FLUX single block: linear1 (act_from) + linear2 (gated, strided x)")
    g = torch.Generator(device="cuda").manual_seed(50)
    mm1 = mold_amd.QMatMul(make_weight(dev, GgmlDType.Q4_K, 3 * h + mlp, h, seed=51))
    lin2 = Linear(make_weight(dev, GgmlDType.Q4_K, h, h + mlp, seed=52))
    x = torch.randn((m, h), device="cuda", generator=g).to(torch.bfloat16)
    y = torch.empty((m, 3 * h + mlp), dtype=torch.bfloat16, device="cuda")
    gate = torch.randn(h, device="cuda", generator=g) * 0.01
    res = torch.zeros((m, h), device="cuda")
    steps = max(50, args.steps)
    _, ms1 = timed(lambda: mm1.forward(x, out=y, act=mold_amd.ACT_GELU_TANH, act_from=3 * h), steps, 5,
                   prewarm_s=0.2)
    _, ms2 = timed(lambda: lin2.gated_add(y[:, 2 * h:], gate, res), steps, 5)
    out = {}
    for name, n, k, ms in (("linear1_act_from", 3 * h + mlp, h, ms1), ("linear2_gated", h, h + mlp, ms2)):
        flop = 2.0 * m * n * k
        out[name] = {"m": m, "n": n, "k": k, "ms": round(ms, 4), "tflops": round(flop / (ms * 1e-3) / 1e12, 1),
                     "frac": round(flop / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
    del mm1, lin2, x, y, res
    return out


def bench_tp8_shards(dev, args):
    """One GPU's share of FLUX's single-block linears under 8-way tensor parallelism, at its real
    shape: linear1 column-split (N/8 = 2688 output features, no exchange) and linear2 row-split.
    linear2's K = 15360 is 60 Q4_K super-blocks, which 8 GPUs cannot split evenly (K/8 = 1920 is
    not a whole number of 256-element blocks): the shares are 8 and 7 super-blocks, and the
    largest (K = 2048) is timed, as the gated update it would feed before the all-reduce."""
    import torch
    import mold_amd
    from mold_amd import GgmlDType
    from mold_amd.quantized import Linear
    m = 4608
    g = torch.Generator(device="cuda").manual_seed(40)
    out = []
    for name, n, k, gated in (("linear1 column shard", 21504 // 8, 3072, False),
                              ("linear2 row shard (largest)", 3072, 2048, True)):
        log(f"tp8 shard: {name} {m}x{k}->{n}")
        qt = make_weight(dev, GgmlDType.Q4_K, n, k, seed=41 + len(out))
        x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
        y = torch.zeros((m, n), device="cuda")
        if gated:
            lin = Linear(qt)
            gate = torch.randn(n, device="cuda", generator=g)
            fn = lambda: lin.gated_add(x, gate, y)
        else:
            mm = mold_amd.QMatMul(qt)
            fn = lambda: mm.forward(x, out=y)
        flop = 2.0 * m * n * k
        _, ms = timed(fn, max(50, args.steps), 5, prewarm_s=0.2)
        out.append({"linear": name, "m": m, "n": n, "k": k, "gated": gated, "ms": round(ms, 4),
                    "tflops": round(flop / (ms * 1e-3) / 1e12, 1),
                    "frac": round(flop / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)})
        del qt, x, y
    return out


def bench_config3(dev, args):
    """MLP fc1 + GELU-tanh -> fc2 at M=4608 for three block layouts."""
    import torch
    import mold_amd
    from mold_amd import GgmlDType
    m, h, f = 4608, 3072, 12288
    g = torch.Generator(device="cuda").manual_seed(30)
    x = torch.randn((m, h), device="cuda", generator=g)
    hid = torch.empty((m, f), device="cuda", dtype=torch.bfloat16)
    y = torch.empty((m, h), device="cuda")
    flop = 2.0 * m * h * f * 2
    out = []
    for tname in ("Q4_K", "Q4_0", "Q6_K"):
        t = GgmlDType[tname]
        log(f"config 3: MLP {tname}")
        fc1 = mold_amd.QMatMul(make_weight(dev, t, f, h, seed=31))
        fc2 = mold_amd.QMatMul(make_weight(dev, t, h, f, seed=32))

        def chain():
            fc1.forward(x, act=mold_amd.ACT_GELU_TANH, out=hid)
            fc2.forward(hid, out=y)
        steps = max(20, args.steps // 4)
        _, ms = timed(chain, steps, 3, prewarm_s=0.2)
        _, ms1 = timed(lambda: fc1.forward(x, act=mold_amd.ACT_GELU_TANH, out=hid), steps, 2)
        _, ms2 = timed(lambda: fc2.forward(hid, out=y), steps, 2)
        out.append({"weight": tname, "ms": round(ms, 4), "tflops": round(flop / (ms * 1e-3) / 1e12, 1),
                    "frac": round(flop / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                    "fc1_ms": round(ms1, 4), "fc2_ms": round(ms2, 4)})
        del fc1, fc2
    return {"m": m, "hidden": h, "mlp": f, "chains": out,
            "what": "fc1 3072->12288 (f32 x staged to bf16, GELU-tanh epilogue, bf16 out) then fc2 12288->3072 "
                    "(bf16 in, f32 out); flop = both GEMMs"}


def bench_dequant(dev, args):
    """QTensor::dequantize of Q4_K 18432x3072 to f32 and bf16, GB/s."""
    import torch
    from mold_amd import GgmlDType
    n, k = 18432, 3072
    log("dequantize Q4_K 18432x3072")
    qt = make_weight(dev, GgmlDType.Q4_K, n, k, seed=7)
    res = {"weight": "Q4_K", "n": n, "k": k, "gguf_bytes": qt.storage_size_in_bytes()}
    for name, dt, es in (("f32", torch.float32, 4), ("bf16", torch.bfloat16, 2)):
        out = torch.empty((n, k), device="cuda", dtype=dt)
        _, ms = timed(lambda: qt.dequantize(dt, out=out), max(20, args.steps // 4), 3, prewarm_s=0.1)
        nbytes = qt.storage_size_in_bytes() + n * k * es
        res[name] = {"us": round(ms * 1e3, 2), "bytes": nbytes, "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    return res


def bench_dense_ceiling(args):
    """torch bf16 linear (hipBLASLt) at the headline shape: the dense-bf16 MFMA ceiling."""
    import torch
    m, n, k = 4608, 21504, 3072
    log("dense bf16 ceiling (torch linear, hipBLASLt)")
    g = torch.Generator(device="cuda").manual_seed(50)
    xb = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    wb = (torch.randn((n, k), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    out = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
    _, ms = timed(lambda: torch.mm(xb, wb.t(), out=out), max(20, args.steps // 2), 5, prewarm_s=0.5)
    flop = 2.0 * m * n * k
    return {"ms": round(ms, 4), "tflops": round(flop / (ms * 1e-3) / 1e12, 1),
            "frac": round(flop / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "what": "torch.mm (x . W^T), bf16 x [4608,3072], dense bf16 W [21504,3072], bf16 out"}


def bench_upload(dev, args):
    """GGUF file -> HBM and host buffer -> HBM upload rates, beside the pinned
    host -> device copy rate of the same process (the PCIe ceiling)."""
    import numpy as np
    import torch
    import mold_amd
    from mold_amd import GgmlDType, gguf
    n, k, distinct, count = 21504, 3072, 8, 32
    t = GgmlDType.Q4_K
    nbytes = n * (k // 256) * 144
    rng = np.random.default_rng(60)
    raw = [rng.integers(0, 256, nbytes, dtype=np.uint8) for _ in range(distinct)]
    names = [f"blk.{i}.weight" for i in range(count)]
    pin = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    pin.copy_(torch.from_numpy(raw[0]))
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    for _ in range(3):
        dst.copy_(pin, non_blocking=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(count):
        dst.copy_(pin, non_blocking=True)
    torch.cuda.synchronize()
    pinned_gbs = count * nbytes / (time.perf_counter() - t0) / 1e9
    del pin, dst
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "w.gguf")
        gguf.write(path, [(nm, t, (n, k), raw[i % distinct]) for i, nm in enumerate(names)])
        log(f"upload: GGUF file {count * nbytes / 1e6:.0f} MB")
        c = gguf.Content.read(path)

        def warm():
            """A short load, then 0.2 s idle: right after hipFree of large buffers
            the copy engine runs at a fraction of its rate for ~10-15 ms (the
            driver's deferred unmapping), which no timing here should absorb."""
            for q in c.tensors(names[:3], dev).values():
                q.free()
            time.sleep(0.2)
        warm()
        t0 = time.perf_counter()
        qts = [c.tensor(nm, dev) for nm in names]
        dt_file = time.perf_counter() - t0
        del qts
        warm()
        t0 = time.perf_counter()
        qts = c.tensors(names, dev)
        dt_batch = time.perf_counter() - t0
        c.close()
    ok = all(np.array_equal(qts[nm].data(), raw[i % distinct]) for i, nm in enumerate(names[:2]))
    del qts
    for q in [mold_amd.QTensor.from_blocks(dev, t, (n, k), r) for r in raw[:3]]:
        q.free()
    time.sleep(0.2)
    t0 = time.perf_counter()
    qts = [mold_amd.QTensor.from_blocks(dev, t, (n, k), raw[i % distinct]) for i in range(count)]
    dt_host = time.perf_counter() - t0
    del qts
    # FP8 E4M3 -> Q8_0 on the device (the FP8 checkpoint cache producer's quantize step)
    import ctypes
    from mold_amd import _lib
    fn, fk = 21504, 3072
    src = torch.randint(0, 126, (fn, fk), dtype=torch.uint8, device="cuda")
    for _ in range(2):
        h = ctypes.c_void_p()
        t0 = time.perf_counter()
        rc = _lib.load().mq_quantize_fp8(dev.handle, int(GgmlDType.Q8_0), fn, fk, src.data_ptr(), fk,
                                         ctypes.c_float(1.0), None, ctypes.byref(h))
        dt_fp8 = time.perf_counter() - t0
        assert rc == 0
        mold_amd.QTensor(dev, h).free()
    return {"bytes": count * nbytes, "tensors": count,
            "fp8_to_q8_0_ms": round(dt_fp8 * 1e3, 3), "fp8_to_q8_0_gbs": round(fn * fk / dt_fp8 / 1e9, 1),
            "gguf_file_gbs": round(count * nbytes / dt_file / 1e9, 2),
            "gguf_file_batched_gbs": round(count * nbytes / dt_batch / 1e9, 2),
            "host_buffer_gbs": round(count * nbytes / dt_host / 1e9, 2),
            "pinned_h2d_ceiling_gbs": round(pinned_gbs, 2), "readback_identical": bool(ok),
            "what": "GGUF file (page cache: PCIe + pipeline, not disk) -> device, 32 Q4_K [21504, 3072] tensors "
                    "(1.19 GB), each timing after a 3-tensor warm-up load and 0.2 s idle (the copy engine runs slow "
                    "for ~10-15 ms after large hipFrees): "
                    "gguf_file = mq_gguf_load_tensor per tensor, gguf_file_batched = one mq_gguf_load_tensors call "
                    "(VarBuilder::from_gguf); host_buffer = mq_qtensor_upload from pageable numpy; "
                    "pinned_h2d_ceiling = torch copy of one tensor's bytes from pinned host memory, same process; "
                    "fp8_to_q8_0: mq_quantize_fp8 of a device-resident FP8 E4M3 [21504, 3072] to Q8_0 including the "
                    "repack and the synchronization (GB/s of FP8 input)"}


def bench_encoder_decode(dev, args):
    """Next-row shapes behind the same boundary: T5-XXL encoder linears at M=512
    (crates/mold-inference/src/encoders/t5_gguf.rs:243-279) and LLM-expand M=1
    decode GEMVs at K=4096 / N=10240 (crates/mold-inference/src/expand.rs:200-203),
    the decode ones rotating through > 256 MB of weight copies in a HIP graph."""
    import torch
    import mold_amd
    from mold_amd import GgmlDType
    enc = []
    m = 512
    g = torch.Generator(device="cuda").manual_seed(70)
    for tname in ("Q8_0", "Q5_K"):
        for label, (n, k) in (("attn_q", (4096, 4096)), ("ffn_up", (10240, 4096)), ("ffn_down", (4096, 10240))):
            mm = mold_amd.QMatMul(make_weight(dev, GgmlDType[tname], n, k, seed=71))
            x = torch.randn((m, k), device="cuda", generator=g)
            y = torch.empty((m, n), device="cuda")
            _, ms = timed(lambda: mm.forward(x, out=y), max(20, args.steps // 4), 3, prewarm_s=0.05)
            fl = 2.0 * m * n * k
            enc.append({"weight": tname, "linear": label, "m": m, "n": n, "k": k, "us": round(ms * 1e3, 2),
                        "tflops": round(fl / (ms * 1e-3) / 1e12, 1),
                        "frac": round(fl / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)})
            log(f"  T5 {tname} {label} m={m}: {ms*1e3:.1f} us {enc[-1]['tflops']} TFLOP/s")
            del mm
    # small-m linears: T5 at a 77-token prompt, Qwen-Image's text stream (256 tokens)
    mid = []
    for label, tname, n, k in (("t5 attn_q", "Q8_0", 4096, 4096), ("t5 ffn_up", "Q8_0", 10240, 4096),
                               ("t5 ffn_down", "Q8_0", 4096, 10240), ("qwen txt add_qkv", "Q3_K", 9216, 3072),
                               ("qwen txt to_add_out", "Q4_K", 3072, 3072)):
        mm = mold_amd.QMatMul(make_weight(dev, GgmlDType[tname], n, k, seed=72))
        for m_ in (77, 256):
            x = torch.randn((m_, k), device="cuda", generator=g)
            y = torch.empty((m_, n), device="cuda")
            _, ms = timed(lambda: mm.forward(x, out=y), max(50, args.steps), 5, prewarm_s=0.05)
            fl = 2.0 * m_ * n * k
            mid.append({"weight": tname, "linear": label, "m": m_, "n": n, "k": k, "us": round(ms * 1e3, 2),
                        "tflops": round(fl / (ms * 1e-3) / 1e12, 1),
                        "frac": round(fl / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)})
            log(f"  {label} {tname} m={m_}: {ms*1e3:.1f} us {mid[-1]['tflops']} TFLOP/s")
        del mm
    dec = []
    for tname in ("Q8_0", "Q6_K", "Q5_K", "Q4_K", "Q4_0"):
        for n, k in ((4096, 4096), (10240, 4096), (4096, 10240)):
            t = GgmlDType[tname]
            first = make_weight(dev, t, n, k, seed=80)
            wbytes = first.storage_size_in_bytes()
            copies = max(2, -(-(300 << 20) // wbytes))
            mms = [mold_amd.QMatMul(first)] + [mold_amd.QMatMul(make_weight(dev, t, n, k, seed=81 + i))
                                               for i in range(copies - 1)]
            x = torch.randn((1, k), device="cuda", generator=g)
            y = torch.empty((1, n), device="cuda")
            cap = torch.cuda.Stream()

            def run():
                for mm in mms:
                    mm.forward(x, out=y)
            torch.cuda.synchronize()
            with torch.cuda.stream(cap):
                run()              # sizes the capture stream's workspace (K-split partials)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=cap):
                run()
            _, ms = timed(graph.replay, max(10, args.steps // 10), 2, prewarm_s=0.05)
            ms /= copies
            nbytes = wbytes + 4 * k + 4 * n
            dec.append({"weight": tname, "m": 1, "n": n, "k": k, "us": round(ms * 1e3, 3), "bytes": nbytes,
                        "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                        "frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)})
            log(f"  decode {tname} {k}->{n}: {ms*1e3:.2f} us {dec[-1]['gbs']} GB/s")
            del graph, mms, first
            torch.cuda.empty_cache()
    return {"t5_encoder_m512": enc, "small_m_gemm": mid, "decode_gemv_m1": dec,
            "what": "T5-XXL encoder linears (f32 x staged to bf16 + fused GEMM) at M=512; small-m GEMMs "
                    "(64- / 128-row tiles) at M=77 and 256; LLM-decode M=1 GEMVs "
                    "(f32 x; Q4_K takes the Q8_K integer-dot GEMV, other types the f32-FMA GEMV)"}


def bench_lora(dev, args):
    """Device LoRA merge of one FLUX single-block linear1 (Q4_K 21504x3072) with
    rank-32 patches on Q, K, V and the MLP rows (mold's gguf_lora_var_builder,
    crates/mold-inference/src/flux/lora.rs:748-849): dequantize -> 4 x
    mq_lora_apply -> quantize, and the same chain on the host (oracle) over a
    256-row sample, scaled to the whole tensor."""
    import numpy as np
    import torch
    from mold_amd import GgmlDType
    from mold_amd import lora as L
    n, k, rank = 21504, 3072, 32
    qt = make_weight(dev, GgmlDType.Q4_K, n, k, seed=90)
    g = torch.Generator(device="cuda").manual_seed(91)
    pts = []
    for comp, size in ((0, 3072), (1, 3072), (2, 3072), (3, 12288)):
        a = torch.randn((rank, k), device="cuda", generator=g) * 0.05
        b = torch.randn((size, rank), device="cuda", generator=g) * 0.05
        pts.append(L.LoraPatch(a, b, 0.5, L.LoraTarget("single_blocks.0.linear1.weight", comp, 0)))
    L.patch_qtensor(qt, pts)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    reps = 3
    for _ in range(reps):
        out, applied = L.patch_qtensor(qt, pts)
        del out
    torch.cuda.synchronize()
    dev_ms = (time.perf_counter() - t0) * 1e3 / reps
    res = {"weight": "Q4_K", "n": n, "k": k, "rank": rank, "patches": applied, "device_ms": round(dev_ms, 2),
           "what": "mq_dequantize + 4 mq_lora_apply (Q, K, V 3072 rows, MLP 12288 rows) + mq_quantize (ggml "
                   "reference Q4_K quantizer), synchronous"}
    if not args.no_cpu:
        from oracle import oracle as O
        rows = 256
        blocks = qt.data()[: rows * O.row_bytes(O.Q4_K, k)]
        a = pts[0].a.cpu().numpy()
        b = pts[0].b[:rows].cpu().numpy()
        t0 = time.perf_counter()
        dq = O.dequantize(O.Q4_K, blocks, rows, k)
        dq = O.lora_apply(dq, b, a, 0.5)
        O.quantize(O.Q4_K, dq)
        dt = time.perf_counter() - t0
        res["cpu_ms_extrapolated"] = round(dt * 1e3 * n / rows, 1)
        res["cpu_sample"] = f"{rows} of {n} rows, one thread (oracle dequantize + merge + reference quantize), x{n // rows}"
    log(f"  LoRA merge: device {dev_ms:.1f} ms" + (f", CPU ~{res['cpu_ms_extrapolated']:.0f} ms" if "cpu_ms_extrapolated" in res else ""))
    return res


def read_ceiling(nbytes, copies, args):
    """The fastest single-launch streaming read of `nbytes` found among a few
    shapes (libmoldq_probe.so: 512-thread workgroups, nontemporal 16-byte
    loads, nothing computed; the GEMV's own layout of one workgroup per CU,
    and contiguous shares over 512 or 1024 workgroups, the fastest shapes of a
    wider sweep), cold: `copies` distinct buffers (> 256 MB together, past the
    Infinity Cache) replayed from a HIP graph.  The ceiling a single GEMV
    launch of the same weight bytes can reach."""
    import ctypes
    import torch
    lib = ctypes.CDLL(os.path.join(ROOT, "mold_amd", "libmoldq_probe.so"))
    lib.mqp_stream_read.restype = ctypes.c_int
    lib.mqp_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_void_p]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    bufs = torch.randint(0, 255, (copies, nbytes), dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4 * cus, dtype=torch.int32, device="cuda")
    cap = torch.cuda.Stream()
    best = None
    for wgs, shape in ((cus, 0), (2 * cus, 1), (4 * cus, 1)):
        def run():
            for i in range(copies):
                rc = lib.mqp_stream_read(bufs[i].data_ptr(), nbytes, sink.data_ptr(), wgs, shape, cap.cuda_stream)
                assert rc == 0, rc
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=cap):
            run()
        graph.replay()
        torch.cuda.synchronize()
        _, ms = timed(graph.replay, max(10, args.steps), 2, prewarm_s=0.1)
        ms /= copies
        del graph
        if best is None or ms < best[0]:
            best = (ms, wgs, shape)
    del bufs
    ms, wgs, shape = best
    return {"bytes": nbytes, "us": round(ms * 1e3, 3), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "shape": f"{wgs} workgroups x 512, " + ("the GEMV's layout" if shape == 0 else "contiguous shares")}


def bench_gemv(dev, args):
    import torch
    import mold_amd
    from mold_amd import GgmlDType
    out, ceilings = [], []
    k = 3072
    for n, copies in ((18432, 12), (9216, 20)):
        log(f"GEMV Q4_K 3072->{n}: quantizing {copies} weight copies")
        qts = [make_weight(dev, GgmlDType.Q4_K, n, k, seed=200 + i) for i in range(copies)]
        wbytes = qts[0].storage_size_in_bytes()
        ceil = read_ceiling(wbytes, copies, args)
        ceil["n"] = n
        ceilings.append(ceil)
        log(f"  streaming-read ceiling of {wbytes} B: {ceil['us']:.2f} us {ceil['gbs']:.0f} GB/s "
            f"({ceil['frac']:.3f} of peak)")
        mms = [mold_amd.QMatMul(q) for q in qts]
        for m in (1, 2, 4):
            g = torch.Generator(device="cuda").manual_seed(m)
            x = torch.randn((m, k), device="cuda", generator=g)
            y = torch.empty((m, n), device="cuda")

            def run():
                for mm in mms:
                    mm.forward(x, out=y)
            run()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                run()
            graph.replay()
            torch.cuda.synchronize()
            iters = max(10, args.steps)
            _, ms = timed(graph.replay, iters, 2, prewarm_s=0.1)
            ms /= copies
            nbytes = wbytes + 4 * m * k + 4 * m * n
            out.append({"m": m, "n": n, "k": k, "us": round(ms * 1e3, 3), "bytes": nbytes,
                        "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                        "frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                        "of_read_ceiling": round(ceil["us"] / (ms * 1e3), 4)})
            del graph
            # the same launches on x quantized once beforehand (mq_quantize_x_q8k): the
            # caller's producer of x (silu(vec) for every modulation of a step) does it once
            xq = mold_amd.Q8KActivations(dev, x)

            def run_q():
                for mm in mms:
                    mm.forward(xq, out=y)
            run_q()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                run_q()
            graph.replay()
            torch.cuda.synchronize()
            _, msq = timed(graph.replay, iters, 2, prewarm_s=0.1)
            msq /= copies
            del graph
            _, msx = timed(lambda: mold_amd.Q8KActivations(dev, x), 200, 10)
            nq = wbytes + m * (k // 256) * 304 + 4 * m * n
            out[-1]["x_q8k"] = {"us": round(msq * 1e3, 3), "bytes": nq,
                                "frac": round(nq / (msq * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                                "of_read_ceiling": round(ceil["us"] / (msq * 1e3), 4),
                                "quantize_us": round(msx * 1e3, 2)}
            log(f"  m={m} n={n}: {ms*1e3:.2f} us  {out[-1]['gbs']:.0f} GB/s; x pre-quantized {msq*1e3:.2f} us "
                f"(quantize {msx*1e3:.2f} us, once per x)")
        del mms, qts
        torch.cuda.empty_cache()
    return {"launches": out, "read_ceiling": ceilings,
            "what": "single Q4_K GEMV launches (f32 x, f32 y) replayed from a HIP graph over distinct weight "
                    "copies (> 256 MB, so reads come from HBM); read_ceiling: the fastest of three single-launch "
                    "streaming-read shapes over the same weight bytes in the same run; of_read_ceiling = ceiling time / GEMV time; x_q8k: the "
                    "same launches on x quantized once beforehand by mq_quantize_x_q8k (bit-identical outputs; "
                    "quantize_us is that one kernel, timed alone with the host call)"}


def bench_stack(stack, ms_list, args):
    """The step's stacked modulation GEMV alone (StackedLinear: every block's
    adaLN modulation weight in one Q4_K tensor, one launch), captured in a HIP
    graph and replayed; its weight is far larger than the Infinity Cache, so
    every replay streams it from HBM."""
    import torch
    lin = stack.linear
    n, k = lin.matmul.w.shape
    wbytes = lin.matmul.w.storage_size_in_bytes()
    out = []
    for m in ms_list:
        x = torch.randn((m, k), device="cuda", generator=torch.Generator(device="cuda").manual_seed(m))
        y = torch.empty((m, n), device="cuda")

        def run():
            lin.matmul.forward(x, bias=lin.bias, out=y)
        run()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run()
        graph.replay()
        torch.cuda.synchronize()
        _, ms = timed(graph.replay, max(10, args.steps), 2, prewarm_s=0.1)
        nbytes = wbytes + 4 * m * k + 4 * n + 4 * m * n
        out.append({"m": m, "n": n, "k": k, "parts": len(stack.names), "us": round(ms * 1e3, 2), "bytes": nbytes,
                    "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                    "frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)})
        log(f"  stacked modulation GEMV m={m}: {len(stack.names)} linears, {n} rows, {ms*1e3:.1f} us, "
            f"{out[-1]['gbs']:.0f} GB/s ({out[-1]['frac']:.3f} of peak)")
        del graph
    return out


def bench_graphed(step, inp, n, eager_out, batched=False):
    """The same forward captured into a HIP graph (mold_amd.graphs.GraphedStep) and replayed:
    ms per step (median of n), and whether a replay equals the eager output bit for bit."""
    import torch
    from mold_amd.graphs import GraphedStep
    g = GraphedStep(step, batched=batched, **inp)
    same = bool(torch.equal(g(**inp), eager_out))
    times = []
    for _ in range(n):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g(**inp)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    del g
    return {"ms": round(sorted(times)[len(times) // 2], 3), "steps_timed": n, "equals_eager": same}


def bench_flux(dev, args):
    """One FLUX.1-dev-shaped Q4_K step at 1024^2, eager, ms per step."""
    import torch
    from mold_amd import flux as F
    cfg = F.FluxConfig.dev()
    log("FLUX step: generating and quantizing the transformer's linears")
    t0 = time.perf_counter()
    params = F.FluxParams.random(cfg, dev, seed=4)
    inp = F.make_inputs(cfg, 1024, 1024, 512, device="cuda", seed=4)
    torch.cuda.synchronize()
    log(f"  {len(params.lin)} quantized linears, {params.quantized_bytes() / 1e9:.2f} GB resident "
        f"({time.perf_counter() - t0:.1f} s)")
    step = F.FluxStep(params)
    for _ in range(max(1, min(2, args.warmup))):
        out = step.forward(**inp)
    torch.cuda.synchronize()
    n = max(3, min(10, args.steps // 4))
    times = []
    for _ in range(n):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = step.forward(**inp)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    assert torch.isfinite(out).all().item(), "non-finite FLUX step output"
    lin, attn = F.step_flop(cfg, 4096, 512)
    ms = sorted(times)[len(times) // 2]
    log(f"  step {ms:.2f} ms (median of {n}), attention backend {F.ATTENTION_BACKEND['name']}")
    graphed = bench_graphed(step, inp, n, out)
    log(f"  graphed step {graphed['ms']:.2f} ms, equals eager: {graphed['equals_eager']}")
    stack = bench_stack(step._mod_stack, (1,), args)
    res = {"ms": round(ms, 3), "steps_timed": n, "all_ms": [round(t, 3) for t in times],
           "graphed": graphed, "modulation_stack": stack,
           "tflops_linear_plus_attention": round((lin + attn) / (ms * 1e-3) / 1e12, 1),
           "flop_linear": lin, "flop_attention": attn,
           "weight_bytes": params.quantized_bytes(), "attention": F.ATTENTION_BACKEND["name"],
           "config": "FLUX.1-dev shape, 1024x1024, batch 1, 4096 img + 512 txt tokens, Q4_K linears, "
                     "f32 activations, bf16 GEMM inputs and attention; attention is PyTorch's fused SDPA "
                     "(on ROCm AOTriton's precompiled attn_fwd kernel), not part of libmoldq"}
    return res, params, inp


def bench_qwen(dev, args):
    """One Qwen-Image-shaped mixed low-bit step at 1328^2, eager, ms per step."""
    import torch
    from mold_amd import qwen_image as Q
    from mold_amd.flux import ATTENTION_BACKEND
    cfg = Q.QwenConfig.image()
    log("Qwen-Image step: generating and quantizing the transformer's linears (Q3_K qkv, Q2_K MLP, Q4_K rest)")
    t0 = time.perf_counter()
    params = Q.QwenParams.random(cfg, dev, seed=5)
    inp = Q.make_inputs(cfg, 1328, 1328, 256, device="cuda", seed=5)
    torch.cuda.synchronize()
    log(f"  {len(params.lin)} quantized linears, {params.quantized_bytes() / 1e9:.2f} GB resident "
        f"({time.perf_counter() - t0:.1f} s)")
    step = Q.QwenImageStep(params)
    for _ in range(max(1, min(2, args.warmup))):
        out = step.forward(**inp)
    torch.cuda.synchronize()
    n = max(3, min(10, args.steps // 4))
    times = []
    for _ in range(n):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = step.forward(**inp)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    assert torch.isfinite(out).all().item(), "non-finite Qwen step output"
    # CFG batching (pipeline.rs:1866-1899): cond + uncond in one batch-2 forward,
    # the uncond prompt 180 of 256 tokens (its padding masked out of attention)
    g = torch.Generator(device="cuda").manual_seed(6)
    txt_u = torch.randn(inp["txt"].shape, device="cuda", generator=g)
    b_args = (torch.stack([inp["img"], inp["img"]]), torch.stack([inp["txt"], txt_u]),
              torch.cat([inp["t"], inp["t"]]), inp["grid"])
    outb = step.forward_batched(*b_args, txt_valid=[256, 180])
    torch.cuda.synchronize()
    btimes = []
    for _ in range(max(2, n // 2)):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        outb = step.forward_batched(*b_args, txt_valid=[256, 180])
        torch.cuda.synchronize()
        btimes.append((time.perf_counter() - t0) * 1e3)
    assert torch.isfinite(outb).all().item(), "non-finite batched Qwen output"
    bms = sorted(btimes)[len(btimes) // 2]
    log(f"  CFG batch-2 forward {bms:.2f} ms (two batch-1 forwards: {2 * sorted(times)[len(times) // 2]:.2f} ms)")
    bgraphed = bench_graphed(step, {"img": b_args[0], "txt": b_args[1], "t": b_args[2], "grid": b_args[3],
                                    "txt_valid": [256, 180]}, len(btimes), outb, batched=True)
    log(f"  graphed CFG batch-2 forward {bgraphed['ms']:.2f} ms, equals eager: {bgraphed['equals_eager']}")
    del outb, b_args, txt_u
    l_img = inp["grid"][0] * inp["grid"][1]
    lin, attn = Q.step_flop(cfg, l_img, 256)
    ms = sorted(times)[len(times) // 2]
    log(f"  step {ms:.2f} ms (median of {n}), attention backend {ATTENTION_BACKEND['name']}")
    graphed = bench_graphed(step, inp, n, out)
    log(f"  graphed step {graphed['ms']:.2f} ms, equals eager: {graphed['equals_eager']}")
    stack = bench_stack(step._mod_stack, (1, 2), args)
    res = {"ms": round(ms, 3), "steps_timed": n, "all_ms": [round(t, 3) for t in times],
           "graphed": graphed, "modulation_stack": stack,
           "tflops_linear_plus_attention": round((lin + attn) / (ms * 1e-3) / 1e12, 1),
           "flop_linear": lin, "flop_attention": attn,
           "cfg_batch2_ms": round(bms, 3), "cfg_batch2_steps_timed": len(btimes), "cfg_batch2_graphed": bgraphed,
           "weight_bytes": params.quantized_bytes(), "attention": ATTENTION_BACKEND["name"],
           "config": f"Qwen-Image shape, 1328x1328, batch 1, {l_img} img + 256 txt tokens, 60 blocks; "
                     "q/k/v Q3_K (stacked per stream), MLP Q2_K, out-projections, modulation, stems Q4_K; "
                     "f32 residuals, bf16 GEMM inputs and attention (joint sequence padded to a multiple of 256 "
                     "with zero keys, corrected by the log-sum-exp), text stream on a second HIP stream; attention is "
                     "PyTorch's fused SDPA (on ROCm AOTriton's precompiled attn_fwd kernel), not part of libmoldq"}
    return res, params, inp


def cpu_qwen_baseline(params, inp):
    """Host-CPU Qwen-Image step: stems, block 0 and the output layer timed on
    the CPU, extrapolated to 60 blocks."""
    import torch
    from mold_amd import qwen_image as Q
    from mold_amd.flux import attention_f32
    threads, _ = host_threads()
    torch.set_num_threads(threads)
    cfg = params.cfg
    names = [nm for nm in params.lin if not nm.startswith("transformer_blocks.")
             or nm.startswith("transformer_blocks.0.")]
    lin = {nm: _CandleCpuLinear(params.lin[nm], threads) for nm in names}
    dense = {nm: v.float().cpu() for nm, v in params.dense.items()
             if not nm.startswith("transformer_blocks.") or nm.startswith("transformer_blocks.0.")}
    step = Q.QwenImageStep(Q.QwenParams(cfg, lin, dense), attn=attention_f32, gemm_dtype=torch.float32,
                           overlap=False)
    x = {k: (v.cpu() if hasattr(v, "cpu") else v) for k, v in inp.items()}
    t0 = time.perf_counter()
    rope = Q.rope_tables(cfg, 1, x["grid"][0], x["grid"][1], x["txt"].shape[0], "cpu")
    img, txt, temb = step.stems(x["img"], x["txt"], x["t"])
    t_stem = time.perf_counter() - t0
    t0 = time.perf_counter()
    img, txt = step.block(0, img, txt, Q.silu(temb), rope)
    t_block = time.perf_counter() - t0
    t0 = time.perf_counter()
    step.output_layer(img, temb)
    t_out = time.perf_counter() - t0
    total = t_stem + cfg.num_layers * t_block + t_out
    return {"value": round(total * 1e3, 1), "unit": "ms", "cores": threads, "kind": "port",
            "sample": f"extrapolated: stems {t_stem:.2f} s + 60 x block {t_block:.2f} s + output {t_out:.2f} s, "
                      f"each measured once (quantized linears: candle CPU algorithm restated; glue and f32 "
                      f"attention: torch CPU)"}


class _CandleCpuLinear:
    """A quantized linear on the host: candle's CPU QMatMul algorithm (oracle
    restatement) on the same GGUF blocks, f32 in and out, bias added after."""

    def __init__(self, lin, threads):
        import torch
        qt = lin.matmul.w
        self.t, (self.n, self.k) = int(qt.dtype()), qt.shape
        self.blocks = qt.data()
        self.bias = lin.bias.cpu() if lin.bias is not None else None
        self.threads = threads
        self.torch = torch

    def forward(self, x, act=0, out_dtype=None):
        import numpy as np
        from oracle import oracle as O
        torch = self.torch
        x2 = np.ascontiguousarray(x.float().reshape(-1, self.k).numpy())
        y = torch.from_numpy(O.matmul_candle(self.t, x2, self.blocks, self.n, self.k, nthreads=self.threads))
        if self.bias is not None:
            y = y + self.bias
        if act == 1:
            y = torch.nn.functional.gelu(y, approximate="tanh")
        return y.to(out_dtype or torch.float32)


def cpu_flux_baseline(params, inp):
    """Host-CPU FLUX step: stems, double block 0, single block 0 and the final
    layer timed on the CPU, extrapolated to 19 + 38 blocks."""
    import torch
    from mold_amd import flux as F
    threads, _ = host_threads()
    torch.set_num_threads(threads)
    cfg = params.cfg
    names = [nm for nm in params.lin if not nm.startswith(("double_blocks.", "single_blocks."))
             or nm.startswith(("double_blocks.0.", "single_blocks.0."))]
    lin = {nm: _CandleCpuLinear(params.lin[nm], threads) for nm in names}
    dense = {nm: v.float().cpu() for nm, v in params.dense.items()
             if not nm.startswith(("double_blocks.", "single_blocks.")) or ".0." in nm}
    step = F.FluxStep(F.FluxParams(cfg, lin, dense), attn=F.attention_f32, gemm_dtype=torch.float32)
    x = {k: v.cpu() for k, v in inp.items()}
    t0 = time.perf_counter()
    cos, sin = step.rope(x["img_ids"], x["txt_ids"])
    img, txt, vec = step.stems(x["img"], x["txt"], x["t"], x["guidance"], x["y"])
    t_stem = time.perf_counter() - t0
    t0 = time.perf_counter()
    img, txt = step.double_block(0, img, txt, vec, cos, sin)
    t_double = time.perf_counter() - t0
    xs = torch.cat([txt, img], dim=0)
    t0 = time.perf_counter()
    xs = step.single_block(0, xs, vec, cos, sin)
    t_single = time.perf_counter() - t0
    t0 = time.perf_counter()
    step.final_layer(xs[txt.shape[0]:], vec)
    t_final = time.perf_counter() - t0
    total = t_stem + cfg.depth * t_double + cfg.depth_single_blocks * t_single + t_final
    return {"value": round(total * 1e3, 1), "unit": "ms", "cores": threads, "kind": "port",
            "sample": f"extrapolated: stems {t_stem:.2f} s + 19 x double block {t_double:.2f} s + "
                      f"38 x single block {t_single:.2f} s + final {t_final:.2f} s, each measured once "
                      f"(quantized linears: candle CPU algorithm restated; glue and f32 attention: torch CPU)"}


def read_traffic():
    """HBM bytes per GEMM launch from the committed counter summary, when the
    summary was taken on these kernel sources (its recorded digest matches);
    else None."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            text = f.read()
    except OSError:
        return None
    mt = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", text)
    md = re.search(r"source_digest:\s*([0-9a-f]{16})", text)
    if not mt or not md or md.group(1) != gemm_source_digest():
        log("traffic summary absent or taken on other kernel sources: roofline.traffic = null")
        return None
    return int(mt.group(1))


def pmc_pass(dev, args):
    """A short run for rocprofv3 counter passes: a 256 MiB device copy (the
    calibration kernel, bytes known exactly), then the GEMM kernel alone
    (bf16 activations, f32 out) and the M=1 3072->18432 Q4_K GEMV."""
    import torch
    import mold_amd
    from mold_amd import GgmlDType
    log(f"kernel source digest {gemm_source_digest()}")
    nbytes = 256 << 20
    a = torch.empty(nbytes // 4, device="cuda").normal_()
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    log(f"copy calibration: {nbytes} bytes read + {nbytes} written per launch")
    m, n, k = 4608, 21504, 3072
    mm = mold_amd.QMatMul(make_weight(dev, GgmlDType.Q4_K, n, k, seed=4))
    g = torch.Generator(device="cuda").manual_seed(40)
    xb = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    y = torch.empty((m, n), device="cuda")
    for _ in range(3):
        mm.forward(xb, out=y)
    torch.cuda.synchronize()
    log("GEMM launches done")
    gv = mold_amd.QMatMul(make_weight(dev, GgmlDType.Q4_K, 18432, k, seed=200))
    x1 = torch.randn((1, k), device="cuda")
    y1 = torch.empty((1, 18432), device="cuda")
    for _ in range(3):
        gv.forward(x1, out=y1)
    torch.cuda.synchronize()
    log("GEMV launches done")


def host_threads():
    """(threads, nproc): the host cores this process may run on (sched_getaffinity,
    what `nproc` prints), used up to 16, the CPU share of one GPU on these boxes."""
    nproc = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return min(16, nproc), nproc


def cpu_baseline(blocks, x, n, k, budget_s=8.0):
    """candle CPU QMatMul algorithm (the oracle's scalar C restatement, portable
    gcc -O3 -march=x86-64-v2 build) on a row sample of the headline workload.
    It is candle's algorithm, not candle's SIMD code, so it understates candle's
    own CPU path; it is a reported baseline only."""
    import numpy as np
    from oracle import oracle as O
    threads, nproc = host_threads()
    builds = ["gcc -O3 -march=x86-64-v2"]
    timings = {}
    for label in builds:
        xs = np.ascontiguousarray(x[:8].float().cpu().numpy())
        t0 = time.perf_counter()
        O.matmul_candle(O.Q4_K, xs, blocks, n, k, nthreads=threads)
        per_row = (time.perf_counter() - t0) / 8
        rows = int(max(8, min(4608, budget_s / max(per_row, 1e-6))))
        xs = np.ascontiguousarray(x[:rows].float().cpu().numpy())
        t0 = time.perf_counter()
        O.matmul_candle(O.Q4_K, xs, blocks, n, k, nthreads=threads)
        dt = time.perf_counter() - t0
        timings[label] = (2.0 * rows * n * k / dt / 1e12, rows, dt)
        log(f"  CPU {label}: {timings[label][0]:.4f} TFLOP/s over {rows} rows ({dt:.1f} s)")
    best = max(timings, key=lambda lb: timings[lb][0])
    tf, rows, dt = timings[best]
    return {"value": tf, "unit": "TFLOP/s", "cores": threads, "nproc": nproc, "kind": "port",
            "cpu_model": cpu_model(), "build": best,
            "sample": f"{rows} of 4608 rows of x [4608,3072] against the full Q4_K W[21504,3072] "
                      f"({dt:.1f} s; candle's CPU algorithm restated as scalar C, not candle's SIMD code: "
                      f"x->Q8_K, integer block dots, {threads} threads over output columns; nproc {nproc})"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemv", action="store_true")
    ap.add_argument("--no-flux", action="store_true")
    ap.add_argument("--flux-only", action="store_true")
    ap.add_argument("--no-qwen", action="store_true")
    ap.add_argument("--qwen-only", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip configs 1/3, dequant, ceiling, upload, encoder legs")
    ap.add_argument("--encoder-only", action="store_true")
    ap.add_argument("--pmc-pass", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: every GPU box in this setup has one GPU, and this build has "
              "no multi-GPU path (the reference runs one whole model per GPU, with no collectives).",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import mold_amd
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    mold_amd.load()
    dev = mold_amd.Device(0)
    if args.pmc_pass:
        pmc_pass(dev, args)
        return
    if args.flux_only:
        flux, _, _ = bench_flux(dev, args)
        print(json.dumps({"flux_step": flux}), flush=True)
        return
    if args.encoder_only:
        print(json.dumps({"encoder_decode": bench_encoder_decode(dev, args), "lora_merge": bench_lora(dev, args),
                          "upload": bench_upload(dev, args)}), flush=True)
        return
    if args.qwen_only:
        qwen, _, _ = bench_qwen(dev, args)
        print(json.dumps({"qwen_step": qwen}), flush=True)
        return
    gemm, blocks, x = bench_gemm(dev, args)
    log(f"GEMM: {gemm['ms_per_step']:.4f} ms/step {gemm['tflops']:.1f} TFLOP/s; kernel {gemm['kernel_ms']:.4f} ms "
        f"{gemm['kernel_tflops']:.1f} TFLOP/s; f32 input {gemm['f32_input']['ms']:.4f} ms")
    extra = {}
    if not args.no_extra:
        extra["config1_q8_0"] = bench_config1(dev, args)
        extra["config3_mlp"] = bench_config3(dev, args)
        extra["flux_single_block"] = bench_single_block(dev, args)
        extra["tp8_shards"] = bench_tp8_shards(dev, args)
        extra["dequant"] = bench_dequant(dev, args)
        extra["dense_bf16_ceiling"] = bench_dense_ceiling(args)
        extra["upload"] = bench_upload(dev, args)
        extra["encoder_decode"] = bench_encoder_decode(dev, args)
        extra["lora_merge"] = bench_lora(dev, args)
        torch.cuda.empty_cache()
        for key, v in extra.items():
            log(f"{key}: {json.dumps(v)[:300]}")
    gemv = None if args.no_gemv else bench_gemv(dev, args)
    flux = None
    if not args.no_flux:
        flux, fparams, finp = bench_flux(dev, args)
        if not args.no_cpu:
            log("FLUX step CPU baseline (one block of each kind, extrapolated)")
            flux["cpu_baseline"] = cpu_flux_baseline(fparams, finp)
            log(f"  CPU: {flux['cpu_baseline']['value']:.0f} ms ({flux['cpu_baseline']['sample']})")
        del fparams, finp
        torch.cuda.empty_cache()
    qwen = None
    if not args.no_qwen:
        qwen, qparams, qinp = bench_qwen(dev, args)
        if not args.no_cpu:
            log("Qwen-Image step CPU baseline (one block, extrapolated)")
            qwen["cpu_baseline"] = cpu_qwen_baseline(qparams, qinp)
            log(f"  CPU: {qwen['cpu_baseline']['value']:.0f} ms ({qwen['cpu_baseline']['sample']})")
        del qparams, qinp
        torch.cuda.empty_cache()
    cpu = None
    if not args.no_cpu:
        log("CPU baseline")
        cpu = cpu_baseline(blocks, x, 21504, 3072)
        log(f"CPU: {cpu['value']:.4f} TFLOP/s ({cpu['sample']})")
    line = {
        "metric": "Q4_K fused-dequant GEMM TFLOP/s at FLUX single-block linear1 (4608x3072->21504)",
        "value": round(gemm["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gemm["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: W ~ N(0, 0.02^2) quantized to Q4_K on the GPU, x ~ N(0, 1) as bf16",
        "config": {"workload": "flux_single_block_linear1_q4k", "m": 4608, "n": 21504, "k": 3072,
                   "weight": "Q4_K", "x": "bf16", "y": "f32"},
        "roofline": {"bound": "mfma", "achieved": round(gemm["kernel_tflops"], 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(gemm["kernel_tflops"] / PEAK_BF16_TFLOPS, 4),
                     "traffic": read_traffic(), "kernel": GEMM_KERNEL,
                     "kernel_ms": round(gemm["kernel_ms"], 4),
                     "algorithmic_flop_per_launch": gemm["flop"], "source_digest": gemm_source_digest()},
        "cpu_baseline": cpu,
        "f32_input": gemm["f32_input"],
        **extra,
        "gemv": gemv,
        "flux_step": flux,
        "qwen_step": qwen,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
