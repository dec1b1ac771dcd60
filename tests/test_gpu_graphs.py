"""GPU tests of mold_amd.graphs.GraphedStep: one FLUX / Qwen-Image forward captured
into a HIP graph.  The captured forward is the eager one (same kernels in the same
order), so every replay must equal the eager forward on the same inputs bit for bit.
Replays run on new inputs each time with eager forwards between them, so a graph
node that kept state from its capture (a stale clear, a cached pointer) would show.
The padded attention's guard inside the graph is checked by forcing it to trip: the
replay then reruns the forward eagerly without padding, as the eager step does."""
import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from mold_amd import flux as F  # noqa: E402
from mold_amd import qwen_image as Q  # noqa: E402

pytestmark = pytest.mark.gpu


def _steps():
    import mold_amd
    dev = mold_amd.Device(0)
    fcfg = F.FluxConfig.tiny()
    qcfg = Q.QwenConfig.tiny()
    return {
        "flux": (F.FluxStep(F.FluxParams.random(fcfg, dev, seed=6)),
                 lambda s: F.make_inputs(fcfg, height=256, width=256, txt_len=32, device="cuda", seed=s)),
        "qwen": (Q.QwenImageStep(Q.QwenParams.random(qcfg, dev, seed=7)),
                 lambda s: Q.make_inputs(qcfg, height=256, width=256, txt_len=32, device="cuda", seed=s)),
    }


@pytest.mark.parametrize("which", ["flux", "qwen"])
def test_graphed_step_equals_eager_forward(which):
    from mold_amd.graphs import GraphedStep
    print(f"[graphs] {which}: capture, then replays against eager forwards", flush=True)
    step, make = _steps()[which]
    g = GraphedStep(step, **make(1))
    for seed in (2, 3, 4):
        inp = make(seed)
        out = g(**inp).clone()
        ref = step.forward(**inp)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all().item()
        assert torch.equal(out, ref), (which, seed)
    # the graph's output tensor is its own: a replay overwrites it
    a = g(**make(5))
    b = g(**make(6)).clone()
    torch.cuda.synchronize()
    assert a.data_ptr() == g.out.data_ptr() and torch.equal(a, b)
    with pytest.raises(ValueError):
        inp = make(7)
        g(**{**inp, "img": inp["img"][:-1]})


def test_graphed_step_guard_reruns_unpadded(monkeypatch):
    """With PAD_MIN_SHARE raised so that any padded row trips the guard, a replay reruns the
    forward unpadded; the eager step (run_guarded) does the same, so both agree bit for bit,
    and both equal the unpadded forward."""
    from mold_amd.graphs import GraphedStep
    step, make = _steps()["flux"]
    g = GraphedStep(step, **make(1))
    monkeypatch.setattr(F, "PAD_MIN_SHARE", 1.0)
    inp = make(2)
    out = g(**inp).clone()
    ref = step.forward(**inp)
    step.pad_attention = False
    try:
        unpadded = step.forward(**inp)
    finally:
        step.pad_attention = True
    torch.cuda.synchronize()
    assert torch.equal(out, ref) and torch.equal(out, unpadded)


def test_graphed_cfg_batch2_equals_eager_forward_batched():
    """Qwen-Image's batched CFG forward (cond + a shorter, masked uncond prompt) captured
    with batched=True: every replay equals the eager forward_batched bit for bit, and a
    txt_valid other than the captured one is refused."""
    from mold_amd.graphs import GraphedStep
    print("[graphs] qwen CFG batch 2: capture, then replays against eager forward_batched", flush=True)
    step, make = _steps()["qwen"]

    def make2(seed):
        inp = make(seed)
        g = torch.Generator(device="cuda").manual_seed(100 + seed)
        txt_u = torch.randn(inp["txt"].shape, device="cuda", generator=g)
        txt_u[27:] = 0.0
        return {"img": torch.stack([inp["img"], inp["img"]]), "txt": torch.stack([inp["txt"], txt_u]),
                "t": torch.cat([inp["t"], inp["t"]]), "grid": inp["grid"], "txt_valid": [32, 27]}

    g = GraphedStep(step, batched=True, **make2(1))
    for seed in (2, 3):
        inp = make2(seed)
        out = g(**inp).clone()
        ref = step.forward_batched(**inp)
        torch.cuda.synchronize()
        assert out.shape == ref.shape and torch.isfinite(out).all().item()
        assert torch.equal(out, ref), seed
    with pytest.raises(ValueError):
        g(**{**make2(4), "txt_valid": [32, 26]})
    for bad in ([32, 0], [33, 27], [32]):     # no valid token, more than L_txt, one count for two
        with pytest.raises(ValueError):
            GraphedStep(step, batched=True, **{**make2(5), "txt_valid": bad})


def test_graphed_cfg_batch2_guard_reruns_unpadded(monkeypatch):
    """The batched capture keeps the guard too: with every padded row tripping it, a replay
    reruns forward_batched unpadded and equals the eager (also rerun) batched forward."""
    from mold_amd.graphs import GraphedStep
    step, make = _steps()["qwen"]
    inp = make(1)
    b = {"img": torch.stack([inp["img"], inp["img"]]), "txt": torch.stack([inp["txt"], inp["txt"]]),
         "t": torch.cat([inp["t"], inp["t"]]), "grid": inp["grid"], "txt_valid": [32, 25]}
    g = GraphedStep(step, batched=True, **b)
    monkeypatch.setattr(F, "PAD_MIN_SHARE", 1.0)
    out = g(**b).clone()
    ref = step.forward_batched(**b)
    step.pad_attention = False
    try:
        unpadded = step.forward_batched(**b)
    finally:
        step.pad_attention = True
    torch.cuda.synchronize()
    assert torch.equal(out, ref) and torch.equal(out, unpadded)
