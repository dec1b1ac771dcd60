"""One denoising forward of a DiT step captured into a HIP graph and replayed.

A step's forward is ~600 (FLUX.1-dev) to ~1300 (Qwen-Image) kernel launches,
many of them short glue kernels; launched from Python, the GPU waits on the
host between some of them (a few ms per step).  `GraphedStep` captures one
forward of a `FluxStep` / `QwenImageStep` (both token streams, the fused glue,
the quantized linears through libmoldq, PyTorch's attention) into one graph and
replays it per denoising step, after copying the step's inputs into the
captured input tensors.

The captured forward is the eager one (same kernels, same order, same values);
before capture it runs twice eagerly on the capture stream, which builds the
stacked modulation weight and grows libmoldq's per-stream workspaces to what
the forward needs, so no call inside the capture allocates device memory.  The
padded attention's guard is a captured tensor cleared at the start of every
replay; after a replay one host synchronization reads it, and if some padded
row's valid-key share fell below flux.PAD_MIN_SHARE the step runs again eagerly
with unpadded attention (exact), as `run_guarded` does for the eager forward.

The output tensor belongs to the graph and is overwritten by the next replay.
Non-tensor arguments (Qwen-Image's `grid`, the batched forward's `txt_valid`)
and tensor shapes are fixed at capture.  With `batched=True` the captured
forward is QwenImageStep.forward_batched (classifier-free guidance's cond and
uncond in one batch-2 forward).
"""
from __future__ import annotations


class GraphedStep:
    """`step` (a FluxStep or QwenImageStep) with its forward on `inputs` (the keyword
    arguments of step.forward, e.g. flux.make_inputs(...)) captured into a HIP graph.
    Call it with inputs of the same shapes to run one forward."""

    def __init__(self, step, batched: bool = False, **inputs):
        import torch
        from .flux import attention_bf16
        self.step = step
        self.batched = batched
        self.static = {k: (v.detach().clone() if torch.is_tensor(v) else v) for k, v in inputs.items()}
        if batched:
            if not hasattr(step, "_forward_batched"):
                raise ValueError(f"GraphedStep: {type(step).__name__} has no batched forward")
            img = self.static["img"]
            b, lt = self.static["txt"].shape[0], self.static["txt"].shape[1]
            if not step._fused(img.reshape(b * img.shape[1], -1)):
                raise ValueError("GraphedStep: the batched forward runs on the GPU with bf16 GEMM inputs")
            tv = self.static.pop("txt_valid", None)
            self.valid = [lt] * b if tv is None else [int(v) for v in tv]
            if len(self.valid) != b or any(v < 1 or v > lt for v in self.valid):
                raise ValueError("GraphedStep: txt_valid needs one count in 1 .. L_txt per batch element")
        dev = next(v.device for v in self.static.values() if torch.is_tensor(v))
        self.guarded = step.attn is attention_bf16 and step.pad_attention
        self.guard = torch.zeros((), dtype=torch.float32, device=dev)
        self.stream = torch.cuda.Stream(device=dev)
        self.graph = torch.cuda.CUDAGraph()
        step._guard = self.guard if self.guarded else None
        try:
            self.stream.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(self.stream):
                for _ in range(2):
                    self._forward()
            torch.cuda.current_stream(dev).wait_stream(self.stream)
            torch.cuda.synchronize(dev)
            with torch.cuda.graph(self.graph, stream=self.stream):
                self.out = self._forward()
        finally:
            step._guard = None

    def _forward(self):
        self.guard.zero_()
        return self._eager()

    def _eager(self):
        s = self.static
        if self.batched:
            return self.step._forward_batched(s["img"], s["txt"], s["t"], s["grid"], self.valid, None)
        return self.step._forward(**s, blocks=None)

    def __call__(self, **inputs):
        import torch
        from .flux import PAD_MIN_SHARE
        for k, v in inputs.items():
            if self.batched and k == "txt_valid":
                if v is not None and [int(c) for c in v] != self.valid:
                    raise ValueError(f"GraphedStep: txt_valid = {v!r}, captured {self.valid!r}")
                continue
            s = self.static[k]
            if torch.is_tensor(v):
                if v.shape != s.shape:
                    raise ValueError(f"GraphedStep: {k} has shape {tuple(v.shape)}, captured {tuple(s.shape)}")
                s.copy_(v)
            elif v != s:
                raise ValueError(f"GraphedStep: {k} = {v!r}, captured {s!r}")
        self.graph.replay()
        if self.guarded and float(self.guard) > 1.0 - PAD_MIN_SHARE:
            # a padded row lost its precision: this forward again, eager and unpadded
            st = self.step
            st.pad_attention = False
            try:
                return self._eager()
            finally:
                st.pad_attention = True
        return self.out
