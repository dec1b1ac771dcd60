"""Host-side argument checks of mold_amd.graphs.GraphedStep that run before any GPU
work: a batched capture of a step without a batched forward (FLUX) is refused."""
import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from mold_amd.graphs import GraphedStep  # noqa: E402


class _NoBatch:
    attn = None
    pad_attention = False


def test_batched_capture_needs_a_batched_forward():
    inp = {"img": torch.zeros(2, 4, 8), "txt": torch.zeros(2, 3, 8), "t": torch.zeros(2), "grid": (2, 2)}
    with pytest.raises(ValueError, match="no batched forward"):
        GraphedStep(_NoBatch(), batched=True, **inp)
