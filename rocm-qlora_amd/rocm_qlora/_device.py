"""Device placement for the codec entry points.

The reference's codecs run on whatever device the tensor is on
(quant_ops.py:86-87).  Here every codec runs as a HIP kernel: GPU tensors are
processed in place; CPU tensors are staged to the current GPU, processed by
the same kernels, and the results copied back, so callers that quantize
CPU-resident weights (model loading) keep working.  Without a GPU the codecs
raise: there is no CPU implementation in this package.
"""
from __future__ import annotations

from contextlib import contextmanager
from typing import Tuple

import torch


def gpu_device_for(t: torch.Tensor) -> torch.device:
    if t.device.type == "cuda":
        return t.device
    if not torch.cuda.is_available():
        raise RuntimeError(
            "rocm_qlora_amd runs its codecs and linears as HIP kernels on an AMD GPU; "
            f"no GPU is available for a tensor on {t.device}")
    return torch.device("cuda", torch.cuda.current_device())


def to_gpu(t: torch.Tensor) -> Tuple[torch.Tensor, torch.device]:
    """Return (tensor on a GPU, original device)."""
    dev = gpu_device_for(t)
    return (t if t.device == dev else t.to(dev)), t.device


@contextmanager
def on(device: torch.device):
    with torch.cuda.device(device):
        yield
