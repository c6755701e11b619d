"""Shared helpers of the GPU tests: device buffers from numpy, and the stream binding."""
from __future__ import annotations

import sys

import numpy as np
import torch

from blog_amd import qlin


def banner(msg: str) -> None:
    """Names the case before a GPU step, flushed, so a crash can be attributed."""
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


def dev(a: np.ndarray) -> torch.Tensor:
    """Copies a numpy array to the GPU as a tensor of the same bytes (uint8 / float32 / int32 / uint16)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16))
    else:
        t = torch.from_numpy(a)
    return t.to("cuda")


def host(t: torch.Tensor, dtype=None) -> np.ndarray:
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def empty_f32(*shape) -> torch.Tensor:
    return torch.full(shape, float("nan"), dtype=torch.float32, device="cuda")


def bind_stream() -> None:
    qlin.set_stream(torch.cuda.current_stream())
