"""Small helpers that turn torch tensors and streams into the raw pointers the C ABI takes."""
from __future__ import annotations

import torch

from ._lib import MODES


def ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("expected a device tensor")
    if not t.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return t.data_ptr()


def stream_handle(stream: torch.cuda.Stream | None = None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def mode_id(mode: int | str) -> int:
    if isinstance(mode, str):
        return MODES[mode]
    return int(mode)
