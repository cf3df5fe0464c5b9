"""Large-bin histogram of uint32 keys (one bin per key value).

Mirrors the reference histogram application
(applications/histogram/src/histogram256_sideaware.cu): "baseline"/"oblivious" is the
locality-oblivious launch (histogram256_chunked_kernel, :51-85), "aware" routes bin ranges
to the XCD that owns them (the persistent side-routed kernel, :87-134), "swapped"/"rotated"
is its reverse=1 launch (:110). The merge (merge_histogram256_kernel, :136-157) is part of
the call here.
"""
from __future__ import annotations

import torch

from . import _lib
from ._torch import mode_id, ptr, stream_handle

HIST_BINS = 1 << 20        # BASELINE config: 2^20 bins (4 MiB of u32 counters)
HIST_KEYS = 1 << 28
HIST_SEED = 1373
ZIPF_S = 1.1


class Histogram:
    """Owns the workspace of xd_hist_u32 for inputs of up to `max_keys` keys. `home_attr` is
    the xd_home_map of the keys buffer the aware and rotated modes route by (None: the
    address-mask prediction)."""

    def __init__(self, max_keys: int, num_bins: int, device: int | str = 0):
        self.num_bins = int(num_bins)
        self.max_keys = int(max_keys)
        nbytes = int(_lib.lib.xd_hist_workspace_size(self.max_keys, self.num_bins))
        if nbytes == 0:
            raise ValueError(f"num_bins {num_bins} out of range")
        dev = torch.device(f"cuda:{device}" if isinstance(device, int) else device)
        # zeroed once; the library leaves it zeroed after every call
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)

    def __call__(self, keys: torch.Tensor, counts: torch.Tensor | None = None, mode="aware",
                 home_attr: torch.Tensor | None = None, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        if keys.dtype not in (torch.int32, torch.uint32) or keys.dim() != 1:
            raise TypeError("keys must be a 1-D 32-bit integer tensor")
        n = keys.numel()
        if n > self.max_keys:
            raise ValueError("more keys than the workspace was sized for")
        if counts is None:
            counts = torch.empty(self.num_bins, dtype=torch.int32, device=keys.device)
        if counts.numel() != self.num_bins or counts.element_size() != 4:
            raise ValueError("counts must hold num_bins 32-bit counters")
        _lib.call("xd_hist_u32", ptr(keys) if n else None, n, ptr(counts), self.num_bins, mode_id(mode),
                  ptr(home_attr), ptr(self.workspace), self.workspace.numel(), stream_handle(stream))
        return counts


def histogram(keys: torch.Tensor, num_bins: int, mode="aware") -> torch.Tensor:
    return Histogram(max(keys.numel(), 1), num_bins, keys.device)(keys, mode=mode)


class ByteHistogram:
    """The reference's own histogram: 256 bins, every byte of every uint32 word counted
    (add_word, histogram256_sideaware.cu:20-25). Owns the workspace of xd_hist256_u32bytes;
    `home_attr` is the xd_home_map of the words buffer the aware mode routes by."""

    def __init__(self, device: int | str = 0):
        dev = torch.device(f"cuda:{device}" if isinstance(device, int) else device)
        nbytes = int(_lib.lib.xd_hist256_workspace_size())
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)  # left zeroed by every call

    def __call__(self, words: torch.Tensor, counts: torch.Tensor | None = None, mode="aware",
                 home_attr: torch.Tensor | None = None, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        if words.dtype not in (torch.int32, torch.uint32) or words.dim() != 1:
            raise TypeError("words must be a 1-D 32-bit integer tensor")
        n = words.numel()
        if counts is None:
            counts = torch.empty(256, dtype=torch.int32, device=words.device)
        if counts.numel() != 256 or counts.element_size() != 4:
            raise ValueError("counts must hold 256 32-bit counters")
        _lib.call("xd_hist256_u32bytes", ptr(words) if n else None, n, ptr(counts), mode_id(mode),
                  ptr(home_attr), ptr(self.workspace), self.workspace.numel(), stream_handle(stream))
        return counts
