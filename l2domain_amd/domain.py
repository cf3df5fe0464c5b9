"""Domain runtime: device topology, DomainScan (workgroup -> XCD map) and cache flush.

Replaces the reference's latency-probed SM->side calibration (utility/latopt.cuh:487-562,
utility/get_smid2side.cu) and its L2 reset (utility/latopt.cuh:103-134).
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from ._torch import ptr, stream_handle


def topology(device: int = 0) -> dict:
    t = _lib.Topology()
    _lib.call("xd_topology_query", device, C.byref(t))
    return {"device": t.device, "num_cu": t.num_cu, "num_xcd": t.num_xcd, "cu_per_xcd": t.cu_per_xcd,
            "wave_size": t.wave_size, "clock_khz": t.clock_khz, "l2_bytes": t.l2_bytes,
            "lds_bytes_per_wg": t.lds_bytes_per_wg, "hbm_bytes": t.hbm_bytes,
            "arch": t.arch.decode(), "name": t.name.decode()}


def decode_placement(word: int) -> dict:
    return {"xcc": (word >> 24) & 0xFF, "se": (word >> 16) & 0xFF, "sh": (word >> 12) & 0xF,
            "cu": (word >> 8) & 0xF, "simd": word & 0xFF}


def domain_scan(num_wg: int, device: int = 0) -> torch.Tensor:
    """Runs DomainScan over `num_wg` workgroups; returns the uint32 placement words (CPU)."""
    out = torch.zeros(num_wg, dtype=torch.int32, device=f"cuda:{device}")
    _lib.call("xd_domain_scan", num_wg, ptr(out), stream_handle())
    torch.cuda.synchronize()
    return out.cpu().view(torch.int32)


class CacheFlusher:
    """Owns the read-stream buffer used to evict the L2s and the Infinity Cache."""

    def __init__(self, device: int = 0):
        self.bytes = int(_lib.lib.xd_cache_flush_bytes())
        self.buf = torch.ones(self.bytes // 4, dtype=torch.int32, device=f"cuda:{device}")

    def flush(self, stream: torch.cuda.Stream | None = None) -> None:
        _lib.call("xd_cache_flush", ptr(self.buf), self.bytes, stream_handle(stream))


def home_map(buf: torch.Tensor, return_latency: bool = False):
    """Measured die (0/1) of every 2 MiB page overlapping `buf` (uint8 device tensor); with
    return_latency, also the (pages, 2) cycle counts of die 0 and die 1."""
    nbytes = buf.numel() * buf.element_size()
    npages = int(_lib.lib.xd_home_map_pages(ptr(buf), nbytes))
    attr = torch.empty(npages, dtype=torch.uint8, device=buf.device)
    ws = torch.empty(int(_lib.lib.xd_home_map_workspace_size(ptr(buf), nbytes)) // 4 + 1, dtype=torch.int32,
                     device=buf.device)
    _lib.call("xd_home_map", ptr(buf), nbytes, ptr(attr), ptr(ws), ws.numel() * 4, stream_handle())
    if return_latency:
        return attr, ws[: 2 * npages].view(npages, 2)
    return attr


def home_parity(buf: torch.Tensor, mask: int | None = None) -> list[int]:
    """Die predicted by the address-bit mask for the first 8 KiB of every 2 MiB page of buf."""
    m = int(_lib.lib.xd_home_mask()) if mask is None else mask
    lo = ptr(buf)
    page0 = lo >> 21
    npages = int(_lib.lib.xd_home_map_pages(lo, buf.numel() * buf.element_size()))
    return [bin(((page0 + p) << 21) & m).count("1") & 1 for p in range(npages)]
