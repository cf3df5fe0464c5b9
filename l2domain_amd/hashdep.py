"""The reference's dependent-probe hash workload (applications/hash/src/hash_probe_dep.cu)
as an input mode: int32 {key, next} entries, two hot pools homed on opposite I/O dies and
chained into cycles, cold keys, serial shuffled CPU build, skewed query stream, and the
chain-following probe in the oblivious / aware / rotated modes ("baseline" / "aware" /
"swapped" in the reference's RESULT line, :367-368).
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib
from ._torch import mode_id, ptr, stream_handle

DEP_SEED = 42          # the reference shuffles with mt19937(42) (HASH.cu:229)
DEP_QSEED = 4242


class DepTable:
    """Device table of `slots` {int32 key, int32 next} entries plus its home map; keys,
    successors and the table contents follow the reference's construction."""

    def __init__(self, K: int, slots: int, H: int, seed: int = DEP_SEED, device: int = 0, map_homes: bool = True):
        if slots & (slots - 1) or K >= slots or 2 * H > K:
            raise ValueError("need slots a power of two, K < slots and 2H <= K")
        self.K, self.slots, self.H = int(K), int(slots), int(H)
        dev = f"cuda:{device}"
        # 2 MiB-aligned table (the reference aligns it the same way, HASH.cu:152-157)
        self._raw = torch.empty(self.slots * 8 + (2 << 20), dtype=torch.uint8, device=dev)
        off = (-self._raw.data_ptr()) % (2 << 20)
        self.table = self._raw[off:off + self.slots * 8].view(torch.int32)
        self.home_attr = None
        attr_host = None
        if map_homes:
            from .domain import home_map
            self.home_attr = home_map(self.table)
            attr_host = np.ascontiguousarray(self.home_attr.cpu().numpy())
        self.keys = np.empty(self.K, dtype=np.int32)
        self.nexts = np.empty(self.K, dtype=np.int32)
        _lib.call("xd_dep_make_keys", self.table.data_ptr(), self.slots,
                  attr_host.ctypes.data if attr_host is not None else None, self.K, self.H,
                  self.keys.ctypes.data, self.nexts.ctypes.data)
        self.host_table = np.empty(2 * self.slots, dtype=np.int32)
        _lib.call("xd_dep_build", self.host_table.ctypes.data, self.slots, self.keys.ctypes.data,
                  self.nexts.ctypes.data, self.K, seed)
        self.table.copy_(torch.from_numpy(self.host_table))

    def queries(self, Q: int, hot_pct: int, seed: int = DEP_QSEED) -> np.ndarray:
        q = np.empty(Q, dtype=np.int32)
        _lib.call("xd_dep_queries", q.ctypes.data, Q, self.keys.ctypes.data, self.K, self.H, hot_pct, seed)
        return q

    def probe(self, queries: torch.Tensor, chain_len: int, mode="aware", out: torch.Tensor | None = None,
              stream=None) -> torch.Tensor:
        n = queries.numel()
        if out is None:
            out = torch.empty(n, dtype=torch.int32, device=queries.device)
        _lib.call("xd_dep_probe", ptr(self.table), self.slots, ptr(queries) if n else None, n, chain_len,
                  ptr(out) if n else None, mode_id(mode), ptr(self.home_attr), stream_handle(stream))
        return out

    def route(self, queries: torch.Tensor, stream=None) -> torch.Tensor:
        """The per-die {key, query id} lists of xd_dep_route (the reference's near/far query
        lists, HASH.cu:244-270), as a device byte buffer for probe_routed()."""
        n = queries.numel()
        buf = torch.empty(int(_lib.lib.xd_dep_route_bytes(n)), dtype=torch.uint8, device=queries.device)
        _lib.call("xd_dep_route", ptr(self.table), self.slots, ptr(queries) if n else None, n, ptr(self.home_attr),
                  ptr(buf), buf.numel(), stream_handle(stream))
        return buf

    def probe_routed(self, route: torch.Tensor, n: int, chain_len: int, mode="aware",
                     out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        """probe_dep_sa (HASH.cu:85-116) over pre-routed lists: die d probes list d (aware)."""
        if out is None:
            out = torch.empty(n, dtype=torch.int32, device=route.device)
        _lib.call("xd_dep_probe_routed", ptr(self.table), self.slots, ptr(route), n, chain_len,
                  ptr(out) if n else None, mode_id(mode), stream_handle(stream))
        return out
