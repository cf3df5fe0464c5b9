"""GPU open-addressing hash table of uint64 keys and values (linear probing).

Mirrors the reference's hash application (applications/hash/src/hash_probe_dep.cu):
"baseline"/"oblivious" is probe_dep_base (:66-83), "aware" the side-routed probe_dep_sa
(:85-116) -- here the keys are routed to the I/O die that homes their slot -- and
"swapped"/"rotated" its swapped launch (:317-323). The reference builds the table on the
CPU (:226-241); this table is filled on the GPU, by `build` (the whole table from scratch, range
by range in LDS) or by `insert` (compare-and-swap claims into a table that may hold keys).
"""
from __future__ import annotations

import torch

from . import _lib
from ._torch import mode_id, ptr, stream_handle

EMPTY = 0xFFFFFFFFFFFFFFFF
HASH_KEYS = 1 << 26        # BASELINE config: 2^26 inserts at load factor 0.5
HASH_SLOTS = 1 << 27
HASH_SEED = 42             # the reference shuffles with mt19937(42) (HASH.cu:229)
HASH_QSEED = 4242


class HashTable:
    """Table storage plus the measured home map of its pages (xd_home_map), which the
    aware/rotated modes use to route each key to the die that homes its slot."""

    def __init__(self, slots: int, device: int | str = 0, stream=None, map_homes: bool = True):
        if slots < 1 or slots & (slots - 1):
            raise ValueError("slots must be a power of two")
        self.slots = int(slots)
        dev = torch.device(f"cuda:{device}" if isinstance(device, int) else device)
        nbytes = int(_lib.lib.xd_hash_table_bytes(self.slots))
        self.table = torch.empty(nbytes // 8, dtype=torch.int64, device=dev)
        self.failed = torch.zeros(1, dtype=torch.int64, device=dev)
        self._build_ws = None
        self.clear(stream)
        self.home_attr = None
        if map_homes:
            from .domain import home_map
            self.home_attr = home_map(self.table)

    def clear(self, stream=None) -> None:
        _lib.call("xd_hash_init", ptr(self.table), self.slots, stream_handle(stream))
        self.failed.zero_()

    def insert(self, keys: torch.Tensor, vals: torch.Tensor, mode="aware", stream=None) -> None:
        n = keys.numel()
        if vals.numel() != n or keys.element_size() != 8 or vals.element_size() != 8:
            raise ValueError("keys and vals must be equal-length 64-bit tensors")
        _lib.call("xd_hash_insert_u64", ptr(self.table), self.slots, ptr(keys) if n else None,
                  ptr(vals) if n else None, n, mode_id(mode), ptr(self.home_attr), ptr(self.failed),
                  stream_handle(stream))

    def build(self, keys: torch.Tensor, vals: torch.Tensor, mode="aware", stream=None) -> None:
        """Replaces the table's contents by the pairs (xd_hash_build_u64): the same lookups as
        clear() followed by insert(). The workspace is kept for later builds of up to as
        many pairs."""
        n = keys.numel()
        if vals.numel() != n or keys.element_size() != 8 or vals.element_size() != 8:
            raise ValueError("keys and vals must be equal-length 64-bit tensors")
        need = int(_lib.lib.xd_hash_build_workspace_size(n, self.slots))
        if need and (self._build_ws is None or self._build_ws.numel() < need):
            self._build_ws = None
            self._build_ws = torch.empty(need, dtype=torch.uint8, device=self.table.device)
        ws = self._build_ws if need else None
        _lib.call("xd_hash_build_u64", ptr(self.table), self.slots, ptr(keys) if n else None,
                  ptr(vals) if n else None, n, mode_id(mode), ptr(self.home_attr), ptr(ws),
                  ws.numel() if ws is not None else 0, ptr(self.failed), stream_handle(stream))

    def lookup(self, queries: torch.Tensor, mode="aware", vals_out=None, found_out=None, stream=None):
        n = queries.numel()
        if vals_out is None:
            vals_out = torch.empty(n, dtype=torch.int64, device=queries.device)
        if found_out is None:
            found_out = torch.empty(n, dtype=torch.uint8, device=queries.device)
        _lib.call("xd_hash_lookup_u64", ptr(self.table), self.slots, ptr(queries) if n else None, n,
                  ptr(vals_out) if n else None, ptr(found_out) if n else None, mode_id(mode),
                  ptr(self.home_attr), stream_handle(stream))
        return vals_out, found_out

    def failures(self) -> int:
        return int(self.failed.item())


def gen_kv(n: int, seed: int = HASH_SEED, device="cuda"):
    keys = torch.empty(n, dtype=torch.int64, device=device)
    vals = torch.empty(n, dtype=torch.int64, device=device)
    _lib.call("xd_gen_hash_kv", ptr(keys) if n else None, ptr(vals) if n else None, n, seed, stream_handle())
    return keys, vals


def gen_queries(n: int, n_keys: int, seed: int = HASH_SEED, qseed: int = HASH_QSEED, device="cuda"):
    q = torch.empty(n, dtype=torch.int64, device=device)
    _lib.call("xd_gen_hash_queries", ptr(q) if n else None, n, n_keys, seed, qseed, stream_handle())
    return q
