"""Direction-optimizing BFS over an undirected CSR graph, and the R-MAT generator.

Mirrors the reference BFS application (applications/bfs/src/bfs.cu): "baseline"/"oblivious"
is the all-SM launch (luo_baseline_level_kernel, :215-252), "aware" the per-side launch
(luo_side_level_kernel, :254-308) -- here the per-I/O-die routing of bottom-up work by the
home of the adjacency chunk -- and "swapped"/"rotated" its inverted launch (:262).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib
from ._torch import mode_id, ptr, stream_handle

UNVISITED = 0xFFFFFFFF
RMAT_SCALE = 22
RMAT_EDGE_FACTOR = 16
RMAT_ABC = (0.57, 0.19, 0.19)
RMAT_SEED = 8201             # applications/bfs/run.sh:18


def rmat_csr(scale: int = RMAT_SCALE, edge_factor: int = RMAT_EDGE_FACTOR, seed: int = RMAT_SEED, abc=RMAT_ABC):
    """Host CSR (rowptr int32[V+1], col int32[nnz]) of the undirected R-MAT graph."""
    V = 1 << scale
    rowptr = np.empty(V + 1, dtype=np.int32)
    col = np.empty(2 * edge_factor * V, dtype=np.int32)
    nnz = C.c_int64()
    _lib.call("xd_rmat_csr", scale, edge_factor, *abc, seed, rowptr.ctypes.data, col.ctypes.data, col.size,
              C.byref(nnz))
    return rowptr, col[: nnz.value].copy()


class Graph:
    """CSR graph resident on the device, with its BFS workspace and its route (the per-die
    block lists of xd_bfs_route, built once from the measured home map of col)."""

    def __init__(self, rowptr: np.ndarray, col: np.ndarray, device: int | str = 0, map_homes: bool = True):
        dev = torch.device(f"cuda:{device}" if isinstance(device, int) else device)
        self.V = int(rowptr.size - 1)
        self.nnz = int(col.size)
        self.rowptr = torch.from_numpy(np.ascontiguousarray(rowptr, dtype=np.int32)).to(dev)
        self.col = torch.from_numpy(np.ascontiguousarray(col, dtype=np.int32)).to(dev) if self.nnz else \
            torch.empty(1, dtype=torch.int32, device=dev)
        ws = int(_lib.lib.xd_bfs_workspace_size(self.V, self.nnz))
        self.workspace = torch.empty(ws, dtype=torch.uint8, device=dev)
        self.level = torch.empty(self.V, dtype=torch.int32, device=dev)
        self.home_attr = None
        if map_homes and self.nnz:
            from .domain import home_map
            self.home_attr = home_map(self.col)
        self.route = torch.empty(int(_lib.lib.xd_bfs_route_bytes(self.V)), dtype=torch.uint8, device=dev)
        _lib.call("xd_bfs_route", ptr(self.rowptr), ptr(self.col) if self.nnz else None, self.V, self.nnz,
                  ptr(self.home_attr), ptr(self.route), self.route.numel(), stream_handle())

    def bfs(self, src: int, mode="aware", stream=None) -> tuple[torch.Tensor, dict]:
        st = _lib.BfsStats()
        _lib.call("xd_bfs_csr", ptr(self.rowptr), ptr(self.col) if self.nnz else None, self.V, self.nnz, src,
                  ptr(self.level), mode_id(mode), ptr(self.route), ptr(self.workspace), self.workspace.numel(),
                  stream_handle(stream), C.byref(st))
        return self.level, {"levels": st.levels, "topdown_steps": st.topdown_steps,
                            "bottomup_steps": st.bottomup_steps, "reached_vertices": st.reached_vertices,
                            "reached_edges": st.reached_edges}
