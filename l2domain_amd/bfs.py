"""Direction-optimizing BFS over an undirected CSR graph, the R-MAT generator, and the
reference's own multi-source fixed-depth workload over its hot-pool graph.

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


# The reference's own BFS workload (applications/bfs/run.sh presets; bfs.cu defaults :329-336)
REF_PAPER = dict(vertices=2000000, degree=64, sources=4096, depth=4, dst_local_pct=95, hot_per_side=200000,
                 seed=8201)
REF_QUICK = dict(vertices=65536, degree=8, sources=128, depth=2, dst_local_pct=95, hot_per_side=4096, seed=8201)


def ref_clamp(vertices, degree, sources, depth, dst_local_pct, hot_per_side):
    """The reference's argument clamps (bfs.cu:338-343)."""
    vertices = max(vertices, 4096)
    degree = max(degree, 1)
    sources = max(1, min(sources, vertices // 4))
    depth = max(1, depth)
    dst_local_pct = max(0, min(dst_local_pct, 100))
    hot_per_side = max(1024, min(hot_per_side, vertices // 3))
    return vertices, degree, sources, depth, dst_local_pct, hot_per_side


class RefGraph:
    """The reference's directed hot-pool graph (xd_bfs_ref_graph), resident on the device with
    the buffers it was generated for: the sides of its vertices come from the measured homes
    of its own col and level arrays, as the reference derives them from its buffers."""

    def __init__(self, vertices: int, degree: int, sources: int, dst_local_pct: int, hot_per_side: int,
                 seed: int = 8201, device: int | str = 0, map_homes: bool = True):
        from .domain import home_map
        dev = torch.device(f"cuda:{device}" if isinstance(device, int) else device)
        V = self.V = int(vertices)
        self.degree, self.nsrc = int(degree), int(sources)
        self.nnz = V * self.degree
        self.col = torch.empty(max(self.nnz, 1), dtype=torch.int32, device=dev)
        self.level = torch.empty(V, dtype=torch.int32, device=dev)
        ch = home_map(self.col).cpu().numpy() if map_homes else None
        lh = home_map(self.level).cpu().numpy() if map_homes else None
        self.col_home, self.level_home = ch, lh
        self.h_rowptr = np.empty(V + 1, dtype=np.int32)
        self.h_col = np.empty(self.nnz, dtype=np.int32)
        self.h_work_side = np.empty(V, dtype=np.uint8)
        self.h_sources = np.empty(max(self.nsrc, 1), dtype=np.int32)
        _lib.call("xd_bfs_ref_graph", V, self.degree, self.nsrc, dst_local_pct, hot_per_side, seed, ptr(self.col),
                  None if ch is None else ch.ctypes.data, ptr(self.level), None if lh is None else lh.ctypes.data,
                  self.h_rowptr.ctypes.data, self.h_col.ctypes.data, self.h_work_side.ctypes.data,
                  self.h_sources.ctypes.data)
        self.h_sources = self.h_sources[: self.nsrc]
        self.col[: self.nnz].copy_(torch.from_numpy(self.h_col))
        self.rowptr = torch.from_numpy(self.h_rowptr).to(dev)
        self.work_side = torch.from_numpy(self.h_work_side).to(dev)
        self.sources = torch.from_numpy(self.h_sources).to(dev)
        ws = int(_lib.lib.xd_bfs_multi_workspace_size(V))
        self.workspace = torch.empty(ws, dtype=torch.uint8, device=dev)

    def bfs(self, max_depth: int, mode="aware", level: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        out = self.level if level is None else level
        _lib.call("xd_bfs_multi", ptr(self.rowptr), ptr(self.col), self.V, self.nnz, ptr(self.sources), self.nsrc,
                  max_depth, ptr(self.work_side), ptr(out), mode_id(mode), ptr(self.workspace),
                  self.workspace.numel(), stream_handle(stream))
        return out


def bfs_multi(rowptr: torch.Tensor, col: torch.Tensor, sources: torch.Tensor, max_depth: int, mode="oblivious",
              work_side: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Multi-source fixed-depth BFS over any directed device CSR (xd_bfs_multi)."""
    V = rowptr.numel() - 1
    ws = torch.empty(int(_lib.lib.xd_bfs_multi_workspace_size(V)), dtype=torch.uint8, device=rowptr.device)
    level = torch.empty(V, dtype=torch.int32, device=rowptr.device)
    _lib.call("xd_bfs_multi", ptr(rowptr), ptr(col) if col.numel() else None, V, col.numel(),
              ptr(sources) if sources.numel() else None, sources.numel(), max_depth, ptr(work_side), ptr(level),
              mode_id(mode), ptr(ws), ws.numel(), stream_handle(stream))
    return level
