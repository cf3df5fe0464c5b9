"""BFS parity on the GPU: xd_bfs_csr (through the C ABI) against the oracle's serial queue
BFS (level rule of bfs.cu:215-252). Levels bit-exact."""
import numpy as np
import pytest

import oracle as ora
from l2domain_amd.bfs import RMAT_EDGE_FACTOR, RMAT_SCALE, RMAT_SEED, Graph, rmat_csr

pytestmark = pytest.mark.gpu
MODES = ["oblivious", "aware", "rotated"]


def check(rowptr, col, src, mode, g=None):
    g = g or Graph(rowptr, col)
    level, st = g.bfs(src, mode=mode)
    got = level.cpu().numpy().view(np.uint32)
    ref, reached = ora.bfs(rowptr, col, src)
    np.testing.assert_array_equal(got, ref)
    assert st["reached_vertices"] == reached
    deg = np.diff(rowptr.astype(np.int64))
    assert st["reached_edges"] == int(deg[ref != 0xFFFFFFFF].sum())
    assert st["levels"] == int(ref[ref != 0xFFFFFFFF].max()) + 1
    return st


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("scale,ef,seed,src", [(10, 16, 8201, 0), (12, 8, 1, 3), (14, 16, 5, 100), (16, 4, 8201, 0)])
def test_rmat_small(scale, ef, seed, src, mode):
    rowptr, col = ora.rmat_csr(scale, ef, seed)
    check(rowptr, col, src, mode)


def csr_from_edges(V, edges):
    adj = [set() for _ in range(V)]
    for u, v in edges:
        if u != v:
            adj[u].add(v)
            adj[v].add(u)
    rowptr = np.zeros(V + 1, dtype=np.int32)
    for u in range(V):
        rowptr[u + 1] = rowptr[u] + len(adj[u])
    col = np.array([v for u in range(V) for v in sorted(adj[u])], dtype=np.int32)
    return rowptr, col


@pytest.mark.parametrize("mode", MODES)
def test_shapes(mode):
    # single vertex, no edges
    check(np.zeros(2, dtype=np.int32), np.zeros(0, dtype=np.int32), 0, mode)
    # isolated source in a graph with edges
    r, c = csr_from_edges(100, [(1, 2), (2, 3)])
    check(r, c, 0, mode)
    # long path: many top-down levels
    r, c = csr_from_edges(3000, [(i, i + 1) for i in range(2999)])
    check(r, c, 1500, mode)
    # star with a hub above the grid-wide expansion threshold, plus a tail
    r, c = csr_from_edges(20000, [(0, i) for i in range(1, 19000)] + [(18999 + i, 19000 + i) for i in range(999)])
    st = check(r, c, 0, mode)
    assert st["levels"] >= 3
    # two components
    r, c = csr_from_edges(200, [(i, i + 1) for i in range(99)] + [(100 + i, 101 + i) for i in range(99)])
    check(r, c, 150, mode)
    # dense random graph: bottom-up steps
    rng = np.random.default_rng(0)
    e = rng.integers(0, 5000, size=(200000, 2))
    r, c = csr_from_edges(5000, [tuple(x) for x in e.tolist()])
    st = check(r, c, 7, mode)
    assert st["bottomup_steps"] >= 1


@pytest.mark.parametrize("mode", MODES)
def test_hub_list_unsorted_with_repeats(mode):
    # The grid-wide hub expansion gathers claims over runs of lanes sharing a visited word:
    # every vertex must still be claimed once (level and reached edges exact) when the hub's
    # list is shuffled and repeats entries.
    rng = np.random.default_rng(11)
    V = 12000
    hub = np.arange(1, 10000, dtype=np.int32)
    hub = np.concatenate([hub, rng.choice(hub, 700)])
    rng.shuffle(hub)
    adj = [hub.tolist()] + [[0] for _ in range(1, 10000)] + [[] for _ in range(10000, V)]
    for i in range(9999, V - 1):  # a path 9999 - 10000 - ... - 11999 behind the star
        adj[i].append(i + 1)
        adj[i + 1].append(i)
    rowptr = np.zeros(V + 1, dtype=np.int32)
    rowptr[1:] = np.cumsum([len(a) for a in adj])
    col = np.array([v for a in adj for v in a], dtype=np.int32)
    st = check(rowptr, col, 0, mode)
    assert st["levels"] >= 3
    # the same hub sorted, repeats kept next to their first copy
    adj[0] = sorted(adj[0])
    col = np.array([v for a in adj for v in a], dtype=np.int32)
    check(rowptr, col, 0, mode)


@pytest.fixture(scope="module")
def config_graph():
    rowptr, col = rmat_csr(RMAT_SCALE, RMAT_EDGE_FACTOR, RMAT_SEED)
    ref, reached = ora.bfs(rowptr, col, 0)
    return rowptr, col, ref, reached, Graph(rowptr, col)


def test_config_generator_matches_oracle_edges(config_graph):
    from l2domain_amd import _lib
    import ctypes as C
    for e in (0, 1, 12345, 16 * (1 << 22) - 1):
        u, v = C.c_int32(), C.c_int32()
        _lib.call("xd_rmat_edge", RMAT_SCALE, 0.57, 0.19, 0.19, RMAT_SEED, e, C.byref(u), C.byref(v))
        assert (u.value, v.value) == ora.rmat_edge(RMAT_SCALE, RMAT_SEED, e)


@pytest.mark.parametrize("mode", MODES)
def test_config_rmat22(config_graph, mode):
    rowptr, col, ref, reached, g = config_graph
    level, st = g.bfs(0, mode=mode)
    np.testing.assert_array_equal(level.cpu().numpy().view(np.uint32), ref)
    assert st["reached_vertices"] == reached
    assert st["bottomup_steps"] >= 1 and st["topdown_steps"] >= 1


def test_route_and_per_call_lists_agree():
    # aware/rotated with the prepared route (measured homes) and with per-call lists
    # (address-mask homes, route=None) give the same levels as the serial oracle
    import ctypes as C
    from l2domain_amd import _lib
    from l2domain_amd._torch import mode_id, ptr, stream_handle
    rowptr, col = rmat_csr(14, 8, 99)
    ref, _ = ora.bfs(rowptr, col, 5)
    g = Graph(rowptr, col)
    for mode in ("aware", "rotated"):
        lev, _ = g.bfs(5, mode=mode)
        np.testing.assert_array_equal(lev.cpu().numpy().view(np.uint32), ref)
        st = _lib.BfsStats()
        _lib.call("xd_bfs_csr", ptr(g.rowptr), ptr(g.col), g.V, g.nnz, 5, ptr(g.level), mode_id(mode), None,
                  ptr(g.workspace), g.workspace.numel(), stream_handle(), C.byref(st))
        np.testing.assert_array_equal(g.level.cpu().numpy().view(np.uint32), ref)


def test_concurrent_host_threads():
    """Two host threads search two graphs at once, each on its own stream: the host side's
    pinned control copies and events come from one process-wide pool, one entry per call in
    flight, and every search still matches the oracle."""
    import threading

    import torch
    graphs = [ora.rmat_csr(13, 8, 11), ora.rmat_csr(12, 16, 12)]
    refs = [ora.bfs(r, c, 5)[0] for r, c in graphs]
    gs = [Graph(r, c) for r, c in graphs]
    errors = []

    def worker(i):
        try:
            s = torch.cuda.Stream()
            for k in range(6):
                level, _ = gs[i].bfs(5, mode=MODES[k % 3], stream=s)
                s.synchronize()
                got = level.cpu().numpy().view(np.uint32)
                if not np.array_equal(got, refs[i]):
                    errors.append((i, k))
        except Exception as e:  # reported below
            errors.append((i, repr(e)))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads)
    assert not errors, errors


def _random_graphs(n, seed):
    """Seeded (scale, edge factor, generator seed, source) draws of small R-MAT graphs."""
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(8, 17)), int(rng.integers(1, 33)), int(rng.integers(1, 1 << 30)),
             int(rng.integers(0, 256))) for _ in range(n)]


@pytest.mark.parametrize("scale,ef,seed,src", _random_graphs(8, 2026))
def test_random_rmat_all_modes(scale, ef, seed, src):
    """Seeded random R-MAT graphs (sparse to dense, sources anywhere, isolated ones included):
    levels bit-exact in every mode, from one route built per graph."""
    rowptr, col = ora.rmat_csr(scale, ef, seed)
    src = src % (len(rowptr) - 1)
    g = Graph(rowptr, col)
    for mode in MODES:
        check(rowptr, col, src, mode, g)

