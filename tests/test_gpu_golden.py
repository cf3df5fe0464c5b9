"""The HIP path (through the C ABI) reproduces every golden fixture, in all three modes."""
from pathlib import Path

import numpy as np
import pytest
import torch

from l2domain_amd.bfs import Graph
from l2domain_amd.gemv import gemv
from l2domain_amd.hashtable import HashTable
from l2domain_amd.histogram import Histogram

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
MODES = ["oblivious", "aware", "rotated"]


def load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("mode", MODES)
def test_gemv_fixtures(mode):
    d = load("gemv_f32_64x256.npz")
    y = gemv(torch.from_numpy(d["A"]).cuda(), torch.from_numpy(d["x"]).cuda(), mode=mode).cpu().numpy()
    assert np.max(np.abs(y - d["y64"])) / np.max(np.abs(d["y64"])) <= 1e-3
    assert np.max(np.abs(y - d["yseq"])) <= 1e-3
    h = load("gemv_f16_64x256.npz")
    y = gemv(torch.from_numpy(h["W"]).cuda(), torch.from_numpy(h["x"]).cuda(), mode=mode).cpu().numpy()
    assert np.max(np.abs(y - h["y64"])) / np.max(np.abs(h["y64"])) <= 2e-2
    i = load("gemv_int_64x256.npz")
    y = gemv(torch.from_numpy(i["A"]).cuda(), torch.from_numpy(i["x"]).cuda(), mode=mode).cpu().numpy()
    np.testing.assert_array_equal(y, i["y"])


@pytest.mark.parametrize("name", ["hist_zipf_2p16_2p10.npz", "hist_uniform_2p16_2p10.npz"])
@pytest.mark.parametrize("mode", MODES)
def test_hist_fixtures(name, mode):
    d = load(name)
    keys = torch.from_numpy(d["keys"].view(np.int32)).cuda()
    h = Histogram(keys.numel(), d["counts"].size)
    got = h(keys, mode=mode).cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(got, d["counts"])


@pytest.mark.parametrize("mode", MODES)
def test_hash_fixture(mode):
    d = load("hash_2p12.npz")
    t = HashTable(2 * d["keys"].size)
    t.insert(torch.from_numpy(d["keys"].view(np.int64)).cuda(), torch.from_numpy(d["vals"].view(np.int64)).cuda(),
             mode=mode)
    v, f = t.lookup(torch.from_numpy(d["queries"].view(np.int64)).cuda(), mode=mode)
    assert t.failures() == 0
    np.testing.assert_array_equal(f.cpu().numpy(), d["found"])
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint64), d["vals_out"])


@pytest.mark.parametrize("mode", MODES)
def test_bfs_fixture(mode):
    d = load("bfs_rmat10.npz")
    g = Graph(d["rowptr"], d["col"])
    lev, st = g.bfs(0, mode=mode)
    np.testing.assert_array_equal(lev.cpu().numpy().view(np.uint32), d["level"])
    assert st["reached_vertices"] == int(np.sum(d["level"] != 0xFFFFFFFF))
