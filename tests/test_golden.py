"""Golden fixtures (tests/golden/*.npz) against the oracle, the product's host-side
generators and methods independent of both.

The fixtures were written by tests/golden/make_fixtures.py after the same independent checks;
a change to the oracle, to a generator or to a seed that alters any output fails here."""
from pathlib import Path

import numpy as np
import pytest

import oracle as ora

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_gemv_f32_fixture():
    d = load("gemv_f32_64x256.npz")
    A, x = d["A"], d["x"]
    np.testing.assert_array_equal(ora.uniform_f32(A.size, 4242).reshape(A.shape), A)
    np.testing.assert_array_equal(ora.uniform_f32(x.size, 4242 + 0x9E37), x)
    y64, _ = ora.gemv_f64(A, x)
    np.testing.assert_array_equal(y64, d["y64"])
    np.testing.assert_array_equal(ora.gemv_f32_seq(A, x), d["yseq"])
    np.testing.assert_allclose(d["y64"], A.astype(np.float64) @ x.astype(np.float64), rtol=0, atol=1e-12)
    # every U[-1,1) value lies on the 2^-23 grid
    assert np.all(np.abs(A) <= 1.0) and np.all((A.astype(np.float64) * 2**23) % 1 == 0)


def test_gemv_f16_fixture():
    d = load("gemv_f16_64x256.npz")
    W, x = d["W"], d["x"]
    np.testing.assert_array_equal(ora.normal_f16(W.size, 0.0, 0.02, 4243).view(np.uint16),
                                  W.reshape(-1).view(np.uint16))
    np.testing.assert_array_equal(ora.normal_f16(x.size, 0.0, 1.0, 4244).view(np.uint16), x.view(np.uint16))
    y64, _ = ora.gemv_f64(W, x)
    np.testing.assert_array_equal(y64, d["y64"])
    np.testing.assert_allclose(y64, W.astype(np.float64) @ x.astype(np.float64), rtol=0, atol=1e-12)


def test_gemv_int_fixture():
    d = load("gemv_int_64x256.npz")
    np.testing.assert_array_equal(ora.gemv_f32_seq(d["A"], d["x"]), d["y"])
    np.testing.assert_array_equal((d["A"].astype(np.int64) @ d["x"].astype(np.int64)).astype(np.float32), d["y"])


@pytest.mark.parametrize("name", ["hist_zipf_2p16_2p10.npz", "hist_uniform_2p16_2p10.npz"])
def test_hist_fixture(name):
    d = load(name)
    keys, counts = d["keys"], d["counts"]
    got, c = ora.histogram(keys, counts.size)
    assert c == keys.size
    np.testing.assert_array_equal(got, counts)
    np.testing.assert_array_equal(np.bincount(keys, minlength=counts.size).astype(np.uint32), counts)
    assert int(counts.sum()) == keys.size


def test_hist_zipf_fixture_keys_regenerate():
    d = load("hist_zipf_2p16_2p10.npz")
    t = ora.zipf_thresholds(1 << 10, 1.1)
    np.testing.assert_array_equal(ora.zipf_keys(1 << 16, t, 1373, scramble=True), d["keys"])


def test_hash_fixture():
    d = load("hash_2p12.npz")
    keys, vals, q = d["keys"], d["vals"], d["queries"]
    k2, v2 = ora.hash_kv(keys.size, 42)
    np.testing.assert_array_equal(k2, keys)
    np.testing.assert_array_equal(v2, vals)
    np.testing.assert_array_equal(ora.hash_queries(q.size, keys.size, 42, 4242), q)
    t = ora.HashTable(2 * keys.size)
    assert t.build(keys, vals) == 0
    vo, fo = t.lookup(q)
    np.testing.assert_array_equal(fo, d["found"])
    np.testing.assert_array_equal(vo, d["vals_out"])
    ref = dict(zip(keys.tolist(), vals.tolist()))
    assert [int(k in ref) for k in q.tolist()] == d["found"].tolist()


def test_bfs_fixture():
    from scipy.sparse import csr_matrix
    from scipy.sparse.csgraph import shortest_path
    d = load("bfs_rmat10.npz")
    rowptr, col = ora.rmat_csr(10, 16, 8201)
    np.testing.assert_array_equal(rowptr, d["rowptr"])
    np.testing.assert_array_equal(col, d["col"])
    level, _ = ora.bfs(rowptr, col, 0)
    np.testing.assert_array_equal(level, d["level"])
    V = rowptr.size - 1
    dist = shortest_path(csr_matrix((np.ones(col.size), col, rowptr), shape=(V, V)), unweighted=True, indices=0)
    np.testing.assert_array_equal(np.where(np.isinf(dist), 0xFFFFFFFF, dist).astype(np.uint32), d["level"])


def test_product_host_generators_match_fixtures():
    """The library's own host generators (libxdom, no oracle code) reproduce the fixture inputs."""
    from l2domain_amd import gen
    from l2domain_amd.bfs import rmat_csr
    d = load("gemv_f32_64x256.npz")
    A, x = gen.gemv_f32_inputs(64, 256)
    np.testing.assert_array_equal(A, d["A"])
    np.testing.assert_array_equal(x, d["x"])
    h = load("gemv_f16_64x256.npz")
    W, xh = gen.gemv_f16_inputs(64, 256)
    np.testing.assert_array_equal(W.view(np.uint16), h["W"].view(np.uint16))
    np.testing.assert_array_equal(xh.view(np.uint16), h["x"].view(np.uint16))
    b = load("bfs_rmat10.npz")
    rp, col = rmat_csr(10, 16, 8201)
    np.testing.assert_array_equal(rp, b["rowptr"])
    np.testing.assert_array_equal(col, b["col"])
    t = np.asarray(gen.zipf_thresholds(1 << 10, 1.1))
    np.testing.assert_array_equal(t, ora.zipf_thresholds(1 << 10, 1.1))
