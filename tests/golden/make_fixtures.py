"""Writes the small golden fixtures of this directory (run from the repository root:
`python tests/golden/make_fixtures.py`).

The reference ships no golden vectors for its kernels, so each fixture is produced by the
CPU oracle and, before it is written, checked against a method that shares no code with the
oracle: numpy float64 products and exact integer sums (GEMV), numpy bincount (histogram), a
Python dict (hash), scipy's unweighted shortest paths (BFS). Inputs come from the seeded
generators whose algorithms are written out in the oracle's header, so the product's
generators are pinned by the same files.

Files (numpy .npz, no pickled objects):
  gemv_f32_64x256.npz   A, x (U[-1,1), seed 4242 / 4242+0x9E37), y64 (fp64 sums), yseq (fp32 loop)
  gemv_f16_64x256.npz   W (N(0,0.02) fp16, seed 4243), x (N(0,1) fp16, seed 4244), y64
  gemv_int_64x256.npz   A, x small integers as fp32, y (exact)
  hist_zipf_2p16_2p10.npz   keys (Zipf(1.1) over 2^10, seed 1373, scrambled), counts
  hist_uniform_2p16_2p10.npz keys (uniform over 2^10, splitmix64 seed 77), counts
  hash_2p12.npz         keys, vals (seed 42), queries (50% hits, seed 4242), found, vals_out (slots 2^13)
  bfs_rmat10.npz        rowptr, col (R-MAT scale 10, edge factor 16, seed 8201), level from source 0
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle as ora  # noqa: E402

GOLDEN_MIX = 0x9E37


def gemv_fixtures() -> None:
    M, K = 64, 256
    A = ora.uniform_f32(M * K, 4242).reshape(M, K)
    x = ora.uniform_f32(K, 4242 + GOLDEN_MIX)
    y64, _ = ora.gemv_f64(A, x)
    yseq = ora.gemv_f32_seq(A, x)
    np.testing.assert_allclose(y64, A.astype(np.float64) @ x.astype(np.float64), rtol=0, atol=1e-12)
    np.savez_compressed(HERE / "gemv_f32_64x256.npz", A=A, x=x, y64=y64, yseq=yseq)

    W = ora.normal_f16(M * K, 0.0, 0.02, 4243).reshape(M, K)
    xh = ora.normal_f16(K, 0.0, 1.0, 4244)
    yh, _ = ora.gemv_f64(W, xh)
    np.testing.assert_allclose(yh, W.astype(np.float64) @ xh.astype(np.float64), rtol=0, atol=1e-12)
    np.savez_compressed(HERE / "gemv_f16_64x256.npz", W=W, x=xh, y64=yh)

    rng = np.random.default_rng(64256)
    Ai = rng.integers(-8, 9, size=(M, K)).astype(np.float32)
    xi = rng.integers(-3, 4, size=K).astype(np.float32)
    yi = (Ai.astype(np.int64) @ xi.astype(np.int64)).astype(np.float32)
    assert np.array_equal(ora.gemv_f32_seq(Ai, xi), yi)
    np.savez_compressed(HERE / "gemv_int_64x256.npz", A=Ai, x=xi, y=yi)


def hist_fixtures() -> None:
    n, bins = 1 << 16, 1 << 10
    t = ora.zipf_thresholds(bins, 1.1)
    keys = ora.zipf_keys(n, t, 1373, scramble=True)
    counts, c = ora.histogram(keys, bins)
    assert c == n and np.array_equal(counts, np.bincount(keys, minlength=bins).astype(np.uint32))
    np.savez_compressed(HERE / "hist_zipf_2p16_2p10.npz", keys=keys, counts=counts)

    ukeys = np.array([ora.splitmix64(77, i) & (bins - 1) for i in range(n)], dtype=np.uint32)
    ucounts, c = ora.histogram(ukeys, bins)
    assert c == n and np.array_equal(ucounts, np.bincount(ukeys, minlength=bins).astype(np.uint32))
    np.savez_compressed(HERE / "hist_uniform_2p16_2p10.npz", keys=ukeys, counts=ucounts)


def hash_fixture() -> None:
    n, slots = 1 << 12, 1 << 13
    keys, vals = ora.hash_kv(n, 42)
    q = ora.hash_queries(n, n, 42, 4242)
    t = ora.HashTable(slots)
    assert t.build(keys, vals) == 0
    vo, fo = t.lookup(q)
    d = dict(zip(keys.tolist(), vals.tolist()))
    assert len(d) == n
    for i, k in enumerate(q.tolist()):
        assert bool(fo[i]) == (k in d)
        assert int(vo[i]) == (d[k] if k in d else 0)
    assert int(fo.sum()) == n // 2
    np.savez_compressed(HERE / "hash_2p12.npz", keys=keys, vals=vals, queries=q, found=fo, vals_out=vo)


def bfs_fixture() -> None:
    from scipy.sparse import csr_matrix
    from scipy.sparse.csgraph import shortest_path

    rowptr, col = ora.rmat_csr(10, 16, 8201)
    level, _ = ora.bfs(rowptr, col, 0)
    V = rowptr.size - 1
    g = csr_matrix((np.ones(col.size), col, rowptr), shape=(V, V))
    dist = shortest_path(g, unweighted=True, indices=0)
    want = np.where(np.isinf(dist), 0xFFFFFFFF, dist).astype(np.uint32)
    assert np.array_equal(level, want)
    np.savez_compressed(HERE / "bfs_rmat10.npz", rowptr=rowptr, col=col, level=level)


if __name__ == "__main__":
    gemv_fixtures()
    hist_fixtures()
    hash_fixture()
    bfs_fixture()
    for f in sorted(HERE.glob("*.npz")):
        print(f"{f.name}: {f.stat().st_size} bytes")
