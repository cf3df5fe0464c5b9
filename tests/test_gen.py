"""The product's seeded generators (libxdom host code) equal the oracle's independent
restatement bit for bit, so GPU inputs are exactly what the CPU checks use."""
import numpy as np

import oracle as ora
from l2domain_amd import gen


def test_rand64_matches_oracle():
    for s in (0, 42, 4242, 2**64 - 1):
        for i in (0, 1, 2, 12345, 2**40):
            assert gen.rand64(s, i) == ora.splitmix64(s, i)


def test_uniform_f32_matches_oracle():
    n = (1 << 17) + 3  # crosses the threaded split
    np.testing.assert_array_equal(gen.uniform_f32(n, 4242).view(np.uint32),
                                  ora.uniform_f32(n, 4242).view(np.uint32))


def test_normal_f16_matches_oracle():
    n = (1 << 17) + 1  # odd length: last element uses only the cosine branch
    for mean, sd, seed in ((0.0, 0.02, 4243), (0.0, 1.0, 4244), (3.0, 1e-6, 9)):
        np.testing.assert_array_equal(gen.normal_f16(n, mean, sd, seed).view(np.uint16),
                                      ora.normal_f16(n, mean, sd, seed).view(np.uint16))


def test_gemv_inputs_shapes_and_seeds():
    A, x = gen.gemv_f32_inputs(8, 16)
    assert A.shape == (8, 16) and x.shape == (16,)
    np.testing.assert_array_equal(x, ora.uniform_f32(16, 4242 + 0x9E37))
    W, xh = gen.gemv_f16_inputs(4, 8)
    assert W.dtype == np.float16 and xh.dtype == np.float16


def test_mix32_generators_match_oracle():
    n = (1 << 17) + 5
    for seed in (0, 4242, 0xFFFFFFFF):
        np.testing.assert_array_equal(gen.mix32_words(n, seed), ora.mix32_words(n, seed))
        for mod, off in ((0, 0), (17, 8), (7, 3)):
            np.testing.assert_array_equal(gen.mix32_f32(n, seed, mod, off).view(np.uint32),
                                          ora.mix32_f32(n, seed, mod, off).view(np.uint32))
    A, x = gen.gemv_mix32_inputs(4, 1024)
    np.testing.assert_array_equal(x, ora.mix32_f32(1024, 4242 + 0x9E37))


def test_bfs_ref_graph_product_matches_oracle():
    import ctypes as C
    from l2domain_amd import _lib
    rng = np.random.default_rng(4)
    for V, deg, nsrc, dl, H, maps in ((9000, 3, 50, 95, 1024, True), (5000, 8, 20, 0, 1024, False)):
        col_addr, level_addr = 0x7E0000000000 + 8192 * 7, 0x7E8000000000 + 4096 * 3
        ch = rng.integers(0, 2, size=(V * deg * 4) // (2 << 20) + 2, dtype=np.uint8) if maps else None
        lh = rng.integers(0, 2, size=(V * 4) // (2 << 20) + 2, dtype=np.uint8) if maps else None
        mask = int(_lib.lib.xd_home_mask())
        ref = ora.bfs_ref_graph(V, deg, nsrc, dl, H, 8201, col_addr, ch, level_addr, lh, mask)
        rowptr = np.empty(V + 1, dtype=np.int32)
        col = np.empty(V * deg, dtype=np.int32)
        ws = np.empty(V, dtype=np.uint8)
        src = np.empty(nsrc, dtype=np.int32)
        rc = _lib.lib.xd_bfs_ref_graph(V, deg, nsrc, dl, H, 8201, col_addr, None if ch is None else ch.ctypes.data,
                                       level_addr, None if lh is None else lh.ctypes.data, rowptr.ctypes.data,
                                       col.ctypes.data, ws.ctypes.data, src.ctypes.data)
        if ref is None:
            assert rc == _lib.XD_ERR_UNSUPPORTED
            continue
        assert rc == 0
        for a, b in zip((rowptr, col, ws, src), ref):
            np.testing.assert_array_equal(a, b)
