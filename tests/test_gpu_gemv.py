"""GEMV parity on the GPU: libxdom (through the C ABI) against the CPU oracle.

Tolerances: fp32 inputs 1e-3 relative, fp16 inputs with fp32
accumulation 2e-2 relative; relative = max_i |y_i - ref_i| / max_i |ref_i| with ref the
fp64-accumulated oracle. Also checked: the reference's own pass rule (max |y - y_seq| <= 1e-3
against its fp32 sequential loop, applications/gemv/run.sh:94-97) and an exact mode with
small-integer inputs, where every summation order gives the same fp32 result.
"""
import numpy as np
import pytest
import torch

import oracle as ora
from l2domain_amd import gen
from l2domain_amd.gemv import gemv, workspace

pytestmark = pytest.mark.gpu
MODES = ["oblivious", "aware", "rotated"]


def device_aligned(a: np.ndarray, align: int = 8192) -> torch.Tensor:
    """Copy of `a` on the GPU starting at an `align`-byte boundary (the home routes need
    8 KiB-aligned matrices)."""
    a = np.ascontiguousarray(a)
    raw = torch.empty(a.nbytes + align, dtype=torch.uint8, device="cuda")
    off = (-raw.data_ptr()) % align
    t = raw[off:off + a.nbytes].view(torch.float16 if a.dtype == np.float16 else torch.float32).view(a.shape)
    t.copy_(torch.from_numpy(a))
    return t


def run(A: np.ndarray, x: np.ndarray, mode, mapped: bool = False, ws=None) -> np.ndarray:
    dA = device_aligned(A) if mapped else torch.from_numpy(np.ascontiguousarray(A)).cuda()
    dx = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    y = torch.full((A.shape[0],), float("nan"), dtype=torch.float32, device="cuda")
    home = None
    if mapped:
        from l2domain_amd.domain import home_map
        home = home_map(dA)
        if ws is None:
            ws = workspace(A.shape[0], A.shape[1], dA.dtype)
    gemv(dA, dx, y, mode=mode, home_attr=home, workspace=ws)
    torch.cuda.synchronize()
    if ws is not None:
        S = A.shape[1] * A.itemsize // 8192
        words = 8 * A.shape[0] if S == 2 else 4 * A.shape[0]  # S == 2: one 64-bit word per row
        assert int(torch.count_nonzero(ws[:words])) == 0, "row words / counters not left at zero"
    return y.cpu().numpy()


def rel_err(y, ref):
    return float(np.max(np.abs(y.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-300))


@pytest.fixture(scope="module")
def f32_config():
    A, x = gen.gemv_f32_inputs(4096, 4096)
    ref, yabs = ora.gemv_f64(A, x, nthreads=8)
    seq = ora.gemv_f32_seq(A, x, nthreads=8)
    return A, x, ref, yabs, seq


@pytest.mark.parametrize("mode", MODES)
def test_f32_4096_config(f32_config, mode):
    A, x, ref, yabs, seq = f32_config
    y = run(A, x, mode)
    assert np.all(np.isfinite(y))
    assert rel_err(y, ref) <= 1e-3
    # element-wise bound: fp32 accumulation error is far below 1e-3 of sum |a x|
    assert np.all(np.abs(y - ref) <= 1e-3 * yabs)
    assert float(np.max(np.abs(y - seq))) <= 1e-3  # the reference's max_abs_error rule


def test_f32_modes_bit_identical(f32_config):
    A, x, *_ = f32_config
    ys = [run(A, x, m) for m in MODES]
    for y in ys[1:]:
        np.testing.assert_array_equal(ys[0].view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("mode", MODES)
def test_f32_integer_inputs_exact(mode):
    rng = np.random.default_rng(1234)
    A = rng.integers(-8, 9, size=(4096, 4096)).astype(np.float32)
    x = rng.integers(-3, 4, size=4096).astype(np.float32)
    y = run(A, x, mode)
    np.testing.assert_array_equal(y, ora.gemv_f32_seq(A, x, nthreads=8))


@pytest.mark.parametrize("M,K", [(1, 4), (7, 12), (9, 256), (1000, 4100), (4097, 64), (33, 16384)])
@pytest.mark.parametrize("mode", ["oblivious", "aware"])
def test_f32_ragged_shapes(M, K, mode):
    A, x = gen.gemv_f32_inputs(M, K, seed=M * 7 + K)
    ref, yabs = ora.gemv_f64(A, x)
    y = run(A, x, mode)
    assert rel_err(y, ref) <= 1e-3
    assert np.all(np.abs(y - ref) <= 1e-3 * yabs + 1e-30)


@pytest.fixture(scope="module", params=[(14336, 4096), (4096, 14336)], ids=["up", "down"])
def f16_config(request):
    M, K = request.param
    W, x = gen.gemv_f16_inputs(M, K)
    ref, yabs = ora.gemv_f64(W, x, nthreads=8)
    return W, x, ref, yabs


@pytest.mark.parametrize("mapped", [False, True], ids=["maskhome", "mappedhome"])
@pytest.mark.parametrize("mode", MODES)
def test_f16_decode_shapes(f16_config, mode, mapped):
    W, x, ref, yabs = f16_config
    y = run(W, x, mode, mapped)
    assert np.all(np.isfinite(y))
    assert rel_err(y, ref) <= 2e-2
    assert np.all(np.abs(y - ref) <= 2e-2 * yabs)


@pytest.mark.parametrize("M,K", [(1, 8), (3, 24), (100, 1000), (4095, 4104)])
def test_f16_ragged_shapes(M, K):
    W, x = gen.gemv_f16_inputs(M, K, w_seed=M, x_seed=K)
    ref, yabs = ora.gemv_f64(W, x)
    for mode in MODES:
        y = run(W, x, mode)
        assert rel_err(y, ref) <= 2e-2
        assert np.all(np.abs(y - ref) <= 2e-2 * yabs + 1e-30)


def test_f16_integer_inputs_exact():
    # Integers |w| <= 8, |x| <= 3 are exact in binary16; K=4096 sums stay below 2^24.
    rng = np.random.default_rng(99)
    W = rng.integers(-8, 9, size=(512, 4096)).astype(np.float16)
    x = rng.integers(-3, 4, size=4096).astype(np.float16)
    ref = (W.astype(np.int64) @ x.astype(np.int64)).astype(np.float32)
    for mode in MODES:
        np.testing.assert_array_equal(run(W, x, mode), ref)


@pytest.mark.parametrize("dtype,M,K", [(np.float16, 34, 14336), (np.float16, 4096, 14336), (np.float32, 34, 3072),
                                       (np.float32, 4096, 7168), (np.float32, 64, 4096), (np.float32, 64, 8192),
                                       (np.float16, 64, 8192)])
@pytest.mark.parametrize("mode", MODES)
def test_home_routes_integer_exact(dtype, M, K, mode):
    """Rows of whole 8 KiB chunks (split-row home route, through the workspace) and rows that
    straddle chunks (28 KiB fp16 and fp32 rows, 12 KiB fp32 rows: every XCD on one contiguous
    eighth of the rows). A dropped, doubled or misplaced 16-byte vector changes an integer sum,
    which is exact in fp32 here (|w| <= 8, |x| <= 3, K <= 14336: |y| < 2^24)."""
    rng = np.random.default_rng(M * 131 + K)
    W = rng.integers(-8, 9, size=(M, K)).astype(dtype)
    x = rng.integers(-3, 4, size=K).astype(dtype)
    ref = (W.astype(np.int64) @ x.astype(np.int64)).astype(np.float32)
    np.testing.assert_array_equal(run(W, x, mode, mapped=True), ref)


def test_f16_row_home_modes_bit_identical():
    # up-projection rows are 8 KiB: the aware/rotated modes route whole rows by home die and
    # must reproduce the oblivious kernel bit for bit (same per-row summation order)
    W, x = gen.gemv_f16_inputs(14336, 4096)
    ys = [run(W, x, m, mapped=True) for m in MODES]
    for y in ys[1:]:
        np.testing.assert_array_equal(ys[0].view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("M,K", [(1, 4096), (7, 4096), (333, 2048), (100, 512), (9, 64)])
def test_f16_row_home_ragged(M, K):
    # row bytes 8192, 4096, 1024, 128 all divide 8 KiB: the home-routed kernel is used
    W, x = gen.gemv_f16_inputs(M, K, w_seed=M + K, x_seed=K)
    ref, yabs = ora.gemv_f64(W, x)
    for mode in MODES:
        y = run(W, x, mode, mapped=True)
        assert rel_err(y, ref) <= 2e-2
        assert np.all(np.abs(y - ref) <= 2e-2 * yabs + 1e-30)


@pytest.mark.parametrize("dtype,K", [("f32", 4096), ("f32", 8192), ("f16", 8192), ("f16", 16384)])
def test_split_row_home_bit_identical(dtype, K):
    # rows of 2 or 4 whole 8 KiB chunks: each chunk is reduced on its home die and the
    # partials meet in chunk order, the same order the oblivious kernel adds them in
    M = 1536
    if dtype == "f32":
        A, x = gen.gemv_f32_inputs(M, K, seed=K + 1)
    else:
        A, x = gen.gemv_f16_inputs(M, K, w_seed=K + 2, x_seed=K + 3)
    assert workspace(M, K, torch.float32 if dtype == "f32" else torch.float16) is not None
    base = run(A, x, "oblivious")
    ref, yabs = ora.gemv_f64(A, x, nthreads=8)
    tol = 1e-3 if dtype == "f32" else 2e-2
    assert rel_err(base, ref) <= tol
    for mode in ("aware", "rotated"):
        y = run(A, x, mode, mapped=True)
        np.testing.assert_array_equal(base.view(np.uint32), y.view(np.uint32))


def test_split_row_home_f32_4096_config(f32_config):
    A, x, ref, yabs, seq = f32_config
    base = run(A, x, "oblivious")
    ws = workspace(4096, 4096, torch.float32)
    for mode in ("aware", "rotated", "aware"):
        y = run(A, x, mode, mapped=True, ws=ws)  # the workspace is reused across calls
        np.testing.assert_array_equal(base.view(np.uint32), y.view(np.uint32))
        assert float(np.max(np.abs(y - seq))) <= 1e-3


@pytest.mark.parametrize("M,K", [(1, 2048), (3, 4096), (1000, 6144), (257, 10240)])
def test_split_row_home_ragged(M, K):
    # S = 2, 2, 3, 5 chunks per row (S = 3 and 5 add in chunk order, not the oblivious order)
    A, x = gen.gemv_f32_inputs(M, K, seed=M * 3 + K)
    ref, yabs = ora.gemv_f64(A, x)
    for mode in MODES:
        y = run(A, x, mode, mapped=True)
        assert rel_err(y, ref) <= 1e-3
        assert np.all(np.abs(y - ref) <= 1e-3 * yabs + 1e-30)


@pytest.mark.parametrize("dtype,M,K", [("f32", 2, 3072), ("f32", 100, 7168), ("f16", 6, 6144), ("f16", 34, 14336),
                                         ("f16", 7, 14336), ("f16", 4096, 14336)])
def test_rows_straddling_chunks(dtype, M, K):
    # rows of an odd number of 4 KiB halves (12, 28 KiB): no workspace, the exact kernel in
    # every mode (aware: contiguous eighths of the rows per XCD), so the same bits as oblivious
    if dtype == "f32":
        A, x = gen.gemv_f32_inputs(M, K, seed=M * 5 + K)
        tol = 1e-3
    else:
        A, x = gen.gemv_f16_inputs(M, K, w_seed=M * 5 + K, x_seed=M * 7 + K)
        tol = 2e-2
    ref, yabs = ora.gemv_f64(A, x)
    assert workspace(M, K, torch.float32 if dtype == "f32" else torch.float16) is None
    base = run(A, x, "oblivious")
    assert rel_err(base, ref) <= tol
    assert np.all(np.abs(base - ref) <= tol * yabs + 1e-30)
    for mode in ("aware", "rotated"):
        y = run(A, x, mode, mapped=True)
        np.testing.assert_array_equal(base.view(np.uint32), y.view(np.uint32))


def test_split_row_without_workspace_falls_back():
    A, x = gen.gemv_f32_inputs(512, 4096, seed=5)
    ref, yabs = ora.gemv_f64(A, x)
    dA = device_aligned(A)
    y = gemv(dA, torch.from_numpy(x).cuda(), mode="aware").cpu().numpy()
    assert rel_err(y, ref) <= 1e-3


@pytest.mark.parametrize("mode", ["aware", "rotated"])
def test_split_row_home_under_a_mask_without_the_die_bit(mode):
    """No page map and a home mask without bit 13 (0x10200000): both segments of a row can sit
    on one die, so a wave can take two segments of one group of 8. The bits still equal the
    oblivious kernel's; the library's mask is restored."""
    from l2domain_amd import _lib
    M, K = 1536, 4096
    A, x = gen.gemv_f32_inputs(M, K, seed=77)
    base = run(A, x, "oblivious")
    dA = device_aligned(A)
    dx = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    ws = workspace(M, K, dA.dtype)
    old = int(_lib.lib.xd_home_mask())
    assert _lib.lib.xd_set_home_mask(0x10200000) == 0
    try:
        y = torch.full((M,), float("nan"), dtype=torch.float32, device="cuda")
        gemv(dA, dx, y, mode=mode, home_attr=None, workspace=ws)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(base.view(np.uint32), y.cpu().numpy().view(np.uint32))
        assert int(torch.count_nonzero(ws[:8 * M])) == 0
    finally:
        assert _lib.lib.xd_set_home_mask(old) == 0


def test_placements_on_queues_that_start_elsewhere():
    """The three aware placements (split-row home route, whole-row home route, contiguous
    eighths of the rows) on new streams, whose queues may deal workgroup 0 to another XCC,
    before and after the library has learned the stream's offset: the oblivious kernel's bits."""
    from l2domain_amd.domain import home_map
    streams = [torch.cuda.Stream() for _ in range(4)]
    for dtype, M, K in [("f32", 512, 4096), ("f16", 512, 4096), ("f16", 256, 14336)]:
        if dtype == "f32":
            A, x = gen.gemv_f32_inputs(M, K, seed=M + K)
        else:
            A, x = gen.gemv_f16_inputs(M, K, w_seed=M + K, x_seed=M + 2 * K)
        base = run(A, x, "oblivious")
        dA = device_aligned(A)
        dx = torch.from_numpy(np.ascontiguousarray(x)).cuda()
        home = home_map(dA)
        ws = workspace(M, K, dA.dtype)
        y = torch.empty(M, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        for s in streams:
            for mode in ("aware", "rotated", "aware"):
                gemv(dA, dx, y, mode=mode, home_attr=home, workspace=ws, stream=s)
                s.synchronize()
                np.testing.assert_array_equal(base.view(np.uint32), y.cpu().numpy().view(np.uint32))


def _random_shapes(n, seed):
    """Seeded (dtype, M, K) draws over every route: K a multiple of 8 up to 16384 (fp16) or
    4 up to 8192 (fp32), so rows of 1 to 4 whole chunks, rows inside a chunk and ragged rows."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        if rng.random() < 0.5:
            out.append((np.float16, int(rng.integers(1, 3000)), 8 * int(rng.integers(1, 2049))))
        else:
            out.append((np.float32, int(rng.integers(1, 3000)), 4 * int(rng.integers(1, 2049))))
    # the route boundaries themselves
    out += [(np.float16, 1000, 4096), (np.float16, 999, 8192), (np.float32, 513, 2048), (np.float32, 77, 4096),
            (np.float16, 5, 12288), (np.float32, 3, 10240)]
    return out


@pytest.mark.parametrize("dtype,M,K", _random_shapes(18, 2026))
def test_random_shapes_integer_exact_all_modes(dtype, M, K):
    """Integer inputs (exact in fp16 and fp32, |y| < 2^24) on seeded random shapes, 8 KiB-aligned
    with a measured home map and a workspace: every mode equals the integer product."""
    rng = np.random.default_rng(M * 7919 + K)
    W = rng.integers(-8, 9, size=(M, K)).astype(dtype)
    x = rng.integers(-3, 4, size=K).astype(dtype)
    ref = (W.astype(np.int64) @ x.astype(np.int64)).astype(np.float32)
    for mode in MODES:
        np.testing.assert_array_equal(run(W, x, mode, mapped=True), ref, err_msg=f"{mode} {M}x{K}")

