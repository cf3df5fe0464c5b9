"""Allocation-free byte histogram: xd_hist256_u32bytes_noalloc, called through the C ABI,
against xd_hist256_u32bytes with a caller-owned workspace, bit-exact. Calls in a row reuse
the library's per-GPU scratch: a large input, then a smaller one, then the large one again
(the scratch must come back zeroed after each call)."""
import numpy as np
import pytest
import torch

from l2domain_amd import _lib

pytestmark = pytest.mark.gpu
MODES = {"oblivious": _lib.MODE_OBLIVIOUS, "aware": _lib.MODE_AWARE, "rotated": _lib.MODE_ROTATED}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _with_workspace(words: torch.Tensor, mode: int) -> np.ndarray:
    ws = torch.zeros(int(_lib.lib.xd_hist256_workspace_size()), dtype=torch.uint8, device="cuda")
    counts = torch.full((256,), -1, dtype=torch.int32, device="cuda")
    _lib.call("xd_hist256_u32bytes", words.data_ptr(), words.numel(), counts.data_ptr(), mode, None, ws.data_ptr(),
              ws.numel(), _stream())
    torch.cuda.synchronize()
    return counts.cpu().numpy().view(np.uint32)


def _noalloc(words: torch.Tensor, mode: int) -> np.ndarray:
    counts = torch.full((256,), -1, dtype=torch.int32, device="cuda")
    _lib.call("xd_hist256_u32bytes_noalloc", words.data_ptr(), words.numel(), counts.data_ptr(), mode, None, _stream())
    torch.cuda.synchronize()
    return counts.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("mode", list(MODES))
def test_noalloc_matches_workspace_entry_point(mode):
    rng = np.random.default_rng(11 + MODES[mode])
    host = rng.integers(0, 1 << 32, size=(1 << 24) + 3, dtype=np.uint64).astype(np.uint32)
    big = torch.from_numpy(host.view(np.int32)).cuda()
    small = big[: (1 << 16) + 5]  # smaller input, same 16-byte aligned start
    for words, n in ((big, host.size), (small, (1 << 16) + 5), (big, host.size)):
        print(mode, n, flush=True)
        got = _noalloc(words, MODES[mode])
        np.testing.assert_array_equal(got, _with_workspace(words, MODES[mode]))
        if n < host.size:
            np.testing.assert_array_equal(got, np.bincount(host[:n].view(np.uint8), minlength=256).astype(np.uint32))
        assert int(got.astype(np.uint64).sum()) == 4 * n


def test_noalloc_rejects_oversized_input():
    buf = torch.zeros(64, dtype=torch.int32, device="cuda")
    counts = torch.zeros(256, dtype=torch.int32, device="cuda")
    rc = _lib.lib.xd_hist256_u32bytes_noalloc(buf.data_ptr(), 1 << 30, counts.data_ptr(), _lib.MODE_AWARE, None,
                                              _stream())
    assert rc == _lib.XD_ERR_INVALID_ARG
    assert b"2^30" in _lib.lib.xd_last_error()
