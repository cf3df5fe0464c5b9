"""The reference's own histogram on the GPU: xd_hist256_u32bytes (through the C ABI) against
the oracle's byte-counting loop (HIST.cu:279-288) on the reference's data (words[i] =
mix32(i), HIST.cu:331-340) and on edge cases. Bit-exact."""
import numpy as np
import pytest
import torch

import oracle as ora
from l2domain_amd import gen
from l2domain_amd.domain import home_map
from l2domain_amd.histogram import ByteHistogram

pytestmark = pytest.mark.gpu
MODES = ["oblivious", "aware", "rotated"]


@pytest.fixture(scope="module")
def bh():
    return ByteHistogram()


def run(bh, words: torch.Tensor, mode, mapped: bool):
    attr = home_map(words.view(torch.uint8)) if (mapped and words.numel()) else None
    counts = torch.full((256,), -7, dtype=torch.int32, device="cuda")
    bh(words, counts, mode=mode, home_attr=attr)
    torch.cuda.synchronize()
    return counts.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("mapped", [True, False])
@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("n", [0, 1, 3, 4, 5, 2047, 2048, 2049, 4096 + 3, 12289, 1 << 20])
def test_random_words(bh, n, mode, mapped):
    host = np.random.default_rng(n + 17).integers(0, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32)
    words = torch.from_numpy(host.view(np.int32)).cuda()
    np.testing.assert_array_equal(run(bh, words, mode, mapped), ora.hist256_bytes(host))


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("offset_words", [4, 2044, 2048, 4092, 6144 - 4])
def test_unaligned_chunk_starts(bh, mode, offset_words):
    """Words that start inside an 8 KiB chunk or a 16 KiB pair (the buffer itself is 2 MiB
    aligned by the allocator's large-block rule; the offsets are 16-byte multiples)."""
    n = 3 * 2048 + 777
    buf = torch.from_numpy(gen.mix32_words(n + offset_words + 8).view(np.int32)).cuda()
    words = buf[offset_words: offset_words + n]
    host = words.cpu().numpy().view(np.uint32)
    for mapped in (True, False):
        np.testing.assert_array_equal(run(bh, words, mode, mapped), ora.hist256_bytes(host))


@pytest.mark.parametrize("mode", MODES)
def test_constant_words(bh, mode):
    n = (1 << 20) + 9
    for val in (0, 0xFFFFFFFF, 0x01020304):
        host = np.full(n, val, dtype=np.uint32)
        words = torch.from_numpy(host.view(np.int32)).cuda()
        ref = ora.hist256_bytes(host)
        assert ref.sum() == 4 * n
        np.testing.assert_array_equal(run(bh, words, mode, True), ref)


def test_reference_data_32mb_all_modes_and_repeats(bh):
    """applications/histogram/run.sh quick preset: data_mb = 32 of mix32(i) words."""
    n = 32 * 1024 * 1024 // 4
    host = gen.mix32_words(n)
    np.testing.assert_array_equal(host[:4], [ora.mix32(i) for i in range(4)])
    ref = ora.hist256_bytes(host, nthreads=8)
    words = torch.from_numpy(host.view(np.int32)).cuda()
    for _ in range(2):  # the workspace tickets are left zeroed: a second call gives the same counts
        for mode in MODES:
            np.testing.assert_array_equal(run(bh, words, mode, True), ref)


def test_reference_data_512mb_full_size(bh):
    """The largest paper-preset size (data_mb = 512): every mode equals the oracle, and the
    counts sum to 4 n."""
    n = 512 * 1024 * 1024 // 4
    host = gen.mix32_words(n)
    ref = ora.hist256_bytes(host, nthreads=16)
    assert int(ref.sum(dtype=np.uint64)) == 4 * n
    words = torch.from_numpy(host.view(np.int32)).cuda()
    del host
    for mode in MODES:
        np.testing.assert_array_equal(run(bh, words, mode, True), ref)


def test_rejects_bad_arguments(bh):
    from l2domain_amd._lib import XdomError
    words = torch.zeros(64, dtype=torch.int32, device="cuda")
    with pytest.raises(XdomError):
        bh(words[1:], mode="aware")  # not 16-byte aligned
    counts = torch.zeros(256, dtype=torch.int32, device="cuda")
    small = torch.zeros(16, dtype=torch.uint8, device="cuda")
    from l2domain_amd import _lib
    from l2domain_amd._torch import ptr, stream_handle
    with pytest.raises(XdomError):
        _lib.call("xd_hist256_u32bytes", ptr(words), 64, ptr(counts), 1, None, ptr(small), 16, stream_handle())
