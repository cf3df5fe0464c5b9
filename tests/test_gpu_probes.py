"""Architecture probes on the GPU: DomainScan placement, XDom-PChase traces and MaskProbe.
The assertions are the MI355X facts the aware kernels rely on: workgroup i runs on XCC
i mod 8; a line chased twice by one XCD is an L2 hit the second time; another XCD does
not hit in that L2; bit 13 moves an address to the other I/O die."""
import numpy as np
import pytest

from l2domain_amd.domain import decode_placement, domain_scan, mask_probe, xdom_pchase

pytestmark = pytest.mark.gpu


def test_domain_scan_round_robin():
    words = domain_scan(4096).cpu().numpy().view(np.uint32)
    xcc = np.array([decode_placement(int(w))["xcc"] for w in words])
    assert np.array_equal(xcc, np.arange(4096) % 8)


@pytest.mark.parametrize("leader,follower", [(0, 0), (0, 1), (0, 4), (3, 6)])
def test_xdom_pchase(leader, follower):
    r = xdom_pchase(leader, follower, numel=2048, stride=128)
    assert r["leader_xcd"] == leader and r["follower_xcd"] == follower
    med = {k: float(np.median(r[k])) for k in ("leader_first", "leader_second", "follower_first", "follower_second")}
    print(leader, follower, med)
    # the second chase of either role hits in that XCD's L2
    assert med["leader_second"] < 0.8 * med["leader_first"]
    assert med["follower_second"] < 0.8 * med["leader_first"]
    if leader == follower:
        assert med["follower_first"] < 0.8 * med["leader_first"]      # same-XCD L2 hit
    else:
        assert med["follower_first"] > 1.2 * med["follower_second"]   # no hit in another XCD's L2


def test_mask_probe_finds_bit13():
    r = mask_probe(first_bit=5, last_bit=29, reps=8)
    print({b: (int(a), int(c)) for b, a, c in zip(r["bits"], r["die0_cycles"], r["die1_cycles"])})
    assert r["xcc"] == (0, 4)
    active = {b for b, on in zip(r["bits"], r["active"]) if on}
    assert 13 in active
    assert all(b >= 13 for b in active)   # nothing below the 8 KiB interleave moves a line between dies


def _stream_seconds(buf, home, flusher, reps):
    """Average duration (dispatch-stamped) of one near-only read of buf, after a flush or warm."""
    import torch
    from l2domain_amd import _lib
    from l2domain_amd.domain import read_stream
    read_stream(buf, "aware", home)
    torch.cuda.synchronize()
    _lib.timing_enable(True)
    for _ in range(reps):
        if flusher is not None:
            flusher.flush()
        read_stream(buf, "aware", home)
    torch.cuda.synchronize()
    t = _lib.timing_read()
    _lib.timing_enable(False)
    ms, n = t["read_stream_kernel"]
    assert n == reps
    return ms / 1e3 / n


def test_cache_flush_evicts_infinity_cache():
    """After xd_cache_flush a 112 MiB buffer (inside the 256 MB Infinity Cache) is read from
    HBM: its near-only read rate stays under the 8 TB/s HBM peak and clearly below the warm
    (cache-resident) rate, and a pointer chase after the flush pays more than a chase served
    by the Infinity Cache (another XCD's first chase of the same lines)."""
    import torch
    from l2domain_amd.domain import CacheFlusher, home_map
    buf = torch.ones((112 << 20) // 4, dtype=torch.int32, device="cuda")
    home = home_map(buf.view(torch.uint8))
    fl = CacheFlusher()
    warm = buf.numel() * 4 / _stream_seconds(buf, home, None, 20) / 1e9
    cold = buf.numel() * 4 / _stream_seconds(buf, home, fl, 10) / 1e9
    print(f"near-only read of 112 MiB: warm {warm:.0f} GB/s, after flush {cold:.0f} GB/s")
    assert cold < 8000.0
    assert warm > 1.2 * cold
    r = xdom_pchase(0, 4, numel=2048, stride=128, flush=True)
    med = {k: float(np.median(r[k])) for k in ("leader_first", "follower_first")}
    print(med)
    assert med["leader_first"] > 1.2 * med["follower_first"]
