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
