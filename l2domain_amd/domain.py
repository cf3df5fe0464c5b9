"""Domain runtime: device topology, DomainScan (workgroup -> XCD map) and cache flush.

Replaces the reference's latency-probed SM->side calibration (utility/latopt.cuh:487-562,
utility/get_smid2side.cu) and its L2 reset (utility/latopt.cuh:103-134).
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from ._torch import ptr, stream_handle


def topology(device: int = 0) -> dict:
    t = _lib.Topology()
    _lib.call("xd_topology_query", device, C.byref(t))
    return {"device": t.device, "num_cu": t.num_cu, "num_xcd": t.num_xcd, "cu_per_xcd": t.cu_per_xcd,
            "wave_size": t.wave_size, "clock_khz": t.clock_khz, "l2_bytes": t.l2_bytes,
            "lds_bytes_per_wg": t.lds_bytes_per_wg, "hbm_bytes": t.hbm_bytes,
            "arch": t.arch.decode(), "name": t.name.decode()}


def decode_placement(word: int) -> dict:
    return {"xcc": (word >> 24) & 0xFF, "se": (word >> 16) & 0xFF, "sh": (word >> 12) & 0xF,
            "cu": (word >> 8) & 0xF, "simd": word & 0xFF}


def domain_scan(num_wg: int, device: int = 0) -> torch.Tensor:
    """Runs DomainScan over `num_wg` workgroups; returns the uint32 placement words (CPU)."""
    out = torch.zeros(num_wg, dtype=torch.int32, device=f"cuda:{device}")
    _lib.call("xd_domain_scan", num_wg, ptr(out), stream_handle())
    torch.cuda.synchronize()
    return out.cpu().view(torch.int32)


def xcd_offset(stream: torch.cuda.Stream | None = None) -> int:
    """XCD of workgroup 0 in the last dispatch of the library's kernels on `stream` (workgroup
    i then ran on XCD (i + offset) mod 8), or -1 if none has run on it yet."""
    return int(_lib.lib.xd_xcd_offset(stream_handle(stream)))


class CacheFlusher:
    """Owns the read-stream buffer used to evict the L2s and the Infinity Cache."""

    def __init__(self, device: int = 0):
        self.bytes = int(_lib.lib.xd_cache_flush_bytes())
        self.buf = torch.ones(self.bytes // 4, dtype=torch.int32, device=f"cuda:{device}")

    def flush(self, stream: torch.cuda.Stream | None = None) -> None:
        _lib.call("xd_cache_flush", ptr(self.buf), self.bytes, stream_handle(stream))


def home_map(buf: torch.Tensor, return_latency: bool = False):
    """Measured die (0/1) of every 2 MiB page overlapping `buf` (uint8 device tensor); with
    return_latency, also the (pages, 2) cycle counts of die 0 and die 1."""
    nbytes = buf.numel() * buf.element_size()
    npages = int(_lib.lib.xd_home_map_pages(ptr(buf), nbytes))
    attr = torch.empty(npages, dtype=torch.uint8, device=buf.device)
    ws = torch.empty(int(_lib.lib.xd_home_map_workspace_size(ptr(buf), nbytes)) // 4 + 1, dtype=torch.int32,
                     device=buf.device)
    _lib.call("xd_home_map", ptr(buf), nbytes, ptr(attr), ptr(ws), ws.numel() * 4, stream_handle())
    if return_latency:
        return attr, ws[: 2 * npages].view(npages, 2)
    return attr


def home_parity(buf: torch.Tensor, mask: int | None = None) -> list[int]:
    """Die predicted by the address-bit mask for the first 8 KiB of every 2 MiB page of buf."""
    m = int(_lib.lib.xd_home_mask()) if mask is None else mask
    lo = ptr(buf)
    page0 = lo >> 21
    npages = int(_lib.lib.xd_home_map_pages(lo, buf.numel() * buf.element_size()))
    return [bin(((page0 + p) << 21) & m).count("1") & 1 for p in range(npages)]


def xdom_pchase(leader_xcd: int, follower_xcd: int, numel: int = 2048, stride: int = 128, flush: bool = True,
                device: int = 0) -> dict:
    """XDom-PChase (run_figure_2, architecture_probe.cu:572-596): four latency traces in
    cycles of a `numel`-element pointer chain at `stride` bytes -- leader first/second and
    follower first/second -- plus the XCC ids the two workgroups ran on."""
    dev = f"cuda:{device}"
    chain = torch.empty(numel * stride // 8, dtype=torch.int64, device=dev)
    out = torch.empty(4 * numel + 4, dtype=torch.int32, device=dev)
    fl = CacheFlusher(device) if flush else None
    _lib.call("xd_xdom_pchase", leader_xcd, follower_xcd, ptr(chain), chain.numel() * 8, numel, stride,
              ptr(fl.buf) if fl else None, fl.bytes if fl else 0, ptr(out), stream_handle())
    o = out.cpu().numpy().view("uint32")
    if o[4 * numel + 2] != 1 or o[4 * numel + 3] != 1:
        raise RuntimeError("xdom_pchase: a role found no workgroup on its XCD")
    return {"leader_xcd": int(o[4 * numel]), "follower_xcd": int(o[4 * numel + 1]),
            "leader_first": o[:numel].copy(), "leader_second": o[numel:2 * numel].copy(),
            "follower_first": o[2 * numel:3 * numel].copy(), "follower_second": o[3 * numel:4 * numel].copy()}


def compute_units(device: int = 0, num_wg: int = 4096) -> list[int]:
    """Placement keys (xcc << 16) | (se << 8) | (sh << 4) | cu of every compute unit that a
    DomainScan of `num_wg` workgroups reaches, sorted (XCD-major)."""
    words = domain_scan(num_wg, device).numpy().view("uint32")
    return sorted({int(w) >> 8 for w in words})


def domain_scan_latency(first_bit: int = 7, last_bit: int = 31, leader_xcd: int = 0, followers=None,
                        flush: bool = True, device: int = 0) -> dict:
    """DomainScan latency curves (run_figure_3, architecture_probe.cu:598-631): for every
    follower compute unit (placement keys; default all that compute_units() finds), the cycles
    of one load of buf + 2^b, b = first_bit..last_bit, right after a leader workgroup on XCD
    `leader_xcd` loaded the same addresses. As in the reference (measure_offsets :440-448) the
    whole protocol -- cache flush, leader, follower -- runs twice per follower and the second
    curve is kept. Returns {"bits": [...], "curves": {key: np.ndarray}}."""
    dev = f"cuda:{device}"
    keys = compute_units(device) if followers is None else [int(k) for k in followers]
    nbytes = (1 << last_bit) + 4096
    buf = torch.zeros(nbytes // 4, dtype=torch.int32, device=dev)
    nb = last_bit - first_bit + 1
    out = torch.zeros(nb + 4, dtype=torch.int32, device=dev)
    fl = CacheFlusher(device) if flush else None
    curves = {}
    for key in keys:
        for _ in range(2):
            _lib.call("xd_domain_scan_latency", ptr(buf), nbytes, first_bit, last_bit, leader_xcd, key,
                      ptr(fl.buf) if fl else None, fl.bytes if fl else 0, ptr(out), stream_handle())
        o = out.cpu().numpy().view("uint32")
        if o[nb] != 1 or o[nb + 1] != 1:
            raise RuntimeError(f"domain_scan_latency: no workgroup ran on the leader XCD or on CU key {key:#x}")
        curves[key] = o[:nb].copy()
    return {"bits": list(range(first_bit, last_bit + 1)), "leader_xcd": leader_xcd, "curves": curves}


def derive_active_bits(a_curve, b_curve) -> list[bool]:
    """The reference's rule (derive_active_bits, architecture_probe.cu:495-523): the relation
    a > b / a < b of the base entry (or the first unequal one) is the baseline; an entry is
    active when its relation is strict and differs from the baseline."""
    def rel(a, b):
        return 0 if a == b else (1 if a > b else -1)
    base = 0
    for a, b in zip(a_curve, b_curve):
        base = rel(a, b)
        if base:
            break
    if base == 0:
        raise ValueError("the two curves are indistinguishable; cannot derive active bits")
    return [rel(a, b) != 0 and rel(a, b) != base for a, b in zip(a_curve, b_curve)]


def mask_probe(first_bit: int = 5, last_bit: int = 29, reps: int = 8, device: int = 0) -> dict:
    """MaskProbe (run_mask_probe, architecture_probe.cu:644-670) for the I/O-die home: latency
    of a memory-side fetch-add at buf and buf + 2^b seen from die 0 (XCD 0) and die 1 (XCD 4);
    `active` marks the bits whose flip moves the address to the other die, `active_mask`
    keeps the page-stable ones (below bit 21) as the reference does."""
    dev = f"cuda:{device}"
    nbytes = (1 << last_bit) + 4096
    buf = torch.zeros(nbytes // 4, dtype=torch.int32, device=dev)
    nb = last_bit - first_bit + 2
    out = torch.empty(2 * nb + 4, dtype=torch.int32, device=dev)
    _lib.call("xd_mask_probe", ptr(buf), nbytes, first_bit, last_bit, reps, ptr(out), stream_handle())
    o = out.cpu().numpy().view("uint32")
    if o[2 * nb + 2] != 1 or o[2 * nb + 3] != 1:
        raise RuntimeError("mask_probe: a die found no workgroup on its XCD")
    a, b = o[:nb].copy(), o[nb:2 * nb].copy()
    flip = derive_active_bits(a, b)
    bits = list(range(first_bit, last_bit + 1))
    active = [f and bit < 21 for f, bit in zip(flip[1:], bits)]
    mask = sum(1 << bit for bit, on in zip(bits, active) if on)
    return {"bits": bits, "die0_cycles": a[1:], "die1_cycles": b[1:], "base": (int(a[0]), int(b[0])),
            "observed_flip": flip[1:], "active": active, "active_mask": mask,
            "xcc": (int(o[2 * nb]), int(o[2 * nb + 1]))}


def read_stream(buf: torch.Tensor, mode: str = "oblivious", home_attr: torch.Tensor | None = None,
                workgroups: int = 0, depth: int = 0, stream: torch.cuda.Stream | None = None) -> None:
    """One read of every 16-byte word of `buf` (the roofline probe of cache-resident data):
    oblivious contiguous, aware near chunks only, rotated far chunks only."""
    nbytes = buf.numel() * buf.element_size()
    _lib.call("xd_read_stream", ptr(buf), nbytes, _lib.MODES[mode], ptr(home_attr) if home_attr is not None else None,
              workgroups, depth, stream_handle(stream))


def _channel_buffer(top_bit: int, device: int):
    """A buffer whose start the library rounds up to 2 MiB, holding offsets below 2^(top_bit+1)."""
    nbytes = (2 << top_bit) + (2 << 20)
    return torch.zeros(nbytes // 4, dtype=torch.int32, device=f"cuda:{device}"), nbytes


def channel_time(vecs, xcd: int = 0, iters: int = 256, device: int = 0) -> float:
    """One channel-probe query (xd_channel_time): microseconds for 128 waves on XCD `xcd` to
    read, `iters` times, the 64 lines base + XOR of the six address vectors `vecs` picked by
    the lane bits."""
    vecs = [int(x) for x in vecs]
    assert len(vecs) == 6
    buf, nbytes = _channel_buffer(max(max(vecs).bit_length() - 1, 7), device)
    vv = (C.c_uint64 * 6)(*vecs)
    us = C.c_float(0.0)
    torch.cuda.synchronize()
    _lib.call("xd_channel_time", ptr(buf), nbytes, xcd, vv, iters, C.byref(us), stream_handle())
    return float(us.value)


def gf2_rank(vectors) -> int:
    """Rank over GF(2) of integers read as bit vectors."""
    basis = []
    for v in vectors:
        for b in basis:
            v = min(v, v ^ b)
        if v:
            basis.append(v)
    return len(basis)


def channel_of(addr: int, masks) -> int:
    """Channel index of an address under XOR masks: bit k = parity of addr & masks[k]."""
    return sum((bin(addr & m).count("1") & 1) << k for k, m in enumerate(masks))


def channel_probe(xcd: int = 0, bits=(7, 20), iters: int = 256, max_sets: int = 256, device: int = 0) -> dict:
    """Channel probe (xd_channel_probe): the XOR masks of address bits that select the L2 channel
    of a line on one XCD. `window_us[b - bits[0]]` times the 64 lines spanned by bits b..b+5;
    `masks` are GF(2)-independent channel-select functions, each with the per-bit curve it was
    read from; `active_mask` is every bit that enters some function (a bit outside it never
    changes the channel). Only bits <= 20 (inside a 2 MiB page) mean the same in virtual and
    physical addresses."""
    b0, b1 = bits
    buf, nbytes = _channel_buffer(b1, device)
    nb, nw = b1 - b0 + 1, b1 - b0 - 4
    win = (C.c_float * nw)()
    fast = C.c_float(0.0)
    masks = (C.c_uint64 * 4)()
    curves = (C.c_float * (4 * nb))()
    nm = C.c_int(0)
    torch.cuda.synchronize()
    _lib.call("xd_channel_probe", ptr(buf), nbytes, xcd, b0, b1, iters, max_sets, win, C.byref(fast), masks, curves,
              C.byref(nm), stream_handle())
    k = int(nm.value)
    ms = [int(masks[i]) for i in range(k)]
    active = 0
    for m in ms:
        active |= m
    return {"xcd": xcd, "bits": list(range(b0, b1 + 1)), "window_bits": list(range(b0, b0 + nw)),
            "window_us": list(win), "fast_us": float(fast.value), "masks": ms,
            "curves": [list(curves[i * nb:(i + 1) * nb]) for i in range(k)], "active_mask": active}


def memchannel_time(vecs, iters: int = 64, device: int = 0) -> float:
    """One memory-side channel query (xd_memchannel_time): microseconds for 2048 waves on all
    XCDs to add 1, `iters` times, to the 64 lines base + XOR of the six address vectors `vecs`
    picked by the lane bits (a distinct dword of each line per wave)."""
    vecs = [int(x) for x in vecs]
    assert len(vecs) == 6
    buf, nbytes = _channel_buffer(max(max(vecs).bit_length() - 1, 7), device)
    vv = (C.c_uint64 * 6)(*vecs)
    us = C.c_float(0.0)
    torch.cuda.synchronize()
    _lib.call("xd_memchannel_time", ptr(buf), nbytes, vv, iters, C.byref(us), stream_handle())
    return float(us.value)


def memchannel_probe(bits=(7, 20), iters: int = 64, nsets: int = 6, device: int = 0) -> dict:
    """Memory-side channel probe (xd_memchannel_probe): which address bits select the unit (an
    Infinity-Cache slice / memory channel) that serves a line's atomics. `ratio[(a, b)]` is the
    smallest slowdown of a five-vector set when bits a and b (a == b: bit a alone) are added
    (about 1: they spread the set; about 2 or more: they never change the unit); `inactive` is
    the mask of bits that never do; `masks` group the other bits into classes of equal effect,
    one XOR mask per class."""
    b0, b1 = bits
    nb = b1 - b0 + 1
    buf, nbytes = _channel_buffer(b1, device)
    ratio = (C.c_float * (nb * nb))()
    inactive = C.c_uint64(0)
    masks = (C.c_uint64 * 32)()
    nm = C.c_int(0)
    torch.cuda.synchronize()
    _lib.call("xd_memchannel_probe", ptr(buf), nbytes, b0, b1, iters, nsets, ratio, C.byref(inactive), masks,
              C.byref(nm), stream_handle())
    k = int(nm.value)
    return {"bits": list(range(b0, b1 + 1)), "inactive": int(inactive.value),
            "masks": [int(masks[i]) for i in range(k)],
            "ratio": {(b0 + a, b0 + b): float(ratio[a * nb + b]) for a in range(nb) for b in range(a, nb)}}
