"""Hash table parity on the GPU: insert + lookup through the C ABI against the oracle's
serial build (HASH.cu:226-241) and probe (HASH.cu:46-64). found/value bit-exact."""
import numpy as np
import pytest
import torch

import oracle as ora
from l2domain_amd.hashtable import (EMPTY, HASH_KEYS, HASH_QSEED, HASH_SEED, HASH_SLOTS, HashTable,
                                    gen_kv, gen_queries)

pytestmark = pytest.mark.gpu
MODES = ["oblivious", "aware", "rotated"]


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint64).view(np.int64)).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint64)


@pytest.mark.parametrize("ins_mode", MODES)
@pytest.mark.parametrize("look_mode", MODES)
def test_small_table_all_mode_pairs(ins_mode, look_mode):
    slots, n = 1 << 12, 1500
    keys, vals = ora.hash_kv(n + 600, 11)
    q = np.concatenate([keys[:n:2], keys[n:], keys[1:n:3]])
    np.random.default_rng(1).shuffle(q)
    ref = ora.HashTable(slots)
    assert ref.build(keys[:n], vals[:n]) == 0
    rv, rf = ref.lookup(q)
    t = HashTable(slots)
    t.insert(dev(keys[:n]), dev(vals[:n]), mode=ins_mode)
    v, f = t.lookup(dev(q), mode=look_mode)
    torch.cuda.synchronize()
    assert t.failures() == 0
    np.testing.assert_array_equal(f.cpu().numpy(), rf)
    np.testing.assert_array_equal(host(v), rv)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("slots,n", [(8, 5), (1 << 9, 300), (1 << 16, 3 * 4096 + 77), (1 << 20, 9 * 4096 + 1)])
def test_ragged_batches_repeats_and_empty(slots, n, mode):
    """Tiny and mid-size tables, batches that are not a multiple of a wave or a workgroup,
    a key repeated far apart in one batch (one slot, one of its values) and an EMPTY key
    (skipped)."""
    keys, vals = ora.hash_kv(n + 40, slots + n)
    keys = keys[:n].copy()
    if n > 4096:
        keys[4100] = keys[3]  # the same key in two tiles
    keys[n // 2] = EMPTY
    vals = vals[:n]
    ref = ora.HashTable(slots)
    assert ref.build(keys, vals) == 0
    q = np.concatenate([keys, ora.hash_kv(n + 40, slots + n)[0][n:]])
    rv, rf = ref.lookup(q)
    t = HashTable(slots)
    t.insert(dev(keys), dev(vals), mode=mode)
    v, f = t.lookup(dev(q), mode=mode)
    torch.cuda.synchronize()
    assert t.failures() == 0
    got_f, got_v = f.cpu().numpy(), host(v)
    if n > 4096:  # the repeated key keeps one of its two values
        assert got_f[3] == 1 and got_v[3] in (vals[3], vals[4100])
        got_v[3] = got_v[4100] = rv[3]
    np.testing.assert_array_equal(got_f, rf)
    np.testing.assert_array_equal(got_v, rv)


@pytest.mark.parametrize("mode", MODES)
def test_full_table_failures_and_reinsert(mode):
    slots = 1 << 10
    keys, vals = ora.hash_kv(slots + 50, 5)
    t = HashTable(slots)
    t.insert(dev(keys), dev(vals), mode=mode)
    torch.cuda.synchronize()
    assert t.failures() == 50  # distinct keys: exactly `slots` of them find a slot
    _, f = t.lookup(dev(keys), mode=mode)
    assert int(f.cpu().numpy().sum()) == slots
    # a fresh table, then the same keys twice: the second pass only updates values
    t.clear()
    t.insert(dev(keys[:700]), dev(vals[:700]), mode=mode)
    t.insert(dev(keys[:700]), dev(vals[::-1][:700]), mode=mode)
    v, f = t.lookup(dev(keys[:700]), mode=mode)
    torch.cuda.synchronize()
    assert t.failures() == 0 and f.cpu().numpy().all()
    np.testing.assert_array_equal(host(v), vals[::-1][:700])


def test_empty_sentinel_and_empty_batches():
    t = HashTable(1 << 8)
    k = np.array([EMPTY, 5, 7], dtype=np.uint64)
    v = np.array([1, 2, 3], dtype=np.uint64)
    t.insert(dev(k), dev(v))
    t.insert(dev(k[:0]), dev(v[:0]))
    vals, f = t.lookup(dev(np.array([EMPTY, 5, 7, 9], dtype=np.uint64)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(f.cpu().numpy(), [0, 1, 1, 0])
    np.testing.assert_array_equal(host(vals), [0, 2, 3, 0])


def test_device_generators_match_oracle():
    keys, vals = gen_kv(5000, HASH_SEED)
    q = gen_queries(3000, 5000, HASH_SEED, HASH_QSEED)
    rk, rv = ora.hash_kv(5000, HASH_SEED)
    np.testing.assert_array_equal(host(keys), rk)
    np.testing.assert_array_equal(host(vals), rv)
    np.testing.assert_array_equal(host(q), ora.hash_queries(3000, 5000, HASH_SEED, HASH_QSEED))


@pytest.fixture(scope="module")
def config_ref():
    keys, vals = gen_kv(HASH_KEYS, HASH_SEED)
    q = gen_queries(HASH_KEYS, HASH_KEYS, HASH_SEED, HASH_QSEED)
    hk, hv, hq = host(keys), host(vals), host(q)
    assert EMPTY not in set(hk[:1 << 16].tolist())
    ref = ora.HashTable(HASH_SLOTS)
    assert ref.build(hk, hv) == 0
    rv, rf = ref.lookup(hq, nthreads=16)
    del ref
    return keys, vals, q, rv, rf


@pytest.mark.parametrize("mode", MODES)
def test_config_2p26_insert_lookup(config_ref, mode):
    keys, vals, q, rv, rf = config_ref
    assert int(rf.sum()) == HASH_KEYS // 2  # 50% hit rate by construction
    t = HashTable(HASH_SLOTS)
    t.insert(keys, vals, mode=mode)
    v, f = t.lookup(q, mode=mode)
    torch.cuda.synchronize()
    assert t.failures() == 0
    np.testing.assert_array_equal(f.cpu().numpy(), rf)
    np.testing.assert_array_equal(host(v), rv)
    del t
    torch.cuda.empty_cache()


@pytest.mark.parametrize("mode", MODES)
def test_config_2p26_build_lookup(config_ref, mode):
    """The bench's step: the range build (xd_hash_build_u64) of the 2^26 pairs into 2^27
    slots, then the 2^26 lookups, against the serial build."""
    keys, vals, q, rv, rf = config_ref
    t = HashTable(HASH_SLOTS)
    t.build(keys, vals, mode=mode)
    v, f = t.lookup(q, mode=mode)
    torch.cuda.synchronize()
    assert t.failures() == 0
    np.testing.assert_array_equal(f.cpu().numpy(), rf)
    np.testing.assert_array_equal(host(v), rv)
    del t
    torch.cuda.empty_cache()


def test_aware_on_queues_that_start_elsewhere():
    """Range build and lookups in every mode on new streams, whose queues may deal workgroup 0
    to another XCC, before and after the library has learned the stream's offset: found and
    values bit-exact."""
    slots, n = 1 << 20, 400000
    keys, vals = ora.hash_kv(n + 50000, 21)
    q = np.concatenate([keys[:n:3], keys[n:]])
    ref = ora.HashTable(slots)
    assert ref.build(keys[:n], vals[:n]) == 0
    rv, rf = ref.lookup(q)
    dk, dv, dq = dev(keys[:n]), dev(vals[:n]), dev(q)
    torch.cuda.synchronize()
    for s in [torch.cuda.Stream() for _ in range(4)]:
        with torch.cuda.stream(s):
            t = HashTable(slots)
            for mode in ("aware", "rotated", "aware"):
                t.build(dk, dv, mode=mode)
                v, f = t.lookup(dq, mode=mode)
                s.synchronize()
                assert t.failures() == 0
                np.testing.assert_array_equal(f.cpu().numpy(), rf)
                np.testing.assert_array_equal(host(v), rv)


def _random_tables(n, seed):
    """Seeded (log2 slots, load factor, hit fraction, bulk build or inserts) draws."""
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(10, 23)), round(float(rng.uniform(0.05, 0.6)), 3), round(float(rng.uniform(0, 1)), 3),
             bool(rng.random() < 0.5)) for _ in range(n)]


@pytest.mark.parametrize("lg,lf,hits,bulk", _random_tables(10, 2026))
def test_random_tables_all_modes(lg, lf, hits, bulk):
    """Seeded random table sizes, load factors and hit fractions, built in bulk or by inserts and
    looked up in every mode: found and values bit-exact against the oracle's serial table."""
    slots = 1 << lg
    n = max(1, int(slots * lf))
    nq = max(1, n // 2)
    keys, vals = ora.hash_kv(n + nq, lg * 1000 + n)
    nh = int(nq * hits)
    rng = np.random.default_rng(n)
    q = np.concatenate([keys[rng.integers(0, n, size=nh)], keys[n:n + nq - nh]])
    rng.shuffle(q)
    ref = ora.HashTable(slots)
    assert ref.build(keys[:n], vals[:n]) == 0
    rv, rf = ref.lookup(q)
    dk, dv, dq = dev(keys[:n]), dev(vals[:n]), dev(q)
    for build_mode in MODES:
        t = HashTable(slots)
        if bulk:
            t.build(dk, dv, mode=build_mode)
        else:
            t.insert(dk, dv, mode=build_mode)
        for look_mode in MODES:
            v, f = t.lookup(dq, mode=look_mode)
            torch.cuda.synchronize()
            assert t.failures() == 0
            np.testing.assert_array_equal(f.cpu().numpy(), rf, err_msg=f"{build_mode} {look_mode}")
            np.testing.assert_array_equal(host(v), rv, err_msg=f"{build_mode} {look_mode}")

