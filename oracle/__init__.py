"""CPU oracle for the XCD-domain kernels -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker or the timed CPU baseline. The product never does.
The functions restate the reference's CPU verification loops (cited in oracle.c).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return C.CDLL(str(LIB_PATH))


lib = _load()
VP, SZ, I, I64, U64, U32, U16, D = (C.c_void_p, C.c_size_t, C.c_int, C.c_int64, C.c_uint64, C.c_uint32,
                                    C.c_uint16, C.c_double)
_SIGS = {
    "ora_splitmix64": (U64, [U64, U64]),
    "ora_mix32": (U32, [U32]),
    "ora_f64_to_f16": (U16, [D]),
    "ora_f16_to_f64": (D, [U16]),
    "ora_gen_uniform_f32": (None, [VP, SZ, U64]),
    "ora_gen_normal_f16": (None, [VP, SZ, D, D, U64]),
    "ora_gemv_f32_seq": (None, [VP, VP, VP, I64, I64, I]),
    "ora_gemv_f32_f64": (None, [VP, VP, VP, VP, I64, I64, I]),
    "ora_gemv_f16_f64": (None, [VP, VP, VP, VP, I64, I64, I]),
    "ora_zipf_thresholds": (None, [VP, U32, D]),
    "ora_gen_zipf_keys": (None, [VP, SZ, VP, U32, U64, I]),
    "ora_zipf_key_at": (U32, [VP, U32, U64, I, U64]),
    "ora_zipf_scramble": (U32, [U32, U32]),
    "ora_histogram": (U64, [VP, SZ, VP, U32, I]),
    "ora_gen_mix32_words": (None, [VP, SZ, U32]),
    "ora_hist256_bytes": (None, [VP, SZ, VP, I]),
    "ora_gen_mix32_f32": (None, [VP, SZ, U32, U32, C.c_int32]),
    "ora_mix64": (U64, [U64]),
    "ora_hash_kv": (None, [VP, VP, U64, U64]),
    "ora_hash_queries": (None, [VP, U64, U64, U64, U64]),
    "ora_hash_build": (U64, [VP, VP, U64, VP, VP, U64]),
    "ora_hash_lookup": (None, [VP, VP, U64, VP, U64, VP, VP, I]),
    "ora_rmat_edge": (None, [I, D, D, D, U64, U64, C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    "ora_rmat_csr": (I64, [I, I, D, D, D, U64, VP, VP]),
    "ora_bfs": (I64, [VP, VP, C.c_int32, C.c_int32, VP]),
    "ora_bfs_multi": (I64, [VP, VP, C.c_int32, VP, C.c_int32, C.c_int32, VP]),
    "ora_bfs_ref_graph": (I, [C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, U64, U64, VP, U64, VP, U64, VP,
                              VP, VP, VP]),
    "ora_dep_build": (I, [VP, U64, VP, VP, C.c_int32, U64]),
    "ora_dep_probe": (None, [VP, U64, VP, I64, I, VP]),
}
for _n, (_r, _a) in _SIGS.items():
    _f = getattr(lib, _n)
    _f.restype = _r
    _f.argtypes = _a


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def splitmix64(seed: int, index: int) -> int:
    return int(lib.ora_splitmix64(seed, index))


def mix32(x: int) -> int:
    return int(lib.ora_mix32(x))


def f64_to_f16_bits(d: float) -> int:
    return int(lib.ora_f64_to_f16(d))


def uniform_f32(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib.ora_gen_uniform_f32(_p(out), n, seed)
    return out


def normal_f16(n: int, mean: float, stddev: float, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib.ora_gen_normal_f16(_p(out), n, mean, stddev, seed)
    return out.view(np.float16)


def gemv_f32_seq(A: np.ndarray, x: np.ndarray, nthreads: int = 1) -> np.ndarray:
    """GEMV.cu:383-390: float running sum, k ascending."""
    A = np.ascontiguousarray(A, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = A.shape
    y = np.empty(M, dtype=np.float32)
    lib.ora_gemv_f32_seq(_p(A), _p(x), _p(y), M, K, nthreads)
    return y


def gemv_f64(A: np.ndarray, x: np.ndarray, nthreads: int = 1):
    """Returns (y, yabs) in float64: y = A.x, yabs[i] = sum_k |A_ik x_k|."""
    M, K = A.shape
    y = np.empty(M, dtype=np.float64)
    yabs = np.empty(M, dtype=np.float64)
    if A.dtype == np.float32:
        A = np.ascontiguousarray(A)
        x = np.ascontiguousarray(x, dtype=np.float32)
        lib.ora_gemv_f32_f64(_p(A), _p(x), _p(y), _p(yabs), M, K, nthreads)
    elif A.dtype == np.float16:
        A = np.ascontiguousarray(A).view(np.uint16)
        x = np.ascontiguousarray(x, dtype=np.float16).view(np.uint16)
        lib.ora_gemv_f16_f64(_p(A), _p(x), _p(y), _p(yabs), M, K, nthreads)
    else:
        raise TypeError(A.dtype)
    return y, yabs


def zipf_thresholds(num_bins: int, s: float) -> np.ndarray:
    t = np.empty(num_bins, dtype=np.uint64)
    lib.ora_zipf_thresholds(_p(t), num_bins, s)
    return t


def zipf_keys(n: int, t: np.ndarray, seed: int, scramble: bool = True) -> np.ndarray:
    keys = np.empty(n, dtype=np.uint32)
    lib.ora_gen_zipf_keys(_p(keys), n, _p(t), len(t), seed, 1 if scramble else 0)
    return keys


def zipf_key_at(t: np.ndarray, seed: int, index: int, scramble: bool = True) -> int:
    return int(lib.ora_zipf_key_at(_p(t), len(t), seed, 1 if scramble else 0, index))


def zipf_scramble(rank: int, num_bins: int) -> int:
    return int(lib.ora_zipf_scramble(rank, num_bins))


def histogram(keys: np.ndarray, num_bins: int, nthreads: int = 1) -> tuple[np.ndarray, int]:
    """HIST.cu:279-288 generalised: returns (counts u32[num_bins], number of keys counted)."""
    keys = np.ascontiguousarray(keys).view(np.uint32)
    counts = np.empty(num_bins, dtype=np.uint32)
    c = lib.ora_histogram(_p(keys), keys.size, _p(counts), num_bins, nthreads)
    return counts, int(c)


def mix32_words(n: int, seed: int = 0) -> np.ndarray:
    """HIST.cu:331-340: words[i] = mix32(i ^ seed) (the reference uses seed 0)."""
    out = np.empty(n, dtype=np.uint32)
    lib.ora_gen_mix32_words(_p(out), n, seed)
    return out


def hist256_bytes(words: np.ndarray, nthreads: int = 1) -> np.ndarray:
    """HIST.cu:279-288: every byte of every word counted into 256 bins."""
    words = np.ascontiguousarray(words).view(np.uint32)
    counts = np.empty(256, dtype=np.uint32)
    lib.ora_hist256_bytes(_p(words), words.size, _p(counts), nthreads)
    return counts


def mix32_f32(n: int, seed: int, modulus: int = 0, offset: int = 0) -> np.ndarray:
    """GEMV.cu:118-139 init_data values (modulus 0: (h & 0xff) / 255 - 0.5)."""
    out = np.empty(n, dtype=np.float32)
    lib.ora_gen_mix32_f32(_p(out), n, seed, modulus, offset)
    return out


EMPTY = 0xFFFFFFFFFFFFFFFF


def mix64(z: int) -> int:
    return int(lib.ora_mix64(z))


def hash_kv(n: int, seed: int):
    k = np.empty(n, dtype=np.uint64)
    v = np.empty(n, dtype=np.uint64)
    lib.ora_hash_kv(_p(k), _p(v), n, seed)
    return k, v


def hash_queries(n: int, n_keys: int, seed: int, qseed: int) -> np.ndarray:
    q = np.empty(n, dtype=np.uint64)
    lib.ora_hash_queries(_p(q), n, n_keys, seed, qseed)
    return q


class HashTable:
    """HASH.cu:226-241 serial insert and HASH.cu:46-64 probing, uint64 keys and values."""

    def __init__(self, slots: int):
        self.slots = slots
        self.keys = np.empty(slots, dtype=np.uint64)
        self.vals = np.empty(slots, dtype=np.uint64)

    def build(self, keys: np.ndarray, vals: np.ndarray) -> int:
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        vals = np.ascontiguousarray(vals, dtype=np.uint64)
        return int(lib.ora_hash_build(_p(self.keys), _p(self.vals), self.slots, _p(keys), _p(vals), keys.size))

    def lookup(self, q: np.ndarray, nthreads: int = 1):
        q = np.ascontiguousarray(q, dtype=np.uint64)
        v = np.empty(q.size, dtype=np.uint64)
        f = np.empty(q.size, dtype=np.uint8)
        lib.ora_hash_lookup(_p(self.keys), _p(self.vals), self.slots, _p(q), q.size, _p(v), _p(f), nthreads)
        return v, f


RMAT_ABC = (0.57, 0.19, 0.19)


def rmat_edge(scale: int, seed: int, e: int, abc=RMAT_ABC) -> tuple[int, int]:
    u, v = C.c_int32(), C.c_int32()
    lib.ora_rmat_edge(scale, *abc, seed, e, C.byref(u), C.byref(v))
    return u.value, v.value


def rmat_csr(scale: int, edge_factor: int, seed: int, abc=RMAT_ABC):
    V = 1 << scale
    rowptr = np.empty(V + 1, dtype=np.int32)
    col = np.empty(2 * edge_factor * V, dtype=np.int32)
    nnz = int(lib.ora_rmat_csr(scale, edge_factor, *abc, seed, _p(rowptr), _p(col)))
    return rowptr, col[:nnz].copy()


def bfs(rowptr: np.ndarray, col: np.ndarray, src: int):
    """Serial queue BFS: (level u32[V], number reached)."""
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    col = np.ascontiguousarray(col, dtype=np.int32)
    V = rowptr.size - 1
    level = np.empty(V, dtype=np.uint32)
    n = int(lib.ora_bfs(_p(rowptr), _p(col) if col.size else None, V, src, _p(level)))
    return level, n


def bfs_multi(rowptr: np.ndarray, col: np.ndarray, sources: np.ndarray, max_depth: int):
    """Multi-source BFS limited to max_depth top-down levels: (level u32[V], number reached)."""
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    col = np.ascontiguousarray(col, dtype=np.int32)
    sources = np.ascontiguousarray(sources, dtype=np.int32)
    V = rowptr.size - 1
    level = np.empty(V, dtype=np.uint32)
    n = int(lib.ora_bfs_multi(_p(rowptr), _p(col) if col.size else None, V, _p(sources) if sources.size else None,
                              sources.size, max_depth, _p(level)))
    return level, n


def bfs_ref_graph(V: int, degree: int, nsrc: int, dst_local_pct: int, H: int, seed: int, col_addr: int,
                  col_home, level_addr: int, level_home, mask: int):
    """bfs.cu:354-409: (rowptr, col, work_side, sources), or None when a hot pool is short."""
    rowptr = np.empty(V + 1, dtype=np.int32)
    col = np.empty(V * degree, dtype=np.int32)
    ws = np.empty(V, dtype=np.uint8)
    src = np.empty(max(nsrc, 1), dtype=np.int32)
    ch = None if col_home is None else np.ascontiguousarray(col_home, dtype=np.uint8)
    lh = None if level_home is None else np.ascontiguousarray(level_home, dtype=np.uint8)
    rc = lib.ora_bfs_ref_graph(V, degree, nsrc, dst_local_pct, H, seed, col_addr, None if ch is None else _p(ch),
                               level_addr, None if lh is None else _p(lh), mask, _p(rowptr), _p(col), _p(ws), _p(src))
    if rc != 0:
        return None
    return rowptr, col, ws, src[:nsrc]


def dep_build(slots: int, keys: np.ndarray, nexts: np.ndarray, seed: int) -> np.ndarray:
    """HASH.cu:226-241: int32 table[slots, 2] = {key, next}, serial shuffled insertion."""
    keys = np.ascontiguousarray(keys, dtype=np.int32)
    nexts = np.ascontiguousarray(nexts, dtype=np.int32)
    t = np.empty(2 * slots, dtype=np.int32)
    rc = lib.ora_dep_build(_p(t), slots, _p(keys), _p(nexts), keys.size, seed)
    if rc:
        raise ValueError("dep_build failed")
    return t


def dep_probe(table: np.ndarray, slots: int, queries: np.ndarray, chain_len: int) -> np.ndarray:
    """HASH.cu:46-83: out[i] = (sum of found slots, -1 per miss) ^ final key."""
    queries = np.ascontiguousarray(queries, dtype=np.int32)
    out = np.empty(queries.size, dtype=np.int32)
    lib.ora_dep_probe(_p(np.ascontiguousarray(table, dtype=np.int32)), slots, _p(queries), queries.size, chain_len,
                      _p(out))
    return out
