"""CPU oracle of the exact k-NN path: TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py load this module, as the
checker; the library (libcertex_amd) never does. The arithmetic lives in oracle.c (built by the
Makefile next to it into _build/liboracle.so); see the header of oracle.c for the score definitions
and the reference lines they follow.
"""

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "liboracle.so")
_DT = {np.dtype(np.float32): 0, np.dtype(np.float16): 1, np.dtype(np.int8): 2, np.dtype(np.uint8): 3}
METRICS = {"l2": 0, "ip": 1, "inner": 1, "cosine": 2}
_lib = None


def build():
    """Compile liboracle.so (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        lib = ctypes.CDLL(LIB)
        p, i64, i32, dbl = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
        lib.oracle_knn.argtypes = [p, i32, i64, i64, p, i64, i32, i32, p, p, p, p, p, p, p]
        lib.oracle_knn.restype = None
        lib.oracle_scores_of.argtypes = [p, i32, i64, i64, p, i64, i32, i32, p, p]
        lib.oracle_scores_of.restype = None
        lib.oracle_score.argtypes = [p, p, i32, i64, i32]
        lib.oracle_score.restype = dbl
        lib.oracle_threads.argtypes = []
        lib.oracle_threads.restype = i32
        lib.oracle_set_generic.argtypes = [i32]
        lib.oracle_set_generic.restype = i32
        _lib = lib
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class generic_scores:
    """Inside the block, searches score through the generic per-coordinate scorer (oracle_score)
    instead of the type-specialised ones; tests compare the two."""

    def __enter__(self):
        self.was = _load().oracle_set_generic(1)
        return self

    def __exit__(self, *exc):
        _load().oracle_set_generic(self.was)
        return False


def cpu_model():
    """The host CPU's model name (from /proc/cpuinfo), for the CPU baseline's record."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def threads():
    """OpenMP threads the oracle runs on."""
    return int(_load().oracle_threads())


def knn(base, queries, k, metric="l2", removed=None, bitset=None, bitmap=None, row_labels=None,
        query_labels=None):
    """Exhaustive fp64 k-NN: (scores [nq, k] float64, ids [nq, k] int64), ascending (score, id).

    Scores are smaller-is-better: l2 = squared distance, ip = -<q, x>, cosine = -cos."""
    base = np.ascontiguousarray(base)
    queries = np.ascontiguousarray(queries, dtype=base.dtype)
    n, d = base.shape
    nq = queries.shape[0]
    s = np.empty((nq, k), np.float64)
    i = np.empty((nq, k), np.int64)
    rem = None if removed is None else np.ascontiguousarray(removed, dtype=np.uint8)
    bs = None if bitset is None else np.ascontiguousarray(bitset).view(np.uint32)
    bm = None if bitmap is None else np.ascontiguousarray(bitmap).view(np.uint32)
    rl = None if row_labels is None else np.ascontiguousarray(row_labels, dtype=np.int32)
    ql = None if query_labels is None else np.ascontiguousarray(query_labels, dtype=np.int32)
    _load().oracle_knn(_ptr(base), _DT[base.dtype], n, d, _ptr(queries), nq, METRICS[metric], k,
                       _ptr(rem), _ptr(bs), _ptr(bm), _ptr(rl), _ptr(ql), _ptr(s), _ptr(i))
    return s, i


def scores_of(base, queries, ids, metric="l2"):
    """Exact scores of the given ids (+inf for -1), same definitions as knn()."""
    base = np.ascontiguousarray(base)
    queries = np.ascontiguousarray(queries, dtype=base.dtype)
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    n, d = base.shape
    nq, k = ids.shape
    out = np.empty((nq, k), np.float64)
    _load().oracle_scores_of(_ptr(base), _DT[base.dtype], n, d, _ptr(queries), nq, METRICS[metric], k,
                             _ptr(ids), _ptr(out))
    return out


def distances(scores, ids, metric="l2"):
    """Output conversion of the reference's finish (certex.cu:224-250) as float32: l2 = score,
    ip = -score, cosine distance = 1 + score; missing entries +inf (-inf for ip)."""
    if metric == "l2":
        d = scores
    elif metric in ("ip", "inner"):
        d = -scores
    else:
        d = 1.0 + scores
    d = d.astype(np.float32)
    miss = ids < 0
    d[miss] = -np.inf if metric in ("ip", "inner") else np.inf
    return d
