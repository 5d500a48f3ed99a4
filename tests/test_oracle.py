"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each check is independent of the oracle's own formula: numpy integer brute force (exact for 8-bit
data), exact rational arithmetic, closed forms for duplicates and ties, the filter semantics of the
reference's C API, the committed golden fixtures, and the reference's known answer for
certex.verify (tests/test_exact.py:440-452: 2/3 after corrupting 100 of 300 queries).
"""

import os
from fractions import Fraction

import numpy as np
import pytest

import oracle
from tests import data

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def numpy_int_knn(X, Q, k, metric, keep=None):
    """Exact integer brute force: int64 scores, ids ordered by (score, id)."""
    Xi, Qi = X.astype(np.int64), Q.astype(np.int64)
    if metric == "l2":
        s = ((Qi[:, None, :] - Xi[None]) ** 2).sum(-1)
    else:
        s = -(Qi @ Xi.T)
    if keep is not None:
        s = np.where(keep, s, np.iinfo(np.int64).max)
    ids = np.tile(np.arange(X.shape[0]), (Q.shape[0], 1))
    order = np.lexsort((ids, s), axis=1)[:, :k]
    return np.take_along_axis(s, order, 1), order


@pytest.mark.parametrize("dtype", [np.uint8, np.int8])
@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_integer_brute_force(dtype, metric):
    X = data.uniform_int(3000, 37, seed=5, dtype=dtype)
    Q = data.uniform_int(40, 37, seed=6, dtype=dtype)
    s, i = oracle.knn(X, Q, 17, metric)
    rs, ri = numpy_int_knn(X, Q, 17, metric)
    np.testing.assert_array_equal(i, ri)
    np.testing.assert_array_equal(s, rs.astype(np.float64))


def test_integer_ties_go_to_lower_id():
    # few distinct values in 2 coordinates: many exactly equal distances
    X = data.uniform_int(5000, 2, seed=1, lo=0, hi=3)
    Q = data.uniform_int(30, 2, seed=2, lo=0, hi=3)
    s, i = oracle.knn(X, Q, 50, "l2")
    rs, ri = numpy_int_knn(X, Q, 50, "l2")
    np.testing.assert_array_equal(i, ri)
    for q in range(30):  # within equal scores the ids ascend
        for j in range(49):
            if s[q, j] == s[q, j + 1]:
                assert i[q, j] < i[q, j + 1]


def test_identical_rows_closed_form():
    X = np.tile(data.gaussian(1, 16, 3), (100, 1))
    Q = data.gaussian(4, 16, 4)
    s, i = oracle.knn(X, Q, 10, "l2")
    np.testing.assert_array_equal(i, np.tile(np.arange(10), (4, 1)))
    assert (s == s[:, :1]).all()


def test_float_scores_against_exact_rationals():
    X = data.gaussian(50, 24, 7)
    Q = data.gaussian(3, 24, 8)
    for metric in ("l2", "ip", "cosine"):
        got = oracle.scores_of(X, Q, np.tile(np.arange(50), (3, 1)), metric)
        for q in range(3):
            for r in range(50):
                a = [Fraction(float(v)) for v in Q[q]]
                b = [Fraction(float(v)) for v in X[r]]
                if metric == "l2":
                    exact = float(sum((u - v) ** 2 for u, v in zip(a, b)))
                elif metric == "ip":
                    exact = -float(sum(u * v for u, v in zip(a, b)))
                else:
                    dot = float(sum(u * v for u, v in zip(a, b)))
                    qq = float(sum(u * u for u in a))
                    xx = float(sum(v * v for v in b))
                    exact = -dot / np.sqrt(qq * xx)
                assert abs(got[q, r] - exact) <= 1e-13 * max(1.0, abs(exact))


def test_float_knn_against_numpy():
    X = data.gaussian(4000, 32, 9)
    Q = data.gaussian(25, 32, 10)
    s, i = oracle.knn(X, Q, 10, "l2")
    ref = ((Q.astype(np.float64)[:, None, :] - X.astype(np.float64)[None]) ** 2).sum(-1)
    ri = np.argsort(ref, axis=1, kind="stable")[:, :10]
    np.testing.assert_array_equal(i, ri)
    np.testing.assert_allclose(s, np.take_along_axis(ref, ri, 1), rtol=1e-12)


def test_filters_and_removed():
    X = data.uniform_int(2000, 8, seed=11)
    Q = data.uniform_int(20, 8, seed=12)
    rng = np.random.default_rng(13)
    keep = rng.random(2000) < 0.3
    words = np.zeros(63, np.uint32)
    for j in np.flatnonzero(keep):
        words[j >> 5] |= np.uint32(1 << (j & 31))
    s, i = oracle.knn(X, Q, 7, "l2", bitset=words)
    rs, ri = numpy_int_knn(X, Q, 7, "l2", keep=keep[None, :])
    np.testing.assert_array_equal(i, ri)
    s2, i2 = oracle.knn(X, Q, 7, "l2", removed=(~keep).astype(np.uint8))
    np.testing.assert_array_equal(i2, ri)
    # bitmap: one row of bits per query
    km = rng.random((20, 2000)) < 0.2
    bits = np.packbits(km.reshape(-1), bitorder="little")
    bits = np.pad(bits, (0, (-bits.size) % 4)).view(np.uint32)
    s3, i3 = oracle.knn(X, Q, 7, "l2", bitmap=bits)
    rs3, ri3 = numpy_int_knn(X, Q, 7, "l2", keep=km)
    np.testing.assert_array_equal(i3, ri3)
    # labels
    rl = rng.integers(0, 4, 2000).astype(np.int32)
    ql = rng.integers(0, 4, 20).astype(np.int32)
    s4, i4 = oracle.knn(X, Q, 7, "l2", row_labels=rl, query_labels=ql)
    rs4, ri4 = numpy_int_knn(X, Q, 7, "l2", keep=rl[None, :] == ql[:, None])
    np.testing.assert_array_equal(i4, ri4)


def test_missing_entries():
    X = data.uniform_int(100, 4, seed=1)
    Q = data.uniform_int(3, 4, seed=2)
    keep = np.zeros(4, np.uint32)
    keep[0] = 0b1011  # ids 0, 1, 3
    s, i = oracle.knn(X, Q, 5, "l2", bitset=keep)
    assert (i[:, 3:] == -1).all() and np.isinf(s[:, 3:]).all()
    assert set(i[0, :3]) == {0, 1, 3}
    d = oracle.distances(s, i, "ip")
    assert np.isneginf(d[:, 3:]).all()


def test_golden_fixtures():
    """The committed fixtures (written by tests/golden/make_golden.py) still match the oracle."""
    for name in sorted(os.listdir(GOLDEN)):
        if not name.endswith(".npz"):
            continue
        f = np.load(os.path.join(GOLDEN, name))
        s, i = oracle.knn(f["base"], f["queries"], int(f["k"]), str(f["metric"]))
        np.testing.assert_array_equal(i, f["ids"], err_msg=name)
        np.testing.assert_array_equal(s, f["scores"], err_msg=name)


def test_verify_known_answer():
    """The reference's known answer for certex.verify (tests/test_exact.py:440-452)."""
    torch = pytest.importorskip("torch")
    from libcertex_amd.index import verify

    g = torch.Generator().manual_seed(7)
    A = torch.randn(32, 32, generator=g) / 32**0.5
    X = (torch.randn(20_000, 32, generator=g) @ A).numpy()
    Q = (torch.randn(300, 32, generator=g) @ A).numpy()
    s, I = oracle.knn(X, Q, 10, "l2")
    assert verify(X, Q, I, sample=None) == 1.0
    wrong = I.copy()
    wrong[:100, 9] = (wrong[:100, 9] + 9_973) % X.shape[0]
    assert abs(verify(X, Q, wrong, sample=None) - 2 / 3) < 1e-6


@pytest.mark.parametrize("dtype", [np.uint8, np.int8, np.float32, np.float16])
@pytest.mark.parametrize("d", [5, 64, 100, 130, 257])
def test_specialised_scorers_equal_the_generic_one(dtype, d):
    """The searches score through type-specialised loops (exact int32 sums for 8-bit data, the
    canonical 64-lane order vectorised for floats); they must give oracle_score's bits exactly,
    ties and ids included."""
    rng = np.random.default_rng(d)
    if dtype in (np.uint8, np.int8):
        info = np.iinfo(dtype)
        X = rng.integers(info.min, info.max + 1, (2_000, d)).astype(dtype)
        Q = rng.integers(info.min, info.max + 1, (16, d)).astype(dtype)
        X[100:110] = X[5]  # exact ties
        metrics = ("l2", "ip")
    else:
        X = (rng.standard_normal((2_000, d)) * 3).astype(dtype)
        Q = (rng.standard_normal((16, d)) * 3).astype(dtype)
        X[100:110] = X[5]
        metrics = ("l2", "ip", "cosine")
    for metric in metrics:
        s1, i1 = oracle.knn(X, Q, 20, metric)
        with oracle.generic_scores():
            s0, i0 = oracle.knn(X, Q, 20, metric)
        np.testing.assert_array_equal(i1, i0)
        np.testing.assert_array_equal(s1.view(np.int64), s0.view(np.int64))
        ids = np.tile(np.arange(0, 2_000, 100), (16, 1))
        fast = oracle.scores_of(X, Q, ids, metric)
        with oracle.generic_scores():
            slow = oracle.scores_of(X, Q, ids, metric)
        np.testing.assert_array_equal(fast.view(np.int64), slow.view(np.int64))
