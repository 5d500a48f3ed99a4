"""k-means lists and the list probe against the CPU oracle.

Lists are a speed option (reference lists.cuh, certex.cu:684-692 and 1031-1050): the rows of the
build are stored in list order and a search first screens the rows of each query's nearest lists,
whose exact scores bound its threshold. Results must not change: ids equal to the oracle's
exhaustive fp64 search, ties to the lower id, for every probe width, after additions (which follow
the lists unordered), removals, filters, labels and a save / load round trip.
"""

import numpy as np
import pytest
import torch

import libcertex_amd as certex
import oracle
from tests import data

pytestmark = pytest.mark.gpu


def check(X, Q, k, metric, D, I, **okw):
    s, i = oracle.knn(X, Q, k, metric, **okw)
    np.testing.assert_array_equal(I, i)
    d = oracle.distances(s, i, metric)
    if metric == "cosine":
        d = np.where(i >= 0, np.float32(1) - d, -np.inf).astype(np.float32)
    np.testing.assert_array_equal(D, d)


def search(idx, Q, k, **kw):
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=k, **kw)
    torch.cuda.synchronize()
    return D.cpu().numpy(), I.cpu().numpy()


@pytest.mark.parametrize("dtype,n_lists", [(np.uint8, 64), (np.uint8, 500), (np.int8, 100)])
def test_integer_lists(gpu, dtype, n_lists):
    if dtype == np.uint8:
        X, Q = data.mixture_u8(40_000, seed=81), data.mixture_u8(600, seed=82)
    else:
        X, Q = data.uniform_int(40_000, 96, 81, np.int8), data.uniform_int(600, 96, 82, np.int8)
    idx = certex.Index(X.shape[1], n_lists=n_lists)
    idx.add(torch.from_numpy(X).cuda())
    assert idx.core.lists == (n_lists, len(X))
    for probe in (0, 1, 2, 8):
        D, I = search(idx, Q, 10, probe_lists=probe)
        check(X, Q, 10, "l2", D, I)
    D, I = search(idx, Q, 100, probe_lists=2, batch=250)
    check(X, Q, 100, "l2", D, I)
    D, I = search(idx, Q, 100, probe_lists=0, batch=250)  # k above 64: the anchors of every row
    check(X, Q, 100, "l2", D, I)


def test_integer_lists_host_source(gpu):
    """A host dataset: the rows are gathered in list order on the host."""
    X, Q = data.mixture_u8(30_000, seed=83), data.mixture_u8(300, seed=84)
    idx = certex.Index(128, n_lists=128)
    idx.add(X)
    D, I = search(idx, Q, 10)
    check(X, Q, 10, "l2", D, I)


@pytest.mark.parametrize("metric,d,n_lists", [("l2", 64, 64), ("cosine", 128, 200), ("ip", 300, 50), ("cosine", 768, 100)])
def test_float_lists(gpu, metric, d, n_lists):
    X = data.powerlaw_unit(30_000, d, seed=85) * np.float32(1.0 if metric != "ip" else 3.0)
    Q = data.powerlaw_unit(300, d, seed=86)
    idx = certex.Index(d, metric=metric, n_lists=n_lists)
    idx.add(torch.from_numpy(X).cuda())
    for probe, k in ((2, 10), (8, 10), (1, 100)):
        D, I = search(idx, Q, k, probe_lists=probe, batch=300)
        check(X, Q, k, metric, D, I)


def test_lists_extend_remove_filter(gpu):
    """Additions after the build follow the lists; removals and filters reach rows in list order."""
    X, Q = data.mixture_u8(50_000, seed=87), data.mixture_u8(400, seed=88)
    idx = certex.Index(128, n_lists=256, capacity=60_000)
    idx.add(torch.from_numpy(X[:35_000]).cuda())
    assert idx.core.capacity == 60_000  # allocated by the build
    idx.add(torch.from_numpy(X[35_000:]).cuda())
    assert idx.core.lists == (256, 35_000) and idx.core.capacity == 60_000
    _, nn = oracle.knn(X, Q, 1, "l2")
    gone = np.unique(np.concatenate([nn[:, 0], np.arange(0, 50_000, 89)]))
    idx.remove(torch.from_numpy(gone))
    removed = np.zeros(len(X), np.uint8)
    removed[gone] = 1
    D, I = search(idx, Q, 10)
    check(X, Q, 10, "l2", D, I, removed=removed)
    keep = np.random.default_rng(90).random(len(X)) < 0.3
    D, I = search(idx, Q, 10, filter=torch.from_numpy(keep))
    check(X, Q, 10, "l2", D, I, removed=(removed.astype(bool) | ~keep).astype(np.uint8))
    km = np.random.default_rng(91).random((len(Q), len(X))) < 0.05
    D, I = search(idx, Q, 5, filter=torch.from_numpy(km))
    bits = np.packbits(km.reshape(-1), bitorder="little")
    bits = np.pad(bits, (0, (-bits.size) % 4)).view(np.uint32)
    check(X, Q, 5, "l2", D, I, removed=removed, bitmap=bits)


def test_lists_with_labels(gpu):
    """Labels and the label partition over an index stored in list order."""
    X, Q = data.mixture_u8(30_000, seed=92), data.mixture_u8(300, seed=93)
    lx, lq = data.labels(len(X), 8, 94), data.labels(len(Q), 8, 95)
    idx = certex.Index(128, n_lists=128)
    idx.add(torch.from_numpy(X).cuda(), labels=torch.from_numpy(lx))
    assert idx.core.n_partitioned == len(X)
    idx.remove(torch.arange(0, 30_000, 7))
    removed = np.zeros(len(X), np.uint8)
    removed[::7] = 1
    D, I = search(idx, Q, 10, labels=torch.from_numpy(lq))
    check(X, Q, 10, "l2", D, I, removed=removed, row_labels=lx, query_labels=lq)
    Xf = data.powerlaw_unit(20_000, 256, seed=96)
    Qf = data.powerlaw_unit(200, 256, seed=97)
    lf, lqf = data.labels(len(Xf), 4, 98), data.labels(len(Qf), 4, 99)
    fidx = certex.Index(256, metric="cosine", n_lists=64)
    fidx.add(torch.from_numpy(Xf).cuda(), labels=torch.from_numpy(lf))
    D, I = search(fidx, Qf, 20, labels=torch.from_numpy(lqf))
    check(Xf, Qf, 20, "cosine", D, I, row_labels=lf, query_labels=lqf)


def test_lists_save_load(gpu, tmp_path):
    X, Q = data.mixture_u8(20_000, seed=100), data.mixture_u8(200, seed=101)
    idx = certex.Index(128, n_lists=100)
    idx.add(torch.from_numpy(X).cuda())
    idx.add(torch.from_numpy(data.mixture_u8(5_000, seed=102)).cuda())
    idx.remove(torch.arange(0, 25_000, 11))
    D0, I0 = search(idx, Q, 10)
    L0 = search(idx, Q, 10, probe_lists=0)  # the list anchors: the loaded lists' offsets
    idx.save(tmp_path / "lists.idx")
    back = certex.Index.load(tmp_path / "lists.idx")
    assert back.core.lists == (100, 20_000)
    D1, I1 = search(back, Q, 10)
    np.testing.assert_array_equal(I0, I1)
    np.testing.assert_array_equal(D0, D1)
    L1 = search(back, Q, 10, probe_lists=0)
    np.testing.assert_array_equal(L0[1], L1[1])
    np.testing.assert_array_equal(L0[0], L1[0])
    np.testing.assert_array_equal(L1[1], I1)
    Xf = data.powerlaw_unit(10_000, 96, seed=103)
    fidx = certex.Index(96, n_lists=40)
    fidx.add(torch.from_numpy(Xf).cuda())
    D0, I0 = search(fidx, Xf[:100], 10)
    fidx.save(tmp_path / "flists.idx")
    D1, I1 = search(certex.Index.load(tmp_path / "flists.idx"), Xf[:100], 10)
    np.testing.assert_array_equal(I0, I1)
    np.testing.assert_array_equal(D0, D1)


def test_lists_tiny_and_errors(gpu):
    """As many lists as vectors, one list, and more lists than vectors (an error)."""
    X, Q = data.uniform_int(300, 32, 104), data.uniform_int(50, 32, 105)
    for n_lists in (300, 1):
        idx = certex.Index(32, n_lists=n_lists)
        idx.add(torch.from_numpy(X).cuda())
        D, I = search(idx, Q, 7)
        check(X, Q, 7, "l2", D, I)
    with pytest.raises(ValueError):
        certex.Index(32, n_lists=301).add(torch.from_numpy(X).cuda())


def test_probe_lowers_survivors(gpu):
    """On clustered data the probe's threshold keeps fewer survivors than the anchors' alone."""
    X, Q = data.mixture_u8(200_000, seed=106), data.mixture_u8(1_000, seed=107)
    idx = certex.Index(128, n_lists=256)
    idx.add(torch.from_numpy(X).cuda())
    counts = {}
    for probe in (0, 2):
        with certex.search_stats() as st:
            D, I = search(idx, Q, 10, probe_lists=probe)
        counts[probe] = st.survivors
        check(X, Q[:64], 10, "l2", D[:64], I[:64])
    assert counts[2] <= counts[0]


def test_list_anchor_threshold(gpu):
    """Without a probe, an index in lists bounds its thresholds by the anchors of each query's 8
    nearest lists instead of the anchors of every row (a bitset filter keeps the latter): the same
    results, and on clustered data about as tight, as the nearest lists hold the anchors that set
    the threshold."""
    X, Q = data.mixture_u8(400_000, seed=112), data.mixture_u8(500, seed=113)
    idx = certex.Index(128, n_lists=160)
    idx.add(torch.from_numpy(X).cuda())
    surv = {}
    for name, kw in (("lists", {}), ("every row", {"filter": torch.ones(len(X), dtype=torch.bool)})):
        with certex.search_stats() as st:
            D, I = search(idx, Q, 10, probe_lists=0, **kw)
        surv[name] = st.survivors
        check(X, Q[:64], 10, "l2", D[:64], I[:64])
    assert surv["lists"] <= 1.25 * surv["every row"], surv


@pytest.mark.parametrize("metric", ["l2", "cosine"])
def test_probe_coarse_groups(gpu, metric):
    """Lists too long for groups of 4 rows in the probe's table: groups of whole steps instead."""
    if metric == "l2":
        X, Q = data.mixture_u8(1_000_000, seed=108), data.mixture_u8(1_000, seed=109)
    else:
        X, Q = data.powerlaw_unit(800_000, 64, seed=108), data.powerlaw_unit(1_000, 64, seed=109)
    idx = certex.Index(X.shape[1], metric=metric, n_lists=2)
    idx.add(torch.from_numpy(X).cuda())
    D, I = search(idx, Q, 10, probe_lists=1)
    check(X, Q[:64], 10, metric, D[:64], I[:64])


def nearest_removed(X, Q, metric):
    """Ids of every query's nearest neighbour, and the removal mask that takes them all out."""
    _, nn = oracle.knn(X, Q, 1, metric)
    gone = np.unique(nn[:, 0])
    removed = np.zeros(len(X), np.uint8)
    removed[gone] = 1
    return gone, removed


def test_listed_anchors_follow_ids(gpu):
    """Anchor j of an index stored in list order is id j * stride, read from that id's stored row.
    With stride 1 every id is an anchor: removing each query's nearest neighbour must take its
    anchor out too, for the thresholds without the probe (all from anchors) and under a bitmap
    filter (which the probe does not serve)."""
    X, Q = data.mixture_u8(30_000, seed=110), data.mixture_u8(300, seed=111)
    idx = certex.Index(128, n_lists=64, anchor_stride=1)
    idx.add(torch.from_numpy(X).cuda())
    gone, removed = nearest_removed(X, Q, "l2")
    idx.remove(torch.from_numpy(gone))
    for k in (1, 10):
        D, I = search(idx, Q, k, probe_lists=0)
        check(X, Q, k, "l2", D, I, removed=removed)
    km = np.random.default_rng(112).random((len(Q), len(X))) < 0.5
    D, I = search(idx, Q, 10, filter=torch.from_numpy(km))
    bits = np.packbits(km.reshape(-1), bitorder="little")
    bits = np.pad(bits, (0, (-bits.size) % 4)).view(np.uint32)
    check(X, Q, 10, "l2", D, I, removed=removed, bitmap=bits)
    keep = np.random.default_rng(113).random(len(X)) < 0.5
    D, I = search(idx, Q, 10, filter=torch.from_numpy(keep))
    check(X, Q, 10, "l2", D, I, removed=(removed.astype(bool) | ~keep).astype(np.uint8))


@pytest.mark.parametrize("stride", [1, 4])
def test_listed_float_anchors_after_load(gpu, tmp_path, stride):
    """A float index in list order with removals, saved and loaded (the anchor copy is gathered
    again from the stored rows): searches without the probe take their thresholds from the anchors
    and must still equal the oracle."""
    X, Q = data.powerlaw_unit(20_000, 96, seed=114), data.powerlaw_unit(200, 96, seed=115)
    idx = certex.Index(96, n_lists=50, anchor_stride=stride)
    idx.add(torch.from_numpy(X).cuda())
    gone, removed = nearest_removed(X, Q, "l2")
    idx.remove(torch.from_numpy(gone))
    D, I = search(idx, Q, 10, probe_lists=0)
    check(X, Q, 10, "l2", D, I, removed=removed)
    idx.save(tmp_path / "flisted.idx")
    back = certex.Index.load(tmp_path / "flisted.idx")
    for probe in (0, 2):
        D, I = search(back, Q, 10, probe_lists=probe)
        check(X, Q, 10, "l2", D, I, removed=removed)


@pytest.mark.parametrize("kind", ["uint8", "float32"])
def test_list_order(gpu, tmp_path, kind):
    """list_order is a permutation of the ids (tests/test_exact.py:479-486): rows of the build in
    list order, later rows in id order; searching stored vectors in that order finds themselves."""
    if kind == "uint8":
        X = data.uniform_int(20_000, 32, 116)
    else:
        X = np.random.default_rng(116).standard_normal((20_000, 32)).astype(np.float32)
    idx = certex.Index(32, n_lists=16)
    idx.add(torch.from_numpy(X[:18_000]).cuda())
    idx.add(torch.from_numpy(X[18_000:]).cuda())
    order = idx.list_order()
    assert order.dtype == torch.int64 and order.is_cuda
    o = order.cpu().numpy()
    np.testing.assert_array_equal(np.sort(o), np.arange(20_000))
    np.testing.assert_array_equal(o[18_000:], np.arange(18_000, 20_000))
    assert not np.array_equal(o[:18_000], np.arange(18_000))  # the build's rows moved into lists
    D, I = search(idx, X[o[:200]], 1)
    np.testing.assert_array_equal(I[:, 0], o[:200])
    idx.save(tmp_path / "order.idx")
    back = certex.Index.load(tmp_path / "order.idx")
    np.testing.assert_array_equal(back.list_order().cpu().numpy(), o)
    with pytest.raises(ValueError):
        plain = certex.Index(32)
        plain.add(torch.from_numpy(X).cuda())
        plain.list_order()
