"""Label search over the label partition (routed) against the CPU oracle.

The partition is a speed option (reference certex.cu:1542-1735): every label's queries screen only
that label's rows, the rows added after the partition go through the label filter, and results
must stay bit-exact: ids equal to the oracle's exhaustive fp64 search among the rows of the
query's label, ties to the lower id. Cases follow the reference's label tests
(tests/test_exact.py label cases, ann_certex.cuh label matrix): skewed and missing labels,
queries whose label has no rows, additions and removals after the partition, ragged batches;
each with the query labels in host memory and in device memory (the device builds the routing).
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


PLACE = {"labels": "host"}


@pytest.fixture(params=["host", "device"], autouse=True)
def label_place(request):
    """Every case twice: query labels in host memory (routing planned on the host) and in device
    memory (routing built on the device, no read-back)."""
    PLACE["labels"] = request.param
    yield
    PLACE["labels"] = "host"


def search(idx, Q, k, ql, batch=2048):
    lq = torch.from_numpy(ql)
    if PLACE["labels"] == "device":
        lq = lq.cuda()
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=k, batch=batch, labels=lq)
    torch.cuda.synchronize()
    return D.cpu().numpy(), I.cpu().numpy()


def skewed_labels(n, seed, n_classes=16):
    """Labels with a skewed histogram: class c has weight 2^-c / ..., class 5 is never used."""
    w = 0.5 ** np.arange(n_classes)
    w[5] = 0
    return np.random.default_rng(seed).choice(n_classes, n, p=w / w.sum()).astype(np.int32)


@pytest.mark.parametrize("dtype", [np.uint8, np.int8])
def test_integer_routed(gpu, dtype):
    X = data.mixture_u8(40_000, seed=61) if dtype == np.uint8 else data.uniform_int(40_000, 96, 61, np.int8)
    Q = data.mixture_u8(700, seed=62) if dtype == np.uint8 else data.uniform_int(700, 96, 62, np.int8)
    lx, lq = skewed_labels(len(X), 63), data.labels(len(Q), 18, 64)  # labels 16, 17 and 5: no rows
    idx = certex.Index(X.shape[1])
    idx.add(torch.from_numpy(X).cuda(), labels=torch.from_numpy(lx))
    assert idx.core is not None
    for batch in (2048, 150):
        D, I = search(idx, Q, 10, lq, batch)
        check(X, Q, 10, "l2", D, I, row_labels=lx, query_labels=lq)


@pytest.mark.parametrize("metric,d", [("l2", 64), ("cosine", 64), ("ip", 300), ("cosine", 768)])
def test_float_routed(gpu, metric, d):
    X = data.powerlaw_unit(30_000, d, seed=65) * np.float32(1.0 if metric != "ip" else 3.0)
    Q = data.powerlaw_unit(400, d, seed=66)
    lx, lq = data.labels(len(X), 16, 67), data.labels(len(Q), 16, 68)
    idx = certex.Index(d, metric=metric)
    idx.add(torch.from_numpy(X).cuda(), labels=torch.from_numpy(lx))
    D, I = search(idx, Q, 50, lq, batch=256)
    check(X, Q, 50, metric, D, I, row_labels=lx, query_labels=lq)


def test_tail_after_partition_and_removals(gpu):
    """Rows added after the partition (the tail) go through the label filter; removals reach the
    partition's copy of the rows."""
    X = data.mixture_u8(50_000, seed=71)
    Q = data.mixture_u8(300, seed=72)
    lx, lq = data.labels(len(X), 8, 73), data.labels(len(Q), 8, 74)
    idx = certex.Index(128)
    idx.add(torch.from_numpy(X[:30_000]).cuda(), labels=torch.from_numpy(lx[:30_000]))
    idx.partition_labels = False  # the next rows stay outside the partition
    idx.add(torch.from_numpy(X[30_000:]).cuda(), labels=torch.from_numpy(lx[30_000:]))
    _, nn = oracle.knn(X, Q, 1, "l2", row_labels=lx, query_labels=lq)
    gone = np.unique(np.concatenate([nn[:, 0], np.arange(0, 50_000, 97)]))
    idx.remove(torch.from_numpy(gone))
    removed = np.zeros(len(X), np.uint8)
    removed[gone] = 1
    D, I = search(idx, Q, 10, lq)
    check(X, Q, 10, "l2", D, I, removed=removed, row_labels=lx, query_labels=lq)


def test_float_tail_wide(gpu):
    X = data.powerlaw_unit(20_000, 256, seed=75)
    Q = data.powerlaw_unit(200, 256, seed=76)
    lx, lq = data.labels(len(X), 4, 77), data.labels(len(Q), 4, 78)
    idx = certex.Index(256, metric="cosine")
    idx.add(torch.from_numpy(X[:15_000]).cuda(), labels=torch.from_numpy(lx[:15_000]))
    idx.partition_labels = False
    idx.add(torch.from_numpy(X[15_000:]).cuda(), labels=torch.from_numpy(lx[15_000:]))
    idx.remove(torch.arange(0, 20_000, 5))
    removed = np.zeros(len(X), np.uint8)
    removed[::5] = 1
    D, I = search(idx, Q, 20, lq)
    check(X, Q, 20, "cosine", D, I, removed=removed, row_labels=lx, query_labels=lq)


def test_rare_label_fewer_than_k(gpu):
    """A label with fewer rows than k: its queries get its rows, then -1 / +inf."""
    X = data.mixture_u8(10_000, seed=79)
    Q = data.mixture_u8(40, seed=80)
    lx = np.zeros(len(X), np.int32)
    lx[[5, 500, 9_999]] = 3
    lq = np.array([3, 0] * 20, np.int32)
    idx = certex.Index(128)
    idx.add(torch.from_numpy(X).cuda(), labels=torch.from_numpy(lx))
    D, I = search(idx, Q, 8, lq)
    assert (I[0::2, 3:] == -1).all()
    check(X, Q, 8, "l2", D, I, row_labels=lx, query_labels=lq)


@pytest.mark.parametrize("metric", ["l2", "cosine"])
def test_paired_layout_odd_starts(gpu, metric):
    """Float rows over 128 halves keep the label partition and the queries in the paired layout,
    and a routed group whose first row or query is odd starts one slot early (that slot is not
    live). Label sizes put group starts at odd rows and odd queries, with one-row and one-query
    groups, groups of several 256-row tiles and of several 128-query tiles, and labels with fewer
    rows than k; ids and distances must still equal the oracle's."""
    rng = np.random.default_rng(90)
    row_counts = {0: 1, 1: 3, 2: 777, 3: 2, 4: 1500, 6: 301, 7: 9}
    query_counts = {0: 1, 1: 2, 2: 131, 3: 1, 4: 257, 5: 3, 6: 20, 7: 5}
    lx = rng.permutation(np.concatenate([np.full(c, l, np.int32) for l, c in row_counts.items()]))
    lq = rng.permutation(np.concatenate([np.full(c, l, np.int32) for l, c in query_counts.items()]))
    X = data.powerlaw_unit(len(lx), 200, seed=91)
    Q = data.powerlaw_unit(len(lq), 200, seed=92)
    idx = certex.Index(200, metric=metric)
    idx.add(torch.from_numpy(X).cuda(), labels=torch.from_numpy(lx))
    assert idx.core.n_partitioned == len(lx)
    for batch in (1024, 100):
        D, I = search(idx, Q, 10, lq, batch)
        check(X, Q, 10, metric, D, I, row_labels=lx, query_labels=lq)


@pytest.mark.parametrize("k", [1, 5])
def test_paired_anchor_pairs_coarse_and_fine(gpu, k):
    """The anchor pass over a paired partition takes row pairs as anchors. Labels of about 70,000
    rows give k = 1 coarse anchor groups (the K-loop anchor pass) and k = 5 fine groups (the anchor
    pass as tiles of the tiled screen); a label with an odd first row and one of 2 rows ride along."""
    rng = np.random.default_rng(93)
    row_counts = {0: 70_001, 1: 2, 2: 68_999}
    lx = rng.permutation(np.concatenate([np.full(c, l, np.int32) for l, c in row_counts.items()]))
    lq = rng.integers(0, 3, 300).astype(np.int32)
    X = data.powerlaw_unit(len(lx), 200, seed=94)
    Q = data.powerlaw_unit(len(lq), 200, seed=95)
    idx = certex.Index(200, metric="l2")
    idx.add(torch.from_numpy(X).cuda(), labels=torch.from_numpy(lx))
    assert idx.core.n_partitioned == len(lx)
    D, I = search(idx, Q, k, lq)
    check(X, Q, k, "l2", D, I, row_labels=lx, query_labels=lq)


@pytest.mark.parametrize("partition", [True, False])
def test_host_and_device_labels(gpu, partition):
    """Query labels in host memory (the routed search plans from them without a read-back; the
    unpartitioned search copies them through pinned staging) and on the GPU give the same results,
    equal to the oracle, over ragged batches and over searches queued back to back without a wait
    in between (the staging is reused only once its last copy is done)."""
    X = data.mixture_u8(30_000, seed=71)
    Q = data.mixture_u8(500, seed=72)
    lx, lq = skewed_labels(len(X), 73), data.labels(len(Q), 18, 74)
    idx = certex.Index(X.shape[1], partition_labels=partition)
    idx.add(torch.from_numpy(X).cuda(), labels=torch.from_numpy(lx))
    assert (idx.core.n_partitioned > 0) == partition
    Qd = torch.from_numpy(Q).cuda()
    host, dev = torch.from_numpy(lq), torch.from_numpy(lq).cuda()
    outs = []
    for batch in (2048, 130, 2048):
        for labels in (host, dev):
            outs.append(idx.search(Qd, k=10, batch=batch, labels=labels))
    torch.cuda.synchronize()
    for D, I in outs:
        check(X, Q, 10, "l2", D.cpu().numpy(), I.cpu().numpy(), row_labels=lx, query_labels=lq)


@pytest.mark.parametrize("kind", ["uint8", "float32"])
def test_equal_labels_in_label_order_after_another_search(gpu, kind):
    """Queries already in label order over labels of equal size: with host labels the routed
    search keeps the batch in place (no gather, no scatter of the results) and its anchor pass
    writes every column of the group table itself (no fill). An earlier search on the same thread
    leaves a table of larger values in the workspace (every query equal to every row), so a
    column left unwritten would raise a threshold and drop true neighbours."""
    n_lab, per, d = 4, 12_000, 128
    if kind == "uint8":
        P = np.full((100_000, d), 255, np.uint8)
        X = data.mixture_u8(n_lab * per, seed=81)
        Q = data.mixture_u8(400, seed=82)
        metric = "l2"
    else:
        v = data.gaussian(1, d, 80)
        P = np.repeat(v, 100_000, axis=0)
        X = data.gaussian(n_lab * per, d, 81)
        Q = data.gaussian(400, d, 82)
        metric = "ip"
    poison = certex.Index(d, metric=metric)
    poison.add(torch.from_numpy(P).cuda())
    poison.search(torch.from_numpy(P[:2048]).cuda(), k=10, batch=2048)
    lx = np.repeat(np.arange(n_lab, dtype=np.int32), per)
    np.random.default_rng(83).shuffle(lx)
    lq = np.sort(data.labels(len(Q), n_lab, 84))
    idx = certex.Index(d, metric=metric)
    idx.add(torch.from_numpy(X).cuda(), labels=torch.from_numpy(lx))
    assert idx.core.n_partitioned == len(X)
    D, I = search(idx, Q, 10, lq)
    check(X, Q, 10, metric, D, I, row_labels=lx, query_labels=lq)


@pytest.mark.parametrize("kind", ["uint8", "float32"])
def test_query_labels_outside_the_partition(gpu, kind):
    """Query labels below 0 and past the partition's labels, mixed with the partition's own, in a
    ragged batch: such queries match no partition row (only rows added later with that label,
    through the filter). On the device the routing sorts them into buckets before and after the
    partition's labels; both placements must give the oracle's results."""
    d = 128
    if kind == "uint8":
        X, Q, metric = data.mixture_u8(20_000, seed=91), data.mixture_u8(1_037, seed=92), "l2"
    else:
        X, Q, metric = data.gaussian(20_000, d, 91), data.gaussian(1_037, d, 92), "ip"
    lx = data.labels(len(X), 5, 93)
    lq = np.random.default_rng(94).choice(np.array([-7, -1, 0, 1, 2, 3, 4, 5, 40], np.int32), len(Q))
    idx = certex.Index(d, metric=metric)
    idx.add(torch.from_numpy(X[:19_000]).cuda(), labels=torch.from_numpy(lx[:19_000]))
    idx.partition_labels = False  # the next rows stay outside the partition: a tail
    idx.add(torch.from_numpy(X[19_000:]).cuda(), labels=torch.from_numpy(lx[19_000:]))
    assert idx.core.n_partitioned == 19_000
    for batch in (2048, 300):
        D, I = search(idx, Q, 10, lq, batch=batch)
        check(X, Q, 10, metric, D, I, row_labels=lx, query_labels=lq)


def test_many_labels(gpu):
    """300 labels, more than the one-workgroup device routing takes (62): device labels go through
    the radix sort and the group-table kernel; host labels through the host's counting sort."""
    X = data.mixture_u8(60_000, seed=101)
    Q = data.mixture_u8(900, seed=102)
    lx = data.labels(len(X), 300, 103)
    lq = data.labels(len(Q), 310, 104)  # labels 300 .. 309: no rows
    idx = certex.Index(X.shape[1])
    idx.add(torch.from_numpy(X).cuda(), labels=torch.from_numpy(lx))
    assert idx.core.n_partitioned == len(X)
    for batch in (2048, 257):
        D, I = search(idx, Q, 10, lq, batch=batch)
        check(X, Q, 10, "l2", D, I, row_labels=lx, query_labels=lq)
