"""Wide vectors against the CPU oracle: 8-bit vectors of more than 256 coordinates and float vectors
of up to 4,096 (the reference takes any dimension through its row lengths, certex.cu:58-62, and
widths up to 4,091, certex/index.py:116).

8-bit rows wider than 256 bytes (stored zero padded to a multiple of 256 bytes) run the tiled int8
screen and the K-loop int8 anchor pass: exact int32 screen values, as the narrow int8 screen.
Float rows of up to 4,096 halves run the tiled fp16 screen and a K-loop anchor pass that holds 16
queries of 8 KB. Ids must be bit-exact, ties to the lower id, distances equal to the oracle's.
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
    np.testing.assert_array_equal(I.cpu().numpy() if torch.is_tensor(I) else I, i)
    d = oracle.distances(s, i, metric)
    if metric == "cosine":
        d = np.where(i >= 0, np.float32(1) - d, -np.inf).astype(np.float32)
    np.testing.assert_array_equal(D.cpu().numpy() if torch.is_tensor(D) else D, d)


def words(mask):
    """A boolean mask (rows of bits per query for a bitmap) as the oracle's uint32 words."""
    b = np.packbits(np.asarray(mask, bool).reshape(-1), bitorder="little")
    return np.pad(b, (0, (-b.size) % 4)).view(np.uint32)


def mixture(n, d, seed):
    return data.mixture_u8(n, d=d, seed=seed)


@pytest.mark.parametrize("dtype", [np.uint8, np.int8])
@pytest.mark.parametrize("metric", ["l2", "ip"])
@pytest.mark.parametrize("d", [384, 960, 4096])
def test_int_wide(gpu, dtype, metric, d):
    n = 6_000 if d == 4096 else 30_011
    if dtype == np.uint8:
        X, Q = mixture(n, d, seed=d), mixture(97, d, seed=d + 1)
    else:
        X, Q = data.uniform_int(n, d, seed=d, dtype=dtype), data.uniform_int(97, d, seed=d + 1, dtype=dtype)
    X[:40] = X[40:80]  # exact ties
    idx = certex.Index(d, metric=metric)
    idx.add(torch.from_numpy(X).cuda())
    Qg = torch.from_numpy(Q).cuda()
    for k in (10, 300):  # the one-wave re-rank and the block re-rank
        D, I = idx.search(Qg, k=k)
        check(X, Q, k, metric, D, I)


def test_int_wide_many_survivors_spill(gpu):
    """d = 384 (the tiled int8 screen): a quarter of the rows repeat one row near every query, so a
    tile of 256 rows keeps thousands of survivors, past its LDS list. The first search moves them
    with a global atomic each and asks for a spill pool; the later ones write the tiles' spill
    regions (entries of one word: query and row offset). Every search must equal the oracle."""
    rng = np.random.default_rng(384)
    X = rng.integers(0, 256, (40_000, 384)).astype(np.uint8)
    base = rng.integers(0, 256, 384).astype(np.uint8)
    X[rng.permutation(40_000)[:10_000]] = base
    Q = np.clip(base.astype(np.int32) + rng.integers(-2, 3, (64, 384)), 0, 255).astype(np.uint8)
    idx = certex.Index(384, metric="l2")
    idx.add(torch.from_numpy(X).cuda())
    for _ in range(3):
        D, I = idx.search(torch.from_numpy(Q).cuda(), k=100)
        torch.cuda.synchronize()
        check(X, Q, 100, "l2", D, I)


def test_int_wide_updates_filters_labels(gpu):
    """d = 960: extend from host memory, removals, a bitset, a bitmap, labels through the filter
    and through the paired label partition (the routed tiled screen and anchor pass)."""
    d, n = 960, 40_000
    X = mixture(n, d, seed=21)
    Q = mixture(120, d, seed=22)
    idx = certex.Index(d, partition_labels=False)
    idx.add(torch.from_numpy(X[:30_000]).cuda(), labels=torch.from_numpy(data.labels(30_000, 5, 23)))
    idx.add(X[30_000:], labels=torch.from_numpy(data.labels(10_000, 5, 24)))
    lx = np.concatenate([data.labels(30_000, 5, 23), data.labels(10_000, 5, 24)])
    gone = np.random.default_rng(25).choice(n, 3_000, replace=False)
    idx.remove(torch.from_numpy(gone))
    removed = np.zeros(n, bool)
    removed[gone] = True
    Qg = torch.from_numpy(Q).cuda()
    D, I = idx.search(Qg, k=20)
    check(X, Q, 20, "l2", D, I, removed=removed)
    keep = np.random.default_rng(26).random(n) < 0.3
    D, I = idx.search(Qg, k=20, filter=torch.from_numpy(keep))
    check(X, Q, 20, "l2", D, I, removed=removed, bitset=words(keep))
    bitmap = np.random.default_rng(27).random((len(Q), n)) < 0.5
    D, I = idx.search(Qg, k=15, filter=torch.from_numpy(bitmap))
    check(X, Q, 15, "l2", D, I, removed=removed, bitmap=words(bitmap))
    lq = data.labels(len(Q), 5, 28)
    D, I = idx.search(Qg, k=20, labels=torch.from_numpy(lq))
    check(X, Q, 20, "l2", D, I, removed=removed, row_labels=lx, query_labels=lq)
    idx.partition()  # the paired label partition: routed tiled screen and anchor pass
    D, I = idx.search(Qg, k=20, labels=torch.from_numpy(lq))
    check(X, Q, 20, "l2", D, I, removed=removed, row_labels=lx, query_labels=lq)
    D, I = idx.search(Qg, k=300, labels=torch.from_numpy(lq))  # the block re-rank over the partition
    check(X, Q, 300, "l2", D, I, removed=removed, row_labels=lx, query_labels=lq)


def test_int_wide_coarse_groups_and_lists(gpu):
    """700,000 rows of 384 bytes: coarse anchor groups (whole steps) in the K-loop pass; then an
    index with k-means lists probed 2 per query."""
    d, n = 384, 700_000
    X = mixture(n, d, seed=31)
    Q = mixture(48, d, seed=32)
    Qg = torch.from_numpy(Q).cuda()
    idx = certex.Index(d)
    idx.add(torch.from_numpy(X).cuda())
    D, I = idx.search(Qg, k=10)
    check(X, Q, 10, "l2", D, I)
    del idx
    listed = certex.Index(d, n_lists=64)
    listed.add(torch.from_numpy(X[:200_000]).cuda())
    for probe in (0, 2):
        D, I = listed.search(Qg, k=10, probe_lists=probe)
        check(X[:200_000], Q, 10, "l2", D, I)


def test_int_wide_save_load(gpu, tmp_path):
    d = 384
    X = mixture(20_000, d, seed=41)
    Q = torch.from_numpy(mixture(50, d, seed=42)).cuda()
    idx = certex.Index(d, metric="ip")
    idx.add(torch.from_numpy(X).cuda())
    D0, I0 = idx.search(Q, k=10)
    idx.save(tmp_path / "wide.cx")
    back = certex.Index.load(tmp_path / "wide.cx")
    D1, I1 = back.search(Q, k=10)
    assert torch.equal(I0, I1) and torch.equal(D0, D1)


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("d", [3000, 4096])
def test_float_wide(gpu, dtype, metric, d):
    g = np.random.default_rng(d)
    X = g.standard_normal((8_000, d)).astype(dtype)
    Q = g.standard_normal((70, d)).astype(dtype)
    X[100:120] = X[200:220]  # exact ties
    idx = certex.Index(d, metric=metric)
    idx.add(torch.from_numpy(X).cuda())
    Qg = torch.from_numpy(Q).cuda()
    for k in (10, 100):
        D, I = idx.search(Qg, k=k)
        check(X, Q, k, metric, D, I)


def test_float_4096_labels_partition(gpu):
    """d = 4,096 with labels through the paired partition (routed tiled screen, tiled anchor pass)
    and a removal."""
    d = 4096
    X = data.powerlaw_unit(12_000, d, seed=51)
    Q = data.powerlaw_unit(64, d, seed=52)
    lx, lq = data.labels(len(X), 4, 53), data.labels(len(Q), 4, 54)
    idx = certex.Index(d, metric="cosine")
    idx.add(torch.from_numpy(X).cuda(), labels=torch.from_numpy(lx))
    gone = np.arange(0, len(X), 13)
    idx.remove(torch.from_numpy(gone))
    removed = np.zeros(len(X), bool)
    removed[gone] = True
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=25, labels=torch.from_numpy(lq))
    check(X, Q, 25, "cosine", D, I, removed=removed, row_labels=lx, query_labels=lq)


def test_widths_beyond_the_limit_refused(gpu):
    with pytest.raises(ValueError, match="4096"):
        certex.Index(4097).add(np.zeros((10, 4097), np.uint8))
    with pytest.raises(ValueError, match="4096"):
        certex.Index(4100).add(np.zeros((10, 4100), np.float32))
