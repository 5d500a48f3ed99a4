"""Parity of the fp16 certified screen path (float32 and float16 vectors) with the CPU oracle.

Ids must be bit-exact, ties to the lower id, and float32 distances equal to the oracle's. Cases
follow the reference's exactness suite (tests/test_exact.py:87-364): metrics, inner products with
unequal norms, near-duplicates and large norms (test_exact.py:446-452), removals, filters, k up
to 2048, float16 storage; plus config 1's shape (100,000 x 128 N(0,1), 1,000 queries, seeds 11/12).
"""

import os

import numpy as np
import pytest
import torch

import libcertex_amd as certex
import oracle
from tests import data

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def correlated(n, d, nq, seed=0, scale_norms=False):
    """The reference's test data (test_exact.py:39-46), drawn with numpy: Gaussian rows times a
    random mixing matrix; optionally unequal row norms."""
    g = np.random.default_rng(seed)
    A = g.standard_normal((d, d)) / d**0.5
    X = (g.standard_normal((n, d)) @ A).astype(np.float32)
    Q = (g.standard_normal((nq, d)) @ A).astype(np.float32)
    if scale_norms:
        X = (X * (0.2 + g.random((n, 1)) * 3)).astype(np.float32)
    return X, Q


def run(X, Q, k, metric="l2", batch=2048, **kw):
    idx = certex.Index(X.shape[1], metric=metric)
    idx.add(torch.from_numpy(X).cuda())
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=k, batch=batch, **kw)
    torch.cuda.synchronize()
    return D.cpu().numpy(), I.cpu().numpy(), idx


def check(X, Q, k, metric, D, I, **okw):
    s, i = oracle.knn(X, Q, k, metric, **okw)
    np.testing.assert_array_equal(I, i)
    d = oracle.distances(s, i, metric)
    if metric == "cosine":
        d = np.where(i >= 0, np.float32(1) - d, -np.inf).astype(np.float32)
    np.testing.assert_array_equal(D, d)


def test_golden_c1(gpu):
    f = np.load(os.path.join(GOLDEN, "c1_f32_l2.npz"))
    D, I, _ = run(f["base"], f["queries"], int(f["k"]))
    np.testing.assert_array_equal(I, f["ids"])
    np.testing.assert_array_equal(D, oracle.distances(f["scores"], f["ids"], "l2"))


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_metrics(gpu, metric, dtype):
    X, Q = correlated(20_011, 64, 333, seed=1)
    X, Q = X.astype(dtype), Q.astype(dtype)
    D, I, _ = run(X, Q, 10, metric)
    check(X, Q, 10, metric, D, I)


def test_dims_and_ragged(gpu):
    for d in (7, 100, 128):
        X, Q = correlated(5_003, d, 130, seed=d)
        D, I, _ = run(X, Q, 17)
        check(X, Q, 17, "l2", D, I)


def test_inner_product_unequal_norms(gpu):
    X, Q = correlated(20_000, 64, 500, scale_norms=True)
    D, I, _ = run(X, Q, 10, "ip")
    check(X, Q, 10, "ip", D, I)


def test_near_duplicates_and_large_norms(gpu):
    X, _ = correlated(5_000, 32, 1, seed=7)
    dup = np.concatenate([X, X + np.float32(1e-6), X * np.float32(1000.0)]).astype(np.float32)
    D, I, _ = run(dup, dup[:200], 4)
    check(dup, dup[:200], 4, "l2", D, I)


def test_exact_ties(gpu):
    X = np.random.default_rng(3).integers(0, 3, (4_000, 16)).astype(np.float32)
    X = np.concatenate([X, X])
    Q = np.random.default_rng(4).integers(0, 3, (50, 16)).astype(np.float32)
    D, I, _ = run(X, Q, 50)
    check(X, Q, 50, "l2", D, I)


def test_k_up_to_2048(gpu):
    """k from 500 to 2,048: the final sort of 1,024 and 2,048 pairs runs in registers (8 or 4 per
    thread, k 513 to 2,048), smaller ones in LDS."""
    X, Q = correlated(12_000, 32, 40, seed=5)
    for k in (2048, 1024, 1000, 513, 500):
        D, I, _ = run(X, Q, k)
        check(X, Q, k, "l2", D, I)


def test_remove_extend_filters(gpu):
    X, Q = correlated(30_000, 48, 100, seed=9)
    idx = certex.Index(48)
    idx.add(torch.from_numpy(X[:20_000]).cuda())
    idx.add(X[20_000:])  # host rows
    _, nn = oracle.knn(X, Q, 1, "l2")
    gone = np.concatenate([nn[:, 0], [0, 29_999]])
    idx.remove(torch.from_numpy(gone))
    removed = np.zeros(30_000, np.uint8)
    removed[gone] = 1
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=10)
    check(X, Q, 10, "l2", D.cpu().numpy(), I.cpu().numpy(), removed=removed)
    keep = np.random.default_rng(10).random(30_000) < 0.1
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=10, filter=torch.from_numpy(keep))
    check(X, Q, 10, "l2", D.cpu().numpy(), I.cpu().numpy(), removed=(removed | ~keep).astype(np.uint8))


def test_config1_shape(gpu):
    """Config 1: 100,000 x 128 fp32 N(0,1), 1,000 queries (seeds 11 / 12), k = 10, every query
    against the oracle."""
    X = data.gaussian(100_000, 128, 11)
    Q = data.gaussian(1_000, 128, 12)
    D, I, _ = run(X, Q, 10)
    check(X, Q, 10, "l2", D, I)


# --- rows of more than 128 halves: the K-loop screen ------------------------------------------


@pytest.mark.parametrize("d", [129, 200, 256, 384, 768])
def test_wide_dims_l2(gpu, d):
    X, Q = correlated(6_007, d, 211, seed=d)
    D, I, _ = run(X, Q, 10)
    check(X, Q, 10, "l2", D, I)


@pytest.mark.parametrize("metric", ["ip", "cosine"])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_wide_metrics(gpu, metric, dtype):
    X, Q = correlated(8_000, 300, 150, seed=3)
    X, Q = X.astype(dtype), Q.astype(dtype)
    D, I, _ = run(X, Q, 25, metric)
    check(X, Q, 25, metric, D, I)


def test_wide_largest_rows(gpu):
    """1,000 and 2,048 coordinates: fewer queries per workgroup (the LDS holds whole queries)."""
    for d in (1000, 2048):
        X, Q = correlated(3_000, d, 70, seed=d)
        D, I, _ = run(X, Q, 7)
        check(X, Q, 7, "l2", D, I)


@pytest.mark.parametrize("nq", [512, 448, 700])
def test_wide_query_tiles(gpu, nq):
    """Batches of 512, 448 and 700 queries over the tiled screen's 128-query tiles: whole tiles,
    and last tiles of 64 and 60 live queries."""
    X, Q = correlated(20_000, 256, nq, seed=nq)
    D, I, _ = run(X, Q, 10)
    check(X, Q, 10, "l2", D, I)


def test_wide_remove_filter_ties(gpu):
    X, Q = correlated(12_000, 256, 97, seed=21)
    X = np.concatenate([X, X[:500]])  # exact duplicates: ties go to the lower id
    idx = certex.Index(256)
    idx.add(torch.from_numpy(X).cuda())
    gone = np.arange(0, 12_500, 7)
    idx.remove(torch.from_numpy(gone))
    removed = np.zeros(len(X), np.uint8)
    removed[gone] = 1
    keep = np.random.default_rng(2).random(len(X)) < 0.3
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=12, filter=torch.from_numpy(keep))
    check(X, Q, 12, "l2", D.cpu().numpy(), I.cpu().numpy(), removed=(removed | ~keep).astype(np.uint8))


def test_config3_shape_labels(gpu):
    """Config 3's kind of data at reduced size: power-law spectrum embeddings, L2-normalised,
    768 coordinates, cosine, k = 100, one of 16 labels per vector and per query; the batch is
    ragged (1,000 queries in batches of 384)."""
    X = data.powerlaw_unit(60_000, 768, seed=41)
    Q = data.powerlaw_unit(1_000, 768, seed=42)
    lx, lq = data.labels(len(X), 16, 43), data.labels(len(Q), 16, 44)
    idx = certex.Index(768, metric="cosine")
    idx.add(torch.from_numpy(X).cuda(), labels=torch.from_numpy(lx))
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=100, batch=384, labels=torch.from_numpy(lq))
    torch.cuda.synchronize()
    check(X, Q, 100, "cosine", D.cpu().numpy(), I.cpu().numpy(), row_labels=lx, query_labels=lq)


@pytest.mark.parametrize("d", [100, 300])
def test_many_survivors_spill(gpu, d):
    """A quarter of the rows repeat one row near every query (narrow screen at d = 100, tiled
    screen at d = 300): thousands of survivors per workgroup pass its LDS list. Repeated searches
    (the later ones with the spill pool, whose entries pack query, row offset and value) must equal
    the oracle."""
    rng = np.random.default_rng(d)
    X = rng.standard_normal((30_000, d)).astype(np.float32)
    base = rng.standard_normal(d).astype(np.float32)
    X[rng.permutation(30_000)[:7_500]] = base
    Q = (base + 0.01 * rng.standard_normal((48, d))).astype(np.float32)
    idx = certex.Index(d, metric="l2")
    idx.add(torch.from_numpy(X).cuda())
    for _ in range(3):
        D, I = idx.search(torch.from_numpy(Q).cuda(), k=50)
        torch.cuda.synchronize()
        check(X, Q, 50, "l2", D.cpu().numpy(), I.cpu().numpy())


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
@pytest.mark.parametrize("d", [64, 300])
def test_bfloat16_vectors(gpu, metric, d, tmp_path):
    """bfloat16 vectors (an addition of this build, which KeyCache uses for bfloat16 keys): kept
    exactly at 2 bytes per coordinate (narrow screen at d = 64, tiled screen at d = 300); the
    results equal the oracle's over the same values in float32, which holds them exactly, and
    again after a save/load round trip, which keeps the type."""
    X, Q = correlated(12_007, d, 200, seed=d + 5)
    Xb, Qb = torch.from_numpy(X).bfloat16(), torch.from_numpy(Q).bfloat16()
    idx = certex.Index(d, metric=metric)
    idx.add(Xb.cuda())
    assert idx.dtype == torch.bfloat16
    D, I = idx.search(Qb.cuda(), k=20)
    torch.cuda.synchronize()
    check(Xb.float().numpy(), Qb.float().numpy(), 20, metric, D.cpu().numpy(), I.cpu().numpy())
    path = tmp_path / "bf16.idx"
    idx.save(path)
    again = certex.Index.load(path)
    assert again.dtype == torch.bfloat16
    D2, I2 = again.search(Qb.cuda(), k=20)
    torch.cuda.synchronize()
    assert torch.equal(I2, I) and torch.equal(D2, D)
