"""Parity of the HIP search path with the CPU oracle (ids bit-exact, ties to the lower id).

Every search here runs through the C API (libcertex_c.so) on the GPU; the expected answers come
from oracle/oracle.c on the same seeded inputs, or from the committed golden fixtures. The cases
follow the reference's exactness suite (tests/test_exact.py, cpp/tests/neighbors/ann_certex.cuh
:277-319, test_updates.cu): metrics, dimensions, ragged sizes, batch sizes, a tiny index, k up to
2048, duplicates and exact ties, removals, extension, bitset / bitmap / label filters.
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


def run(X, Q, k, metric="l2", batch=2048, anchor_stride=16, **kw):
    idx = certex.Index(X.shape[1], metric=metric, anchor_stride=anchor_stride)
    idx.add(torch.from_numpy(X).cuda())
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=k, batch=batch, **kw)
    torch.cuda.synchronize()
    return D.cpu().numpy(), I.cpu().numpy(), idx


def check(X, Q, k, metric, D, I, **okw):
    s, i = oracle.knn(X, Q, k, metric, **okw)
    np.testing.assert_array_equal(I, i)
    d = oracle.distances(s, i, metric)
    if metric == "cosine":
        d = np.where(i >= 0, 1 - d, -np.inf).astype(np.float32)
    np.testing.assert_array_equal(D, d)


@pytest.mark.parametrize("name", ["c2_u8_l2", "u8_ties_l2", "i8_ip"])
def test_golden(gpu, name):
    f = np.load(os.path.join(GOLDEN, name + ".npz"))
    X, Q, k, metric = f["base"], f["queries"], int(f["k"]), str(f["metric"])
    D, I, _ = run(X, Q, k, metric)
    np.testing.assert_array_equal(I, f["ids"])
    np.testing.assert_array_equal(D, oracle.distances(f["scores"], f["ids"], metric))


@pytest.mark.parametrize("dtype", [np.uint8, np.int8])
@pytest.mark.parametrize("metric", ["l2", "ip"])
@pytest.mark.parametrize("d", [128, 37, 200])
def test_metrics_dims(gpu, dtype, metric, d):
    X = data.uniform_int(20_011, d, seed=d, dtype=dtype)
    Q = data.uniform_int(257, d, seed=d + 1, dtype=dtype)
    D, I, _ = run(X, Q, 10, metric)
    check(X, Q, 10, metric, D, I)


@pytest.mark.parametrize("k", [1, 10, 100])
def test_mixture_u8(gpu, k):
    X = data.mixture_u8(60_013, seed=2)
    Q = data.mixture_u8(300, seed=3)
    D, I, _ = run(X, Q, k)
    check(X, Q, k, "l2", D, I)


def test_k_2048_and_batches(gpu):
    X = data.mixture_u8(9_000, seed=4)
    Q = data.mixture_u8(40, seed=5)
    for k, batch in ((2048, 2048), (300, 7), (10, 1)):
        D, I, _ = run(X, Q, k, batch=batch)
        check(X, Q, k, "l2", D, I)


def test_tiny_index(gpu):
    X = data.uniform_int(50, 16, seed=6)
    Q = data.uniform_int(9, 16, seed=7)
    for k in (1, 10, 50):
        D, I, _ = run(X, Q, k)
        check(X, Q, k, "l2", D, I)


def test_duplicates_and_ties(gpu):
    base = data.uniform_int(3_000, 16, seed=8, lo=0, hi=2)
    X = np.concatenate([base, base, base[:777]])
    Q = data.uniform_int(64, 16, seed=9, lo=0, hi=2)
    D, I, _ = run(X, Q, 64)
    check(X, Q, 64, "l2", D, I)


def test_remove(gpu):
    X = data.mixture_u8(30_000, seed=10)
    Q = data.mixture_u8(200, seed=11)
    _, nn = oracle.knn(X, Q, 1, "l2")
    gone = np.concatenate([nn[:, 0], nn[:5, 0], [29_999, 0]])
    idx = certex.Index(128)
    idx.add(torch.from_numpy(X).cuda())
    idx.remove(torch.from_numpy(gone))
    removed = np.zeros(30_000, np.uint8)
    removed[gone] = 1
    assert idx.ntotal == 30_000 - int(removed.sum())
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=10)
    I = I.cpu().numpy()
    assert not removed[I].any()
    check(X, Q, 10, "l2", D.cpu().numpy(), I, removed=removed)


def test_extend_and_reserve(gpu):
    X = data.mixture_u8(25_000, seed=12)
    Q = data.mixture_u8(100, seed=13)
    idx = certex.Index(128, capacity=5_000)
    ids = [idx.add(X[:1000]), idx.add(X[1000:17_000]), idx.add(torch.from_numpy(X[17_000:]).cuda())]
    assert np.concatenate([np.asarray(i.cpu() if torch.is_tensor(i) else i) for i in ids]).tolist() == list(range(25_000))
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=10)
    check(X, Q, 10, "l2", D.cpu().numpy(), I.cpu().numpy())


def test_bitset_bitmap_labels(gpu):
    X = data.mixture_u8(20_000, seed=14)
    Q = data.mixture_u8(64, seed=15)
    rng = np.random.default_rng(16)
    keep = rng.random(20_000) < 0.05
    idx = certex.Index(128)
    idx.add(torch.from_numpy(X).cuda())
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=10, filter=torch.from_numpy(keep))
    check(X, Q, 10, "l2", D.cpu().numpy(), I.cpu().numpy(), removed=(~keep).astype(np.uint8))
    km = rng.random((64, 20_000)) < 0.01
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=10, filter=torch.from_numpy(km))
    bits = np.packbits(km.reshape(-1), bitorder="little")
    bits = np.pad(bits, (0, (-bits.size) % 4)).view(np.uint32)
    check(X, Q, 10, "l2", D.cpu().numpy(), I.cpu().numpy(), bitmap=bits)
    rl = rng.integers(0, 16, 20_000)
    ql = rng.integers(0, 16, 64)
    lab = certex.Index(128)
    lab.add(torch.from_numpy(X).cuda(), labels=torch.from_numpy(rl))
    D, I = lab.search(torch.from_numpy(Q).cuda(), k=10, labels=torch.from_numpy(ql))
    check(X, Q, 10, "l2", D.cpu().numpy(), I.cpu().numpy(), row_labels=rl, query_labels=ql)


def test_fewer_candidates_than_k(gpu):
    X = data.uniform_int(5_000, 32, seed=17)
    Q = data.uniform_int(20, 32, seed=18)
    keep = np.zeros(5_000, bool)
    keep[[3, 70, 4_999]] = True
    idx = certex.Index(32)
    idx.add(torch.from_numpy(X).cuda())
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=5, filter=torch.from_numpy(keep))
    I = I.cpu().numpy()
    assert (I[:, 3:] == -1).all() and np.isinf(D.cpu().numpy()[:, 3:]).all()
    check(X, Q, 5, "l2", D.cpu().numpy(), I, removed=(~keep).astype(np.uint8))


def test_search_stats(gpu):
    X = data.mixture_u8(50_000, seed=19)
    Q = data.mixture_u8(500, seed=20)
    idx = certex.Index(128)
    idx.add(torch.from_numpy(X).cuda())
    with certex.search_stats() as st:
        idx.search(torch.from_numpy(Q).cuda(), k=10)
    assert st.queries == 500
    assert 500 * 10 <= st.verified <= st.survivors < 500 * 50_000 // 4


def test_c2_shape_subset_parity(gpu):
    """Config 2's generator at 2,000,000 rows: 48 queries against the oracle, and for all 2,000
    queries the properties that hold at any size (ascending (distance, id), returned distances equal
    to fp64 recomputation, the k-th distance equal to a GPU fp64 brute force)."""
    X = data.mixture_u8(2_000_000, seed=2)
    Q = data.mixture_u8(2_000, seed=3)
    D, I, _ = run(X, Q, 10, batch=2_000)
    check(X, Q[:48], 10, "l2", D[:48], I[:48])
    assert (np.diff(D, axis=1) >= 0).all()
    Xg = torch.from_numpy(X).cuda()
    Qg = torch.from_numpy(Q).cuda().double()
    rows = Xg[torch.from_numpy(I).cuda()].double()
    exact = ((Qg[:, None, :] - rows) ** 2).sum(-1)
    np.testing.assert_array_equal(D, exact.float().cpu().numpy())
    kth = torch.full((2_000,), float("inf"), dtype=torch.float64, device="cuda")
    best = torch.empty((2_000, 0), dtype=torch.float64, device="cuda")
    for c in range(0, 2_000_000, 250_000):
        Xc = Xg[c : c + 250_000].double()
        s = (Qg * Qg).sum(1, keepdim=True) + (Xc * Xc).sum(1)[None] - 2.0 * (Qg @ Xc.T)
        best = torch.topk(torch.cat([best, s], 1), 10, dim=1, largest=False).values
    kth = best[:, 9].cpu().numpy()
    np.testing.assert_array_equal(exact[:, 9].cpu().numpy(), kth)


def test_many_survivors_spill(gpu):
    """A quarter of the rows are one repeated row near every query: each screen workgroup keeps
    thousands of survivors, past its LDS list. The first search of the resources moves them with a
    global atomic each and asks for a spill pool; the later ones write the workgroups' spill regions.
    Every search must equal the oracle (ties to the lower id)."""
    rng = np.random.default_rng(5)
    X = rng.integers(0, 256, (40_000, 128)).astype(np.uint8)
    base = rng.integers(0, 256, 128).astype(np.uint8)
    X[rng.permutation(40_000)[:10_000]] = base
    Q = np.clip(base.astype(np.int32) + rng.integers(-2, 3, (64, 128)), 0, 255).astype(np.uint8)
    idx = certex.Index(128, metric="l2")
    idx.add(torch.from_numpy(X).cuda())
    s, i = oracle.knn(X, Q, 100, "l2")
    for _ in range(3):
        D, I = idx.search(torch.from_numpy(Q).cuda(), k=100)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(I.cpu().numpy(), i)
        np.testing.assert_array_equal(D.cpu().numpy(), oracle.distances(s, i, "l2"))


@pytest.mark.parametrize("k", [10, 64])
def test_small_and_large_buckets(gpu, k):
    """Half of the queries sit next to 2,000 copies of one row (buckets of thousands, the block
    re-rank), the other half are random (buckets of a few hundred at most, the one-wave re-rank):
    one search runs both paths and must equal the oracle (ties to the lower id)."""
    rng = np.random.default_rng(11)
    X = rng.integers(0, 256, (40_000, 128)).astype(np.uint8)
    base = rng.integers(0, 256, 128).astype(np.uint8)
    X[rng.permutation(40_000)[:2_000]] = base
    near = np.clip(base.astype(np.int32) + rng.integers(-2, 3, (32, 128)), 0, 255).astype(np.uint8)
    far = rng.integers(0, 256, (32, 128)).astype(np.uint8)
    Q = np.concatenate([near, far])[rng.permutation(64)]
    D, I, _ = run(X, Q, k)
    check(X, Q, k, "l2", D, I)
