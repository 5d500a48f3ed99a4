"""Index options: host storage of the float vectors (the reference's host_vectors, certex.cu:253-289)
and the options this build refuses instead of ignoring (a projection width below the dimension,
local projections, int8 rows of float vectors). Results are checked against the oracle's
exhaustive fp64 search, ties to the lower id."""

import numpy as np
import pytest
import torch

import libcertex_amd as certex
import oracle
from tests import data

pytestmark = pytest.mark.gpu


def check(X, Q, k, metric, D, I):
    s, i = oracle.knn(X, Q, k, metric)
    np.testing.assert_array_equal(I.cpu().numpy(), i)
    d = oracle.distances(s, i, metric)
    if metric == "cosine":
        d = np.where(i >= 0, np.float32(1) - d, -np.inf).astype(np.float32)
    np.testing.assert_array_equal(D.cpu().numpy(), d)


@pytest.mark.parametrize("d, dtype, metric", [(64, np.float32, "l2"), (300, np.float16, "cosine"),
                                              (128, np.float32, "ip")])
def test_host_vectors(gpu, tmp_path, d, dtype, metric):
    """storage="host": the exact scores read the vectors from pinned host memory. Build, extend,
    save and load keep them there, and every search equals the oracle."""
    rng = np.random.default_rng(d)
    X = rng.standard_normal((9_000, d)).astype(dtype)
    Q = rng.standard_normal((70, d)).astype(dtype)
    idx = certex.Index(d, metric=metric, storage="host")
    idx.add(torch.from_numpy(X[:6_000]).cuda())
    assert idx.core.host_vectors
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=9)
    check(X[:6_000], Q, 9, metric, D, I)
    idx.add(X[6_000:])  # a host source into host storage, with capacity growth
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=9)
    check(X, Q, 9, metric, D, I)
    path = tmp_path / "host.certex"
    idx.save(path)
    back = certex.Index.load(path)
    assert back.storage == "host" and back.core.host_vectors
    D2, I2 = back.search(torch.from_numpy(Q).cuda(), k=9)
    assert torch.equal(I2, I) and torch.equal(D2, D)


def test_host_vectors_8bit(gpu):
    """8-bit vectors are their own screening codes: there is no second copy to keep on the host.
    The option is recorded and the results are unchanged."""
    X = data.mixture_u8(20_000, seed=5)
    Q = data.mixture_u8(50, seed=6)
    idx = certex.Index(128, storage="host")
    idx.add(torch.from_numpy(X).cuda())
    assert idx.core.host_vectors
    D, I = idx.search(torch.from_numpy(Q).cuda(), k=10)
    check(X, Q, 10, "l2", D, I)


def test_full_widths_accepted(gpu):
    """width 0 (auto) and any width of at least the dimension screen full-dimension rows."""
    rng = np.random.default_rng(7)
    X = rng.standard_normal((3_000, 32)).astype(np.float32)
    Q = rng.standard_normal((20, 32)).astype(np.float32)
    for w in ("auto", 32, 64):
        idx = certex.Index(32, width=w)
        idx.add(torch.from_numpy(X).cuda())
        assert idx.core.width == 32
        D, I = idx.search(torch.from_numpy(Q).cuda(), k=5)
        check(X, Q, 5, "l2", D, I)


@pytest.mark.parametrize(
    "dtype, options, message",
    [
        (np.float32, {"width": 16}, "projection width"),
        (np.uint8, {"width": 64}, "projection width"),
        (np.float32, {"local_projections": True}, "local_projections"),
        (np.float32, {"int8_rows": True}, "int8_rows"),
        (np.float16, {"int8_rows": True}, "int8_rows"),
    ],
)
def test_unsupported_options_refused(gpu, dtype, options, message):
    X = (np.random.default_rng(1).random((500, 128)) * 100).astype(dtype)
    idx = certex.Index(128, **options)
    with pytest.raises(ValueError, match=message):
        idx.add(torch.from_numpy(X).cuda())
    assert idx.core is None


def test_int8_rows_of_8bit_vectors(gpu):
    """8-bit vectors are screened as exact int8 rows whatever int8_rows says."""
    X = data.mixture_u8(5_000, seed=8)
    Q = data.mixture_u8(30, seed=9)
    for flag in (False, True):
        idx = certex.Index(128, int8_rows=flag)
        idx.add(torch.from_numpy(X).cuda())
        D, I = idx.search(torch.from_numpy(Q).cuda(), k=10)
        check(X, Q, 10, "l2", D, I)


def test_trim_pool(gpu):
    """trim_pool frees the scratch the thread's searches grew (reference certex/index.py:165-169);
    the next search grows it again and returns the same results."""
    X = data.mixture_u8(200_000, seed=160)
    Q = torch.from_numpy(data.mixture_u8(4_000, seed=161)).cuda()
    idx = certex.Index(128)
    idx.add(torch.from_numpy(X).cuda())
    D0, I0 = idx.search(Q, k=100, batch=4_000)
    torch.cuda.synchronize()
    before = torch.cuda.mem_get_info()[0]
    certex.trim_pool()
    freed = torch.cuda.mem_get_info()[0] - before
    assert freed >= 4_000 * 100 * 12  # at least the batch's best lists (score f64 + row i64 per entry)
    D1, I1 = idx.search(Q, k=100, batch=4_000)
    assert torch.equal(I0, I1) and torch.equal(D0, D1)
    check(X, Q[:50].cpu().numpy(), 100, "l2", D1[:50], I1[:50])
