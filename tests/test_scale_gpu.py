"""Config 5's kind of workload at a scale one test can afford: 100,000,000 x 128 uint8 rows (the
config 2 / 5 mixture), with an extend of 1,000,000 rows and a removal of 1,000,000 random ids
running while searches run (reference tests/test_updates: searches during updates return exact
results over a snapshot of the live set). Checked by a GPU fp64 brute force, which is exact for
8-bit data (every distance is an integer below 2^23): ids bit-exact with ties to the lower id.
"""

import threading

import numpy as np
import pytest
import torch

import libcertex_amd as certex
from tests import data

pytestmark = pytest.mark.gpu

N, N_NEW, N_GONE, K = 100_000_000, 1_000_000, 1_000_000, 10


def brute_force(X, live, Q, k, chunk=250_000):
    """Exact (distance, id) top k of Q over the live rows of X, ties to the lower id: distances are
    integers below 2^23 and ids below 2^30, so distance * 2^30 + id is exact in fp64."""
    Qd = Q.double()
    qq = (Qd * Qd).sum(1, keepdim=True)
    best = torch.empty((Q.shape[0], 0), dtype=torch.float64, device="cuda")
    for c in range(0, X.shape[0], chunk):
        Xc = X[c : c + chunk].double()
        d = qq + (Xc * Xc).sum(1)[None] - 2.0 * (Qd @ Xc.T)
        key = d * float(1 << 30) + torch.arange(c, c + Xc.shape[0], device="cuda", dtype=torch.float64)[None]
        key[:, ~live[c : c + chunk]] = float("inf")
        best = torch.topk(torch.cat([best, key], 1), k, dim=1, largest=False).values
    ids = torch.remainder(best, float(1 << 30)).long()
    dist = torch.floor(best / float(1 << 30))
    return dist, ids


def test_hundred_million_rows_with_concurrent_updates(gpu):
    X = data.mixture_u8_cuda(N + N_NEW, seed=2)
    Q = data.mixture_u8_cuda(1_000, seed=3)
    idx = certex.Index(128)
    for c in range(0, N, 10_000_000):
        idx.add(X[c : c + 10_000_000])
    torch.cuda.synchronize()
    gone = torch.randperm(N, generator=torch.Generator().manual_seed(4))[:N_GONE].cuda()
    errors, results = [], []

    def writer():
        try:
            with torch.cuda.stream(torch.cuda.Stream()):
                idx.add(X[N:])
                idx.remove(gone)
                torch.cuda.current_stream().synchronize()
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    def reader():
        try:
            with torch.cuda.stream(torch.cuda.Stream()):
                for _ in range(3):
                    D, I = idx.search(Q[:256], k=K)
                    torch.cuda.current_stream().synchronize()
                    results.append((D, I))
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    threads = [threading.Thread(target=writer), threading.Thread(target=reader)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[0]
    assert idx.core.size == N + N_NEW and idx.ntotal == N + N_NEW - N_GONE

    # every search during the updates: ascending, returned distances exact for the returned ids
    Qd = Q[:256].double()
    for D, I in results:
        assert (I >= 0).all() and (I < N + N_NEW).all()
        assert (D[:, 1:] >= D[:, :-1]).all()
        exact = ((Qd[:, None, :] - X[I].double()) ** 2).sum(-1)
        assert torch.equal(D.double(), exact)

    # after the updates: every query against the live set
    live = torch.ones(N + N_NEW, dtype=torch.bool, device="cuda")
    live[gone] = False
    D, I = idx.search(Q, k=K)
    dist, ids = brute_force(X, live, Q, K)
    assert torch.equal(I, ids)
    assert torch.equal(D.double(), dist)
