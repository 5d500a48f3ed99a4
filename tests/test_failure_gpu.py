"""Failure paths and update races of the search, against the CPU oracle.

- Allocation failure: the reference halves a batch on rmm::bad_alloc or batch_too_large and
  retries (certex.cu:1477-1502). The testing-only call cuvsCertexTestScratchCap makes every
  scratch request of the thread's resources above the cap fail as an allocation would, so the
  halving runs; results must equal the oracle, and a single query that cannot fit is an error.
- Fractional queries of an integer index are rejected (tests/test_exact.py:342-350).
- Searches of a float index during concurrent additions each equal the exact top k of one
  published snapshot (cpp/tests/neighbors/ann_certex/test_updates.cu:504-591).
"""

import threading

import numpy as np
import pytest
import torch

import libcertex_amd as certex
import oracle
from libcertex_amd import _capi as C
from tests import data

pytestmark = pytest.mark.gpu


def in_fresh_resources(fn, cap):
    """Run fn() in a new thread, whose C resources get the scratch cap (a testing-only call)."""
    out, errors = [], []

    def body():
        try:
            C.check(C.lib().cuvsCertexTestScratchCap(C.resources(), cap))
            out.append(fn())
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    t = threading.Thread(target=body)
    t.start()
    t.join()
    if errors:
        raise errors[0]
    return out[0]


@pytest.mark.parametrize("kind", ["uint8", "float32"])
def test_batches_halve_on_allocation_failure(gpu, kind):
    if kind == "uint8":
        X, Q, metric = data.mixture_u8(60_000, seed=150), data.mixture_u8(2_000, seed=151), "l2"
    else:
        X, Q, metric = data.powerlaw_unit(40_000, 192, seed=150), data.powerlaw_unit(2_000, 192, seed=151), "cosine"
    idx = certex.Index(X.shape[1], metric=metric)
    idx.add(torch.from_numpy(X).cuda())
    Qg = torch.from_numpy(Q).cuda()

    def search():
        D, I = idx.search(Qg, k=10, batch=2_000)
        torch.cuda.synchronize()
        return D.cpu().numpy(), I.cpu().numpy()

    # the buckets of a 2,000-query batch take 2,048 x 1,024 x 4 bytes, four times the cap: the
    # batch halves until its slots fit
    D, I = in_fresh_resources(search, 2 << 20)
    s, i = oracle.knn(X, Q, 10, metric)
    np.testing.assert_array_equal(I, i)
    d = oracle.distances(s, i, metric)
    if metric == "cosine":
        d = (np.float32(1) - d).astype(np.float32)
    np.testing.assert_array_equal(D, d)
    with pytest.raises((ValueError, C.CertexError)):
        in_fresh_resources(search, 64)  # not even one query fits


def test_fractional_queries_rejected(gpu):
    X = torch.randint(0, 255, (5_000, 16), dtype=torch.uint8, device="cuda")
    idx = certex.Index(16)
    idx.add(X)
    with pytest.raises(ValueError):
        idx.search(torch.full((4, 16), 0.5, device="cuda"), k=5)
    with pytest.raises(ValueError):
        idx.search(torch.full((4, 16), 256.0, device="cuda"), k=5)
    D, I = idx.search(X[:4].float(), k=1)  # integral floats are taken as the index's type
    assert bool((D[:, 0] == 0).all())


@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_float_search_during_extend(gpu, metric):
    X = data.powerlaw_unit(36_000, 96, seed=152) * np.float32(2.0)
    Q = data.powerlaw_unit(150, 96, seed=153)
    idx = certex.Index(96, metric=metric)
    idx.add(torch.from_numpy(X[:12_000]).cuda())
    sizes = list(range(12_000, 36_001, 3_000))
    refs = [oracle.knn(X[:n], Q, 10, metric)[1] for n in sizes]
    errors, matched = [], set()
    done = threading.Event()

    def writer():
        try:
            with torch.cuda.stream(torch.cuda.Stream()):
                for i in range(12_000, 36_000, 3_000):
                    idx.add(torch.from_numpy(X[i : i + 3_000]).cuda())
                torch.cuda.current_stream().synchronize()
        except Exception as e:  # noqa: BLE001
            errors.append(e)
        finally:
            done.set()

    def reader():
        try:
            with torch.cuda.stream(torch.cuda.Stream()):
                Qg = torch.from_numpy(Q).cuda()
                n = 0
                while not done.is_set() or n < 3:
                    _, I = idx.search(Qg, k=10)
                    torch.cuda.current_stream().synchronize()
                    I = I.cpu().numpy()
                    hits = [j for j, r in enumerate(refs) if np.array_equal(I, r)]
                    assert hits, "a search during the additions equals no published snapshot"
                    matched.update(hits)
                    n += 1
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    threads = [threading.Thread(target=writer)] + [threading.Thread(target=reader) for _ in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[0]
    _, I = idx.search(torch.from_numpy(Q).cuda(), k=10)
    np.testing.assert_array_equal(I.cpu().numpy(), refs[-1])
