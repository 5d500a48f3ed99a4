"""Full-size workloads of configs 2 and 5 under the GPU tests, checked by an exact GPU brute force
(tests/exact_gpu.py: fp64 is exact for 8-bit data; ids bit-exact with ties to the lower id).

Config 2 runs at its full size: 10,000,000 x 128 uint8 rows of the config 2 mixture, all 10,000
queries in one batch, every id row checked; in id order and in the order of 4,096 k-means lists
(the bench's index), searched with and without a probe.

Config 5's workload runs at 100,000,000 rows (a tenth of config 5's rows, which one test can afford):
4,096 k-means lists probed 2 per query (config 5's setting), and while searches run another thread
extends the index by 1,000,000 rows (two additions) and removes 1,000,000 random ids. As in the
reference's SearchDuringExtend (cpp/tests/neighbors/ann_certex/test_updates.cu:504-591), every
search made during the updates must equal the exact top k of one published snapshot of the index;
afterwards all 1,000 queries must equal the brute force over the live rows.
"""

import threading

import pytest
import torch

import libcertex_amd as certex
from tests import data
from tests.exact_gpu import topk_u8

pytestmark = pytest.mark.gpu

K = 10


def test_config2_full_size(gpu):
    # the bench's data: the same generators and chunks
    X = data.mixture_u8_cuda(10_000_000, seed=2, chunk=1 << 20)
    Q = data.mixture_u8_cuda(10_000, seed=3, chunk=1 << 20)
    idx = certex.Index(128)
    idx.add(X)
    D, I = idx.search(Q, k=K, batch=10_000)
    torch.cuda.synchronize()
    print("config 2: searched 10,000 queries; brute force next", flush=True)
    ((dist, ids),) = topk_u8(X, Q, K, chunk=50_000)
    assert torch.equal(I, ids)
    assert torch.equal(D.double(), dist)
    # the bench's index: rows stored in the order of 4,096 k-means lists, searched without a probe
    # (every row screened) and with one
    del idx
    listed = certex.Index(128, n_lists=4096)
    listed.add(X)
    assert listed.core.lists == (4096, 10_000_000)
    for probe in (0, 2):
        D, I = listed.search(Q, k=K, batch=10_000, probe_lists=probe)
        torch.cuda.synchronize()
        print(f"config 2 in list order, probe {probe}: searched", flush=True)
        assert torch.equal(I, ids)
        assert torch.equal(D.double(), dist)


N, N_NEW, N_GONE, N_LISTS = 100_000_000, 1_000_000, 1_000_000, 4_096


def test_config5_workload_lists_during_updates(gpu):
    X = data.mixture_u8_cuda(N + N_NEW, seed=2)
    Q = data.mixture_u8_cuda(1_000, seed=3)
    idx = certex.Index(128, n_lists=N_LISTS, capacity=N + N_NEW)
    idx.add(X[:N])
    torch.cuda.synchronize()
    print("config 5 workload: built 10^8 rows with 4,096 lists", flush=True)
    assert idx.core.lists == (N_LISTS, N)
    gone = torch.randperm(N, generator=torch.Generator().manual_seed(4))[:N_GONE].cuda()
    half = N + N_NEW // 2
    errors, results = [], []
    done = threading.Event()

    def writer():
        try:
            with torch.cuda.stream(torch.cuda.Stream()):
                idx.add(X[N:half])
                idx.add(X[half:])
                idx.remove(gone)
                torch.cuda.current_stream().synchronize()
        except Exception as e:  # noqa: BLE001
            errors.append(e)
        finally:
            done.set()

    def reader():
        try:
            with torch.cuda.stream(torch.cuda.Stream()):
                while not done.is_set() or len(results) < 4:
                    # the list anchors (no probe, config 5's default) and the probe in turn
                    D, I = idx.search(Q[:256], k=K, probe_lists=(0, 2)[len(results) % 2])
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
    print(f"config 5 workload: {len(results)} searches during the updates; brute force next", flush=True)
    assert idx.core.size == N + N_NEW and idx.ntotal == N + N_NEW - N_GONE
    assert idx.core.lists == (N_LISTS, N)

    # the published snapshots: the build, each addition, then the removal
    live = torch.ones(N + N_NEW, dtype=torch.bool, device="cuda")
    live[gone] = False
    prefix = lambda n: torch.ones(n, dtype=torch.bool, device="cuda")  # noqa: E731
    snaps = topk_u8(X, Q, K, live_masks=(prefix(N), prefix(half), None, live))
    for D, I in results:
        matches = [
            j
            for j, (dist, ids) in enumerate(snaps)
            if torch.equal(I, ids[:256]) and torch.equal(D.double(), dist[:256])
        ]
        assert matches, "a search during the updates equals no published snapshot"

    # after the updates: all queries against the live rows, with and without the probe
    dist, ids = snaps[-1]
    for probe in (2, 0):
        D, I = idx.search(Q, k=K, probe_lists=probe)
        torch.cuda.synchronize()
        assert torch.equal(I, ids)
        assert torch.equal(D.double(), dist)
