"""Save / load (reference tests/test_exact.py:219-239, test_updates.cu:459-498) and searches that
run while another thread adds vectors (test_exact.py:367-405): every search must equal the exact
answer over one of the published prefixes."""

import os
import threading

import numpy as np
import pytest
import torch

import libcertex_amd as certex
import oracle
from tests import data

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [np.uint8, np.float32, np.float16])
def test_save_load(gpu, tmp_path, dtype):
    if dtype == np.uint8:
        X, Q = data.mixture_u8(20_000, seed=1), data.mixture_u8(100, seed=2)
    else:
        X, Q = data.gaussian(20_000, 64, 1, dtype), data.gaussian(100, 64, 2, dtype)
    idx = certex.Index(X.shape[1], metric="l2")
    idx.add(X)
    idx.remove(torch.arange(0, 20_000, 7))
    labels = None
    D0, I0 = idx.search(Q, k=10)
    path = tmp_path / "index.cx"
    idx.save(path)
    back = certex.Index.load(path)
    assert back.ntotal == idx.ntotal and back.dtype == idx.dtype and back.metric == "l2"
    D1, I1 = back.search(Q, k=10)
    np.testing.assert_array_equal(I0, I1)
    np.testing.assert_array_equal(D0, D1)
    back.add(X[:1000])  # a loaded index keeps growing
    assert back.ntotal == idx.ntotal + 1000


@pytest.mark.parametrize("dtype", [np.uint8, np.float32])
def test_save_load_in_chunks(gpu, tmp_path, dtype):
    """Arrays larger than the 64 MiB staging buffers move in several chunks each (an odd count for
    the rows), with labels and lists; the loaded index answers exactly as the saved one."""
    if dtype == np.uint8:
        X = data.mixture_u8(1_300_000, seed=7)  # 166 MB of rows: 3 chunks
        Q = data.mixture_u8(300, seed=8)
    else:
        X = data.gaussian(330_000, 128, 7, np.float32)  # 169 MB of vectors: 3 chunks
        Q = data.gaussian(300, 128, 8, np.float32)
    labels = torch.from_numpy(np.random.default_rng(9).integers(0, 5, len(X)).astype(np.int32))
    idx = certex.Index(128, metric="l2", n_lists=32)
    idx.add(X, labels=labels)
    idx.remove(torch.arange(3, len(X), 101))
    D0, I0 = idx.search(Q, k=10)
    ql = torch.from_numpy(np.random.default_rng(10).integers(0, 5, len(Q)).astype(np.int32))
    Dl0, Il0 = idx.search(Q, k=10, labels=ql)
    path = tmp_path / "big.cx"
    idx.save(path)
    back = certex.Index.load(path)
    assert back.ntotal == idx.ntotal and back.core.lists == idx.core.lists
    assert torch.equal(back.list_order(), idx.list_order())
    D1, I1 = back.search(Q, k=10)
    np.testing.assert_array_equal(I0, I1)
    np.testing.assert_array_equal(D0, D1)
    Dl1, Il1 = back.search(Q, k=10, labels=ql)
    np.testing.assert_array_equal(Il0, Il1)
    np.testing.assert_array_equal(Dl0, Dl1)


def test_load_rejects_foreign_files(gpu, tmp_path):
    bad = tmp_path / "bad.cx"
    bad.write_bytes(b"<f4\x00" + (0x43455258).to_bytes(4, "little") + (1).to_bytes(4, "little") + b"\x00" * 64)
    with pytest.raises(ValueError, match="another version"):
        certex.Index.load(bad)
    with pytest.raises(ValueError):
        (tmp_path / "junk").write_bytes(b"hello world")
        certex.Index.load(tmp_path / "junk")


@pytest.mark.parametrize("dtype", [np.uint8, np.float32])
def test_concurrent_search_and_add(gpu, dtype):
    """Searches on three streams while a fourth adds rows: every search equals the oracle on one
    published snapshot. Float rows of 256 coordinates take the tiled screen, and additions raise
    the index's fp16 maxima (the certificate's operand bounds) while searches read them."""
    if dtype == np.uint8:
        X = data.mixture_u8(40_000, seed=5)
        Q = data.mixture_u8(200, seed=6)
    else:
        X = data.powerlaw_unit(40_000, 256, seed=5) * np.linspace(1, 3, 40_000, dtype=np.float32)[:, None]
        Q = data.powerlaw_unit(200, 256, seed=6)
    idx = certex.Index(X.shape[1])
    idx.add(X[:20_000])
    sizes = list(range(20_000, 40_001, 2_000))
    refs = [oracle.knn(X[:n], Q, 10, "l2")[1] for n in sizes]
    errors = []

    def writer():
        with torch.cuda.stream(torch.cuda.Stream()):
            for i in range(20_000, 40_000, 2_000):
                idx.add(X[i : i + 2_000])
            torch.cuda.current_stream().synchronize()

    def reader():
        try:
            with torch.cuda.stream(torch.cuda.Stream()):
                Qg = torch.from_numpy(Q).cuda()
                for _ in range(10):
                    _, I = idx.search(Qg, k=10)
                    torch.cuda.current_stream().synchronize()
                    I = I.cpu().numpy()
                    ok = np.zeros(len(Q), bool)
                    for r in refs:
                        ok |= (I == r).all(1)
                    assert ok.all(), f"{int((~ok).sum())} queries match no snapshot"
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    threads = [threading.Thread(target=writer)] + [threading.Thread(target=reader) for _ in range(3)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[0]
    assert idx.ntotal == 40_000
    _, I = idx.search(Q, k=10)
    np.testing.assert_array_equal(I, refs[-1])
