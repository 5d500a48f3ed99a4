"""cuvsCertexSearchNoAlloc against cuvsCertexSearch, both called through the C ABI.

The search without allocation takes its scratch from one fixed 128 MiB array per GPU instead of
growing buffers. Its results must equal the allocating search's bit for bit (ids and distances),
on two calls in a row, the second with fewer queries, when a batch outgrows the array and is
split, and when two threads with their own resources and streams call one after the other. The
device's free memory must not move during a call.
"""

import ctypes

import numpy as np
import pytest
import torch

import libcertex_amd as certex
from libcertex_amd import _capi as C
from tests import data

pytestmark = pytest.mark.gpu


def c_search(idx, Q, k, entry, batch=2048, mask=None, probe=2):
    """One call of `entry` (cuvsCertexSearch or cuvsCertexSearchNoAlloc) on torch's stream."""
    Q = Q.contiguous()
    I = torch.full((Q.shape[0], k), -7, dtype=torch.int64, device="cuda")
    D = torch.full((Q.shape[0], k), -7.0, dtype=torch.float32, device="cuda")
    sp = C.SearchParams(128, int(batch), int(probe))
    qb, ib, db = C.Borrowed(Q), C.Borrowed(I), C.Borrowed(D)
    f, wb = C.Filter(0, C.NO_FILTER), None
    if mask is not None:
        from libcertex_amd.index import _pack

        wb = C.Borrowed(_pack(mask.cuda()), dtype_override=(C.kDLUInt, 32))
        f = C.Filter(ctypes.addressof(wb.m), C.BITSET if mask.ndim == 1 else C.BITMAP)
    C.check(getattr(C.lib(), entry)(C.resources(), ctypes.byref(sp), idx.core.h, qb.ptr, ib.ptr, db.ptr, f))
    torch.cuda.synchronize()
    del wb
    return D.cpu().numpy(), I.cpu().numpy()


def same(idx, Q, k, **kw):
    D0, I0 = c_search(idx, Q, k, "cuvsCertexSearch", **kw)
    D1, I1 = c_search(idx, Q, k, "cuvsCertexSearchNoAlloc", **kw)
    np.testing.assert_array_equal(I1, I0)
    np.testing.assert_array_equal(D1, D0)
    assert (I1 >= 0).all()


def test_uint8_two_calls(gpu):
    X = data.mixture_u8(300_000, seed=140)
    Q = torch.from_numpy(data.mixture_u8(3_000, seed=141)).cuda()
    idx = certex.Index(128)
    idx.add(torch.from_numpy(X).cuda())
    same(idx, Q, 10, batch=3000)
    same(idx, Q[:500], 10, batch=3000)  # the second call, smaller


def test_uint8_lists_without_probe_two_calls(gpu):
    """An index stored in k-means lists, searched without a probe: the thresholds come from the
    anchors of each query's nearest lists (their scratch carved from the array as well)."""
    X = data.mixture_u8(200_000, seed=146)
    Q = torch.from_numpy(data.mixture_u8(2_000, seed=147)).cuda()
    idx = certex.Index(128, n_lists=64)
    idx.add(torch.from_numpy(X).cuda())
    same(idx, Q, 10, batch=2000, probe=0)
    same(idx, Q[:300], 64, batch=2000, probe=0)  # the second call, smaller


def test_float_filtered_two_calls(gpu):
    X = data.powerlaw_unit(60_000, 256, seed=142)
    Q = torch.from_numpy(data.powerlaw_unit(1_500, 256, seed=143)).cuda()
    idx = certex.Index(256, metric="cosine")
    idx.add(torch.from_numpy(X).cuda())
    keep = torch.from_numpy(np.random.default_rng(144).random(len(X)) < 0.6)
    same(idx, Q, 50, mask=keep)
    same(idx, Q[:200], 50, mask=keep)
    bitmap = torch.from_numpy(np.random.default_rng(145).random((200, len(X))) < 0.5)
    same(idx, Q[:200], 20, mask=bitmap)


def test_batch_outgrows_the_scratch(gpu):
    """k = 2048 over 1,024 queries keeps far more than 128 MiB of candidates and best lists in one
    batch: the search splits it, with the same results."""
    X = np.random.default_rng(146).standard_normal((80_000, 128)).astype(np.float32)
    Q = torch.from_numpy(np.random.default_rng(147).standard_normal((1_024, 128)).astype(np.float32)).cuda()
    idx = certex.Index(128, metric="ip")
    idx.add(torch.from_numpy(X).cuda())
    same(idx, Q, 2048, batch=1024)
    same(idx, Q[:100], 2048, batch=1024)


def test_lists_and_free_memory(gpu):
    """An index with lists (the probe runs), and no device memory taken by the call itself."""
    X = data.mixture_u8(100_000, seed=148)
    Q = torch.from_numpy(data.mixture_u8(800, seed=149)).cuda()
    idx = certex.Index(128, n_lists=64)
    idx.add(torch.from_numpy(X).cuda())
    same(idx, Q, 10)
    I = torch.empty((800, 10), dtype=torch.int64, device="cuda")
    D = torch.empty((800, 10), dtype=torch.float32, device="cuda")
    sp = C.SearchParams(128, 2048, 2)
    qb, ib, db = C.Borrowed(Q), C.Borrowed(I), C.Borrowed(D)

    def call():
        C.check(C.lib().cuvsCertexSearchNoAlloc(C.resources(), ctypes.byref(sp), idx.core.h, qb.ptr, ib.ptr,
                                                db.ptr, C.Filter(0, C.NO_FILTER)))
        torch.cuda.synchronize()

    call()  # the same shape once before: code objects the runtime loads lazily are loaded by now
    before = torch.cuda.mem_get_info()[0]
    call()
    # the smallest slot the allocating search would carve is 1 MiB; nothing else allocates here
    assert abs(torch.cuda.mem_get_info()[0] - before) < (1 << 20)


def test_two_threads_take_turns(gpu):
    """Two threads, each with its own resources and stream, call one after the other without a
    sync between them. Each call returns with its verify still queued; the second call's stream
    must wait for it on the GPU before it reuses the scratch array."""
    import threading

    X = np.random.default_rng(150).standard_normal((120_000, 128)).astype(np.float32)
    Qs = [torch.from_numpy(np.random.default_rng(151 + i).standard_normal((512, 128)).astype(np.float32)).cuda()
          for i in range(2)]
    idx = certex.Index(128, metric="ip")
    idx.add(torch.from_numpy(X).cuda())
    k = 1024
    want = [c_search(idx, Q, k, "cuvsCertexSearch", batch=512) for Q in Qs]
    out = [None, None]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()

    def run(i):
        with torch.cuda.stream(streams[i]):
            I = torch.full((512, k), -7, dtype=torch.int64, device="cuda")
            D = torch.full((512, k), -7.0, dtype=torch.float32, device="cuda")
            sp = C.SearchParams(128, 512, 2)
            qb, ib, db = C.Borrowed(Qs[i]), C.Borrowed(I), C.Borrowed(D)
            C.check(C.lib().cuvsCertexSearchNoAlloc(C.resources(), ctypes.byref(sp), idx.core.h, qb.ptr, ib.ptr,
                                                    db.ptr, C.Filter(0, C.NO_FILTER)))
            out[i] = (D, I, (qb, ib, db))  # no sync here: the next call starts while these kernels run

    for i in range(2):
        t = threading.Thread(target=run, args=(i,))
        t.start()
        t.join()
    torch.cuda.synchronize()
    for i in range(2):
        np.testing.assert_array_equal(out[i][1].cpu().numpy(), want[i][1])
        np.testing.assert_array_equal(out[i][0].cpu().numpy(), want[i][0])
