"""KeyCache and topk (config 4 path): the exact top k keys by inner product, as
torch.topk(q @ keys.mT, k) with exact fp64 scores and ties to the lower key id (reference
tests/test_attention.py:45-72). Expected ids come from the CPU oracle on the same values."""

import numpy as np
import pytest
import torch

import libcertex_amd as certex
import oracle

pytestmark = pytest.mark.gpu


def data(n_kv, H, n, m, d=128, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    keys = torch.randn((n_kv, n, d), generator=g, device="cuda", dtype=torch.float32).half()
    q = torch.randn((H, m, d), generator=g, device="cuda", dtype=torch.float32).half()
    return q, keys


def assert_exact(q, keys, scores, ids, k):
    """ids equal the oracle's top k of every query head against its KV head; scores descend."""
    H, m, d = q.shape
    r = H // keys.shape[0]
    qn, kn = q.cpu().numpy(), keys.cpu().numpy()
    ids, scores = ids.cpu().numpy(), scores.cpu().numpy()
    for h in range(H):
        s, i = oracle.knn(kn[h // r], qn[h], k, "ip")
        np.testing.assert_array_equal(ids[h], i)
        np.testing.assert_array_equal(scores[h], (-s).astype(np.float32))
    assert (scores[..., :-1] >= scores[..., 1:]).all()


@pytest.mark.parametrize("k", [10, 64, 2048])
def test_gqa_exact(gpu, k):
    q, keys = data(n_kv=2, H=4, n=50_000, m=16)
    scores, ids = certex.KeyCache(2, 128, k=k).append(keys).topk(q, k)
    assert scores.shape == ids.shape == (4, 16, k)
    assert_exact(q, keys, scores, ids, k)


def test_append_in_steps(gpu):
    q, keys = data(n_kv=2, H=2, n=40_000, m=8)
    cache = certex.KeyCache(2, 128, k=64, capacity=40_000)
    for s in range(0, 40_000, 10_000):
        cache.append(keys[:, s : s + 10_000])
    scores, ids = cache.topk(q, 64)
    assert_exact(q, keys, scores, ids, 64)


def test_single_query_and_function(gpu):
    q, keys = data(n_kv=1, H=2, n=30_000, m=1)
    s1, i1 = certex.topk(q[:, 0], keys, 32)
    assert s1.shape == (2, 32)
    assert_exact(q, keys, s1[:, None], i1[:, None], 32)


def test_bf16_inputs(gpu):
    q, keys = data(n_kv=2, H=4, n=30_000, m=8)
    scores, ids = certex.topk(q.bfloat16(), keys.bfloat16(), 64)
    assert_exact(q.bfloat16().float(), keys.bfloat16().float(), scores, ids, 64)


def test_outlier_channels(gpu):
    """Keys with 4 channels scaled by 20 (config 4's outliers)."""
    q, keys = data(n_kv=2, H=8, n=20_000, m=4, seed=3)
    keys = keys.float()
    keys[..., :4] *= 20
    scores, ids = certex.topk(q, keys.half(), 100)
    assert_exact(q, keys.half(), scores, ids, 100)


@pytest.mark.parametrize("key_type", [torch.bfloat16, torch.float16])
def test_queries_of_another_type(gpu, key_type):
    """float32 queries against a bfloat16 or float16 cache are rounded to the cache's type, as
    the reference rounds them; the top k is exact for the rounded queries."""
    q, keys = data(n_kv=2, H=4, n=30_000, m=8, seed=5)
    q32 = q.float() + 1e-3 * torch.randn(q.shape, generator=torch.Generator(device="cuda").manual_seed(6),
                                         device="cuda")
    cache = certex.KeyCache(2, 128, k=64).append(keys.to(key_type))
    scores, ids = cache.topk(q32, 64)
    assert_exact(q32.to(key_type).float(), keys.to(key_type).float(), scores, ids, 64)
    s16, i16 = cache.topk(q32.half(), 64)  # float16 queries against the same cache
    assert_exact(q32.half().to(key_type).float(), keys.to(key_type).float(), s16, i16, 64)


def test_queries_that_overflow_the_cache(gpu):
    q, keys = data(n_kv=1, H=1, n=5_000, m=2, seed=7)
    cache = certex.KeyCache(1, 128, k=8).append(keys)  # a float16 cache
    big = q.float()
    big[0, 0, 0] = 1e6  # beyond float16's range
    with pytest.raises(ValueError, match="overflow"):
        cache.topk(big, 8)


def test_group_table_of_an_earlier_search(gpu):
    """A KeyCache's search (KV heads of equal size, queries in head order) writes every column of
    its group table itself: a table of larger values that an earlier search on the same thread
    left in the workspace (every query equal to every row) changes nothing."""
    v = torch.randn((1, 128), generator=torch.Generator(device="cuda").manual_seed(9), device="cuda")
    P = v.repeat(100_000, 1)
    poison = certex.Index(128, metric="ip")
    poison.add(P)
    poison.search(P[:2048].contiguous(), k=16, batch=2048)
    q, keys = data(n_kv=2, H=4, n=20_000, m=16, seed=11)
    cache = certex.KeyCache(2, 128, k=16)
    cache.append(keys[:, :19_000]).append(keys[:, 19_000:])  # the partition, then a tail
    scores, ids = cache.topk(q, 16)
    assert_exact(q, keys, scores, ids, 16)
