"""Configs 3 and 4 at their full sizes under the GPU tests.

Config 3: 1,000,000 x 768 power-law embeddings (L2-normalised, cosine), 10,000 queries, k = 100,
one of 16 labels per vector and per query, labels in device memory (the routing built on the
device), one batch of 10,000 and the API's default batch of 2,048. Config 4: the KeyCache of 8 KV
heads x 131,072 bfloat16 keys x 128 with 4 outlier channels x 20, 32 query heads (GQA 4:1) x 64
queries, k = 2,048, and two appends of 256 keys per head between searches.

Two checks (the bench's generators, seeded as the bench seeds them):
- the CPU oracle on a subset of the queries: ids bit-exact (ties to the lower id) and distances
  equal to the oracle's;
- a GPU fp64 brute force over every query (torch, float64 products): the exact scores of the
  returned ids, recomputed in fp64, equal the brute force's k best scores, in order, to 1e-12
  relative (the summation order differs from the oracle's only in the last bits, so ids are
  compared on the oracle's subset).
"""

import numpy as np
import pytest
import torch

import libcertex_amd as certex
import oracle

pytestmark = pytest.mark.gpu

REL = 1e-12


def powerlaw_unit(n, d, seed, basis, dev):
    """The bench's config 3 rows (torch generator seeded `seed`)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    out = torch.empty((n, d), dtype=torch.float32, device=dev)
    for i in range(0, n, 1 << 17):
        m = min(1 << 17, n - i)
        x = torch.randn((m, d), generator=g, device=dev) @ basis
        out[i : i + m] = x / x.norm(dim=1, keepdim=True)
    return out


def assert_scores_close(got, want):
    np.testing.assert_allclose(got, want, rtol=REL, atol=0)


def test_config3_full_size(gpu):
    dev = torch.device("cuda")
    n, d, nq, k = 1_000_000, 768, 10_000, 100
    qm, _ = torch.linalg.qr(torch.randn((d, d), generator=torch.Generator().manual_seed(31), dtype=torch.float64))
    basis = (torch.sqrt(1.0 / torch.arange(1, d + 1, dtype=torch.float64))[:, None] * qm.T).float().to(dev)
    X = powerlaw_unit(n, d, 32, basis, dev)
    Q = powerlaw_unit(nq, d, 33, basis, dev)
    gl = torch.Generator(device=dev).manual_seed(34)
    lx = torch.randint(0, 16, (n,), generator=gl, device=dev, dtype=torch.int32)
    lq = torch.randint(0, 16, (nq,), generator=gl, device=dev, dtype=torch.int32)
    idx = certex.Index(d, metric="cosine")
    idx.add(X, labels=lx)
    D, I = idx.search(Q, k=k, batch=10_000, labels=lq)
    D2, I2 = idx.search(Q, k=k, labels=lq)  # batches of 2,048
    torch.cuda.synchronize()
    assert torch.equal(I, I2) and torch.equal(D, D2)
    print("config 3: searched; GPU fp64 brute force next", flush=True)

    # every query: the exact cosine scores of the returned ids against the k best of its label
    Xd = X.double()
    xn = Xd.norm(dim=1)
    for lab in range(16):
        qs = torch.nonzero(lq == lab).flatten()
        rows = torch.nonzero(lx == lab).flatten()
        Qd = Q[qs].double()
        qn = Qd.norm(dim=1)
        sim = (Qd @ Xd[rows].T) / (qn[:, None] * xn[rows][None, :])
        best = torch.topk(sim, k, dim=1).values
        got = ((Qd[:, None, :] * Xd[I[qs]]).sum(-1)) / (qn[:, None] * xn[I[qs]])
        assert bool((lx[I[qs]] == lab).all()), f"label {lab}: an id of another label"
        assert_scores_close(got.cpu().numpy(), best.cpu().numpy())
    print("config 3: brute force equal; oracle on the first 48 queries next", flush=True)

    c = 48
    Xh, Qh = X.cpu().numpy(), Q[:c].cpu().numpy()
    s, i = oracle.knn(Xh, Qh, k, "cosine", row_labels=lx.cpu().numpy(), query_labels=lq[:c].cpu().numpy())
    np.testing.assert_array_equal(I[:c].cpu().numpy(), i)
    want = np.where(i >= 0, np.float32(1) - oracle.distances(s, i, "cosine"), -np.inf).astype(np.float32)
    np.testing.assert_array_equal(D[:c].cpu().numpy(), want)


def test_config4_full_size(gpu):
    dev = torch.device("cuda")
    n_kv, n, d, H, m, k, grow = 8, 131_072, 128, 32, 64, 2048, 256
    g = torch.Generator(device=dev).manual_seed(41)
    outliers = torch.randperm(d, generator=torch.Generator().manual_seed(42))[:4].to(dev)

    def keys(count):
        x = torch.randn((n_kv, count, d), generator=g, device=dev)
        x[:, :, outliers] *= 20.0
        return x.to(torch.bfloat16)

    cache = certex.KeyCache(n_kv, d, k=k, capacity=n + 2 * grow)
    all_keys = [keys(n)]
    cache.append(all_keys[0])
    q = torch.randn((H, m, d), generator=g, device=dev).to(torch.bfloat16)
    for step in range(3):  # a search on the first keys, then after each of two appends
        if step:
            all_keys.append(keys(grow))
            cache.append(all_keys[-1])
        scores, ids = cache.topk(q, k)
        torch.cuda.synchronize()
        K = torch.cat(all_keys, 1).double()  # (n_kv, n_now, d), bf16 held exactly
        r = H // n_kv
        for h in range(H):
            qd = q[h].double()
            sim = qd @ K[h // r].T
            best = torch.topk(sim, k, dim=1).values
            got = (qd[:, None, :] * K[h // r][ids[h]]).sum(-1)
            assert_scores_close(got.cpu().numpy(), best.cpu().numpy())
            assert bool((scores[h, :, :-1] >= scores[h, :, 1:]).all())
        print(f"config 4 step {step}: brute force equal over all {H} query heads", flush=True)
    # the oracle on query heads 0 and 31 (KV heads 0 and 7), ids bit-exact
    Kf = torch.cat(all_keys, 1).float().cpu().numpy()
    for h in (0, H - 1):
        s, i = oracle.knn(Kf[h // (H // n_kv)], q[h].float().cpu().numpy(), k, "ip")
        np.testing.assert_array_equal(ids[h].cpu().numpy(), i)
        np.testing.assert_array_equal(scores[h].cpu().numpy(), (-s).astype(np.float32))
