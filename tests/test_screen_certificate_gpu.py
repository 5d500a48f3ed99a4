"""The screen and its certificate checked kernel by kernel, on the arrays one search batch produced
(reference harness: cpp/tests/neighbors/certex_kernels.cu:62-180, which screens random rows
against an fp64 product and asserts no missing pair, no wrong product, no duplicate and correct
anchor-group maxima).

A testing-only capture (cuvsCertexTestCaptureBegin / Get) copies, from the search's own launches,
the encoded queries, the anchor group table, the thresholds, the buckets and, for float indexes,
the certified bound U of each query and the certificate's two bounds of every bucket entry. Then,
against a CPU brute force:

int8 rows (exact integer screen):
- the stored codes and row terms are the encoding of the vectors (x ^ 0x80, -floor(|x'|^2 / 2)),
  for rows of 128 bytes (the narrow screen) and of 512 bytes (the tiled screen, K-loop anchors);
- every group maximum equals the largest <q', x'> + rowc over the group's anchors;
- theta is the k-th largest group maximum (floored at the keep-all value), and no row of the true
  top k (ties at the k-th value included) lies below it;
- the survivors are exactly {rows with <q', x'> + rowc >= theta}, each once.

fp16 rows (certified screen):
- every survivor has a screen value >= theta and appears once;
- the fp32 accumulation of the MFMA stays within the model the certificate assumes:
  |v - (<w~, z~> + rowc)| <= gamma (|w~| |z~| + |rowc|), with gamma = 2 (K + 1) 2^-24;
- lb(v) <= exact fp64 score <= ub(v) for every survivor (the bounds the verification and the
  threshold use, evaluated on the device);
- U >= the true k-th score, and every row whose exact score is <= U is a survivor.
Inputs include rows at the maximum norm, coordinates on both sides of fp16's smallest normal,
queries far outside the data (cancellation in l2), cosine near-duplicates, and d in
{7, 128, 768, 2048}. The worst margins seen are printed (run with -s).
"""

import ctypes

import numpy as np
import pytest
import torch

import libcertex_amd as certex
import oracle
from libcertex_amd import _capi as C
from tests import data

pytestmark = pytest.mark.gpu

DEAD = -(1 << 30)
KEEP_ALL = -(1 << 29)


def captured(run):
    """Runs run() (one search batch) with the capture on; returns a getter of the arrays."""
    L = C.lib()
    C.check(L.cuvsCertexTestCaptureBegin())
    run()
    torch.cuda.synchronize()

    def get(name, dtype=np.int64, shape=None):
        n = ctypes.c_int64()
        C.check(L.cuvsCertexTestCaptureGet(name.encode(), None, ctypes.byref(n)))
        buf = np.empty(n.value, np.uint8)
        C.check(L.cuvsCertexTestCaptureGet(name.encode(), buf.ctypes.data_as(ctypes.c_void_p), ctypes.byref(n)))
        a = buf.view(dtype)
        return a.reshape(shape) if shape is not None else (a[0] if a.size == 1 and dtype == np.int64 else a)

    return get


def buckets(get, B):
    cap = int(get("cap"))
    count = get("count", np.uint32)
    rows = get("rows", np.uint32, (B, cap))
    assert (count <= cap).all(), "a bucket overflowed without a re-run"
    return cap, count, rows


def groups_of(n_anchor, fine, group_steps):
    """The group column of every anchor (coarse: group_steps steps of 64 anchors; fine: 4)."""
    j = np.arange(n_anchor)
    return j // 4 if fine else (j // 64) // group_steps


# --- int8 rows -------------------------------------------------------------------------------


def int8_case(n, nq, kind, seed, d=128):
    rng = np.random.default_rng(seed)
    if kind == "uint8":
        X = data.mixture_u8(n, d=d, seed=seed)
        Q = data.mixture_u8(nq, d=d, seed=seed + 1)
        X[:50] = 0  # extreme codes (-128) and exact ties
        X[50:100] = 255
        X[100:400] = X[400:700]  # duplicated rows: ties at every distance
        Q[:4] = X[400:404]  # queries on duplicated rows
    else:
        X = data.uniform_int(n, d, seed, np.int8)
        Q = data.uniform_int(nq, d, seed + 1, np.int8)
        X[:64] = -128
    removed = rng.choice(n, n // 50, replace=False)
    return X, Q, removed


@pytest.mark.parametrize("n, k, kind, metric, d", [
    (200_000, 10, "uint8", "l2", 128),     # fine anchor groups (4 anchors each)
    (200_000, 64, "uint8", "ip", 128),
    (1_200_000, 10, "uint8", "l2", 128),   # coarse anchor groups (whole 64-anchor steps)
    (150_000, 32, "int8", "l2", 128),
    (150_000, 10, "int8", "ip", 128),
    (120_000, 10, "uint8", "l2", 384),     # rows of 512 bytes: the tiled int8 screen, K-loop anchors
    (700_000, 10, "uint8", "ip", 300),     # coarse groups in the K-loop anchor pass
])
def test_int8_screen(gpu, n, k, kind, metric, d):
    nq = 96
    X, Q, removed = int8_case(n, nq, kind, seed=n % 97 + k, d=d)
    idx = certex.Index(d, metric=metric)
    idx.add(torch.from_numpy(X).cuda())
    idx.remove(torch.from_numpy(removed))
    Qg = torch.from_numpy(Q).cuda()
    get = captured(lambda: idx.search(Qg, k=k, batch=nq))
    B, size, rb = int(get("B")), int(get("size")), int(get("row_bytes"))
    assert (B, size, rb) == (nq, n, 128 if d <= 128 else (d + 255) // 256 * 256) and not get("all_rows")

    # the encoding of the rows and queries
    flip = 0x80 if kind == "uint8" else 0
    codes = get("codes", np.int8, (size, rb)).astype(np.int64)
    rowc = get("rowc", np.int32).astype(np.int64)
    qrows = get("qrows", np.int8, (B, rb)).astype(np.int64)
    xc = (X.view(np.uint8) ^ flip).view(np.int8).astype(np.int64)
    assert np.array_equal(codes[:, :d], xc) and not codes[:, d:].any()
    assert np.array_equal(qrows[:, :d], (Q.view(np.uint8) ^ flip).view(np.int8).astype(np.int64))
    live = np.ones(n, bool)
    live[removed] = False
    if metric == "l2":
        want = -((xc * xc).sum(1) // 2)
    else:
        want = 128 * xc.sum(1) if kind == "uint8" else np.zeros(n, np.int64)
    assert np.array_equal(rowc[live], want[live])
    assert (rowc[~live] == DEAD).all()

    # acc = <q', x'> + rowc, exact (float64 products of integers below 2^53)
    acc = np.empty((B, size), np.int64)
    for c in range(0, size, 1 << 17):
        acc[:, c : c + (1 << 17)] = (qrows.astype(np.float64) @ codes[c : c + (1 << 17)].T.astype(np.float64)).astype(np.int64)
    acc += rowc[None, :]

    # group maxima of the anchors (every anchor_stride-th row)
    s, fine, gs = int(get("anchor_stride")), bool(get("fine")), int(get("group_steps"))
    n_groups = int(get("n_groups"))
    gmax = get("gmax", np.int32, (B, n_groups)).astype(np.int64)
    anchors = np.arange(0, size, s)
    col = groups_of(len(anchors), fine, gs)
    assert col.max() == n_groups - 1
    want_g = np.full((B, n_groups), -(1 << 62))
    np.maximum.at(want_g.T, col, acc[:, anchors].T)
    assert np.array_equal(gmax, want_g), "anchor group maxima"

    theta = get("theta", np.int32).astype(np.int64)
    kth_group = -np.sort(-gmax, axis=1)[:, k - 1]
    assert np.array_equal(theta, np.maximum(kth_group, KEEP_ALL)), "theta is the k-th best group"
    kth_true = -np.sort(-np.where(live, acc, -(1 << 62)), axis=1)[:, k - 1]
    assert (theta <= kth_true).all(), "a row of the true top k lies below theta"

    cap, count, rows = buckets(get, B)
    for q in range(B):
        got = rows[q, : count[q]]
        assert len(np.unique(got)) == len(got), f"query {q}: a survivor twice"
        assert set(got.tolist()) == set(np.nonzero(acc[q] >= theta[q])[0].tolist()), f"query {q}: survivors"


@pytest.mark.parametrize("k, metric, stride, d", [
    (10, "l2", 16, 128),
    (64, "ip", 4, 128),
    (1, "l2", 1, 200),  # rows of 256 bytes
])
def test_int8_list_anchors(gpu, k, metric, stride, d):
    """An index stored in k-means lists and searched without a probe takes its thresholds from the
    anchors of each query's 8 nearest lists: column 64 t + g of the group table holds the largest
    <q', x'> + rowc over the anchors i = g, g + 64, ... of the query's t-th list (its stored rows
    offset + i stride / 4). Checked against the brute force as above: the table, theta as its k-th
    largest column, no true top-k row below theta, the survivors exactly the rows at or above it."""
    nq, n = 96, 120_000
    X, Q, removed = int8_case(n, nq, "uint8", seed=k + stride, d=d)
    idx = certex.Index(d, metric=metric, n_lists=64, anchor_stride=stride)
    idx.add(torch.from_numpy(X).cuda())
    idx.remove(torch.from_numpy(removed))
    Qg = torch.from_numpy(Q).cuda()
    get = captured(lambda: idx.search(Qg, k=k, batch=nq, probe_lists=0))
    B, size, rb = int(get("B")), int(get("size")), int(get("row_bytes"))
    p, ls = int(get("list_anchors")), int(get("list_anchor_stride"))
    assert (B, size, rb, p) == (nq, n, 128 if d <= 128 else 256, 8) and not get("all_rows")
    assert ls == max(1, stride // 2)
    codes = get("codes", np.int8, (size, rb)).astype(np.int64)
    rowc = get("rowc", np.int32).astype(np.int64)
    qrows = get("qrows", np.int8, (B, rb)).astype(np.int64)
    live = rowc != DEAD
    assert (~live).sum() == len(removed)
    acc = (qrows.astype(np.float64) @ codes.T.astype(np.float64)).astype(np.int64) + rowc[None, :]

    lists = get("lists", np.int32, (B, p)).astype(np.int64)
    off = get("list_offsets", np.int64)
    assert off[0] == 0 and off[-1] == size and (np.diff(off) >= 0).all()
    assert ((lists >= 0) & (lists < 64)).all()
    assert all(len(set(r)) == p for r in lists.tolist()), "a list twice among a query's nearest"
    n_anchor = (np.diff(off) + ls - 1) // ls
    assert (n_anchor[lists] >= 32).all(), "a list of fewer than 32 anchors among the nearest"
    gmax = get("gmax", np.int32, (B, 64 * p)).astype(np.int64)
    want = np.full((B, 64 * p), np.iinfo(np.int32).min, np.int64)
    for q in range(B):
        for t in range(p):
            j = lists[q, t]
            rows = np.arange(off[j], off[j + 1], ls)
            np.maximum.at(want[q], t * 64 + np.arange(len(rows)) % 64, acc[q, rows])
    assert np.array_equal(gmax, want), "list anchor group maxima"

    theta = get("theta", np.int32).astype(np.int64)
    kth_group = -np.sort(-gmax, axis=1)[:, k - 1]
    assert np.array_equal(theta, np.maximum(kth_group, KEEP_ALL)), "theta is the k-th best group"
    kth_true = -np.sort(-np.where(live, acc, -(1 << 62)), axis=1)[:, k - 1]
    assert (theta <= kth_true).all(), "a row of the true top k lies below theta"
    cap, count, rows = buckets(get, B)
    for q in range(B):
        got = rows[q, : count[q]]
        assert len(np.unique(got)) == len(got), f"query {q}: a survivor twice"
        assert set(got.tolist()) == set(np.nonzero(acc[q] >= theta[q])[0].tolist()), f"query {q}: survivors"


# --- fp16 rows -------------------------------------------------------------------------------


def float_case(kind, n, nq, d, metric, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, d))
    Q = rng.standard_normal((nq, d))
    if kind == "maxnorm":
        # 2% of the rows on the sphere of the largest radius: |Z| = 64 exactly for them
        r = np.linalg.norm(X - X.mean(0), axis=1).max() * 1.5
        m = rng.choice(n, n // 50, replace=False)
        u = rng.standard_normal((len(m), d))
        X[m] = X.mean(0) + r * u / np.linalg.norm(u, axis=1, keepdims=True)
        Q[: nq // 4] = X[m[: nq // 4]] + 1e-3 * rng.standard_normal((nq // 4, d))
    elif kind == "subnormal":
        # one large coordinate sets the scale (|Z| up to 64); the others sit on both sides of
        # fp16's smallest normal 2^-14 after scaling, so that some round to zero
        X = np.zeros((n, d))
        X[:, 0] = rng.choice([-64.0, 64.0], n) * rng.uniform(0.5, 1.0, n)
        X[:, 1:] = 2.0 ** -14 * rng.uniform(0.5, 1.5, (n, d - 1)) * rng.choice([-1, 1], (n, d - 1))
        Q = X[rng.choice(n, nq)] + 2.0 ** -14 * rng.uniform(-1, 1, (nq, d))
    elif kind == "far":
        # queries far outside the data: |W|^2 dominates the l2 distances (cancellation)
        u = rng.standard_normal((nq, d))
        Q = 200.0 * u / np.linalg.norm(u, axis=1, keepdims=True) * np.sqrt(d)
    elif kind == "neardup":
        base = rng.standard_normal((n // 20, d))
        X = np.repeat(base, 20, axis=0) + 1e-6 * rng.standard_normal((n, d))
        Q = X[rng.choice(n, nq)] + 1e-7 * rng.standard_normal((nq, d))
    return X.astype(np.float32), Q.astype(np.float32)


WORST = {"accumulation": np.inf, "lower": np.inf, "upper": np.inf, "U": np.inf}


def float_cases():
    out = []
    for d in (7, 128, 768, 2048):
        for metric in ("l2", "ip", "cosine"):
            out.append(("gauss", d, metric, 10))
    out += [("gauss", 128, "l2", 100), ("gauss", 768, "cosine", 100)]
    for d in (128, 768):
        out += [("maxnorm", d, "l2", 10), ("maxnorm", d, "ip", 10)]
        out += [("subnormal", d, m, 10) for m in ("l2", "ip", "cosine")]
        out += [("far", d, "l2", 10), ("neardup", d, "cosine", 10), ("neardup", d, "l2", 10)]
    return out


@pytest.mark.parametrize("kind, d, metric, k", float_cases())
def test_fp16_certificate(gpu, kind, d, metric, k):
    n = 4_000 if d == 2048 else 20_000
    nq = 64
    X, Q, = float_case(kind, n, nq, d, metric, seed=d + k)
    removed = np.random.default_rng(d).choice(n, n // 40, replace=False)
    idx = certex.Index(d, metric=metric)
    idx.add(torch.from_numpy(X).cuda())
    idx.remove(torch.from_numpy(removed))
    Qg = torch.from_numpy(Q).cuda()
    get = captured(lambda: idx.search(Qg, k=k, batch=nq))
    B, size, halves = int(get("B")), int(get("size")), int(get("halves"))
    assert (B, size) == (nq, n)
    live = np.ones(n, bool)
    live[removed] = False
    theta = get("theta", np.float32).astype(np.float64)
    if get("all_rows"):
        pytest.skip("fewer than k anchor groups: every row is scored, no screen to check")
    cap, count, rows = buckets(get, B)
    with np.errstate(invalid="ignore"):  # slots past a query's count hold whatever was there
        vals = get("vals", np.float32, (B, cap)).astype(np.float64)
    lb = get("lb", np.float64, (B, cap))
    ub = get("ub", np.float64, (B, cap))
    U = get("ub_q", np.float64)
    gamma = float(get("gamma", np.float64)[0])
    z = get("codes", np.float16, (size, halves)).astype(np.float64)
    w = get("qrows", np.float16, (B, halves)).astype(np.float64)
    rowc = get("rowc", np.float32).astype(np.float64)
    assert np.isinf(rowc[~live]).all() and (rowc[~live] < 0).all()

    ids = np.broadcast_to(np.arange(n), (B, n))
    S = oracle.scores_of(X, Q, np.ascontiguousarray(ids), metric)  # exact fp64 scores, all pairs
    S_live = np.where(live, S, np.inf)
    kth = np.sort(S_live, axis=1)[:, k - 1]
    assert (U >= kth).all(), "U below the true k-th score"
    nz, nw = np.linalg.norm(z, axis=1), np.linalg.norm(w, axis=1)
    for q in range(B):
        got = rows[q, : count[q]].astype(np.int64)
        assert len(np.unique(got)) == len(got), f"query {q}: a survivor twice"
        assert live[got].all(), f"query {q}: a removed row survived"
        v = vals[q, : count[q]]
        assert (v >= theta[q]).all(), f"query {q}: a survivor below theta"
        # the fp32 accumulation against the model: |v - (<w~, z~> + rowc)| <= gamma (|w~||z~| + |rowc|)
        exact = z[got] @ w[q] + rowc[got]
        bound = gamma * (nw[q] * nz[got] + np.abs(rowc[got]))
        err = np.abs(v - exact)
        assert (err <= bound).all(), f"query {q}: MFMA accumulation error beyond gamma"
        nzero = err > 0
        if nzero.any():
            WORST["accumulation"] = min(WORST["accumulation"], float((bound[nzero] / err[nzero]).min()))
        s = S[q, got]
        assert (lb[q, : count[q]] <= s).all(), f"query {q}: lower bound above the exact score"
        assert (ub[q, : count[q]] >= s).all(), f"query {q}: upper bound below the exact score"
        scale = np.maximum(np.abs(s), 1e-300)
        WORST["lower"] = min(WORST["lower"], float(((s - lb[q, : count[q]]) / scale).min()))
        WORST["upper"] = min(WORST["upper"], float(((ub[q, : count[q]] - s) / scale).min()))
        need = np.nonzero(S_live[q] <= U[q])[0]
        missing = np.setdiff1d(need, got)
        assert missing.size == 0, f"query {q}: rows with exact score <= U missing: {missing[:5]}"
    WORST["U"] = min(WORST["U"], float(((U - kth) / np.maximum(np.abs(kth), 1e-300)).min()))
    print(f"\n{kind} d={d} {metric} k={k}: survivors/query {count.mean():.1f}; worst so far: "
          f"gamma bound / accumulation error {WORST['accumulation']:.3g}, "
          f"(score - lb) / |score| {WORST['lower']:.3g}, (ub - score) / |score| {WORST['upper']:.3g}, "
          f"(U - kth) / |kth| {WORST['U']:.3g}")
