"""certex.Index: exact k-nearest-neighbour search on the MI355X, over the C API.

Mirrors the reference's Python interface (certex/index.py:191-548): the same classes, functions,
argument names, defaults, validation and errors. Every call goes through libcertex_c.so's
cuvsCertex* entry points on torch's current stream; arrays are converted here and the ids are
kept here.
"""

import ctypes
import threading

import numpy as np
import torch

from . import _capi as C

METRICS = ("l2", "cosine", "ip")
_DTYPES = {
    torch.float32: "float32",
    torch.float16: "float16",
    torch.bfloat16: "bfloat16",  # an addition of this build: bfloat16 vectors kept exactly
    torch.int8: "int8",
    torch.uint8: "uint8",
}
_TORCH = {v: k for k, v in _DTYPES.items()}
_METRIC_C = {"l2": C.L2Expanded, "cosine": C.CosineExpanded, "ip": C.InnerProduct}
_METRIC_PY = {v: k for k, v in _METRIC_C.items()}
_PREFIX = {b"f4": "float32", b"f2": "float16", b"b2": "bfloat16", b"i1": "int8", b"u1": "uint8"}


def row_len(m):
    """Halves per screening row of width m: m + 1 lifted and 4 certificate coordinates, padded to
    64 or 128n (reference certex/index.py:46-49, certex.cu:58-62)."""
    L = m + 5
    return 64 if L <= 64 else 128 * ((L + 127) // 128)


def _as_tensor(x):
    """(tensor, restore): a torch view of a numpy array, torch tensor or DLPack-capable array, and
    a function that returns a result tensor in the caller's array family (numpy arrays come back
    as numpy on the host, torch as torch, other DLPack producers through their module's
    from_dlpack when it has one). Reference interface: certex/index.py:54-84."""
    if isinstance(x, torch.Tensor):
        return x, lambda t: t
    if isinstance(x, np.ndarray) or not hasattr(x, "__dlpack__"):
        return torch.from_numpy(np.ascontiguousarray(np.asarray(x))), lambda t: t.cpu().numpy()
    family = type(x).__module__.partition(".")[0]

    def restore(t):
        import importlib

        try:
            return importlib.import_module(family).from_dlpack(t)
        except (ImportError, AttributeError, TypeError):
            return t

    return torch.from_dlpack(x), restore


def _to_torch(x):
    """The tensor of _as_tensor alone."""
    return _as_tensor(x)[0]


def _require(ok, message):
    """Reject a call with a ValueError (certex/index.py:66-69)."""
    if not ok:
        raise ValueError(message)


def _cast(t, dtype):
    """t in the index's vector type. An integer index takes only values that its type holds
    exactly; anything else (fractions, out-of-range values) is a ValueError, as in the reference
    (certex/index.py:87-96, tests/test_exact.py:342-350)."""
    if t.dtype == dtype:
        return t
    if dtype.is_floating_point:
        return t.to(dtype)
    info = torch.iinfo(dtype)
    y = t.to(dtype)
    exact = t.numel() == 0 or (
        bool(torch.equal(y.to(torch.float64), t.to(torch.float64)))
        and float(t.min()) >= info.min
        and float(t.max()) <= info.max
    )
    _require(exact, f"the index holds {dtype} vectors: values must be integers in [{info.min}, {info.max}]")
    return y


_BIT_WEIGHTS = {}


def _pack(mask):
    """A boolean mask, flattened row-major, as 32-bit filter words on the mask's device: entry e is
    bit e % 32 of word e // 32 (the reference's layout, certex/index.py:99-104). Eight entries
    become one byte by a weighted sum, and four consecutive bytes are read as one little-endian
    word; the returned words are int32."""
    flat = mask.reshape(-1).to(torch.uint8)
    flat = torch.nn.functional.pad(flat, (0, (-flat.numel()) % 32))
    w = _BIT_WEIGHTS.get(flat.device)
    if w is None:
        w = _BIT_WEIGHTS[flat.device] = torch.tensor([1 << b for b in range(8)], dtype=torch.int32, device=flat.device)
    octets = (flat.view(-1, 8).to(torch.int32) * w).sum(1).to(torch.uint8)
    return octets.contiguous().view(torch.int32)


def auto_width(X, metric, target=0.95, sample=200_000):
    """The screening width the reference's rule picks (certex/index.py:107-121): the smallest
    m = L - 5 over the tile lengths L = 64, 128, 256, 384, ... whose m leading principal directions
    hold `target` of the variance (of the centred rows; raw rows for inner products), capped at the
    dimension. Here the sample is every (n / sample)-th row, and the spectrum comes from the
    singular values of the sample in float64."""
    X = _to_torch(X)
    n, d = X.shape
    S = X[:: max(1, -(-n // sample))].to(torch.float64)
    if metric != "ip":
        S = S - S.mean(0, keepdim=True)
    var = torch.linalg.svdvals(S).square()
    held = torch.cumsum(var, 0) / var.sum().clamp_min(1e-300)
    # directions needed: the first count whose share reaches the target (1-based)
    need = int(torch.searchsorted(held, torch.tensor([target], dtype=held.dtype), right=False)[0]) + 1
    L = 64
    while L - 5 < min(need, d):
        L = 128 if L == 64 else L + 128
    return min(L - 5, d)


def trim_pool():
    """Free the scratch memory that the calling thread's searches on the current device have grown
    (certex/index.py:165-169, which returns the unused memory of the device's stream-ordered pool
    to the driver), after waiting for the thread's current stream; later searches grow it again."""
    C.check(C.lib().cuvsCertexTrimPool(C.resources()))


class search_stats:
    """Counters of the searches of the calling thread inside the block: queries, certified
    survivors and verified exact distances (certex/index.py:171-188).

        with certex.search_stats() as st:
            index.search(q)
        st.survivors / st.queries
    """

    def __enter__(self):
        C.check(C.lib().cuvsCertexStatsBegin())
        self.queries = self.survivors = self.verified = 0
        return self

    def __exit__(self, *exc):
        torch.cuda.current_stream().synchronize()
        q, s, v = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        C.check(C.lib().cuvsCertexStatsEnd(ctypes.byref(q), ctypes.byref(s), ctypes.byref(v)))
        self.queries, self.survivors, self.verified = q.value, s.value, v.value
        return False


class _Core:
    """One cuvsCertexIndex handle."""

    def __init__(self):
        self.h = ctypes.POINTER(C.IndexHandle)()
        C.check(C.lib().cuvsCertexIndexCreate(ctypes.byref(self.h)))

    def __del__(self):
        try:
            if self.h:
                C.lib().cuvsCertexIndexDestroy(self.h)
                self.h = None
        except Exception:  # interpreter shutdown
            pass

    def _get(self, fn, ctype):
        v = ctype()
        C.check(getattr(C.lib(), fn)(self.h, ctypes.byref(v)))
        return v.value

    @property
    def size(self):
        return self._get("cuvsCertexIndexGetSize", ctypes.c_int64)

    @property
    def dim(self):
        return self._get("cuvsCertexIndexGetDim", ctypes.c_int64)

    @property
    def n_removed(self):
        return self._get("cuvsCertexIndexGetRemoved", ctypes.c_int64)

    @property
    def capacity(self):
        return self._get("cuvsCertexIndexGetCapacity", ctypes.c_int64)

    @property
    def width(self):
        return self._get("cuvsCertexIndexGetWidth", ctypes.c_int32)

    @property
    def metric(self):
        return _METRIC_PY[self._get("cuvsCertexIndexGetMetric", ctypes.c_int)]

    @property
    def anchor_stride(self):
        return self._get("cuvsCertexIndexGetAnchorStride", ctypes.c_int32)

    @property
    def has_labels(self):
        return self._get("cuvsCertexIndexHasLabels", ctypes.c_bool)

    @property
    def host_vectors(self):
        return self._get("cuvsCertexIndexGetHostVectors", ctypes.c_bool)

    @property
    def n_partitioned(self):
        return self._get("cuvsCertexIndexGetPartitioned", ctypes.c_int64)

    @property
    def lists(self):
        """(number of k-means lists, vectors they cover)."""
        n, m = ctypes.c_int32(), ctypes.c_int64()
        C.check(C.lib().cuvsCertexIndexGetLists(self.h, ctypes.byref(n), ctypes.byref(m)))
        return n.value, m.value

    @property
    def dtype(self):
        d = self.h.contents.dtype
        return {
            (C.kDLFloat, 32): "float32",
            (C.kDLFloat, 16): "float16",
            (C.kDLBfloat, 16): "bfloat16",
            (C.kDLInt, 8): "int8",
            (C.kDLUInt, 8): "uint8",
        }[(d.code, d.bits)]


class Index:
    """Exact k-NN index: every search returns the exact k nearest stored vectors of every query,
    ranked by the fp64 score and, on equal scores, by the lower id (certex/index.py:191-216).

    metric: "l2" (squared Euclidean distances, ascending), "ip" (inner products, descending) or
    "cosine" (cosine similarities, descending). width, storage, capacity, anchor_stride,
    partition_labels, n_lists, local_projections and int8_rows have the reference's meaning; they
    change the speed or the memory, never the results.
    """

    def __init__(
        self,
        dim,
        metric="l2",
        width="auto",
        storage="device",
        capacity=None,
        anchor_stride=16,
        partition_labels=True,
        n_lists=0,
        local_projections=False,
        int8_rows=False,
    ):
        _require(metric in METRICS, f"metric must be one of {METRICS}, not {metric!r}")
        _require(storage in ("device", "host"), f'storage must be "device" or "host", not {storage!r}')
        self.d, self.metric, self.width, self.storage = dim, metric, width, storage
        self.capacity, self.anchor_stride = capacity, anchor_stride
        self.partition_labels = partition_labels
        self.n_lists, self.local_projections, self.int8_rows = n_lists, local_projections, int8_rows
        self.core = None
        self._writer = threading.Lock()

    @property
    def ntotal(self):
        return 0 if self.core is None else int(self.core.size - self.core.n_removed)

    @property
    def dtype(self):
        return None if self.core is None else _TORCH[self.core.dtype]

    def _vectors(self, x, device):
        t, kind = _as_tensor(x)
        if t.ndim == 1:
            t = t.reshape(1, -1)
        _require(
            t.ndim == 2 and t.shape[1] == self.d,
            f"expected vectors of dimension {self.d} (a matrix (n, {self.d}) or one vector), "
            f"got shape {tuple(t.shape)}",
        )
        if device or t.is_cuda:
            t = t.cuda()
        if self.core is not None:
            t = _cast(t, self.dtype)
        elif t.dtype not in _DTYPES or (self.metric == "cosine" and not t.dtype.is_floating_point):
            t = t.float()
        return t.contiguous(), kind

    def add(self, x, labels=None):
        """Add vectors, optionally with one non-negative label each; returns their ids
        (certex/index.py:266-305)."""
        return self._add(x, labels, check_labels=True)

    def _add(self, x, labels, check_labels):
        """add(); labels the caller built itself (check_labels false) are not checked, which
        spares a read of the labels back from the GPU and the wait for the stream it needs."""
        X, kind = self._vectors(x, device=False)
        if labels is not None:
            labels = _to_torch(labels).reshape(-1).to(device="cuda", dtype=torch.int32).contiguous()
            _require(labels.shape[0] == X.shape[0], "one non-negative label per vector")
            if check_labels:
                _require(labels.numel() == 0 or int(labels.min()) >= 0, "one non-negative label per vector")
        L = C.lib()
        with self._writer:
            if self.core is not None and self.core.has_labels:
                _require(labels is not None, "this index is labeled: add labels with every addition")
            if self.core is not None and labels is not None and not self.core.has_labels:
                raise ValueError("labels must be given from the first addition on")
            res = C.resources()
            if self.core is None:
                core = _Core()
                p = ctypes.POINTER(C.IndexParams)()
                C.check(L.cuvsCertexIndexParamsCreate(ctypes.byref(p)))
                try:
                    p.contents.metric = _METRIC_C[self.metric]
                    p.contents.width = 0 if self.width == "auto" else int(self.width)
                    p.contents.anchor_stride = int(self.anchor_stride)
                    p.contents.host_vectors = self.storage == "host"
                    p.contents.n_lists = int(self.n_lists)
                    p.contents.local_projections = bool(self.local_projections)
                    p.contents.int8_rows = bool(self.int8_rows)
                    if self.capacity is not None and self.capacity > X.shape[0]:
                        C.check(L.cuvsCertexReserve(res, int(self.capacity), core.h))  # for the build
                    x = C.Borrowed(X)
                    C.check(L.cuvsCertexBuild(res, p, x.ptr, core.h))
                finally:
                    C.check(L.cuvsCertexIndexParamsDestroy(p))
                self.core = core
                n0 = 0
            else:
                n0 = self.core.size
                x = C.Borrowed(X)
                C.check(L.cuvsCertexExtend(res, x.ptr, self.core.h))
            if labels is not None:
                lb = C.Borrowed(labels)
                C.check(L.cuvsCertexSetLabels(res, lb.ptr, n0, self.core.h))
                if self.partition_labels:
                    C.check(L.cuvsCertexPartitionByLabels(res, self.core.h))
        ids = torch.arange(n0, n0 + X.shape[0])
        return kind(ids)

    def partition(self):
        """Copy the screening rows into label order now (reference index.partition_by_labels): each
        label's queries then screen only that label's rows; vectors added later go through the
        label filter until the next partition. Results do not change."""
        _require(self.core is not None and self.core.has_labels, "add labeled vectors first")
        with self._writer:
            C.check(C.lib().cuvsCertexPartitionByLabels(C.resources(), self.core.h))

    def remove(self, ids):
        """Remove vectors by id; they never appear in later results (certex/index.py:314-319)."""
        _require(self.core is not None, "add vectors first")
        t = _to_torch(ids).reshape(-1).to(device="cuda", dtype=torch.int64).contiguous()
        with self._writer:
            b = C.Borrowed(t)
            C.check(C.lib().cuvsCertexRemove(C.resources(), b.ptr, self.core.h))

    def search(self, q, k=10, batch=2048, labels=None, filter=None, anchors=128, probe_lists=2):
        """Exact k nearest neighbours of every query: (distances or similarities, ids), best first
        (certex/index.py:320-351)."""
        _require(self.core is not None, "the index is empty: add vectors first")
        single = _to_torch(q).ndim == 1
        Q, kind = self._vectors(q, device=True)
        nq = Q.shape[0]
        _require(1 <= k <= 2048, f"k must be between 1 and 2048, not {k}")
        _require(k <= self.core.size, f"k = {k} exceeds the {int(self.core.size)} vectors added to the index")
        I = torch.empty((nq, k), dtype=torch.int64, device="cuda")
        D = torch.empty((nq, k), dtype=torch.float32, device="cuda")
        ql = words = None
        ftype = C.NO_FILTER
        if labels is not None:
            _require(self.core.has_labels, "the index has no labels")
            # labels on the GPU stay there; labels from the host stay in host memory, where the
            # search plans its label routing without reading them back from the GPU
            ql = _to_torch(labels).reshape(-1)
            ql = ql.to(dtype=torch.int32).contiguous()
            _require(ql.shape[0] == nq, "one label per query")
        if filter is not None:
            m = _to_torch(filter).to(torch.bool)
            _require(m.shape[-1] == self.core.size, "the filter needs one entry per id")
            _require(m.ndim == 1 or (m.ndim == 2 and m.shape[0] == nq), "a mask over the ids, or one row per query")
            words = _pack(m.cuda())
            ftype = C.BITSET if m.ndim == 1 else C.BITMAP
        if nq > 0:
            L = C.lib()
            sp = C.SearchParams(int(anchors), int(batch), int(probe_lists))
            qb, ib, db = C.Borrowed(Q), C.Borrowed(I), C.Borrowed(D)
            res = C.resources()
            if ql is not None:
                lb = C.Borrowed(ql)
                C.check(L.cuvsCertexSearchWithLabels(res, ctypes.byref(sp), self.core.h, qb.ptr, lb.ptr, ib.ptr, db.ptr))
            else:
                wb = None
                f = C.Filter(0, C.NO_FILTER)
                if words is not None:
                    wb = C.Borrowed(words, dtype_override=(C.kDLUInt, 32))
                    f = C.Filter(ctypes.addressof(wb.m), ftype)
                C.check(L.cuvsCertexSearch(res, ctypes.byref(sp), self.core.h, qb.ptr, ib.ptr, db.ptr, f))
                del wb
        if self.metric == "cosine":
            D = 1 - D
        if single:
            D, I = D[0], I[0]
        return kind(D), kind(I)

    def list_order(self):
        """The ids in the order of the stored rows of an index with lists, list by list (rows added
        after the build follow in id order); queries taken in this order share their nearest lists
        within a batch (certex/index.py:353-359). An int64 tensor on the GPU."""
        _require(self.core is not None and self.n_lists, "an index with lists")
        out = torch.empty(self.core.size, dtype=torch.int32, device="cuda")
        b = C.Borrowed(out)
        C.check(C.lib().cuvsCertexIndexListOrder(C.resources(), self.core.h, b.ptr))
        torch.cuda.current_stream().synchronize()
        return out.long()

    def save(self, path):
        """Write the index to a file; load() restores it without rebuilding (certex/index.py:361-365)."""
        _require(self.core is not None, "add vectors first")
        C.check(C.lib().cuvsCertexSerialize(C.resources(), str(path).encode(), self.core.h))

    @classmethod
    def load(cls, path):
        """An index saved by save() (certex/index.py:367-385)."""
        with open(path, "rb") as f:
            prefix = f.read(4)
        _require(prefix[1:3] in _PREFIX, "not a certex index file")
        core = _Core()
        C.check(C.lib().cuvsCertexDeserialize(C.resources(), str(path).encode(), core.h))
        idx = cls(core.dim, metric=core.metric, anchor_stride=core.anchor_stride, n_lists=core.lists[0],
                  storage="host" if core.host_vectors else "device")
        idx.core = core
        return idx

    def info(self):
        c = self.core
        return {
            "metric": self.metric,
            "width": None if c is None else c.width,
            "dtype": None if c is None else c.dtype,
            "storage": self.storage,
            "ntotal": self.ntotal,
            "n_lists": 0 if c is None else c.lists[0],
        }


def search(xb, xq=None, k=10, metric="l2", **index_options):
    """The exact k nearest neighbours in one call (certex/index.py:422-447)."""
    X = _to_torch(xb)
    _require(X.ndim == 2, "xb must be a matrix (n, dim)")
    index_options.setdefault("storage", "device")
    index = Index(dim=X.shape[1], metric=metric, **index_options)
    index.add(X)
    D, I = index.search(xb if xq is None else xq, k=k)
    del index
    return D, I


def _exact_scores(X, Q, dev, metric, rows_per_chunk):
    """Exact float64 scores (smaller is better: l2 sum (q - x)^2, ip -<q, x>, cosine -cos) of every
    query of Q against every row of X, yielded chunk by chunk of rows as (first row, scores)."""
    for r0 in range(0, X.shape[0], rows_per_chunk):
        R = X[r0 : r0 + rows_per_chunk].to(dev, torch.float64)
        if metric == "l2":
            s = (Q[:, None, :] - R[None]).square().sum(-1)
        else:
            if metric == "cosine":
                R = R / torch.linalg.vector_norm(R, dim=1, keepdim=True)
            s = -(Q @ R.T)
        yield r0, s


def verify(xb, xq, I, metric="l2", sample=100, seed=0):
    """Fraction of checked queries whose returned neighbours have exactly the k best float64 scores
    (the reference's semantics, certex/index.py:450-548): queries are sampled at random (torch CPU
    generator seeded with `seed`; all when sample is None), and ties count as exact whichever tied
    vector was returned.

    The check is a counting certificate rather than a second search. Let r_1 <= ... <= r_k be the
    sorted exact scores of a query's k returned (distinct) ids. Those ids are the k best, up to the
    tolerance t = 1e-9 max|r|, iff for every rank i fewer than i rows score below r_i - t. One pass
    over the rows scores them exactly and, per query, histograms how many of the k bounds each score
    falls under; a cumulative sum gives the counts. Runs on the GPU when one is present."""
    _require(metric in METRICS, f"metric must be one of {METRICS}, not {metric!r}")
    X, Q, ids = _to_torch(xb), _to_torch(xq), _to_torch(I)
    if Q.ndim == 1:
        Q, ids = Q.reshape(1, -1), ids.reshape(1, -1)
    _require(X.ndim == 2 and Q.ndim == 2 and Q.shape[1] == X.shape[1], "xb and xq need the same dimension")
    _require(ids.shape[0] == Q.shape[0], "one row of ids per query")
    dev = torch.device("cuda" if torch.cuda.is_available() else "cpu")
    nq, k = ids.shape
    if sample is None or sample >= nq:
        chosen = torch.arange(nq)
    else:
        chosen = torch.randperm(nq, generator=torch.Generator().manual_seed(seed))[:sample]
    Qs = Q[chosen.to(Q.device)].to(dev, torch.float64)
    got = ids[chosen.to(ids.device)].to(dev, torch.int64)
    if metric == "cosine":
        Qs = Qs / torch.linalg.vector_norm(Qs, dim=1, keepdim=True)
    ns, n = Qs.shape[0], X.shape[0]
    # the returned ids must be k distinct valid rows
    ok = ((got >= 0) & (got < n)).all(1)
    srt = got.sort(1).values
    ok &= (srt[:, 1:] != srt[:, :-1]).all(1)
    # exact scores of the returned rows, sorted: the bounds r_i
    rows = X[got.clamp(0, n - 1).reshape(-1).to(X.device)].to(dev, torch.float64).reshape(ns, k, -1)
    if metric == "l2":
        r = (Qs[:, None, :] - rows).square().sum(-1)
    else:
        if metric == "cosine":
            rows = rows / torch.linalg.vector_norm(rows, dim=-1, keepdim=True)
        r = -(rows * Qs[:, None, :]).sum(-1)
    r = r.sort(1).values
    bound = (r - 1e-9 * r.abs().amax(1, keepdim=True).clamp_min(1e-30)).contiguous()
    # under[q, j] = rows of query q whose score lies below exactly the bounds j, j + 1, ..., k - 1
    under = torch.zeros((ns, k + 1), dtype=torch.int64, device=dev)
    per_chunk = max(1, (1 << 26) // max(1, ns * X.shape[1]))
    for _, s in _exact_scores(X, Qs, dev, metric, per_chunk):
        first = torch.searchsorted(bound, s.contiguous(), right=True)  # bounds <= the score
        under.scatter_add_(1, first, torch.ones_like(first))
    below = torch.cumsum(under, 1)[:, :k]  # below[:, i] = rows scoring under bound i
    ok &= (below <= torch.arange(k, device=dev)).all(1)
    return float(ok.double().mean())
