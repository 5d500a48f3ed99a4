"""Exact sparse-attention top-k over a growing KV cache (reference certex/attention.py:1-114).

KeyCache keeps one inner-product index per KV head; query head h reads KV head h // (n_heads /
n_kv_heads). topk(q, keys, k) equals torch.topk(q @ keys.mT, k, dim=-1) with exact fp64 scores and,
on equal scores, the lower key id first.
"""

import torch

from .index import Index, _require

def _stride(n, k):
    """An anchor stride between 1 and 16 (the reference picks one from n and k,
    certex/attention.py:30-34): here it leaves about 8k groups of 4 anchors, so that the k-th best
    group stays close to the k-th best key while the anchor pass reads a fraction of the keys
    (at config 4, 131,072 keys and k = 2,048: stride 2, measured against 4 and 1: 851k, 776k and
    793k queries/s)."""
    s = n // (32 * k)
    return int(max(1, min(16, s)))


def _keys(x):
    """Keys or queries on the GPU as float16, or float32 when float16 would overflow
    (certex/attention.py:37-41). bfloat16 inputs stay bfloat16: the index keeps them exactly at
    2 bytes per coordinate (float16 would round bfloat16 values below its normal range), and the
    exact re-rank reads half the bytes of float32 rows."""
    x = torch.as_tensor(x, device="cuda")
    if x.dtype == torch.bfloat16:
        return x
    if x.dtype == torch.float16:
        return x  # nothing to convert (no check that would wait for the GPU)
    h = x.to(torch.float16)
    return h if bool(torch.isfinite(h).all()) else x.to(torch.float32)


def _queries(q, dtype):
    """Queries in the cache's vector type, rounded to nearest as the reference rounds them
    (certex/attention.py:97, `.to(self.dtype)`): the top k is then exact for the rounded queries.
    Queries are converted once from the type they come in (float32 queries against bfloat16 keys
    are not rounded to float16 first). A finite value that the cache's type overflows is an error."""
    x = torch.as_tensor(q, device="cuda")
    if x.dtype == dtype:
        return x
    y = x.to(dtype)
    _require(
        bool((torch.isfinite(y) | ~torch.isfinite(x)).all()),
        f"these queries overflow the cache's {dtype} keys: start the cache with float32 keys",
    )
    return y


def _fit(x, dtype, what):
    """Keys in the cache's vector type; a conversion that would change a key (float32 or bfloat16
    values that float16 rounds or overflows, float32 or float16 values that bfloat16 rounds) is an
    error rather than a silent rounding of the cache."""
    if x.dtype == dtype:
        return x
    y = x.to(dtype)
    _require(
        bool(torch.equal(y.to(x.dtype), x)),
        f"the cache holds {dtype} keys, which cannot represent these {what} exactly: "
        "start the cache with keys of this type (float32 keys give a float32 cache, which holds "
        "float16 and bfloat16 values exactly)",
    )
    return y


class KeyCache:
    """Exact top-k over the keys of a growing KV cache (attention.py:44-106).

    The reference keeps one index per KV head. Here all heads share one inner-product index whose
    keys carry their head as a label, so that one label-routed search serves every query head of
    a step (each query head screens only its KV head's keys, in one launch per phase). Keys
    appended after the label partition are screened through the label filter; the partition is
    rebuilt when they exceed a sixteenth of the cache.
    """

    def __init__(self, n_kv_heads, head_dim, k=2048, capacity=None):
        _require(n_kv_heads >= 1 and head_dim >= 1, "n_kv_heads and head_dim must be positive")
        _require(1 <= k <= 2048, f"k must be between 1 and 2048, not {k}")
        self.n_kv_heads, self.head_dim, self.k, self.capacity = int(n_kv_heads), int(head_dim), int(k), capacity
        self.index, self.dtype = None, None
        self.local = None  # key id within its head, per id of the shared index (grown in place)
        self.size = 0
        self._labels = {}  # cached label vectors: appends of n keys, and searches of (H, m)

    def append(self, keys):
        """Append keys of shape (n_kv_heads, n, head_dim); ids continue from the keys before."""
        K = _keys(keys)
        _require(
            K.ndim == 3 and K.shape[0] == self.n_kv_heads and K.shape[2] == self.head_dim,
            f"keys must have shape ({self.n_kv_heads}, n, {self.head_dim}), not {tuple(K.shape)}",
        )
        n = K.shape[1]
        if n == 0:
            return self
        if self.index is None:
            self.dtype = K.dtype
            cap = max(n, int(self.capacity or 0))
            self.index = Index(
                self.head_dim,
                metric="ip",
                # the reference narrows the screening rows below the head dimension
                # (certex/attention.py:25-27); this build screens full-dimension rows
                width="auto",
                storage="device",
                capacity=cap * self.n_kv_heads,
                anchor_stride=_stride(cap, self.k),
                partition_labels=False,
            )
        key = ("append", n)
        if key not in self._labels:
            heads = torch.arange(self.n_kv_heads, device="cuda", dtype=torch.int32)
            self._labels[key] = heads.repeat_interleave(n)
        n0 = self.n_kv_heads * self.size  # the shared index's first new id
        # the head labels are built here (non-negative): no check that would wait for the GPU
        self.index._add(
            _fit(K, self.dtype, "keys").reshape(self.n_kv_heads * n, self.head_dim).contiguous(),
            self._labels[key],
            check_labels=False,
        )
        need = n0 + self.n_kv_heads * n
        if self.local is None or self.local.shape[0] < need:
            grown = torch.empty(max(need, 2 * (0 if self.local is None else self.local.shape[0])),
                                device="cuda", dtype=torch.int64)
            if self.local is not None:
                grown[:n0] = self.local[:n0]
            self.local = grown
        self.local[n0:need].view(self.n_kv_heads, n).copy_(
            torch.arange(self.size, self.size + n, device="cuda", dtype=torch.int64))
        self.size += n
        core = self.index.core
        if (core.size - core.n_partitioned) * 16 > core.size:
            self.index.partition()
        return self

    def topk(self, q, k=None, batch=None):
        """The exact top k keys of every query: q (n_heads, m, head_dim) or (n_heads, head_dim);
        returns (scores, ids) of shape (n_heads, m, k) or (n_heads, k)."""
        _require(self.index is not None, "the cache is empty: append keys first")
        k = self.k if k is None else int(k)
        _require(1 <= k <= min(2048, self.size), f"k must be between 1 and {min(2048, self.size)}, not {k}")
        Q = _queries(q, self.dtype)
        single = Q.ndim == 2
        if single:
            Q = Q[:, None, :]
        _require(
            Q.ndim == 3 and Q.shape[2] == self.head_dim and Q.shape[0] % self.n_kv_heads == 0,
            f"queries must have shape (n_heads, m, {self.head_dim}) with n_heads a multiple of {self.n_kv_heads}",
        )
        H, m, d = Q.shape
        r = H // self.n_kv_heads
        key = ("search", H, m)
        if key not in self._labels:
            # in host memory: the label-routed search plans its launches from them without a
            # read-back from the GPU
            self._labels[key] = (torch.arange(H, dtype=torch.int32) // r).repeat_interleave(m)
        labels = self._labels[key]
        D, I = self.index.search(
            Q.reshape(H * m, d), k=k, batch=batch or max(2048, H * m), labels=labels
        )
        scores = D.reshape(H, m, k)
        ids = self.local[I].reshape(H, m, k)
        return (scores[:, 0], ids[:, 0]) if single else (scores, ids)


def topk(q, keys, k):
    """The exact top k keys of every query in one call (certex/attention.py:109-114)."""
    K = torch.as_tensor(keys)
    _require(K.ndim == 3, "keys must have shape (n_kv_heads, n, head_dim)")
    return KeyCache(K.shape[0], K.shape[2], k=k).append(K).topk(q, k)
