"""Exact GPU brute force for 8-bit vectors, the checker of the full-size tests.

For uint8 / int8 rows every squared L2 distance is an integer below 2^23 and every fp64 product
and sum of the expanded form |q|^2 + |x|^2 - 2<q, x> is exact, so the fp64 brute force equals the
oracle's exhaustive search. Ties go to the lower id: rows are ranked by the key distance * 2^30 + id,
exact in fp64 for ids below 2^30.
"""

import torch

_ID_BITS = float(1 << 30)


def topk_u8(X, Q, k, live_masks=(None,), chunk=100_000):
    """For each mask in live_masks (bool [rows] of live rows, or None for all rows of X), the exact
    (distances, ids) top k of every query of Q over the live rows: float64 [nq, k] and int64
    [nq, k]. One pass over X serves all masks; masks shorter than X leave the rows past them out."""
    Qd = Q.double()
    qq = (Qd * Qd).sum(1, keepdim=True)
    best = [torch.empty((Q.shape[0], 0), dtype=torch.float64, device=Q.device) for _ in live_masks]
    for c in range(0, X.shape[0], chunk):
        Xc = X[c : c + chunk].double()
        d = qq + (Xc * Xc).sum(1)[None] - 2.0 * (Qd @ Xc.T)
        key = d * _ID_BITS + torch.arange(c, c + Xc.shape[0], device=Q.device, dtype=torch.float64)[None]
        del d
        for j, m in enumerate(live_masks):
            kj = key
            if m is not None:
                alive = torch.zeros(Xc.shape[0], dtype=torch.bool, device=Q.device)
                if c < m.shape[0]:
                    part = m[c : c + chunk]
                    alive[: part.shape[0]] = part
                kj = key.masked_fill(~alive[None], float("inf"))
            best[j] = torch.topk(torch.cat([best[j], kj], 1), k, dim=1, largest=False).values
    out = []
    for b in best:
        out.append((torch.floor(b / _ID_BITS), torch.remainder(b, _ID_BITS).long()))
    return out
