"""Measurement, not a test (pytest does not collect it): survivors per query of the reference's
int8 certificate for float vectors (index_params::int8_rows) against this build's full-row fp16
certificate, at config 3 (1,000,000 x 768 power-law unit vectors, cosine, 16 labels, k = 100), on
the CPU.

    python tests/measure_int8_certificate.py [n_queries]     # about 2 minutes at 200 queries

The reference codes each screening vector z as int8 with one scale per vector, z = s (c + e) with
s = max |z_j| / 127 and |e_j| <= 1/2 (cpp/src/neighbors/certex/detail/int8.cuh:30-77), and bounds
<z_q, z_x> <= s_q s_x (<c_q, c_x> + |e_x| (|c_q| + |e_q|) + |e_q| |c_x|) by Cauchy-Schwarz
(int8.cuh:11-19), so that |q - x|^2 >= a_q + a_x - 2 (that bound). Here z is the full-dimension
vector (no PCA, as this build screens), centred like the fp16 rows. Both certificates get the same
threshold U, the k-th best fine group of 4 anchors every 16 rows of the query's label, scored
exactly; the fp32 epilogue margin of the int8 pass (int8.cuh:18-20) and the fp16 rounding of the
full-row rows are left out (each only widens its bound).
"""

import os
import sys
import time

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from tests import data  # noqa: E402

n, d, nq, k, L_labels, stride = 1_000_000, 768, int(sys.argv[1]) if len(sys.argv) > 1 else 200, 100, 16, 16
t0 = time.time()
X = data.powerlaw_unit(n, d, seed=32)
Q = data.powerlaw_unit(nq, d, seed=33)
lx = data.labels(n, L_labels, 34)
lq = data.labels(nq, L_labels, 35)
c = X.mean(0, dtype=np.float64)
print(f"data {time.time()-t0:.1f}s", flush=True)


def int8_code(Z):
    """Codes c, the scale s and |e|, |c| of every row of Z (fp64), the reference's rule."""
    s = np.maximum(np.abs(Z).max(1), 1e-30) / 127.0
    v = Z / s[:, None]
    cq = np.clip(np.rint(v), -127, 127)
    return cq, s, np.sqrt(((v - cq) ** 2).sum(1)), np.sqrt((cq ** 2).sum(1))


Zq = Q.astype(np.float64) - c
aq = (Zq ** 2).sum(1)
Cq, sq, eq, cnq = int8_code(Zq)
order = np.argsort(lx, kind="stable")
starts = np.searchsorted(lx[order], np.arange(L_labels + 1))
full_s, int8_s = [], []
for lab in range(L_labels):
    qs = np.nonzero(lq == lab)[0]
    if len(qs) == 0:
        continue
    rows = order[starts[lab]:starts[lab + 1]]
    Zx = X[rows].astype(np.float64) - c
    ax = (Zx ** 2).sum(1)
    Cx, sx, ex, cnx = int8_code(Zx)
    dist = aq[qs, None] + ax[None, :] - 2.0 * (Zq[qs] @ Zx.T)  # exact squared distance
    acc = Cq[qs] @ Cx.T  # exact: integers below 2^53
    ub = (sq[qs, None] * sx[None, :]) * (acc + ex[None, :] * (cnq[qs, None] + eq[qs, None])
                                         + eq[qs, None] * cnx[None, :])
    lb = aq[qs, None] + ax[None, :] - 2.0 * ub
    # U: the k-th best fine group (4 consecutive anchors, every 16th row of the label's partition)
    an = np.arange(0, len(rows), stride)
    ad = dist[:, an]
    g = len(an) // 4 * 4
    grp = ad[:, :g].reshape(len(qs), -1, 4).min(2)
    if len(an) > g:
        grp = np.concatenate([grp, ad[:, g:].min(1, keepdims=True)], 1)
    U = np.sort(grp, 1)[:, k - 1]
    full_s += list((dist <= U[:, None]).sum(1))
    int8_s += list((lb <= U[:, None]).sum(1))
    print(f"label {lab}: {len(qs)} queries, {len(rows)} rows", flush=True)
print(f"done {time.time()-t0:.1f}s")
print(f"survivors per query (bound <= U): full rows {np.mean(full_s):.1f}, int8 codes {np.mean(int8_s):.1f} "
      f"(x{np.mean(int8_s) / np.mean(full_s):.2f}); median {np.median(full_s):.0f} / {np.median(int8_s):.0f}; "
      f"max {np.max(full_s)} / {np.max(int8_s)}")
