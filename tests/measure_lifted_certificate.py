"""Measurement, not a test (pytest does not collect it): survivors per query of the reference's
lifted PCA certificate against this build's full-row certificate, at config 3 (1,000,000 x 768
power-law unit vectors, cosine, 16 labels, k = 100), on the CPU.

    python tests/measure_lifted_certificate.py [n_queries]     # about 2 minutes at 400 queries

The reference lifts a vector to m principal coordinates z and the residual norm r
(cpp/src/neighbors/certex/detail/certex_kernels.cuh:66-112) and screens the lower bound
|q - x|^2 >= a_q + a_x - 2 (<z_q, z_x> + r_q r_x) (Cauchy-Schwarz on the residuals); m comes from
its width rule (certex.cu:418-438, variance 0.95). Both certificates get the same threshold U, the
k-th best fine group of 4 anchors every 16 rows of the query's label, scored exactly; fp16
rounding is left out on both sides (it only widens the bounds, the lifted one more).
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
print(f"data {time.time()-t0:.1f}s", flush=True)

# PCA of the (unit, centred) vectors, as fit_projection (certex.cu:354-446): all rows (pca_sample 1M)
c = X.mean(0, dtype=np.float64)
cov = np.zeros((d, d))
for i in range(0, n, 100_000):
    y = X[i:i+100_000].astype(np.float64) - c
    cov += y.T @ y
vals, vecs = np.linalg.eigh(cov)
vals, vecs = vals[::-1], vecs[:, ::-1]
frac = np.cumsum(np.maximum(vals, 0)) / np.maximum(vals, 0).sum()
m = d
L = 64
while L <= 4096:
    cand = L - 5
    if cand >= d or frac[cand - 1] >= 0.95:
        m = min(cand, d)
        break
    L = L + 64 if L < 128 else L + 128
row_len = m + 5
row_len = 64 if row_len <= 64 else (128 if row_len <= 128 else (row_len + 127) // 128 * 128)
print(f"PCA {time.time()-t0:.1f}s: width m = {m} (variance {frac[m-1]:.4f}), row length {row_len} halves "
      f"(full rows: {d} halves)", flush=True)
V = vecs[:, :m].astype(np.float32)  # d x m

def lift(A):
    p = A.astype(np.float32) - c.astype(np.float32)
    z = p @ V
    pp = (p.astype(np.float64) ** 2).sum(1)
    zz = (z.astype(np.float64) ** 2).sum(1)
    r = np.sqrt(np.maximum(pp - zz, 0))
    return z, r, pp

zq, rq, aq = lift(Q)
order = np.argsort(lx, kind="stable")
starts = np.searchsorted(lx[order], np.arange(L_labels + 1))
full_s, lift_s, full_v, lift_v = [], [], [], []
for lab in range(L_labels):
    qs = np.nonzero(lq == lab)[0]
    if len(qs) == 0:
        continue
    rows = order[starts[lab]:starts[lab + 1]]
    Xl = X[rows]
    zx, rx, ax = lift(Xl)
    dist = 2.0 - 2.0 * (Q[qs].astype(np.float64) @ Xl.T.astype(np.float64))  # exact l2 of unit vectors
    lb = aq[qs, None] + ax[None, :] - 2.0 * (zq[qs].astype(np.float64) @ zx.T.astype(np.float64) + rq[qs, None] * rx[None, :])
    # U: the k-th best fine group (4 consecutive anchors, every 16th row of the label's partition)
    an = np.arange(0, len(rows), stride)
    ad = dist[:, an]
    g = len(an) // 4 * 4
    grp = ad[:, :g].reshape(len(qs), -1, 4).min(2)
    if len(an) > g:
        grp = np.concatenate([grp, ad[:, g:].min(1, keepdims=True)], 1)
    U = np.sort(grp, 1)[:, k - 1]
    dk = np.sort(dist, 1)[:, k - 1]  # the true k-th score
    full_s += list((dist <= U[:, None]).sum(1))
    lift_s += list((lb <= U[:, None]).sum(1))
    full_v += list((dist <= dk[:, None]).sum(1))
    lift_v += list((lb <= dk[:, None]).sum(1))
    print(f"label {lab}: {len(qs)} queries, {len(rows)} rows, U/dk {np.mean(U/dk):.4f}", flush=True)
print(f"done {time.time()-t0:.1f}s")
print(f"survivors per query (bound <= U): full rows {np.mean(full_s):.1f}, lifted m={m} {np.mean(lift_s):.1f} "
      f"(x{np.mean(lift_s)/np.mean(full_s):.2f})")
print(f"rows an ordered verification must score (bound <= true k-th score): full {np.mean(full_v):.1f}, "
      f"lifted {np.mean(lift_v):.1f}")
print(f"median survivors: full {np.median(full_s):.0f}, lifted {np.median(lift_s):.0f}; max: full {np.max(full_s)}, lifted {np.max(lift_s)}")
