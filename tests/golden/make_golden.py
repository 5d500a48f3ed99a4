"""Write the small golden fixtures of this directory from the CPU oracle (oracle/oracle.c).

    python tests/golden/make_golden.py

Each fixture holds its inputs (base, queries, k, metric) and the oracle's exact answer (fp64
scores and ids in (score, id) order). They are C1- and C2-shaped at small sizes, plus a case with
many exactly tied distances, so that a GPU path and later oracle changes are checked against
fixed data.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from tests import data  # noqa: E402

CASES = {
    "c1_f32_l2": lambda: (data.gaussian(1000, 128, 11), data.gaussian(16, 128, 12), 10, "l2"),
    "c2_u8_l2": lambda: (data.mixture_u8(3000, seed=2), data.mixture_u8(16, seed=3), 10, "l2"),
    "u8_ties_l2": lambda: (
        data.uniform_int(2500, 16, seed=21, lo=0, hi=2),
        data.uniform_int(8, 16, seed=22, lo=0, hi=2),
        40,
        "l2",
    ),
    "i8_ip": lambda: (
        data.uniform_int(2000, 64, seed=31, dtype=np.int8),
        data.uniform_int(8, 64, seed=32, dtype=np.int8),
        12,
        "ip",
    ),
}


def main():
    for name, make in CASES.items():
        base, queries, k, metric = make()
        s, i = oracle.knn(base, queries, k, metric)
        np.savez_compressed(
            os.path.join(HERE, name + ".npz"), base=base, queries=queries, k=k, metric=metric, scores=s, ids=i
        )
        print("wrote", name, base.shape, queries.shape, k, metric)


if __name__ == "__main__":
    main()
