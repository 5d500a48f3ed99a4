"""Seeded synthetic inputs of the configurations, shared by the tests and the bench."""

import numpy as np


def gaussian(n, d, seed, dtype=np.float32):
    """i.i.d. N(0, 1) rows (config 1 shape: 100,000 x 128 fp32, seeds 11 / 12)."""
    return np.random.default_rng(seed).standard_normal((n, d)).astype(dtype)


def mixture_u8(n, d=128, n_centres=1000, seed=2, centre_seed=1, sigma=20.0, hi=80.0):
    """Descriptor-like uint8 rows (config 2): a centre drawn uniformly from n_centres centres
    U[0, hi]^d, plus N(0, sigma^2) per coordinate, rounded half-to-even and clipped to [0, 255]."""
    centres = np.random.default_rng(centre_seed).uniform(0.0, hi, (n_centres, d))
    rng = np.random.default_rng(seed)
    out = np.empty((n, d), np.uint8)
    step = 1 << 16
    for i in range(0, n, step):
        m = min(step, n - i)
        c = rng.integers(0, n_centres, m)
        v = centres[c] + rng.standard_normal((m, d)) * sigma
        out[i : i + m] = np.clip(np.rint(v), 0, 255).astype(np.uint8)
    return out


def uniform_int(n, d, seed, dtype=np.uint8, lo=None, hi=None):
    info = np.iinfo(dtype)
    lo = info.min if lo is None else lo
    hi = info.max if hi is None else hi
    return np.random.default_rng(seed).integers(lo, hi + 1, (n, d)).astype(dtype)


def powerlaw_unit(n, d, seed, basis_seed=31, dtype=np.float32, chunk=1 << 15):
    """Embedding-like rows (config 3): Gaussian with covariance eigenvalues lambda_i ~ 1 / i
    (i = 1..d) in a random orthogonal basis (seeded by basis_seed), then L2-normalised."""
    q, _ = np.linalg.qr(np.random.default_rng(basis_seed).standard_normal((d, d)))
    m = (np.sqrt(1.0 / np.arange(1, d + 1))[:, None] * q.T).astype(np.float32)
    rng = np.random.default_rng(seed)
    out = np.empty((n, d), dtype)
    for i in range(0, n, chunk):
        r = min(chunk, n - i)
        x = rng.standard_normal((r, d), dtype=np.float32) @ m
        out[i : i + r] = (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(dtype)
    return out


def labels(n, n_classes, seed):
    """uint32-valued labels uniform over n_classes (stored as int32, as the index takes them)."""
    return np.random.default_rng(seed).integers(0, n_classes, n).astype(np.int32)


def mixture_u8_cuda(n, d=128, n_centres=1000, seed=2, centre_seed=1, sigma=20.0, hi=80.0, chunk=1 << 22):
    """The config 2 / config 5 generator on the GPU (torch generators): for large n. Centres come
    from a CPU generator seeded centre_seed, rows from a CUDA generator seeded seed."""
    import torch

    centres = (torch.rand((n_centres, d), generator=torch.Generator().manual_seed(centre_seed), dtype=torch.float64) * hi)
    centres = centres.float().cuda()
    g = torch.Generator(device="cuda").manual_seed(seed)
    out = torch.empty((n, d), dtype=torch.uint8, device="cuda")
    for i in range(0, n, chunk):
        m = min(chunk, n - i)
        c = torch.randint(0, n_centres, (m,), generator=g, device="cuda")
        v = centres[c] + torch.randn((m, d), generator=g, device="cuda") * sigma
        out[i : i + m] = v.round().clamp_(0, 255).to(torch.uint8)
    return out
