"""Seeded synthetic workloads for the benchmark configurations.

Every generator uses numpy's PCG64 seeded through ``SeedSequence`` and fills
rows in fixed 1,000,000-row chunks, each chunk drawing from its own spawned
child sequence, so any host produces identical bytes for a given seed and the
chunks can be generated independently. Values are computed in float32 and
rounded to float16 (round to nearest even) at the end.

Configurations (base / query seeds follow the benchmark definition):
  * ``gaussian``   -- i.i.d. N(0, 1)                              (config 1)
  * ``clustered``  -- mixture of isotropic Gaussians: centers U[0, 128]^d,
                      sigma 20, clipped to [0, 218], rounded to integers
                      (config 2; config 5 uses 10,000 clusters). The centers
                      are drawn from their own fixed seed, so base and queries
                      share one mixture.
  * ``unit_sphere``-- N(0, 1) rows normalised to unit L2 norm      (config 3)
  * ``sparse_abs`` -- |N(0, 1)| * 0.05 with 20% of the coordinates of every
                      row set to zero                               (config 4)
"""

from __future__ import annotations

import numpy as np

CHUNK = 1_000_000
CENTERS_SEED = 7919  # fixed seed of the cluster centres (shared by base and queries)


def _chunks(n: int, seed: int):
    ss = np.random.SeedSequence(seed)
    n_chunks = max(1, (n + CHUNK - 1) // CHUNK)
    for c, child in enumerate(ss.spawn(n_chunks)):
        lo = c * CHUNK
        hi = min(n, lo + CHUNK)
        if lo >= hi:
            break
        yield lo, hi, np.random.Generator(np.random.PCG64(child))


def gaussian(n: int, dim: int, seed: int) -> np.ndarray:
    out = np.empty((n, dim), dtype=np.float16)
    for lo, hi, rng in _chunks(n, seed):
        out[lo:hi] = rng.standard_normal((hi - lo, dim), dtype=np.float32).astype(np.float16)
    return out


def cluster_centers(n_clusters: int, dim: int, seed: int = CENTERS_SEED) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, n_clusters, dim])))
    return rng.uniform(0.0, 128.0, size=(n_clusters, dim)).astype(np.float32)


def clustered(n: int, dim: int, seed: int, n_clusters: int = 1000, sigma: float = 20.0,
              lo: float = 0.0, hi: float = 218.0) -> np.ndarray:
    centers = cluster_centers(n_clusters, dim)
    out = np.empty((n, dim), dtype=np.float16)
    for a, b, rng in _chunks(n, seed):
        lab = rng.integers(0, n_clusters, size=b - a)
        x = rng.standard_normal((b - a, dim), dtype=np.float32)
        x *= np.float32(sigma)
        x += centers[lab]
        np.clip(x, lo, hi, out=x)
        np.rint(x, out=x)
        out[a:b] = x.astype(np.float16)
    return out


def unit_sphere(n: int, dim: int, seed: int) -> np.ndarray:
    out = np.empty((n, dim), dtype=np.float16)
    for a, b, rng in _chunks(n, seed):
        x = rng.standard_normal((b - a, dim), dtype=np.float32)
        x /= np.linalg.norm(x, axis=1, keepdims=True)
        out[a:b] = x.astype(np.float16)
    return out


def sparse_abs(n: int, dim: int, seed: int, zero_frac: float = 0.2, scale: float = 0.05) -> np.ndarray:
    out = np.empty((n, dim), dtype=np.float16)
    n_zero = int(round(zero_frac * dim))
    for a, b, rng in _chunks(n, seed):
        x = np.abs(rng.standard_normal((b - a, dim), dtype=np.float32)) * np.float32(scale)
        if n_zero:
            idx = np.argsort(rng.random((b - a, dim), dtype=np.float32), axis=1)[:, :n_zero]
            np.put_along_axis(x, idx, 0.0, axis=1)
        out[a:b] = x.astype(np.float16)
    return out


def config(name: str, n: int | None = None, nq: int | None = None):
    """(base, queries, params) for a benchmark configuration name
    ('c1'..'c5'); n / nq override the row counts for reduced-size runs."""
    if name == "c1":
        n, nq = n or 10_000, nq or 100
        return gaussian(n, 128, 0), gaussian(nq, 128, 1), dict(R=32, distance="l2", alpha=1.2)
    if name == "c2":
        n, nq = n or 1_000_000, nq or 10_000
        return (clustered(n, 128, 0), clustered(nq, 128, 1),
                dict(R=64, distance="l2", alpha=1.2))
    if name == "c3":
        n, nq = n or 1_000_000, nq or 10_000
        return unit_sphere(n, 96, 0), unit_sphere(nq, 96, 1), dict(R=64, distance="ip", alpha=1.2)
    if name == "c4":
        n, nq = n or 1_000_000, nq or 1_000
        return sparse_abs(n, 960, 0), sparse_abs(nq, 960, 1), dict(R=64, distance="l2", alpha=1.2)
    if name == "c5":
        n, nq = n or 100_000_000, nq or 10_000
        return (clustered(n, 128, 0, n_clusters=10_000), clustered(nq, 128, 1, n_clusters=10_000),
                dict(R=64, distance="l2", alpha=1.2))
    raise ValueError(f"unknown config {name!r}")


def clustered_device(n: int, dim: int, seed: int, device, n_clusters: int = 10_000, sigma: float = 20.0,
                     lo: float = 0.0, hi: float = 218.0, chunk: int = 1 << 22):
    """The clustered integer mixture generated on the GPU, for sizes whose
    host generation would dominate a benchmark (config 5: 100M rows). Same
    centres as `clustered` (cluster_centers), labels and noise from torch's
    device generator seeded with `seed`, so the values differ from the host
    generator's. Returns a device fp16 tensor [n, dim]."""
    import torch
    dev = torch.device(device)
    centers = torch.from_numpy(cluster_centers(n_clusters, dim)).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    out = torch.empty((n, dim), dtype=torch.float16, device=dev)
    for a in range(0, n, chunk):
        b = min(n, a + chunk)
        lab = torch.randint(0, n_clusters, (b - a,), generator=gen, device=dev)
        x = torch.randn((b - a, dim), generator=gen, device=dev, dtype=torch.float32)
        x.mul_(sigma).add_(centers[lab]).clamp_(lo, hi).round_()
        out[a:b] = x.to(torch.float16)
        del x, lab
    return out


def sparse_abs_device(n: int, dim: int, seed: int, device, zero_frac: float = 0.2, scale: float = 0.05,
                      chunk: int = 1 << 18):
    """`sparse_abs` generated on the GPU (config 4: 1M x 960): |N(0,1)| *
    scale with round(zero_frac * dim) coordinates per row set to zero,
    chosen uniformly. Uses torch's device generator seeded with `seed`, so
    the values differ from the host generator's. Returns a device fp16
    tensor [n, dim]."""
    import torch
    dev = torch.device(device)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    n_zero = int(round(zero_frac * dim))
    out = torch.empty((n, dim), dtype=torch.float16, device=dev)
    for a in range(0, n, chunk):
        b = min(n, a + chunk)
        x = torch.randn((b - a, dim), generator=gen, device=dev, dtype=torch.float32).abs_().mul_(scale)
        if n_zero:
            idx = torch.rand((b - a, dim), generator=gen, device=dev).argsort(dim=1)[:, :n_zero]
            x.scatter_(1, idx, 0.0)
        out[a:b] = x.to(torch.float16)
        del x
    return out
