"""Shared test helpers: seeded data and oracle-built graphs."""

from __future__ import annotations

import numpy as np

from jasper_amd import datasets


def gaussian(n, dim, seed):
    return datasets.gaussian(n, dim, seed)


def integer_clustered(n, dim, seed, n_clusters=20):
    return datasets.clustered(n, dim, seed, n_clusters=n_clusters)


def unit(n, dim, seed):
    return datasets.unit_sphere(n, dim, seed)


def hub_mix(n, dim, seed, shell_frac=0.7, spread=0.3, scale=8.0, integer=False):
    """Rows where one vertex is a hub: about shell_frac of the rows lie on a
    thin shell (radius 1 .. 1 + spread) around row 0 = the origin, the rest
    in a Gaussian blob away from it; times `scale`, rounded to integers when
    asked, fp16. In high dim the shell's rows are farther from each other
    than from the hub, so nearly every shell row links to row 0 and, in one
    batch of the build, row 0 receives more than 256 + R reverse
    candidates."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, dim)).astype(np.float32)
    shell = rng.random(n) < shell_frac
    shell[0] = True
    d = x[shell] / np.linalg.norm(x[shell], axis=1, keepdims=True)
    x[shell] = d * rng.uniform(1.0, 1.0 + spread, size=(int(shell.sum()), 1))
    x[~shell] = x[~shell] * 0.5 + 4.0
    x[0] = 0.0
    x *= scale
    if integer:
        x = np.round(x)
    return x.astype(np.float16)


def compare_search(gpu_ids, gpu_d, ref_ids, ref_d):
    """Bit-exact comparison; returns a short diagnostic on mismatch."""
    gi = np.asarray(gpu_ids)
    gd = np.asarray(gpu_d)
    bad = np.nonzero((gi != ref_ids).any(axis=1) | (gd.view(np.uint32) != ref_d.view(np.uint32)).any(axis=1))[0]
    if len(bad) == 0:
        return None
    q = bad[0]
    return (f"{len(bad)} of {len(gi)} queries differ; first q={q}\n gpu ids {gi[q].tolist()}\n ref ids "
            f"{ref_ids[q].tolist()}\n gpu d {gd[q].tolist()}\n ref d {ref_d[q].tolist()}")
