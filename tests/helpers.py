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
