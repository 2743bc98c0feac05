"""How well the one-bit RaBitQ estimate ranks a row's nearest neighbours:
the evidence behind the RaBitQ-estimated build's recall at narrow beams.

Test infrastructure, like the rest of this package: it runs on the host
with the oracle's RaBitQ quantizer (`rabitq_quantize`, the one-bit closed
form of rabitq/quantize.cuh:144-276) and estimator (`rq_estimates`, the
published RaBitQ estimator over the quantizer's factors).

The construction's search stage with `build_search="rabitq"` ranks the
beam by this estimate, with the inserted row as the query. This script
takes the rows as that build stores them: the clustered integer mixture of
`jasper_amd.datasets.clustered`, prerotated with the seed-42 rotation, and
coded against their mean. For a sample of rows it compares the exact L2
distances to every other row with the estimates, and reports:

- how many of the 10 true nearest rows rank within the estimate's top 64
  (the build's beam) and top 256;
- the median estimate rank of those 10;
- the estimate's median relative error over the 1,000 nearest rows;
- the spread of exact distances: d_10 / d_1 - 1 and d_100 / d_1 - 1.

Usage: python3 -m oracle.rabitq_build_study N CLUSTERS [SAMPLES]
(one JSON line; about 4 minutes for N = 1,000,000 and 200 samples).
"""

import json
import sys

import numpy as np

import oracle
from jasper_amd import datasets


def study(n: int, n_clusters: int, samples: int = 200, seed: int = 3) -> dict:
    dim = 128
    x16 = datasets.clustered(n, dim, 0, n_clusters=n_clusters)
    P, _ = oracle.rotation_matrix(dim, 42)
    xr16 = oracle.rotate_rows(x16.view(np.uint16), dim, P.astype(np.float16).view(np.uint16))
    xr = xr16.view(np.float16)[:, :dim].astype(np.float32)
    cent = xr.mean(axis=0, dtype=np.float64).astype(np.float32)
    identity = np.eye(dim, dtype=np.float32).ravel(order="F")  # the rows are already rotated
    nodes, _, _, _ = oracle.rabitq_quantize(xr, identity, cent, "l2")
    rq = oracle.RqArtifacts(dim, nodes, cent)
    x64 = xr.astype(np.float64)
    norms = (x64 ** 2).sum(1)
    rng = np.random.default_rng(seed)
    in64, in256, med_rank, rel_err, gap10, gap100 = [], [], [], [], [], []
    for s in rng.choice(n, samples, replace=False):
        q = x64[s]
        exact = norms - 2.0 * (x64 @ q) + float(q @ q)
        exact[s] = np.inf
        est = oracle.rq_estimates(rq, xr16[s:s + 1], "l2")[0].astype(np.float64)
        est[s] = np.inf
        order = np.argsort(exact, kind="stable")
        rank = np.empty(n, dtype=np.int64)
        rank[np.argsort(est, kind="stable")] = np.arange(n)
        r10 = rank[order[:10]]
        in64.append(np.mean(r10 < 64))
        in256.append(np.mean(r10 < 256))
        med_rank.append(np.median(r10))
        near = order[:1000]
        rel_err.append(np.median(np.abs(est[near] - exact[near]) / exact[near]))
        gap10.append(exact[order[9]] / exact[order[0]] - 1.0)
        gap100.append(exact[order[99]] / exact[order[0]] - 1.0)
    return {"n": n, "clusters": n_clusters, "samples": samples,
            "top10_in_est_top64": float(np.mean(in64)), "top10_in_est_top256": float(np.mean(in256)),
            "median_est_rank_of_top10": float(np.median(med_rank)),
            "est_rel_error_median_top1000": float(np.median(rel_err)),
            "d10_over_d1_minus1": float(np.median(gap10)), "d100_over_d1_minus1": float(np.median(gap100))}


if __name__ == "__main__":
    args = [int(a) for a in sys.argv[1:]]
    print(json.dumps(study(*args)), flush=True)
