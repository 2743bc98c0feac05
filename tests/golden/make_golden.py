"""Writes the small golden fixtures of tests/golden/ (test infrastructure).

Each fixture is data only: seeded inputs and the CPU oracle's outputs for
them (graphs, search results, estimator artifacts, file byte images). They
freeze the oracle (tests/test_golden.py regenerates them and compares bit
for bit) and give the GPU tests fixed expected outputs that do not need the
oracle at run time. Regenerate with `python tests/golden/make_golden.py`
after an intended change of the oracle, and say why in the commit.
"""

from __future__ import annotations

import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle  # noqa: E402
from jasper_amd import datasets  # noqa: E402


def plain_fixture(name: str, base: np.ndarray, q: np.ndarray, R: int, distance: str, bws=(8, 24)) -> dict:
    g = oracle.build(base, R=R, distance=distance, alpha=1.2)
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "g.bin"
        oracle.save_graph(g, path)
        file_bytes = np.frombuffer(path.read_bytes(), dtype=np.uint8).copy()
    out = dict(base=base.astype(np.float16), queries=q.astype(np.float16), R=np.int64(R),
               metric=np.int64(oracle.metric_code(distance)), medoid=np.int64(g.medoid), counts=g.counts,
               edges=g.edges, edge_dist=g.edge_dist, file_bytes=file_bytes, bws=np.array(bws, dtype=np.int64))
    for bw in bws:
        ids, dists = oracle.beam_search(g, q, k=5, beam_width=bw)
        out[f"ids_bw{bw}"] = ids
        out[f"dists_bw{bw}"] = dists
    return out, g


def directional_fixture(g, q: np.ndarray) -> dict:
    lsh = oracle.build_lsh(g, K=4, pbytes=1, n_samples=500, seed=5)
    pq = oracle.build_pq(g, M=4, n_train=500, iters=3, seed=6)
    q16 = oracle.as_padded_f16(q)
    out = dict(lsh_c=lsh.c_per_rank, lsh_norm_denom=np.float32(lsh.norm_denom), lsh_rows=lsh.rows,
               pq_centroids=pq.centroids, pq_codes=pq.codes, pq_norms=pq.norms)
    for unique in (False, True):
        tag = "_unique" if unique else ""
        ids, d = oracle.directional_search(g, q16, lsh=lsh, k=5, beam_width=16, unique=unique)
        out[f"lsh_ids{tag}"], out[f"lsh_dists{tag}"] = ids, d
        ids, d = oracle.directional_search(g, q16, pq=pq, k=5, beam_width=16, unique=unique)
        out[f"pq_ids{tag}"], out[f"pq_dists{tag}"] = ids, d
    return out


def rabitq_fixture() -> dict:
    x = datasets.gaussian(16, 24, 9).astype(np.float32)
    m, _ = oracle.rotation_matrix(24, 7)
    c = (np.arange(24, dtype=np.float32) - 12.0) / 24.0
    nodes_l2, *_ = oracle.rabitq_quantize(x, m, c, "l2")
    nodes_ip, *_ = oracle.rabitq_quantize(x, m, None, "ip")
    return dict(x=x, rotation=m.astype(np.float32), centroid=c, nodes_l2=nodes_l2, nodes_ip=nodes_ip)


def make_all() -> dict[str, dict]:
    out = {}
    base, q = datasets.gaussian(300, 24, 1), datasets.gaussian(8, 24, 2)
    out["plain_l2"], g = plain_fixture("plain_l2", base, q, 8, "l2")
    out["directional_l2"] = directional_fixture(g, q)
    base, q = datasets.unit_sphere(300, 16, 3), datasets.unit_sphere(8, 16, 4)
    out["plain_ip"], _ = plain_fixture("plain_ip", base, q, 8, "ip")
    out["rabitq"] = rabitq_fixture()
    m, _ = oracle.rotation_matrix(24, 42)
    out["rotation"] = dict(dim=np.int64(24), seed=np.int64(42), matrix=m.astype(np.float32))
    return out


def main() -> None:
    for name, arrays in make_all().items():
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print("wrote", HERE / f"{name}.npz")


if __name__ == "__main__":
    main()
