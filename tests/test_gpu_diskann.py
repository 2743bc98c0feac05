"""GPU DiskANN build against the oracle restatement (reference
index/construct_diskann.cuh, construct_diskann_kernels.cuh,
cmd/create_diskann_index.cu).

The shard assignment must equal the oracle's row for row (the same mean,
the same fp16 rotation, accumulated in the same order), and the merged
graph must equal the oracle's bit for bit: edge counts, neighbour ids slot
by slot and bf16 edge distances. Shard batches stay at or below 256 rows,
so no reverse group reaches the 256 + R cap inside a shard build.
"""

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import gaussian, integer_clustered, unit

pytestmark = pytest.mark.gpu


def _compare(gg, og):
    edges, edist, counts = gg.export_edges()
    assert np.array_equal(counts, og.counts), (
        f"edge counts differ at {np.nonzero(counts != og.counts)[0][:10].tolist()}")
    n, R = edges.shape
    mask = np.arange(R)[None, :] < counts[:, None]
    bad = np.nonzero(((edges != og.edges) & mask).any(axis=1))[0]
    assert len(bad) == 0, (f"{len(bad)} adjacency rows differ; first {bad[0]}: gpu "
                           f"{edges[bad[0], :counts[bad[0]]].tolist()} ref "
                           f"{og.edges[bad[0], :og.counts[bad[0]]].tolist()}")
    assert np.array_equal(edist[mask], og.edge_dist[mask])


ASSIGN = [
    ("integer_d128", lambda: integer_clustered(3000, 128, 41), 8, 2),
    ("gaussian_d96", lambda: gaussian(2000, 96, 42), 5, 3),
    ("gaussian_d50", lambda: gaussian(1500, 50, 43), 7, 2),
    ("gaussian_d200", lambda: gaussian(1200, 200, 44), 16, 4),
    ("unit_d64_one_shard", lambda: unit(800, 64, 45), 1, 2),
]


@pytest.mark.parametrize("case", ASSIGN, ids=[c[0] for c in ASSIGN])
def test_diskann_assign_matches_oracle(jasper, oracle_lib, case):
    name, make, n_parts, n_dup = case
    x = make()
    print(f"case {name}: n={x.shape[0]} dim={x.shape[1]} n_parts={n_parts} n_dup={n_dup}", flush=True)
    so, mean = oracle.diskann_assign(x, n_parts=n_parts, n_dup=n_dup, seed=42)
    gso, gmean = jasper.diskann_assign(torch.from_numpy(np.ascontiguousarray(x)).cuda(), n_parts, n_dup, 42)
    assert np.array_equal(gmean, mean)
    bad = np.nonzero((gso != so).any(axis=1))[0]
    assert len(bad) == 0, f"{len(bad)} rows differ; first {bad[0]}: gpu {gso[bad[0]]} ref {so[bad[0]]}"


BUILD = [
    # name, rows, R_int, R_fin, distance, n_parts, n_dup, batch cap
    ("integer_32_32", lambda: integer_clustered(3000, 128, 46), 32, 32, "l2", 5, 2, 25),
    ("integer_32_64", lambda: integer_clustered(3000, 128, 47), 32, 64, "l2", 4, 2, 30),
    ("gaussian_16_32_dup3", lambda: gaussian(2000, 96, 48), 16, 32, "l2", 6, 3, 20),
    ("ip_32_32", lambda: unit(2000, 64, 49), 32, 32, "ip", 4, 2, 25),
    ("gaussian_d50_one_copy", lambda: gaussian(1500, 50, 50), 16, 16, "l2", 3, 1, 16),
]


@pytest.mark.parametrize("case", BUILD, ids=[c[0] for c in BUILD])
def test_diskann_build_matches_oracle(jasper, oracle_lib, case):
    name, make, R_int, R_fin, distance, n_parts, n_dup, cap = case
    x = make()
    print(f"case {name}: n={x.shape[0]} dim={x.shape[1]} R_int={R_int} R_fin={R_fin} {distance} "
          f"n_parts={n_parts} n_dup={n_dup} cap={cap}", flush=True)
    og = oracle.build_diskann(x, R_int=R_int, R_fin=R_fin, distance=distance, alpha=1.2, n_parts=n_parts,
                              n_dup=n_dup, seed=42, batch_cap=cap)
    t = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    gg = jasper.Graph.build_diskann(t, n_neighbors=R_fin, r_int=R_int, distance=distance, alpha=1.2,
                                    n_parts=n_parts, n_dup=n_dup, max_batch_size=cap, seed=42)
    torch.cuda.synchronize()
    _compare(gg, og)
    st = jasper.last_diskann_stats()
    sizes = np.bincount(og.shard_of[og.shard_of != 0xFFFFFFFF].ravel(), minlength=n_parts)
    assert st["shards"] == int((sizes > 0).sum()) and st["max_shard"] == int(sizes.max())


def test_diskann_build_then_search(jasper, oracle_lib):
    x = integer_clustered(3000, 128, 51)
    q = integer_clustered(300, 128, 52)
    og = oracle.build_diskann(x, R_int=32, R_fin=64, n_parts=4, n_dup=2, batch_cap=30)
    gg = jasper.Graph.build_diskann(torch.from_numpy(x).cuda(), n_neighbors=64, r_int=32, n_parts=4, n_dup=2,
                                    max_batch_size=30)
    _compare(gg, og)
    ids, d = gg.search(torch.from_numpy(q).cuda(), k=10, beam_width=64)
    rid, rd = oracle.beam_search(og, q, k=10, beam_width=64)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.array_equal(d.cpu().numpy().view(np.uint32), rd.view(np.uint32))
    gt, _ = oracle.bruteforce_exact(x, q, k=10)
    assert oracle.recall(gt, ids.cpu().numpy(), 10) > 0.95


def test_diskann_bad_arguments(jasper):
    t = torch.zeros((16, 8), dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        jasper.Graph.build_diskann(t, n_neighbors=8, r_int=8, n_parts=2, n_dup=17)
    with pytest.raises(ValueError):
        jasper.Graph.build_diskann(t, n_neighbors=8, r_int=65, n_parts=2, n_dup=2)


@pytest.mark.parametrize("max_shard", [400, 999])
def test_diskann_build_split_shards_matches_oracle(jasper, oracle_lib, max_shard):
    """A shard graph cap (the device budget a shard may take) below the
    shards' sizes: each shard is built as equal sub-shards of its ascending
    ids, at most max_shard rows each, largest first
    (construct_diskann.cuh:386-417), and merged as shards are; the graph
    equals the oracle's with the same cap."""
    x = integer_clustered(3000, 128, 53)
    og = oracle.build_diskann(x, R_int=32, R_fin=32, n_parts=4, n_dup=2, batch_cap=25, max_shard=max_shard)
    gg = jasper.Graph.build_diskann(torch.from_numpy(x).cuda(), n_neighbors=32, r_int=32, n_parts=4, n_dup=2,
                                    max_batch_size=25, max_shard=max_shard)
    _compare(gg, og)
    st = jasper.last_diskann_stats()
    sizes = np.bincount(og.shard_of[og.shard_of != 0xFFFFFFFF].ravel(), minlength=4)
    subs = [-(-int(s) // max_shard) for s in sizes if s]
    assert st["shards"] == sum(subs) and st["shards"] > int((sizes > 0).sum())
    assert st["max_shard"] <= max_shard
