"""GPU partitioned ("scale") build against the oracle restatement
(reference index/construct_scale.cuh, construct_scale_kernels.cuh,
cmd/create_scale_index.cu).

Batches stay at or below 256 rows, so no reverse group reaches the 256 + R
candidate cap and the reference's result does not depend on arrival order;
the GPU graph must then equal the oracle's bit for bit: edge counts,
neighbour ids slot by slot and bf16 edge distances. The cases cover integer
rows (the partitions' exact integer paths), non-integer rows, inner product,
a dimension that is not a multiple of 8, odd and even partition counts
(merge cycles of both kinds) and several merge batches per partition pair.
"""

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import gaussian, integer_clustered, unit

pytestmark = pytest.mark.gpu


def _budget(batch, R):
    # max_batch_size_for_budget (construct.cuh:238-262): per item
    # 8 L + 8 * 256 + 4 + 8 (256 + R) + 4 + 16 R bytes, plus 4
    return f"{batch * (4616 + 24 * R) + 4}B"


def _gpu_scale(jasper, base, R, distance, n_parts, part_batch, merge_batch):
    t = torch.from_numpy(np.ascontiguousarray(base)).cuda()
    g = jasper.Graph.build_scale(t, n_neighbors=R, distance=distance, alpha=1.2, n_parts=n_parts,
                                 workspace_budget=_budget(merge_batch, R), max_batch_size=part_batch)
    torch.cuda.synchronize()
    return g


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


CASES = [
    # name, rows, R, distance, n_parts, part batch, merge batch
    ("integer_p3", lambda: integer_clustered(3000, 128, 31), 32, "l2", 3, 30, 256),
    ("gaussian_p4_batches", lambda: gaussian(2500, 96, 32), 32, "l2", 4, 25, 100),
    ("ip_p2", lambda: unit(2000, 64, 33), 16, "ip", 2, 20, 128),
    ("dim50_p3", lambda: gaussian(1500, 50, 34), 16, "l2", 3, 16, 64),
    ("integer_r64_p5", lambda: integer_clustered(4000, 128, 35), 64, "l2", 5, 40, 200),
    ("gaussian_p6", lambda: gaussian(2400, 32, 36), 16, "l2", 6, 8, 50),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_scale_build_matches_oracle(jasper, oracle_lib, case):
    name, make, R, distance, P, pb, mb = case
    base = make()
    print(f"case {name}: n={base.shape[0]} dim={base.shape[1]} R={R} {distance} P={P} "
          f"part batch {pb} merge batch {mb}", flush=True)
    og = oracle.build_scale(base, R=R, distance=distance, alpha=1.2, n_parts=P, part_batch=pb,
                            merge_batch=mb)
    gg = _gpu_scale(jasper, base, R, distance, P, pb, mb)
    _compare(gg, og)
    st = jasper.last_scale_stats()
    assert st["merges"] == P * (P - 1) // 2
    part = -(-base.shape[0] // P)
    per_pair = -(-part // mb)
    assert st["merge_batches"] >= st["merges"] and st["merge_batches"] <= st["merges"] * per_pair


def test_scale_one_partition_is_the_plain_build(jasper, oracle_lib):
    base = gaussian(1200, 64, 37)
    og = oracle.build(base, R=16, distance="l2", alpha=1.2, max_batch=24)
    gg = _gpu_scale(jasper, base, 16, "l2", 1, 24, 64)
    _compare(gg, og)


def test_scale_build_then_search(jasper, oracle_lib):
    base = integer_clustered(3000, 128, 38)
    q = integer_clustered(300, 128, 39)
    og = oracle.build_scale(base, R=32, n_parts=4, part_batch=30, merge_batch=128)
    gg = _gpu_scale(jasper, base, 32, "l2", 4, 30, 128)
    _compare(gg, og)
    ids, d = gg.search(torch.from_numpy(q).cuda(), k=10, beam_width=64)
    rid, rd = oracle.beam_search(og, q, k=10, beam_width=64)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.array_equal(d.cpu().numpy().view(np.uint32), rd.view(np.uint32))
    gt, _ = oracle.bruteforce_exact(base, q, k=10)
    assert oracle.recall(gt, ids.cpu().numpy(), 10) > 0.95


def test_scale_empty_partition_rejected(jasper):
    t = torch.zeros((9, 8), dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        jasper.Graph.build_scale(t, n_neighbors=8, n_parts=4)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_scale_build_staged_matches_oracle(jasper, oracle_lib, case):
    """on_host: the graph in pinned host memory, each partition built on the
    device and written back, every merge with its two partitions staged
    into two device slots (a partition shared with the previous pair stays
    resident; five and six partitions switch cycles). The graph equals the
    oracle's partitioned build edge for edge, as the in-HBM build does."""
    name, make, R, distance, P, pb, mb = case
    base = make()
    print(f"staged case {name}: n={base.shape[0]} dim={base.shape[1]} R={R} {distance} P={P}", flush=True)
    og = oracle.build_scale(base, R=R, distance=distance, alpha=1.2, n_parts=P, part_batch=pb,
                            merge_batch=mb)
    t = torch.from_numpy(np.ascontiguousarray(base))  # host rows
    gg = jasper.Graph.build_scale(t, n_neighbors=R, distance=distance, alpha=1.2, n_parts=P,
                                  workspace_budget=_budget(mb, R), max_batch_size=pb, on_host=True)
    torch.cuda.synchronize()
    _compare(gg, og)
    st = jasper.last_scale_stats()
    assert st["merges"] == P * (P - 1) // 2


def test_scale_build_staged_then_search(jasper, oracle_lib):
    base = integer_clustered(3000, 128, 38)
    q = integer_clustered(300, 128, 39)
    og = oracle.build_scale(base, R=32, n_parts=4, part_batch=30, merge_batch=128)
    gg = jasper.Graph.build_scale(torch.from_numpy(base), n_neighbors=32, n_parts=4,
                                  workspace_budget=_budget(128, 32), max_batch_size=30, on_host=True)
    _compare(gg, og)
    ids, d = gg.search(torch.from_numpy(q).cuda(), k=10, beam_width=64)
    rid, rd = oracle.beam_search(og, q, k=10, beam_width=64)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.array_equal(d.cpu().numpy().view(np.uint32), rd.view(np.uint32))
