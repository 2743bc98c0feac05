"""Oracle partitioned ("scale") build (reference index/construct_scale.cuh,
index/construct_scale_kernels.cuh).

Pinned by:
  * the merge order, worked out by hand from the reference's loop for P = 4,
    and its general properties (every unordered pair once, consecutive calls
    sharing a partition within a cycle);
  * the merge prune on a hand-made candidate list, where the answer follows
    from the rule itself (a candidate whose vector is in neither partition is
    kept untested and never prunes others);
  * one partition: the build is the plain construction with the same batch
    schedule, bit for bit;
  * several partitions: degree <= R, no self loops or duplicates, stored
    distances equal bf16(exact distance), cross-partition edges present and
    recall against brute force.
"""

import numpy as np
import pytest

import oracle
from jasper_amd import datasets


def test_merge_order_hand_p4():
    # itv 1: one cycle of 4 calls from B1 = 0; itv 2: gcd 2 -> two cycles of
    # length 2 (one call each), the second starting at (2 + 1) % 4 = 3
    assert oracle.scale_merge_order(4) == [(0, 1), (1, 2), (2, 3), (3, 0), (0, 2), (3, 1)]
    assert oracle.scale_merge_order(2) == [(0, 1)]
    assert oracle.scale_merge_order(1) == []


@pytest.mark.parametrize("P", [3, 5, 6, 7, 8, 9, 12])
def test_merge_order_covers_every_pair_once(P):
    order = oracle.scale_merge_order(P)
    pairs = [tuple(sorted(p)) for p in order]
    assert len(pairs) == P * (P - 1) // 2
    assert len(set(pairs)) == len(pairs)
    assert all(a != b for a, b in order)
    # a call's B1 is the previous call's B2 or, at a cycle start, one past it
    for (a0, b0), (a1, _) in zip(order, order[1:]):
        assert a1 in (b0, (b0 + 1) % P)


def _line_vectors():
    # 8 dimensions: the reference's fp16 L2 reads whole 8-value chunks
    x = np.zeros((6, 8), dtype=np.float32)
    x[:, :2] = [[0, 0], [1, 0], [2, 0], [0, 3.5], [10, 0], [0, 3]]
    return x


def test_prune_scale_hand():
    x = _line_vectors()
    inv = 0xFFFFFFFF
    # self 0; B1 = rows {0, 1}, B2 = rows {2, 3}; rows 4 and 5 in neither
    ids = [0, 1, 2, 5, 3, 4, inv]
    d = [0.0, 1.0, 4.0, 9.0, 12.25, 100.0, np.inf]
    sel, sd = oracle.prune_scale(x, (0, 2), (2, 2), 0, ids, d, R=8, alpha=1.2)
    # 1 kept; 2 pruned by 1 (1 * 1.2 < 4); 5 unresolvable -> kept untested;
    # 3 tested against 1 only (13.25 * 1.2 > 12.25; 5 would prune it) -> kept;
    # 4 unresolvable -> kept
    assert sel.tolist() == [1, 5, 3, 4]
    assert sd.tolist() == [1.0, 9.0, 12.25, 100.0]
    sel, _ = oracle.prune_scale(x, (0, 2), (2, 2), 0, ids, d, R=3, alpha=1.2)
    assert sel.tolist() == [1, 5, 3]
    # every row resolvable: the plain rule, 5 pruned by 1 (10 * 1.2 < 9 is
    # false -> kept), 3 pruned by 5 (0.25 * 1.2 < 12.25), 4 pruned by 1
    sel, _ = oracle.prune_scale(x, (0, 6), (0, 0), 0, ids, d, R=8, alpha=1.2)
    assert sel.tolist() == [1, 5]


def test_one_partition_is_the_plain_build():
    x = datasets.gaussian(2000, 32, 3)
    g1 = oracle.build(x, R=24, max_batch=40)
    gs = oracle.build_scale(x, R=24, n_parts=1, part_batch=40)
    assert np.array_equal(g1.counts, gs.counts)
    for i in range(x.shape[0]):
        c = g1.counts[i]
        assert np.array_equal(g1.edges[i, :c], gs.edges[i, :c])
        assert np.array_equal(g1.edge_dist[i, :c], gs.edge_dist[i, :c])


def test_empty_partition_rejected():
    x = datasets.gaussian(9, 8, 0)
    with pytest.raises(ValueError):
        oracle.build_scale(x, R=8, n_parts=4, part_batch=1)


@pytest.fixture(scope="module", params=[2, 3, 4])
def scale_built(request):
    x = datasets.clustered(3000, 48, 5, n_clusters=16)
    P = request.param
    return x, P, oracle.build_scale(x, R=32, n_parts=P, part_batch=30, merge_batch=256)


def test_scale_invariants(scale_built):
    x, P, g = scale_built
    n = x.shape[0]
    part = (n + P - 1) // P
    c = g.counts.astype(np.int64)
    assert (c <= g.R).all() and (c > 0).all()
    rows = np.repeat(np.arange(n), c)
    cols = np.concatenate([g.edges[i, :c[i]] for i in range(n)]).astype(np.int64)
    stored = np.concatenate([g.edge_dist[i, :c[i]] for i in range(n)])
    assert (cols < n).all() and (cols != rows).all()
    assert len(np.unique(rows * n + cols)) == len(rows)
    exact = oracle.distance_pairs(g.vecs16[rows], g.vecs16[cols], "l2")
    bf = np.array([oracle.f2bf(v) for v in exact], dtype=np.uint16)
    assert np.array_equal(bf, stored)
    # the merges wire partitions together
    assert (rows // part != cols // part).mean() > 0.3


def test_scale_recall(scale_built):
    x, P, g = scale_built
    q = datasets.clustered(200, 48, 99, n_clusters=16)
    gt, _ = oracle.bruteforce_exact(x, q, k=10)
    ids, _ = oracle.beam_search(g, q, k=10, beam_width=32)
    assert oracle.recall(gt, ids, 10) > 0.98
