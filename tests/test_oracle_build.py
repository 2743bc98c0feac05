"""Oracle Vamana construction (reference index/construct.cuh:743-1160).

Pinned by the properties the algorithm guarantees:
  * the batch schedule and maximum batch size of the reference
    (construct.cuh:238-262, :913-958; ffi/jasper_ffi_common.cuh:245-248);
  * degree <= R, no self loops, no INVALID ids in a row's valid prefix;
  * rows sorted by stored distance, and the alpha-pruning dominance
    property: for selected s_i before s_j, d(s_j, s_i) * alpha >= d_j
    (up to the bf16 rounding of the stored d_j);
  * stored distances are bf16(exact distance);
  * recall against brute force, and connectivity from the medoid.
"""

import numpy as np
import pytest

import oracle
from jasper_amd import datasets


def test_reference_max_batch_sizes():
    # per_item = 6152 B at R = 64 -> floor((1e10 - 4) / 6152) = 1625487
    assert oracle.max_batch_size(100_000_000, 64, 10 ** 10) == 1_625_487
    assert oracle.max_batch_size(1_000_000, 64, 10 ** 10) == 20_000
    assert oracle.max_batch_size(10_000, 32, 10 ** 10) == 200
    assert oracle.max_batch_size(49, 32, 10 ** 10) == 0       # the reference's n < 50 hang
    assert oracle.max_batch_size(10_000, 32, 1000) == 0       # budget below one item


def test_batch_schedule_count():
    x = datasets.gaussian(1000, 32, 0)
    g = oracle.build(x, R=16, max_batch=20)
    # 1 + 2 + 4 + 8 = 15, then 16, then 20s: (1000 - 31) / 20 -> 49 (last partial)
    assert g.n_batches == 4 + 1 + int(np.ceil((1000 - 31) / 20))


@pytest.fixture(scope="module")
def built():
    x = datasets.gaussian(3000, 64, 1)
    return x, oracle.build(x, R=24, distance="l2", alpha=1.2)


def test_rows_are_valid(built):
    x, g = built
    n = g.n
    assert g.counts.max() <= g.R
    assert (g.counts > 0).all()
    for v in range(n):
        row = g.edges[v, :g.counts[v]]
        assert (row < n).all()
        assert v not in row.tolist()


def test_stored_distances_are_bf16_of_exact(built):
    x, g = built
    x16 = oracle.as_padded_f16(x)
    rng = np.random.default_rng(0)
    for v in rng.choice(g.n, 200, replace=False):
        c = g.counts[v]
        row = g.edges[v, :c]
        exact = oracle.distance_pairs(np.repeat(x16[v:v + 1], c, 0), x16[row], "l2")
        assert [oracle.f2bf(float(e)) for e in exact] == g.edge_dist[v, :c].tolist()


def test_alpha_prune_dominance(built):
    x, g = built
    x16 = oracle.as_padded_f16(x)
    alpha = np.float32(1.2)
    rng = np.random.default_rng(1)
    for v in rng.choice(g.n, 150, replace=False):
        c = g.counts[v]
        row = g.edges[v, :c]
        dd = g.edge_dist[v, :c].astype(np.uint32) << 16
        dv = dd.view(np.float32)
        assert np.all(np.diff(dv) >= 0), "row not sorted by stored distance"
        for j in range(1, c):
            prev = row[:j]
            dsj = oracle.distance_pairs(np.repeat(x16[row[j]:row[j] + 1], j, 0), x16[prev], "l2")
            # stored d_j is bf16-rounded (relative error <= 2^-9)
            assert np.all(dsj * alpha >= dv[j] * (1 - 2 ** -8)), (v, j)


def test_connected_from_medoid(built):
    x, g = built
    seen = np.zeros(g.n, bool)
    stack = [g.medoid]
    seen[g.medoid] = True
    while stack:
        u = stack.pop()
        for w in g.edges[u, :g.counts[u]]:
            if not seen[w]:
                seen[w] = True
                stack.append(int(w))
    assert seen.mean() > 0.95  # single alpha pass: a few vertices can lose every in-edge


def test_recall_against_bruteforce():
    x, q, _ = datasets.config("c1", n=5000, nq=50)
    g = oracle.build(x, R=32, distance="l2", alpha=1.2)
    gt, _ = oracle.bruteforce_exact(x, q, k=10)
    r64 = oracle.recall(gt, oracle.beam_search(g, q, k=10, beam_width=64)[0], 10)
    r256 = oracle.recall(gt, oracle.beam_search(g, q, k=10, beam_width=256)[0], 10)
    assert r64 > 0.8 and r256 > 0.97 and r256 >= r64


def test_ip_build_valid():
    x = datasets.unit_sphere(1500, 32, 2)
    g = oracle.build(x, R=16, distance="ip", alpha=1.2)
    assert g.counts.max() <= 16 and (g.counts > 0).all()
    q = datasets.unit_sphere(20, 32, 3)
    gt, _ = oracle.bruteforce_exact(x, q, k=10, distance="ip")
    r = oracle.recall(gt, oracle.beam_search(g, q, k=10, beam_width=128)[0], 10)
    assert r > 0.9


def test_tiny_inputs_build():
    # n < 50: the reference's batch size would be 0; the oracle clamps it to 1
    for n in (1, 2, 3, 10):
        x = datasets.gaussian(n, 16, 20 + n)
        g = oracle.build(x, R=8)
        assert g.n_batches == n
        assert (g.counts <= min(n - 1, 8)).all()
        if n > 1:
            assert (g.counts >= 1).all()


# ---------------------------------------------------- hand-computed tiny build
# Six points on a line (coordinate 0 of d = 8) at 0, 10, 3, 20, 21, 12;
# alpha = 1.2, L2 (squared distances), R = 2 or 8 (no row keeps more than two
# candidates after the alpha prune, so both give the same graph). The expected graphs below were worked
# out by hand from the contract (batched search from the medoid 0 against the
# pre-batch graph, forward RobustPrune of existing edges + visited nodes,
# reverse merge of the target's existing edges with its new sources, then
# RobustPrune; prune c when d(c, s) * alpha < d_c). Batches of two (schedule
# 1, 2, 2, 1) make the result sensitive to three plausible mistakes:
#   * leaving the target's existing edges out of the reverse merge gives row
#     2 = [3] after the third batch (and changes rows 2, 3, 5 at the end);
#   * searching the graph as it stands after earlier members of the batch
#     were inserted lets row 4 see row 3: [3, 2] instead of [2];
#   * applying alpha to the other side (d_c * alpha < d(c, s)) keeps 2 in
#     row 3: [5, 2] instead of [5].
# With batches of one (n < 50 forces them on the device) every search sees
# the previous insertions, and the graph is the second one.
LINE = [0.0, 10.0, 3.0, 20.0, 21.0, 12.0]
HAND_BATCH2 = {0: [(2, 9)], 1: [(0, 100)], 2: [(0, 9), (5, 81)], 3: [(5, 64)], 4: [(2, 324)],
               5: [(3, 64), (2, 81)]}
HAND_BATCH1 = {0: [(2, 9)], 1: [(5, 4), (2, 49)], 2: [(0, 9), (1, 49)], 3: [(4, 1), (5, 64)],
               4: [(3, 1), (2, 324)], 5: [(1, 4), (3, 64)]}


def line_points():
    x = np.zeros((6, 8), dtype=np.float32)
    x[:, 0] = LINE
    return x


def check_hand_graph(edges, edist, counts, want):
    for v, row in want.items():
        assert int(counts[v]) == len(row), (v, counts[v], row)
        assert edges[v, :len(row)].tolist() == [w for w, _ in row], (v, edges[v, :counts[v]], row)
        got = (np.asarray(edist[v, :len(row)], dtype=np.uint32) << 16).view(np.float32).tolist()
        assert got == [float(d) for _, d in row], (v, got, row)


@pytest.mark.parametrize("R", [2, 8])
@pytest.mark.parametrize("max_batch,want", [(2, HAND_BATCH2), (1, HAND_BATCH1)])
def test_hand_computed_line_build(max_batch, want, R):
    g = oracle.build(line_points(), R=R, distance="l2", alpha=1.2, max_batch=max_batch)
    assert g.n_batches == (4 if max_batch == 2 else 6)
    check_hand_graph(g.edges, g.edge_dist, g.counts, want)


def test_rabitq_search_build_quality():
    """The construction with the RaBitQ build search (an extension) keeps
    the build's invariants and a graph whose plain-search recall is near the
    exact construction's on clustered data."""
    dim = 64
    x = datasets.clustered(4000, dim, 31, n_clusters=40).astype(np.float32)
    q = datasets.clustered(60, dim, 32, n_clusters=40).astype(np.float32)
    c = x.mean(0).astype(np.float32)
    nodes, *_ = oracle.rabitq_quantize(x, np.eye(dim, dtype=np.float32).ravel(), centroid=c)
    g_rq = oracle.build(x, R=32, rq=oracle.RqArtifacts(dim, nodes, c))
    g_ex = oracle.build(x, R=32)
    R = 32
    for g in (g_rq, g_ex):
        assert (g.counts <= R).all() and g.counts.min() >= 1
        for v in range(g.n):
            row = g.edges[v, :g.counts[v]]
            assert v not in row and (row < g.n).all()
    gt, _ = oracle.bruteforce_exact(x, q, k=10)
    rec = [oracle.recall(gt, oracle.beam_search(g, q, k=10, beam_width=32)[0], 10) for g in (g_rq, g_ex)]
    assert rec[0] >= rec[1] - 0.05, rec
