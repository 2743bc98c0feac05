"""Oracle plain traversal (reference beam_search/beam_search.cuh:27-225).

Pinned by what the algorithm fixes independently of the restatement:
  * bw >= N on a connected graph -> the result is the brute-force top-k;
  * complete graph -> one expansion of the medoid already holds every
    vertex, so the result after a single hop is the brute-force top-k;
  * a path graph with a hand-computed pop order;
  * the loop bounds (limit + 1 iterations, max_result pops);
  * invariants: sorted by (distance, id), unique ids, distances are the
    distance function's values.
"""

import numpy as np
import pytest

import oracle
from jasper_amd import datasets


def _graph(vecs, adj, R, distance="l2", medoid=0):
    n = len(adj)
    edges = np.full((n, R), 0xFFFFFFFF, dtype=np.uint32)
    counts = np.zeros(n, dtype=np.uint8)
    for i, nb in enumerate(adj):
        edges[i, :len(nb)] = nb
        counts[i] = len(nb)
    v16 = oracle.as_padded_f16(vecs)
    return oracle.OracleGraph(v16, edges, np.zeros((n, R), np.uint16), counts, R, vecs.shape[1], distance,
                              medoid=medoid)


def test_complete_graph_one_hop_is_exact():
    n, dim = 40, 16
    x = datasets.gaussian(n, dim, 3)
    adj = [[j for j in range(n) if j != i] for i in range(n)]
    g = _graph(x, adj, R=64)
    q = datasets.gaussian(8, dim, 4)
    gt, gd = oracle.bruteforce_exact(x, q, k=5)
    # limit = 0: one iteration = pop the medoid and expand it
    ids, dist, vis_ids, vis_d, vis_c = oracle.beam_search(g, q, k=5, beam_width=64, limit=0,
                                                          get_visited=True)
    assert (vis_c == 1).all() and (vis_ids[:, 0] == 0).all()
    assert np.array_equal(ids, gt) and np.array_equal(dist, gd)


def test_large_beam_on_connected_graph_is_exact():
    # a ring (connectivity) plus the 12 nearest neighbours of every vertex
    n = 300
    x = datasets.gaussian(n, 32, 5)
    nn, _ = oracle.bruteforce_exact(x, x, k=13)
    adj = [[(i + 1) % n] + [int(j) for j in nn[i] if j != i][:12] for i in range(n)]
    g = _graph(x, adj, R=16)
    q = datasets.gaussian(20, 32, 6)
    gt, gd = oracle.bruteforce_exact(x, q, k=10)
    ids, dist = oracle.beam_search(g, q, k=10, beam_width=400, limit=1000)
    assert np.array_equal(ids, gt)
    assert np.array_equal(dist, gd)


def test_path_graph_pop_order():
    # points on a line at x = 0..9, path edges, query at x = 5.25, bw = 2
    n = 10
    x = np.zeros((n, 8), dtype=np.float32)
    x[:, 0] = np.arange(n)
    adj = [[j for j in (i - 1, i + 1) if 0 <= j < n] for i in range(n)]
    g = _graph(x, adj, R=2)
    q = np.zeros((1, 8), dtype=np.float32)
    q[0, 0] = 5.25
    ids, dist, vis_ids, vis_d, vis_c = oracle.beam_search(g, q, k=2, beam_width=2, limit=20,
                                                          get_visited=True)
    # walk 0 -> 1 -> ... -> 5, then 6 is expanded; 7 never beats {5, 6}
    assert vis_c[0] == 7
    assert vis_ids[0, :7].tolist() == [0, 1, 2, 3, 4, 5, 6]
    assert ids[0].tolist() == [5, 6]
    assert dist[0].tolist() == [0.0625, 0.5625]
    assert vis_d[0, :7].tolist() == [(5.25 - i) ** 2 for i in range(7)]


def test_max_result_caps_pops():
    x = datasets.gaussian(500, 32, 8)
    g = oracle.build(x, R=16, distance="l2", alpha=1.2)
    q = datasets.gaussian(5, 32, 9)
    *_, vis_c = oracle.beam_search(g, q, k=10, beam_width=64, limit=500, max_result=3, get_visited=True)
    assert (vis_c == 3).all()
    *_, vis_c = oracle.beam_search(g, q, k=10, beam_width=64, limit=4, max_result=2048, get_visited=True)
    assert (vis_c <= 5).all()  # limit + 1 iterations


def test_output_invariants_and_distances():
    x = datasets.gaussian(2000, 64, 10)
    g = oracle.build(x, R=32, distance="l2", alpha=1.2)
    q = datasets.gaussian(30, 64, 11)
    ids, dist = oracle.beam_search(g, q, k=20, beam_width=32)
    x16 = oracle.as_padded_f16(x)
    q16 = oracle.as_padded_f16(q)
    for i in range(len(q)):
        row = ids[i]
        assert len(set(row.tolist())) == len(row)
        assert np.all(np.diff(dist[i]) >= 0)
        exp = oracle.distance_pairs(np.repeat(q16[i:i + 1], len(row), 0), x16[row], "l2")
        assert np.array_equal(exp, dist[i])


def test_out_of_range_edges_are_ignored():
    # edges pointing past n enter as visited INVALID entries and never surface
    n = 6
    x = datasets.gaussian(n, 8, 12)
    adj = [[1, 2, 99, 3], [0, 4, 1000], [5], [0], [1], [2]]
    g = _graph(x, adj, R=4)
    q = datasets.gaussian(3, 8, 13)
    ids, dist = oracle.beam_search(g, q, k=6, beam_width=8)
    gt, gd = oracle.bruteforce_exact(x, q, k=6)
    assert np.array_equal(ids, gt) and np.array_equal(dist, gd)


def test_deleted_vertices_are_skipped_in_output():
    x = datasets.gaussian(300, 16, 14)
    g = oracle.build(x, R=16, distance="l2", alpha=1.2)
    q = datasets.gaussian(4, 16, 15)
    ids, _ = oracle.beam_search(g, q, k=5, beam_width=64)
    victim = int(ids[0, 0])
    g.deleted_bits[victim >> 5] |= np.uint32(1 << (victim & 31))
    ids2, _ = oracle.beam_search(g, q, k=5, beam_width=64)
    assert victim not in ids2[0].tolist()
    assert ids2[0, :4].tolist() == ids[0, 1:5].tolist()
