"""The oracle's live updates, pinned without the GPU.

append: with batches of one vertex, appending to a graph built with batches
of one is the same computation as building the whole set with batches of
one (the construction's schedule is then 1, 1, 1, ...), so the graphs must
be identical; and appended vectors must find themselves (the reference's
gate, cmd/test_append.cu:110-121).
consolidate: the repair candidates are recounted by plain loops from their
definition (deletion.cuh:45-109); rows with no deleted neighbour are left as
they were; no edge leads into a deleted vertex; deleted rows are empty; each
repaired row satisfies the alpha rule against its own earlier members.
mark_deleted: the medoid replacement rule on a hand-made graph.
"""

import numpy as np

import oracle
from tests.helpers import gaussian, integer_clustered


def test_append_with_unit_batches_equals_build():
    x = gaussian(400, 32, 41)
    full = oracle.build(x, R=16, max_batch=1)
    part = oracle.build(x[:250], R=16, max_batch=1)
    grown, ids = oracle.append(part, x[250:], max_batch=1)
    assert ids.tolist() == list(range(250, 400))
    assert np.array_equal(grown.counts, full.counts)
    mask = np.arange(16)[None, :] < full.counts[:, None]
    assert np.array_equal(grown.edges[mask], full.edges[mask])
    assert np.array_equal(grown.edge_dist[mask], full.edge_dist[mask])


def test_append_self_recall_gate():
    x = integer_clustered(2400, 64, 42)
    g = oracle.build(x[:1600], R=32)
    g2, ids = oracle.append(g, x[1600:])
    out, _ = oracle.beam_search(g2, x[1600:], k=10, beam_width=64)
    hit = np.mean([ids[i] in out[i] for i in range(len(ids))])
    assert hit >= 0.99, hit
    assert g2.next_id == 2400 and (g2.counts[1600:] > 0).all()


def _dead(g, v):
    return bool((int(g.deleted_bits[v >> 5]) >> (v & 31)) & 1)


def test_consolidate_against_definition():
    x = integer_clustered(1500, 64, 43)
    g = oracle.build(x, R=16)
    rng = np.random.default_rng(44)
    dels = rng.choice(1500, size=300, replace=False)
    oracle.mark_deleted(g, dels)
    dead = np.array([_dead(g, v) for v in range(g.n)])
    before_e, before_c, before_d = g.edges.copy(), g.counts.copy(), g.edge_dist.copy()
    # repair candidates by definition
    expect = 0
    touched = np.zeros(g.n, bool)
    for N in range(g.n):
        if dead[N]:
            continue
        for j in range(before_c[N]):
            D = int(before_e[N, j])
            if D >= g.n or not dead[D]:
                continue
            touched[N] = True
            for k in range(before_c[D]):
                M = int(before_e[D, k])
                if M < g.n and not dead[M] and M != N:
                    expect += 1
    n_rep = oracle.consolidate(g)
    assert n_rep == expect
    assert not g.deleted_bits.any()
    assert (g.counts[dead] == 0).all()
    for N in range(g.n):
        row = g.edges[N, :g.counts[N]]
        assert not dead[row].any()
        assert N not in row
        if not dead[N] and not touched[N]:
            assert g.counts[N] == before_c[N]
            assert np.array_equal(row, before_e[N, :before_c[N]])
            assert np.array_equal(g.edge_dist[N, :g.counts[N]], before_d[N, :before_c[N]])
    # alpha rule inside each repaired row: no member is pruned by an earlier
    # one (the candidate distance the prune saw is the exact one or, for an
    # edge that was already there, its bf16 rounding: 1/128 of slack)
    for N in np.nonzero(touched)[0][:200]:
        row = g.edges[N, :g.counts[N]]
        for i in range(1, len(row)):
            cd = min(oracle.distance(x[N], x[row[i]]),
                     float((np.uint32(g.edge_dist[N, i]) << np.uint32(16)).view(np.float32)))
            for j in range(i):
                assert oracle.distance(x[row[i]], x[row[j]]) * 1.2 >= cd * (1 - 1 / 128)


def test_mark_deleted_medoid_rule():
    # medoid 0 with edges [3, 1, 2]; deleting 0 and 3 moves it to 1, the first
    # live neighbour in edge order; then deleting all of 0's neighbours moves
    # it to the lowest live vertex
    x = np.arange(6 * 8, dtype=np.float32).reshape(6, 8)
    g = oracle.build(x, R=4)
    g.edges[0, :3] = [3, 1, 2]
    g.counts[0] = 3
    g.medoid = 0
    assert oracle.mark_deleted(g, [0, 3, 3, 99, -5]) == 2
    assert g.medoid == 1
    g2 = oracle.build(x, R=4)
    g2.edges[0, :3] = [3, 1, 2]
    g2.counts[0] = 3
    assert oracle.mark_deleted(g2, [0, 1, 2, 3]) == 4
    assert g2.medoid == 4
