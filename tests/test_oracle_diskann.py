"""Oracle DiskANN build (reference index/construct_diskann.cuh,
construct_diskann_kernels.cuh, cmd/create_diskann_index.cu).

Pinned by:
  * the shard assignment on rows built as m +- s * (column j of P), whose
    centred rotation is +-s e_j: rank 0 must pick coordinate j with the sign
    of s (taking P's rows instead of its columns, or skipping the centring,
    picks other coordinates);
  * the mean's row sampling worked out by hand: n = 4,000,001 gives stride 2,
    so only the even rows count;
  * n_dup semantics (distinct shards per row, INVALID for repeats);
  * with n_dup = 1 and R_fin = R_int the build is each shard's plain build
    with ids mapped to global ones, bit for bit;
  * with n_dup = 2: degree, uniqueness, sorted rows, stored distance =
    bf16(exact distance), and the merge rule (the first R_fin distinct ids of
    the shard rows in task order, stably sorted by stored distance) checked
    against the shards' plain builds;
  * recall against brute force.
"""

import numpy as np
import pytest

import oracle
from jasper_amd import datasets

INV = 0xFFFFFFFF


def test_assign_rank0_follows_the_rotation():
    dim, seed = 16, 42
    P, _ = oracle.rotation_matrix(dim, seed)
    cols = P.reshape(dim, dim)          # column-major: row j of this view = column j of P
    m = np.full(dim, 100.0, dtype=np.float64)
    rows, want = [], []
    for j in range(dim):
        for s in (40.0, -40.0):
            rows.append(m + s * cols[j])
            want.append(2 * j + (1 if s < 0 else 0))
    x = np.array(rows, dtype=np.float32)
    so, mean = oracle.diskann_assign(x, n_parts=2 * dim, n_dup=2, seed=seed)
    assert so[:, 0].tolist() == want
    # the +-s pairs centre on m
    assert np.abs(oracle_mean(mean) - 100.0).max() <= 0.5
    # with P's rows in place of its columns rank 0 would differ
    other = [2 * int(np.argmax(np.abs(cols.T @ (r - m)))) for r in rows]
    assert other != [w - (w & 1) for w in want]


def oracle_mean(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float64)


def test_assign_mean_samples_every_stride_row():
    # n = 4,000,001: target = 2,000,000, stride = 4,000,001 // 2,000,000 = 2,
    # rows 0, 2, ..., 4,000,000 (2,000,001 of them) are averaged
    n, dim = 4_000_001, 8
    x = np.empty((n, dim), dtype=np.float32)
    x[0::2] = 3.0
    x[1::2] = -7.0
    so, mean = oracle.diskann_assign(x, n_parts=4, n_dup=1)
    assert np.array_equal(oracle_mean(mean), np.full(dim, 3.0))
    # a smaller set averages every row
    so, mean = oracle.diskann_assign(x[:1000], n_parts=4, n_dup=1)
    assert np.array_equal(oracle_mean(mean), np.full(dim, -2.0))


@pytest.mark.parametrize("n_parts,n_dup", [(1, 3), (3, 2), (8, 4), (64, 2)])
def test_assign_ranks_are_distinct_shards(n_parts, n_dup):
    x = datasets.gaussian(500, 24, 7)
    so, _ = oracle.diskann_assign(x, n_parts=n_parts, n_dup=n_dup)
    assert (so[:, 0] != INV).all() and (so[so != INV] < n_parts).all()
    for row in so:
        v = row[row != INV]
        assert len(set(v.tolist())) == len(v)
    if n_parts == 1:
        assert (so[:, 1:] == INV).all()


def _shards(so, n_parts):
    ids = [[] for _ in range(n_parts)]
    for v, row in enumerate(so):
        for s in row:
            if s != INV:
                ids[s].append(v)
    return [np.array(i, dtype=np.int64) for i in ids]


def _tasks(shards):
    order = [p for p in range(len(shards)) if len(shards[p])]
    return sorted(order, key=lambda p: -len(shards[p]))  # stable: equal sizes by index


def test_one_copy_is_the_shards_plain_builds():
    x = datasets.clustered(2400, 32, 4, n_clusters=12)
    n_parts, R = 4, 16
    g = oracle.build_diskann(x, R_int=R, R_fin=R, n_parts=n_parts, n_dup=1, batch_cap=20)
    shards = _shards(g.shard_of, n_parts)
    assert sum(len(s) for s in shards) == len(x)
    for ids in shards:
        if not len(ids):
            continue
        sg = oracle.build(x[ids], R=R, max_batch=max(1, min(20, len(ids))))
        for i, gid in enumerate(ids):
            c = sg.counts[i]
            assert g.counts[gid] == c
            assert np.array_equal(g.edges[gid, :c], ids[sg.edges[i, :c]])
            assert np.array_equal(g.edge_dist[gid, :c], sg.edge_dist[i, :c])


@pytest.fixture(scope="module", params=[(32, 32), (16, 48)])
def diskann_built(request):
    R_int, R_fin = request.param
    x = datasets.clustered(3000, 48, 6, n_clusters=16)
    g = oracle.build_diskann(x, R_int=R_int, R_fin=R_fin, n_parts=5, n_dup=2, batch_cap=25)
    return x, R_int, R_fin, g


def test_diskann_invariants(diskann_built):
    x, R_int, R_fin, g = diskann_built
    n = len(x)
    c = g.counts.astype(np.int64)
    assert (c > 0).all() and (c <= R_fin).all()
    rows = np.repeat(np.arange(n), c)
    cols = np.concatenate([g.edges[i, :c[i]] for i in range(n)]).astype(np.int64)
    stored = np.concatenate([g.edge_dist[i, :c[i]] for i in range(n)])
    assert (cols < n).all() and (cols != rows).all()
    assert len(np.unique(rows * n + cols)) == len(rows)
    exact = oracle.distance_pairs(g.vecs16[rows], g.vecs16[cols], "l2")
    assert np.array_equal(np.array([oracle.f2bf(v) for v in exact], dtype=np.uint16), stored)
    f = (stored.astype(np.uint32) << 16).view(np.float32)
    starts = np.concatenate([[0], np.cumsum(c)[:-1]])
    for s, k in zip(starts, c):
        assert (np.diff(f[s:s + k]) >= 0).all()


def test_diskann_merge_rule(diskann_built):
    x, R_int, R_fin, g = diskann_built
    n_parts = 5
    shards = _shards(g.shard_of, n_parts)
    per_node = [[] for _ in range(len(x))]  # (dist, order, id) in task order
    order = 0
    for p in _tasks(shards):
        ids = shards[p]
        sg = oracle.build(x[ids], R=R_int, max_batch=max(1, min(25, len(ids))))
        for i, gid in enumerate(ids):
            for j in range(sg.counts[i]):
                d = float((np.uint32(sg.edge_dist[i, j]) << np.uint32(16)).view(np.float32))
                per_node[gid].append((d, order, int(ids[sg.edges[i, j]]), int(sg.edge_dist[i, j])))
                order += 1
    for v in range(len(x)):
        seen, want = set(), []
        for d, _, w, bits in sorted(per_node[v]):
            if w in seen:
                continue
            seen.add(w)
            want.append((w, bits))
            if len(want) == R_fin:
                break
        c = g.counts[v]
        assert [(int(a), int(b)) for a, b in zip(g.edges[v, :c], g.edge_dist[v, :c])] == want, v


def test_diskann_recall(diskann_built):
    x, R_int, R_fin, g = diskann_built
    q = datasets.clustered(200, 48, 61, n_clusters=16)
    gt, _ = oracle.bruteforce_exact(x, q, k=10)
    ids, _ = oracle.beam_search(g, q, k=10, beam_width=32)
    assert oracle.recall(gt, ids, 10) > 0.95
