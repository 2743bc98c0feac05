"""Oracle of the directional path (reference beam_search/graph_beam_search.cuh,
beam_search_common.cuh, directional_beam_search.cuh, pq_beam_search.cuh,
lsh/lsh_globals.cuh, lsh/lsh_kernels.cuh, pq/pq_kernels.cuh).

Pinned by checks that do not restate the oracle's code:
  * fp16 arithmetic against numpy's correctly rounded float64 -> float16;
  * splitmix64 / pq_hash against the published splitmix64 sequence;
  * frontier insertion against numpy's stable argsort;
  * per-edge LSH words and PQ codes against numpy sorts / argmins;
  * one k-means step against numpy means;
  * closed forms: on a grid graph every edge is a unit axis step, so the
    LSH estimate (c = [1, 0, ...]) and the PQ estimate with a {0, +1, -1}
    codebook are exact, and a wide-beam directional search must return the
    exact k nearest (L2) or largest inner products (IP).
"""

import numpy as np
import pytest

import oracle
from jasper_amd import datasets


def f16(x):
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float64).astype(np.float16)


def bits(x16):
    return np.asarray(x16, dtype=np.float16).view(np.uint16)


# ------------------------------------------------------------ fp16 arithmetic

def test_d2h_matches_numpy():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.normal(0, 1, 2000), rng.normal(0, 1e4, 500), rng.normal(0, 1e-5, 500),
        [0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001,
         3 * 2.0 ** -26, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 2.0 ** -14 - 2.0 ** -25],
    ])
    for v in vals:
        assert oracle.d2h(v) == int(bits(f16(v))), v


def test_hsub_hmul_match_numpy():
    rng = np.random.default_rng(1)
    a = f16(rng.normal(0, 30, 3000))
    b = f16(rng.normal(0, 30, 3000))
    a[:20] = f16(rng.normal(0, 1e-4, 20))
    for x, y in zip(a, b):
        xb, yb = int(bits(x)), int(bits(y))
        exact_sub = f16(np.float64(x) - np.float64(y))   # float64 holds the exact difference
        exact_mul = f16(np.float64(x) * np.float64(y))   # ... and the exact product
        assert oracle.hsub(xb, yb) == int(bits(exact_sub))
        assert oracle.hmul(xb, yb) == int(bits(exact_mul))


def test_visit_exact_integer_data():
    rng = np.random.default_rng(2)
    for dp in (8, 64, 128, 136, 256, 1024):
        q = rng.integers(-40, 40, dp).astype(np.float16)
        u = rng.integers(-40, 40, dp).astype(np.float16)
        ex, diff = oracle.visit_exact(bits(q), bits(u), l2=True)
        d = q.astype(np.int64) - u.astype(np.int64)
        assert ex == float((d * d).sum())
        assert np.array_equal(diff, bits(d.astype(np.float16)))
        ip, _ = oracle.visit_exact(bits(q), bits(u), l2=False)
        assert ip == float((q.astype(np.int64) * u.astype(np.int64)).sum())


def test_visit_exact_float_data_close():
    rng = np.random.default_rng(3)
    q = f16(rng.normal(0, 3, 200))
    u = f16(rng.normal(0, 3, 200))
    ex, _ = oracle.visit_exact(bits(np.pad(q, (0, 8))), bits(np.pad(u, (0, 8))), l2=True)
    d = f16(q.astype(np.float64) - u.astype(np.float64)).astype(np.float64)
    assert abs(ex - (d * d).sum()) <= 1e-5 * (d * d).sum()


# ------------------------------------------------------------ hashes / sampler

def test_splitmix_known_answers():
    # splitmix64 with state 0: published first outputs
    assert oracle.splitmix(0) == 0xE220A8397B1DCDAF
    assert oracle.splitmix(0x9E3779B97F4A7C15) == 0x6E789E6AA1B965F4
    assert oracle.splitmix((2 * 0x9E3779B97F4A7C15) % 2 ** 64) == 0x06C45D188009454F
    # pq_hash(x, seed) is the splitmix64 output for state x + seed
    assert oracle.pq_hash(0, 0) == 0xE220A8397B1DCDAF
    assert oracle.pq_hash(5, 0x9E3779B97F4A7C15 - 5) == 0x6E789E6AA1B965F4


def _small_graph(n=600, dim=32, R=16, seed=5, distance="l2", data="gauss"):
    if data == "int":
        x = np.round(datasets.gaussian(n, dim, seed) * 8)
    else:
        x = datasets.gaussian(n, dim, seed) * 4
    return x, oracle.build(x, R=R, distance=distance, alpha=1.2)


def test_sampler_returns_graph_edges():
    _, g = _small_graph()
    seen = 0
    for s in range(500):
        r = oracle.sample_edge(g, 42, s)
        if r is None:
            continue
        u, nb = r
        assert nb in g.edges[u, :g.counts[u]].tolist()
        seen += 1
    assert seen == 500  # every vertex of a built graph has out-edges


# ------------------------------------------------------------ frontier list

def test_frontier_insert_is_stable_topk():
    rng = np.random.default_rng(4)
    for k in (1, 3, 10, 40):
        d = rng.integers(0, 12, 60).astype(np.float32)   # many ties
        ids = np.arange(60, dtype=np.uint32)
        oi, od = oracle.frontier_insert_seq(d, ids, k)
        order = np.argsort(d, kind="stable")[:k]
        assert np.array_equal(oi, ids[order]) and np.array_equal(od, d[order])


# ------------------------------------------------------------ LSH artifacts

def _edge_diffs(g):
    x = g.vecs16.view(np.float16).astype(np.float64)
    for u in range(g.n):
        for e in range(g.counts[u]):
            nb = g.edges[u, e]
            yield u, e, (x[nb] - x[u]).astype(np.float16)   # exact difference, one rounding


@pytest.mark.parametrize("K,pbytes,dim", [(4, 1, 32), (8, 1, 128), (3, 2, 200)])
def test_populate_lsh_words(K, pbytes, dim):
    _, g = _small_graph(n=300, dim=dim, R=8)
    rows = oracle.populate_lsh(g, K, pbytes)
    cb = pbytes * 8 - 1
    for u, e, d in _edge_diffs(g):
        mag = np.abs(d).astype(np.float64)
        neg = np.signbit(d)
        idx = np.arange(g.dp)
        # rank: |d| descending, then negative before positive, then larger index
        order = np.lexsort((-idx, -neg.astype(int), -mag))[:K]
        words = (neg[order].astype(np.uint32) << cb) | order.astype(np.uint32)
        if pbytes == 1:
            got = rows[u, e * K:(e + 1) * K].astype(np.uint32)
        else:
            got = rows[u, 2 * e * K:2 * (e + 1) * K].view(np.uint16).astype(np.uint32)
        assert np.array_equal(got, words), (u, e)
        off = g.R * K * pbytes + 2 * e
        mb = rows[u, off:off + 2].view(np.uint16)[0]
        want = float((d.astype(np.float64) ** 2).sum())
        got_mag = float((np.array([mb], dtype=np.uint32) << 16).view(np.float32)[0])
        assert abs(got_mag - want) <= 2 ** -7 * want + 1e-30   # one bf16 ulp
    # slots past the count stay zero
    for u in range(g.n):
        c = g.counts[u]
        assert not rows[u, c * K * pbytes:g.R * K * pbytes].any()


def test_lsh_globals_against_numpy():
    _, g = _small_graph(n=500, dim=48, R=16)
    K = 6
    c, nd, nv = oracle.lsh_globals(g, K, n_samples=3000, seed=9)
    x = g.vecs16.view(np.float16).astype(np.float64)
    acc = []
    for s in range(3000):
        r = oracle.sample_edge(g, 9, s)
        if r is None:
            continue
        u, nb = r
        d = (x[nb] - x[u]).astype(np.float16).astype(np.float64)
        nrm = np.sqrt((d * d).sum())
        if nrm == 0:
            continue
        acc.append(np.sort(np.abs(d))[::-1][:K] / nrm)
    want = np.mean(acc, axis=0)
    assert nv == len(acc)
    assert np.allclose(c, want, rtol=1e-5, atol=1e-7)
    assert abs(nd - float((want ** 2).sum())) < 1e-5
    assert np.all(np.diff(c) <= 0) and nd <= 1.0


# ------------------------------------------------------------ PQ artifacts

def test_pq_training_rows_and_one_kmeans_step():
    _, g = _small_graph(n=400, dim=32, R=8)
    M, nt, seed = 8, 1000, 77
    dsub = g.dp // M
    cent0, X = oracle.pq_train(g, M, n_train=nt, iters=0, seed=seed)
    x = g.vecs16.view(np.float16).astype(np.float64)
    for p in range(nt):
        u, nb = oracle.sample_edge(g, seed, p)
        assert np.array_equal(X[p], bits((x[nb] - x[u]).astype(np.float16)))
    Xf = X.view(np.float16).astype(np.float64)
    init_seed = seed ^ 0xA5A5A5A5
    init = np.zeros((M, 256, dsub))
    for j in range(M):
        for c in range(256):
            r = oracle.pq_hash(j * 256 + c, init_seed) % nt
            init[j, c] = Xf[r, j * dsub:(j + 1) * dsub]
    assert np.array_equal(cent0.reshape(M, 256, dsub), init.astype(np.float32))
    cent1, _ = oracle.pq_train(g, M, n_train=nt, iters=1, seed=seed)
    cent1 = cent1.reshape(M, 256, dsub)
    for j in range(M):
        sub = Xf[:, j * dsub:(j + 1) * dsub]
        dist = ((sub[:, None, :] - init[j][None]) ** 2).sum(-1)
        lab = np.argmin(dist, axis=1)   # first minimum: the smaller index on ties
        for c in range(256):
            members = sub[lab == c]
            if len(members):
                assert np.allclose(cent1[j, c], members.mean(0), rtol=1e-5, atol=1e-5)
            else:
                r = oracle.pq_hash((j * 256 + c) ^ 0, init_seed) % nt
                assert np.array_equal(cent1[j, c], Xf[r, j * dsub:(j + 1) * dsub].astype(np.float32))


def test_pq_encode_is_argmin():
    _, g = _small_graph(n=300, dim=32, R=8)
    M = 4
    art = oracle.build_pq(g, M, n_train=2000, iters=3, seed=5)
    C = art.centroids.reshape(M, 256, art.dsub).astype(np.float64)
    for u, e, d in _edge_diffs(g):
        r = d.astype(np.float64)
        for j in range(M):
            dist = ((C[j] - r[j * art.dsub:(j + 1) * art.dsub]) ** 2).sum(-1)
            code = art.codes[u, j * g.R + e]
            assert dist[code] <= dist.min() * (1 + 1e-5) + 1e-9
    assert np.array_equal(art.norms, (g.vecs16.view(np.float16).astype(np.float64) ** 2).sum(1).astype(np.float32)) \
        or np.allclose(art.norms, (g.vecs16.view(np.float16).astype(np.float64) ** 2).sum(1), rtol=1e-6)


# ------------------------------------------------------------ closed forms

def grid_graph(gx=14, gy=11, dim=16, distance="l2", R=4):
    """Points (i, j, 1, 0, ...) with 4-neighbour edges: every edge is a unit
    axis step."""
    n = gx * gy
    x = np.zeros((n, dim), dtype=np.float32)
    adj = []
    for i in range(gx):
        for j in range(gy):
            v = i * gy + j
            x[v, 0], x[v, 1], x[v, 2] = i, j, 1
            nb = []
            for di, dj in ((1, 0), (-1, 0), (0, 1), (0, -1)):
                a, b = i + di, j + dj
                if 0 <= a < gx and 0 <= b < gy:
                    nb.append(a * gy + b)
            adj.append(nb)
    edges = np.full((n, R), 0xFFFFFFFF, dtype=np.uint32)
    counts = np.zeros(n, dtype=np.uint8)
    for v, nb in enumerate(adj):
        edges[v, :len(nb)] = nb
        counts[v] = len(nb)
    g = oracle.OracleGraph(oracle.as_padded_f16(x), edges, np.zeros((n, R), np.uint16), counts, R, dim, distance,
                           medoid=0)
    return x, g


def grid_queries(dim=16):
    """Queries whose products with every grid coordinate are exact in fp16
    (the visit's IP arithmetic rounds each product to fp16)."""
    q = np.zeros((6, dim), dtype=np.float32)
    q[:, :3] = [[5.25, 3.125, 0.5], [0.375, 9.75, 2.0], [12.5, 0.25, -1.0], [7.125, 5.5625, 1.0],
                [-3.25, 4.875, 0.0], [13.5, 10.375, 3.0]]
    q[:, 3] = 0.75
    coords = np.arange(0, 14, dtype=np.float64)
    prods = q[:, :3, None].astype(np.float64) * coords[None, None, :]
    assert np.array_equal(prods.astype(np.float16).astype(np.float64), prods)
    return q


def exact_topk(x, q, k, distance):
    xd, qd = x.astype(np.float64), q.astype(np.float16).astype(np.float64)
    if distance == "l2":
        s = ((qd[:, None, :] - xd[None]) ** 2).sum(-1)
    else:
        s = -(qd @ xd.T)
    order = np.argsort(s, axis=1, kind="stable")[:, :k]
    return order, np.take_along_axis(s, order, 1)


@pytest.mark.parametrize("distance", ["l2", "ip"])
def test_lsh_estimate_exact_on_grid(distance):
    x, g = grid_graph(distance=distance)
    c, nd, nv = oracle.lsh_globals(g, 2, n_samples=4000, seed=3)
    assert nv > 0 and abs(c[0] - 1.0) < 1e-6 and c[1] == 0.0 and abs(nd - 1.0) < 1e-6
    lsh = oracle.build_lsh(g, K=2, pbytes=1, n_samples=4000, seed=3)
    q = grid_queries()
    ids, d = oracle.directional_search(g, q, lsh=lsh, k=8, beam_width=g.n, limit=2 * g.n)
    want_ids, want_d = exact_topk(x, q, 8, distance)
    assert np.array_equal(d.astype(np.float64), want_d)
    assert np.array_equal(ids, want_ids)


@pytest.mark.parametrize("distance", ["l2", "ip"])
def test_pq_estimate_exact_on_grid(distance):
    x, g = grid_graph(distance=distance)
    M = g.dp  # one coordinate per subspace
    cent = np.full((M, 256, 1), 1000.0, dtype=np.float32) + np.arange(256, dtype=np.float32)[None, :, None]
    cent[:, 0, 0], cent[:, 1, 0], cent[:, 2, 0] = 0.0, 1.0, -1.0
    codes = oracle.pq_encode(g, M, cent.ravel())
    # each code is the residual's coordinate: 0 -> 0, +1 -> 1, -1 -> 2
    for u, e, dd in _edge_diffs(g):
        want = np.where(dd == 0, 0, np.where(dd > 0, 1, 2))
        assert np.array_equal(codes[u, np.arange(M) * g.R + e], want)
    pq = oracle.PqArtifacts(M, 1, cent.ravel(), codes, oracle.vector_norms(g.vecs16))
    q = grid_queries()
    ids, d = oracle.directional_search(g, q, pq=pq, k=8, beam_width=g.n, limit=2 * g.n)
    want_ids, want_d = exact_topk(x, q, 8, distance)
    assert np.array_equal(d.astype(np.float64), want_d)
    assert np.array_equal(ids, want_ids)


def _grid_dsub8(distance, dim, swap=False):
    """The grid with its coordinates at dims 0, 9 and 18 (subspaces 0, 1
    and 2 at dsub = 8) and the queries' extra value at dim 27, and a PQ of
    M = dim / 8 whose codebooks hold the zero vector and +-1 steps along
    each of the subspace's 8 axes. swap=True exchanges the +1 and -1 steps of
    axis 0 (a wrong codebook, for the sensitivity check)."""
    x0, g0 = grid_graph(distance=distance)
    at = [0, 9, 18, 27]
    x = np.zeros((len(x0), dim), dtype=np.float32)
    x[:, at] = x0[:, :4]
    g = oracle.OracleGraph(oracle.as_padded_f16(x), g0.edges, g0.edge_dist, g0.counts, g0.R, dim, distance,
                           medoid=0)
    M, dsub = dim // 8, 8
    cent = np.full((M, 256, dsub), 1000.0, dtype=np.float32) + np.arange(256, dtype=np.float32)[None, :, None]
    cent[:, 0] = 0.0
    for t in range(dsub):
        cent[:, 1 + 2 * t] = 0.0
        cent[:, 1 + 2 * t, t] = 1.0
        cent[:, 2 + 2 * t] = 0.0
        cent[:, 2 + 2 * t, t] = -1.0
    codes = oracle.pq_encode(g, M, cent.ravel())
    if swap:
        cent[:, [1, 2]] = cent[:, [2, 1]]
    pq = oracle.PqArtifacts(M, dsub, cent.ravel(), codes, oracle.vector_norms(g.vecs16))
    q0 = grid_queries()
    q = np.zeros((len(q0), dim), dtype=np.float32)
    q[:, at] = q0[:, :4]
    return x, g, pq, q, codes


@pytest.mark.parametrize("distance", ["l2", "ip"])
@pytest.mark.parametrize("dim", [32, 960])
def test_pq_estimate_exact_on_grid_dsub8(distance, dim):
    """One subspace per 8 dims (M = 4 and 120): every edge residual's PQ
    reconstruction is exact, so a wide search returns the exact top-k."""
    x, g, pq, q, codes = _grid_dsub8(distance, dim)
    M, dsub = pq.M, pq.dsub
    for u, e, dd in _edge_diffs(g):
        for j in range(M):
            sub = dd[j * dsub:(j + 1) * dsub]
            nz = np.nonzero(sub)[0]
            want = 0 if len(nz) == 0 else (1 if sub[nz[0]] > 0 else 2) + 2 * int(nz[0])
            assert codes[u, j * g.R + e] == want
    ids, d = oracle.directional_search(g, q, pq=pq, k=8, beam_width=g.n, limit=2 * g.n)
    want_ids, want_d = exact_topk(x, q, 8, distance)
    assert np.array_equal(d.astype(np.float64), want_d)
    assert np.array_equal(ids, want_ids)


@pytest.mark.parametrize("distance", ["l2", "ip"])
def test_exact_estimators_visit_in_the_same_order(distance):
    """At a narrow beam the pop order is the order of the estimates. On the
    grid the LSH estimate (c = (1, 0)), the one-coordinate PQ and the
    8-dim-subspace PQ (d = 32 and 960) all equal the exact distance, so
    their visit sequences (ids and exact distances) must be identical; a
    codebook with the +-1 steps of one axis swapped must change it."""
    x, g = grid_graph(distance=distance)
    q = grid_queries()
    lsh = oracle.build_lsh(g, K=2, pbytes=1, n_samples=4000, seed=3)
    M = g.dp
    cent = np.full((M, 256, 1), 1000.0, dtype=np.float32) + np.arange(256, dtype=np.float32)[None, :, None]
    cent[:, 0, 0], cent[:, 1, 0], cent[:, 2, 0] = 0.0, 1.0, -1.0
    pq1 = oracle.PqArtifacts(M, 1, cent.ravel(), oracle.pq_encode(g, M, cent.ravel()),
                             oracle.vector_norms(g.vecs16))
    runs = [oracle.directional_search(g, q, lsh=lsh, k=8, beam_width=4, limit=40, get_visited=True),
            oracle.directional_search(g, q, pq=pq1, k=8, beam_width=4, limit=40, get_visited=True)]
    for dim in (32, 960):
        _, g8, pq8, q8, _ = _grid_dsub8(distance, dim)
        runs.append(oracle.directional_search(g8, q8, pq=pq8, k=8, beam_width=4, limit=40, get_visited=True))
    _, _, vi0, vd0, vc0 = runs[0]
    assert vc0.min() >= 5 and vc0.sum() > 60
    for _, _, vi, vd, vc in runs[1:]:
        assert np.array_equal(vc, vc0)
        assert np.array_equal(vi, vi0)
        assert np.array_equal(vd.view(np.uint32), vd0.view(np.uint32))
    _, gs, pqs, qs, _ = _grid_dsub8(distance, 32, swap=True)
    _, _, vis, _, vcs = oracle.directional_search(gs, qs, pq=pqs, k=8, beam_width=4, limit=40, get_visited=True)
    assert not (np.array_equal(vcs, vc0) and np.array_equal(vis, vi0))


def test_output_is_stable_topk_of_visits():
    _, g = _small_graph(n=800, dim=32, R=16)
    lsh = oracle.build_lsh(g, K=4, pbytes=1, n_samples=2000, seed=1)
    q = datasets.gaussian(20, 32, 99) * 4
    ids, d, vi, vd, vc = oracle.directional_search(g, q, lsh=lsh, k=10, beam_width=32, get_visited=True)
    for i in range(len(q)):
        m = vc[i]
        order = np.argsort(vd[i, :m], kind="stable")[:10]
        assert np.array_equal(ids[i, :len(order)], vi[i, :m][order].astype(np.int32))
        assert np.array_equal(d[i, :len(order)], vd[i, :m][order])


def _replay_frontier(vi, vd, k):
    """The exact top-k list after each visit (frontier_insert_sorted,
    beam_search_common.cuh:156-185: ascending distance, a new entry after
    equal ones, full list only takes strictly smaller)."""
    F, states = [], []
    for u, dist in zip(vi.tolist(), vd.tolist()):
        states.append([f[0] for f in F])
        if len(F) < k or dist < F[-1][1]:
            j = len(F) if len(F) < k else k - 1
            if len(F) < k:
                F.append(None)
            while j > 0 and F[j - 1][1] > dist:
                F[j] = F[j - 1]
                j -= 1
            F[j] = (u, dist)
    return F, states


def test_reference_mode_repeats_nodes_unique_mode_does_not():
    _, g = _small_graph(n=800, dim=32, R=16)
    lsh = oracle.build_lsh(g, K=4, pbytes=1, n_samples=2000, seed=1)
    q = datasets.gaussian(20, 32, 99) * 4
    ids, *_ = oracle.directional_search(g, q, lsh=lsh, k=10, beam_width=32)
    assert any(len(set(r.tolist())) < len(r) for r in ids), "expected repeated ids in the reference mode"
    uids, ud, vi, vd, vc = oracle.directional_search(g, q, lsh=lsh, k=10, beam_width=32, get_visited=True,
                                                     unique=True)
    for i in range(len(q)):
        m = int(vc[i])
        F, states = _replay_frontier(vi[i, :m], vd[i, :m], 10)
        # a pop is skipped exactly when the node is in the top-k list: no
        # visit is of a node that list held at that moment
        for t in range(m):
            assert int(vi[i, t]) not in states[t], f"query {i}: visit {t} re-visits a listed node"
        assert [f[0] for f in F] == uids[i, :len(F)].astype(np.int64).tolist()
        assert np.array_equal(np.array([f[1] for f in F], dtype=np.float32), ud[i, :len(F)])
        assert len(set(uids[i, :len(F)].tolist())) == len(F)


def test_unique_mode_pq_distinct():
    _, g = _small_graph(n=600, dim=32, R=16)
    pq = oracle.build_pq(g, M=4, n_train=600, iters=3, seed=2)
    q = datasets.gaussian(10, 32, 97) * 4
    ids, d = oracle.directional_search(g, q, pq=pq, k=10, beam_width=24, unique=True)
    for r in ids:
        assert len(set(r.tolist())) == len(r)


def test_limit_and_max_result():
    _, g = _small_graph(n=500, dim=32, R=16)
    lsh = oracle.build_lsh(g, K=4, pbytes=1, n_samples=1000, seed=1)
    q = datasets.gaussian(5, 32, 98) * 4
    *_, vc = oracle.directional_search(g, q, lsh=lsh, k=10, beam_width=64, limit=500, max_result=7,
                                       get_visited=True)
    assert (vc == 7).all()
    *_, vc = oracle.directional_search(g, q, lsh=lsh, k=10, beam_width=64, limit=3, get_visited=True)
    assert (vc <= 4).all()


def test_k_larger_than_visits_pads():
    x, g = grid_graph()
    lsh = oracle.build_lsh(g, K=2, pbytes=1, n_samples=100, seed=3)
    ids, d = oracle.directional_search(g, grid_queries()[:1], lsh=lsh, k=20, beam_width=4, limit=2)
    # limit 2 -> at most 3 visits; the rest is padding
    assert (ids[0, 3:] == 0x7FFFFFFF).all() and (d[0, 3:] == np.finfo(np.float32).max).all()


# ------------------------------------------------------------ rotation rows

def test_rotate_rows_close_to_float64():
    d = 24
    m, _ = oracle.rotation_matrix(d, 42)
    P16 = bits(f16(m))
    rng = np.random.default_rng(6)
    x = f16(rng.normal(0, 10, (50, d)))
    xp = np.zeros((50, 24), dtype=np.uint16)
    xp[:, :d] = bits(x)
    out = oracle.rotate_rows(xp, d, P16).view(np.float16).astype(np.float64)
    P = P16.view(np.float16).astype(np.float64).reshape(d, d).T    # P[k, i] = flat[k + i*d]
    want = x.astype(np.float64) @ P                                  # row r: sum_k x_k P[k, i]
    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    # one fp16 rounding of the fp32 sum, whose own error is below d ulp(fp32) of sum |x_k P_ki|
    acc_err = d * 2.0 ** -23 * (np.abs(x.astype(np.float64)) @ np.abs(P))
    assert np.all(np.abs(out - want) <= ulp * 0.5 + acc_err)
