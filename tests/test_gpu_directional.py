"""GPU parity of the directional path against the oracle.

Each case builds a directional graph on the GPU (Vamana build, optional
prerotation, LSH and/or PQ artifacts), saves it in the reference format,
reads the base section back with the oracle's loader, and checks:
  * prerotated rows (matrix-core GEMM, fp32 accumulation) are within one
    fp16 rounding plus the fp32 accumulation bound of the oracle's rotation;
    the same holds for rotated queries;
  * the graph equals the oracle's build of the stored rows;
  * LSH calibration constants and per-edge rows are bit-identical to the
    oracle's, and so are PQ centroids, codes and vector norms;
  * directional_search / pq_search ids and distances are bit-identical to
    the oracle's traversal with the same artifacts;
  * a save -> load round trip (trailer included) searches identically.
"""

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import compare_search, gaussian, integer_clustered, unit

pytestmark = pytest.mark.gpu


def assert_rotation_close(got16, x, dim, seed=42):
    """GEMM rows vs the exact product P^T x (fp16 P): at most half an fp16
    ulp from rounding plus the fp32 accumulation bound."""
    m, _ = oracle.rotation_matrix(dim, seed)
    P = m.astype(np.float16).astype(np.float64).reshape(dim, dim).T   # P[k, i]
    xf = x.astype(np.float16).astype(np.float64)
    want = xf @ P
    got = got16[:, :dim].view(np.float16).astype(np.float64)
    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    acc = dim * 2.0 ** -23 * (np.abs(xf) @ np.abs(P))
    bad = np.abs(got - want) > 0.5 * ulp + acc
    assert not bad.any(), f"{bad.sum()} rotated entries off, worst {np.abs(got - want).max()}"
    assert not got16[:, dim:].any()


def _search(gg, fn, q, k, bw, limit=None, unique=False):
    qt = torch.from_numpy(np.ascontiguousarray(q.astype(np.float16))).cuda()
    ids, d = getattr(gg, fn)(qt, k=k, beam_width=bw, limit=limit, unique=unique)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), d.cpu().numpy()


def _check_unique(gg, g, fn, q, q_rows, bw, **art):
    """unique=True (distinct results) against the oracle's same mode."""
    ids, d = _search(gg, fn, q, 10, bw, unique=True)
    rid, rd = oracle.directional_search(g, q_rows, k=10, beam_width=bw, unique=True, **art)
    msg = compare_search(ids, d, rid, rd)
    assert msg is None, f"{fn} unique bw={bw}: {msg}"
    for row in ids:
        live = row[row != 0x7FFFFFFF]
        assert len(set(live.tolist())) == len(live), f"{fn} unique bw={bw}: repeated id in {row}"


def _case(jasper, tmp_path, x, q, *, R, distance, k_ranks, prerotate, lsh, pq, bws=(16, 64),
          lsh_samples=4000, pq_train=3000, pq_iters=4, pq_m=None):
    n, dim = x.shape
    M = pq_m or k_ranks
    xt = torch.from_numpy(x.astype(np.float16)).cuda()
    gg = jasper.Graph.build(xt, n_neighbors=R, distance=distance, build_lsh=lsh, build_pq=pq, k_ranks=k_ranks,
                            prerotate=prerotate, lsh_samples=lsh_samples, lsh_seed=7, pq_train=pq_train,
                            pq_kmeans_iter=pq_iters, pq_seed=11, pq_m=pq_m)
    path = tmp_path / "dir.bin"
    gg.save(str(path))
    g = oracle.load_graph(path, dim, R, distance)

    rows = gg.export_vectors()
    if prerotate:
        assert_rotation_close(rows, x, dim)
    else:
        assert np.array_equal(rows, oracle.as_padded_f16(x)), "stored rows differ"
    assert np.array_equal(g.vecs16, rows)
    ref = oracle.build(rows.view(np.float16)[:, :dim].astype(np.float32), R=R, distance=distance, alpha=1.2)
    assert g.medoid == ref.medoid
    assert np.array_equal(g.counts, ref.counts)
    for i in range(n):
        c = int(ref.counts[i])
        assert np.array_equal(g.edges[i, :c], ref.edges[i, :c]), f"vertex {i}"

    q_rows = gg.directional_query_rows(torch.from_numpy(q.astype(np.float16)).cuda())
    if prerotate:
        assert_rotation_close(q_rows, q, dim)
    else:
        assert np.array_equal(q_rows, oracle.as_padded_f16(q))
    pbytes = 1 if dim <= 128 else 2
    out = {}
    if lsh:
        c, nd, lrows = gg.export_lsh()
        rc, rnd, nv = oracle.lsh_globals(g, k_ranks, n_samples=lsh_samples, seed=7)
        assert nv > 0
        assert np.array_equal(c.view(np.uint32), rc.view(np.uint32)), (c, rc)
        assert np.float32(nd).view(np.uint32) == np.float32(rnd).view(np.uint32)
        want_rows = oracle.populate_lsh(g, k_ranks, pbytes)
        assert np.array_equal(lrows, want_rows), "LSH rows differ"
        art = oracle.LshArtifacts(k_ranks, pbytes, c, nd, lrows)
        for bw in bws:
            ids, d = _search(gg, "directional_search", q, 10, bw)
            rid, rd = oracle.directional_search(g, q_rows, lsh=art, k=10, beam_width=bw)
            msg = compare_search(ids, d, rid, rd)
            assert msg is None, f"lsh bw={bw}: {msg}"
            out[("lsh", bw)] = (ids, d)
            _check_unique(gg, g, "directional_search", q, q_rows, bw, lsh=art)
    if pq:
        cent, codes, norms = gg.export_pq()
        rcent, _ = oracle.pq_train(g, M, n_train=pq_train, iters=pq_iters, seed=11)
        assert np.array_equal(cent.view(np.uint32), rcent.view(np.uint32)), "PQ centroids differ"
        rcodes = oracle.pq_encode(g, M, rcent)
        assert codes.shape == rcodes.shape == (n, M * R)
        assert np.array_equal(codes, rcodes), "PQ codes differ"
        rnorms = oracle.vector_norms(g.vecs16)
        assert np.array_equal(norms.view(np.uint32), rnorms.view(np.uint32)), "vector norms differ"
        art = oracle.PqArtifacts(M, g.dp // M, cent, codes, norms)
        for bw in bws:
            ids, d = _search(gg, "pq_search", q, 10, bw)
            rid, rd = oracle.directional_search(g, q_rows, pq=art, k=10, beam_width=bw)
            msg = compare_search(ids, d, rid, rd)
            assert msg is None, f"pq bw={bw}: {msg}"
            out[("pq", bw)] = (ids, d)
            _check_unique(gg, g, "pq_search", q, q_rows, bw, pq=art)

    # save -> load round trip keeps the artifacts and the results
    g2 = jasper.Graph.load(str(path), dim=dim, n_neighbors=R, distance=distance, k_ranks=k_ranks,
                           prerotate=prerotate)
    if pq:
        assert np.array_equal(g2.export_pq()[1], codes), "PQ codes changed in the file round trip"
    for (kind, bw), (ids, d) in out.items():
        ids2, d2 = _search(g2, "directional_search" if kind == "lsh" else "pq_search", q, 10, bw)
        msg = compare_search(ids2, d2, ids, d)
        assert msg is None, f"after load, {kind} bw={bw}: {msg}"
    g2.free()
    gg.free()


def test_lsh_pq_l2_small_dim(jasper, oracle_lib, tmp_path):
    x = gaussian(2000, 96, 20)
    q = gaussian(48, 96, 21)
    _case(jasper, tmp_path, x, q, R=32, distance="l2", k_ranks=4, prerotate=False, lsh=True, pq=True)


def test_lsh_pq_l2_prerotated(jasper, oracle_lib, tmp_path):
    x = integer_clustered(2500, 128, 22)
    q = integer_clustered(40, 128, 23)
    _case(jasper, tmp_path, x, q, R=64, distance="l2", k_ranks=16, prerotate=True, lsh=True, pq=True,
          bws=(32, 96, 256))


def test_lsh_pq_long_rows(jasper, oracle_lib, tmp_path):
    """Config 4's shape at small n: dim 960 (u16 LSH words, PQ M=16 with
    dsub=60), prerotated as the Python default for build_pq does."""
    from jasper_amd import datasets
    x = datasets.sparse_abs(1200, 960, 26)
    q = datasets.sparse_abs(24, 960, 27)
    _case(jasper, tmp_path, x, q, R=32, distance="l2", k_ranks=16, prerotate=True, lsh=True, pq=True,
          bws=(16, 64), pq_train=1500, pq_iters=3)


def test_config3_shape(jasper, oracle_lib, tmp_path):
    """Config 3's parameters at reduced n: unit-sphere d = 96, inner
    product, R = 64, LSH k_ranks = 4 with u8 words, prerotated, 32768
    calibration samples, beam widths 32..128."""
    x = unit(3000, 96, 40)
    q = unit(40, 96, 41)
    _case(jasper, tmp_path, x, q, R=64, distance="ip", k_ranks=4, prerotate=True, lsh=True, pq=False,
          bws=(32, 64, 128), lsh_samples=32768)


@pytest.mark.parametrize("pq_m", [16, 120])
def test_config4_shape(jasper, oracle_lib, tmp_path, pq_m):
    """Config 4's parameters at reduced n: sparse non-negative d = 960, L2,
    R = 64, prerotated, PQ with 8-bit codebooks; M = 16 (the largest the
    reference's configs offer, dsub = 60) and M = 120 (one subspace per
    8 dims as the config asks, a 120 KB table per query)."""
    from jasper_amd import datasets
    x = datasets.sparse_abs(1500, 960, 42)
    q = datasets.sparse_abs(24, 960, 43)
    _case(jasper, tmp_path, x, q, R=64, distance="l2", k_ranks=16, prerotate=True, lsh=False, pq=True,
          bws=(32, 64), pq_train=2000, pq_iters=3, pq_m=pq_m)


@pytest.mark.parametrize("pq_m", [80, 96, 120])
def test_pq_table_split(jasper, oracle_lib, pq_m):
    """More queries than the device has CUs with a table of more than 64
    subspaces: each query's wave keeps the first 4 groups of 16 subspaces'
    table rows in LDS and reads the rest from global memory, so that two
    queries share a CU. 600 queries at d = 960, R = 64, M = 80 (one group
    gathered), 96 (two) and 120 (config 4: the last group's 8 rows in LDS
    beside the first 4 groups at beam width 64, gathered with groups 4-6
    at 256), plain and distinct-results traversals: bit-identical to the
    oracle, and to the first 24 queries searched alone (a launch that keeps
    the whole table in LDS)."""
    from jasper_amd import datasets
    dim, R = 960, 64
    x = datasets.sparse_abs(1500, dim, 42)
    q = datasets.sparse_abs(600, dim, 43)
    xt = torch.from_numpy(x.astype(np.float16)).cuda()
    print(f"[pq split] M={pq_m} n=1500 nq=600", flush=True)
    gg = jasper.Graph.build(xt, n_neighbors=R, distance="l2", build_pq=True, prerotate=True, pq_train=1500,
                            pq_kmeans_iter=2, pq_seed=11, pq_m=pq_m)
    rows = gg.export_vectors()
    g = oracle.build(rows.view(np.float16)[:, :dim].astype(np.float32), R=R, distance="l2", alpha=1.2)
    cent, codes, norms = gg.export_pq()
    assert np.array_equal(codes, oracle.pq_encode(g, pq_m, cent)), "PQ codes differ"
    art = oracle.PqArtifacts(pq_m, g.dp // pq_m, cent, codes, norms)
    q_rows = gg.directional_query_rows(torch.from_numpy(q.astype(np.float16)).cuda())
    for bw in (64, 256):
        for unique in (False, True):
            print(f"[pq split] M={pq_m} bw={bw} unique={unique}", flush=True)
            ids, d = _search(gg, "pq_search", q, 10, bw, unique=unique)
            rid, rd = oracle.directional_search(g, q_rows, pq=art, k=10, beam_width=bw, unique=unique)
            msg = compare_search(ids, d, rid, rd)
            assert msg is None, f"M={pq_m} bw={bw} unique={unique}: {msg}"
            ids24, d24 = _search(gg, "pq_search", q[:24], 10, bw, unique=unique)
            msg = compare_search(ids24, d24, ids[:24], d[:24])
            assert msg is None, f"M={pq_m} bw={bw} unique={unique}, 24 queries alone: {msg}"
    gg.free()


@pytest.mark.parametrize("pq_m", [8, 12, 24, 32])
def test_pq_subspace_counts(jasper, oracle_lib, tmp_path, pq_m):
    """PQ at subspace counts between the reference's 4 and 16 and beyond:
    8-code groups (m = 8), a partly filled 16-code group (12), two and
    three groups (24, 32), and dsub = 12, 8, 4, 3 for the table kernels."""
    x = gaussian(1500, 96, 44)
    q = gaussian(32, 96, 45)
    _case(jasper, tmp_path, x, q, R=32, distance="l2", k_ranks=4, prerotate=False, lsh=False, pq=True,
          bws=(16, 64), pq_m=pq_m)


def test_pq_ip_wide(jasper, oracle_lib, tmp_path):
    x = unit(1500, 64, 46)
    q = unit(32, 64, 47)
    _case(jasper, tmp_path, x, q, R=32, distance="ip", k_ranks=4, prerotate=True, lsh=False, pq=True,
          bws=(32,), pq_m=32)


def test_lsh_ip(jasper, oracle_lib, tmp_path):
    x = unit(2000, 64, 24)
    q = unit(40, 64, 25)
    _case(jasper, tmp_path, x, q, R=32, distance="ip", k_ranks=4, prerotate=True, lsh=True, pq=True)


def test_large_dim_u16_words(jasper, oracle_lib, tmp_path):
    x = gaussian(1200, 200, 26)
    q = gaussian(24, 200, 27)
    _case(jasper, tmp_path, x, q, R=32, distance="l2", k_ranks=4, prerotate=False, lsh=True, pq=True,
          bws=(32,))


@pytest.mark.parametrize("dim,R,k_ranks", [(40, 32, 16), (40, 32, 4), (100, 64, 16), (128, 32, 4)])
def test_lsh_rows_short_dims(jasper, oracle_lib, tmp_path, dim, R, k_ranks):
    """LSH rows of the at-most-128-coordinate kernel against the oracle: row
    widths that leave lanes without coordinates (dim 40, and dim 100 whose
    rows pad to 104), K below and equal to the lane count, vertices with
    fewer than R edges, and repeated rows (zero differences, whose keys
    carry only the coordinate index)."""
    x = gaussian(900, dim, 33)
    x[300:330] = x[200:230]
    x[600] = x[601]
    gg = jasper.Graph.build(torch.from_numpy(x.astype(np.float16)).cuda(), n_neighbors=R, build_lsh=True,
                            k_ranks=k_ranks, lsh_samples=500, prerotate=False)
    path = tmp_path / "dir.bin"
    gg.save(str(path))
    g = oracle.load_graph(path, dim, R, "l2")
    assert (g.counts < R).any()
    _, _, lrows = gg.export_lsh()
    want = oracle.populate_lsh(g, k_ranks, 1)
    assert lrows.shape == want.shape
    bad = np.nonzero((lrows != want).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} LSH rows differ, first vertex {bad[0] if bad.size else None}"
    gg.free()


def test_lsh_wide_beam(jasper, oracle_lib, tmp_path):
    """A beam of 1024 at R = 64, K = 16: the general merge on a head of
    more than 128 entries on most hops, with more than 8 rows to move on
    many (the row masks then come from the keys' positions in scalar
    registers), and LDS bounds residency, so the square roots are computed
    instead of read from the LDS table. Both traversals against the oracle,
    for LSH and for PQ (M = 16) on the same graph."""
    x = integer_clustered(3000, 128, 34)
    q = integer_clustered(24, 128, 35)
    gg = jasper.Graph.build(torch.from_numpy(x.astype(np.float16)).cuda(), n_neighbors=64, build_lsh=True,
                            build_pq=True, k_ranks=16, lsh_samples=2000, pq_train=2000, pq_kmeans_iter=3,
                            pq_seed=11, prerotate=False)
    path = tmp_path / "dir.bin"
    gg.save(str(path))
    g = oracle.load_graph(path, 128, 64, "l2")
    c, nd, lrows = gg.export_lsh()
    lsh = oracle.LshArtifacts(16, 1, c, nd, lrows)
    cent, codes, norms = gg.export_pq()
    pq = oracle.PqArtifacts(16, g.dp // 16, cent, codes, norms)
    q_rows = oracle.as_padded_f16(q)
    for fn, art in (("directional_search", {"lsh": lsh}), ("pq_search", {"pq": pq})):
        for unique in (False, True):
            ids, d = _search(gg, fn, q, 10, 1024, unique=unique)
            rid, rd = oracle.directional_search(g, q_rows, k=10, beam_width=1024, unique=unique, **art)
            msg = compare_search(ids, d, rid, rd)
            assert msg is None, f"{fn} unique={unique}: {msg}"
    gg.free()


def test_lsh_only_then_pq_search_rejected(jasper, oracle_lib):
    x = gaussian(600, 64, 28)
    gg = jasper.Graph.build(torch.from_numpy(x.astype(np.float16)).cuda(), n_neighbors=32, build_lsh=True,
                            k_ranks=4, lsh_samples=1000)
    with pytest.raises(RuntimeError):
        gg.pq_search(torch.from_numpy(x[:4].astype(np.float16)).cuda(), k=5)
    gg.free()


def test_directional_k_larger_than_visits(jasper, oracle_lib):
    x = gaussian(600, 64, 29)
    gg = jasper.Graph.build(torch.from_numpy(x.astype(np.float16)).cuda(), n_neighbors=32, build_lsh=True,
                            k_ranks=4, lsh_samples=1000, prerotate=False)
    ids, d = _search(gg, "directional_search", x[:3], k=30, bw=4, limit=2)
    assert (ids[:, 3:] == 0x7FFFFFFF).all()
    assert (d[:, 3:] == np.finfo(np.float32).max).all()
    gg.free()


@pytest.mark.parametrize("dim", [40, 100, 200])
def test_prerotated_build_rows(jasper, oracle_lib, dim):
    """Prerotated build: stored rows and query rows at dims that exercise the
    K/M padding cases of the matrix-core rotation."""
    x = gaussian(300, dim, 30) * 3
    q = gaussian(37, dim, 31) * 3
    gg = jasper.Graph.build(torch.from_numpy(x.astype(np.float16)).cuda(), n_neighbors=32, build_lsh=True,
                            k_ranks=4, lsh_samples=500, prerotate=True)
    assert_rotation_close(gg.export_vectors(), x, dim)
    assert_rotation_close(gg.directional_query_rows(torch.from_numpy(q.astype(np.float16)).cuda()), q, dim)
    gg.free()


@pytest.mark.parametrize("dim,n", [(8, 5), (33, 70), (96, 1000), (128, 4099), (160, 500), (200, 777), (250, 64),
                                   (960, 300), (960, 2100), (1000, 130)])
def test_rotate_operator(jasper, oracle_lib, dim, n):
    """The stand-alone rotation (device and host inputs, unaligned strides,
    more than 64 KB of LDS per block at dim 160, the LDS-tiled GEMM above
    dim 192: partial output and row blocks, dim 1000 with K padded to 1024
    and outputs past the row's stride)."""
    x = (gaussian(n, dim, 32) * 4).astype(np.float16)
    got = jasper.rotate(torch.from_numpy(x).cuda(), seed=42)
    torch.cuda.synchronize()
    g16 = np.zeros((n, (dim + 7) // 8 * 8), dtype=np.uint16)
    g16[:, :dim] = got.cpu().numpy().view(np.uint16)
    assert_rotation_close(g16, x.astype(np.float32), dim)
    got_h = jasper.rotate(torch.from_numpy(x), seed=42)     # host input
    assert torch.equal(got_h.cpu(), got.cpu())


def test_prerotation_recorded_in_file(jasper, oracle_lib, tmp_path):
    # the trailer records the prerotation (flag 8 and the seed); a load that
    # does not ask for it still rotates queries the same way
    x = integer_clustered(1500, 64, 71)
    q = integer_clustered(32, 64, 72)
    xt = torch.from_numpy(x.astype(np.float16)).cuda()
    gg = jasper.Graph.build(xt, n_neighbors=32, distance="l2", build_lsh=True, k_ranks=4, prerotate=True,
                            prerotate_seed=7, lsh_samples=4000, lsh_seed=7)
    path = tmp_path / "rot.bin"
    gg.save(str(path))
    ids, d = _search(gg, "directional_search", q, 10, 32)
    g2 = jasper.Graph.load(str(path), dim=64, n_neighbors=32, distance="l2", k_ranks=4, prerotate=False)
    assert g2._prerotate and g2._prerotate_seed == 7
    assert "prerotate=True" in repr(g2)
    ids2, d2 = _search(g2, "directional_search", q, 10, 32)
    assert compare_search(ids2, d2, ids, d) is None
    # the base section is the reference's format: its loader reads it as before
    g = oracle.load_graph(path, 64, 32, "l2")
    assert np.array_equal(g.vecs16, gg.export_vectors())
    g2.free()
    gg.free()


# ---------------------------------------------------------------- RaBitQ --

def _rq_case(jasper, tmp_path, x, q, *, R, distance, prerotate, bws):
    """build_rabitq on a directional graph: the codes are the oracle
    quantizer's on the stored rows against the stored rows' mean (codes
    bit-exact, factors within the fp32 reduction-order bound), and
    rabitq_search returns the oracle traversal's ids and distances bit for
    bit on the exported codes; a file round trip keeps them."""
    n, dim = x.shape
    xt = torch.from_numpy(x.astype(np.float16)).cuda()
    gg = jasper.Graph.build(xt, n_neighbors=R, distance=distance, build_lsh=True, build_rabitq=True, k_ranks=4,
                            prerotate=prerotate, lsh_samples=2000)
    rows = gg.export_vectors()
    stored = rows.view(np.float16)[:, :dim].astype(np.float32)
    cent, nodes = gg.export_rabitq()
    mean = stored.astype(np.float64).mean(0)
    assert np.abs(cent - mean).max() <= 1e-5 * (np.abs(mean).max() + 1.0)
    ref_nodes, ref_codes, ref_add, ref_res = oracle.rabitq_quantize(stored, np.eye(dim, dtype=np.float32).ravel(),
                                                                    centroid=cent, metric=distance)
    cb = oracle.rabitq_code_bytes(dim)
    assert nodes.shape == ref_nodes.shape
    assert np.array_equal(nodes[:, :cb], ref_codes), "RaBitQ codes differ"
    f = np.ascontiguousarray(nodes[:, cb:]).view(np.float32)
    assert np.allclose(f[:, 0], ref_add, rtol=2e-5, atol=1e-5 * np.abs(ref_add).max())
    assert np.allclose(f[:, 1], ref_res, rtol=2e-5)

    path = tmp_path / "rq.bin"
    gg.save(str(path))
    g = oracle.load_graph(path, dim, R, distance)
    rq = oracle.RqArtifacts(dim, nodes, cent)
    q_rows = gg.directional_query_rows(torch.from_numpy(q.astype(np.float16)).cuda())
    qt = torch.from_numpy(np.ascontiguousarray(q.astype(np.float16))).cuda()
    out = {}
    for bw in bws:
        for unique in (False, True):
            ids, d = gg.rabitq_search(qt, k=10, beam_width=bw, unique=unique)
            torch.cuda.synchronize()
            ids, d = ids.cpu().numpy(), d.cpu().numpy()
            rid, rd = oracle.directional_search(g, q_rows, rq=rq, k=10, beam_width=bw, unique=unique)
            msg = compare_search(ids, d, rid, rd)
            assert msg is None, f"rabitq bw={bw} unique={unique}: {msg}"
            out[(bw, unique)] = (ids, d)
    g2 = jasper.Graph.load(str(path), dim=dim, n_neighbors=R, distance=distance, k_ranks=4, prerotate=prerotate)
    assert g2._has_rabitq and g2._has_lsh
    c2, n2 = g2.export_rabitq()
    assert np.array_equal(c2.view(np.uint32), cent.view(np.uint32)) and np.array_equal(n2, nodes)
    for (bw, unique), (ids, d) in out.items():
        ids2, d2 = g2.rabitq_search(qt, k=10, beam_width=bw, unique=unique)
        torch.cuda.synchronize()
        assert compare_search(ids2.cpu().numpy(), d2.cpu().numpy(), ids, d) is None
    g2.free()
    gg.free()


def test_rabitq_l2_prerotated(jasper, oracle_lib, tmp_path):
    x = integer_clustered(3000, 128, 50)
    q = integer_clustered(40, 128, 51)
    _rq_case(jasper, tmp_path, x, q, R=64, distance="l2", prerotate=True, bws=(16, 64, 160))


def test_rabitq_ip_d96(jasper, oracle_lib, tmp_path):
    # d = 96: 12 code bytes, 20-byte nodes (4-byte aligned only)
    x = unit(2500, 96, 52)
    q = unit(32, 96, 53)
    _rq_case(jasper, tmp_path, x, q, R=32, distance="ip", prerotate=True, bws=(32, 96))


def test_rabitq_l2_d200_unrotated(jasper, oracle_lib, tmp_path):
    # d = 200: 28 code bytes (seven code words, the eight-word kernel)
    x = gaussian(2000, 200, 54)
    q = gaussian(32, 200, 55)
    _rq_case(jasper, tmp_path, x, q, R=32, distance="l2", prerotate=False, bws=(32,))


def test_exact_search_on_directional_and_plain_graphs(jasper, oracle_lib, tmp_path):
    """exact_search (an extension): the plain beam search on the stored rows
    with the queries rotated as directional_search rotates them; on a
    prerotated directional graph it equals the oracle's plain search of the
    saved graph with the rotated query rows, on a plain graph it equals
    search()."""
    x = integer_clustered(3000, 128, 60)
    q = integer_clustered(40, 128, 61)
    qt = torch.from_numpy(q.astype(np.float16)).cuda()
    gg = jasper.Graph.build(torch.from_numpy(x.astype(np.float16)).cuda(), n_neighbors=32, build_lsh=True,
                            k_ranks=4, prerotate=True, lsh_samples=2000)
    path = tmp_path / "ex.bin"
    gg.save(str(path))
    g = oracle.load_graph(path, 128, 32, "l2")
    q_rows = gg.directional_query_rows(qt)
    for bw in (16, 64):
        ids, d = gg.exact_search(qt, k=10, beam_width=bw)
        torch.cuda.synchronize()
        rid, rd = oracle.beam_search(g, q_rows, k=10, beam_width=bw)
        assert compare_search(ids.cpu().numpy(), d.cpu().numpy(), rid, rd) is None
    gg.free()
    pg = jasper.Graph.build(torch.from_numpy(x.astype(np.float16)).cuda(), n_neighbors=32)
    a, ad = pg.search(qt, k=10, beam_width=48)
    b, bd = pg.exact_search(qt, k=10, beam_width=48)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(ad, bd)
    pg.free()
