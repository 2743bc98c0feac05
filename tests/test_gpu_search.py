"""GPU parity of plain beam search against the oracle, on fixed graphs.

A graph is built by the oracle (CPU), written in the reference file format,
loaded by the HIP library, and searched by both. Ids and distances must be
bit-identical (reference contract: bit-exact ids on a fixed graph with the
same entry point and beam width; distances are the same fp32 bits because
the accumulation order is reproduced).
"""

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import compare_search, gaussian, integer_clustered, unit

pytestmark = pytest.mark.gpu


def _load(jasper, g, tmp_path, name="g.bin"):
    path = tmp_path / name
    oracle.save_graph(g, path)
    return jasper.Graph.load(str(path), dim=g.dim, n_neighbors=g.R, distance=g.distance)


def _run(jasper, gg, q, k, bw):
    qt = torch.from_numpy(np.ascontiguousarray(q)).cuda()
    ids, d = gg.search(qt, k=k, beam_width=bw)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), d.cpu().numpy()


@pytest.fixture(scope="module")
def c1_small(oracle_lib):
    base = gaussian(3000, 128, 0)
    q = gaussian(64, 128, 1)
    g = oracle.build(base, R=32, distance="l2", alpha=1.2)
    return base, q, g


@pytest.mark.parametrize("bw", [16, 64, 128, 300])
def test_search_matches_oracle_gaussian_l2(jasper, c1_small, tmp_path, bw):
    base, q, g = c1_small
    gg = _load(jasper, g, tmp_path)
    ids, d = _run(jasper, gg, q, 10, bw)
    rid, rd = oracle.beam_search(g, q, k=10, beam_width=bw)
    msg = compare_search(ids, d, rid, rd)
    assert msg is None, msg


def test_search_matches_oracle_integer_l2_r64(jasper, oracle_lib, tmp_path):
    base = integer_clustered(4000, 128, 0)
    q = integer_clustered(64, 128, 1)
    g = oracle.build(base, R=64, distance="l2", alpha=1.2)
    gg = _load(jasper, g, tmp_path)
    for bw in (32, 96, 256, 600):
        ids, d = _run(jasper, gg, q, 10, bw)
        rid, rd = oracle.beam_search(g, q, k=10, beam_width=bw)
        msg = compare_search(ids, d, rid, rd)
        assert msg is None, f"bw={bw}: {msg}"


@pytest.mark.parametrize("R,dim", [(8, 64), (16, 96), (64, 200)])
def test_search_matches_oracle_shapes(jasper, oracle_lib, tmp_path, R, dim):
    base = gaussian(1500, dim, 3)
    q = gaussian(40, dim, 4)
    g = oracle.build(base, R=R, distance="l2", alpha=1.2)
    gg = _load(jasper, g, tmp_path)
    ids, d = _run(jasper, gg, q, 10, 48)
    rid, rd = oracle.beam_search(g, q, k=10, beam_width=48)
    msg = compare_search(ids, d, rid, rd)
    assert msg is None, msg


def test_search_matches_oracle_ip(jasper, oracle_lib, tmp_path):
    base = unit(2500, 96, 5)
    q = unit(48, 96, 6)
    g = oracle.build(base, R=32, distance="ip", alpha=1.2)
    gg = _load(jasper, g, tmp_path)
    for bw in (16, 64, 160):
        ids, d = _run(jasper, gg, q, 10, bw)
        rid, rd = oracle.beam_search(g, q, k=10, beam_width=bw)
        msg = compare_search(ids, d, rid, rd)
        assert msg is None, f"bw={bw}: {msg}"


def test_search_k_larger_than_beam_pads(jasper, c1_small, tmp_path):
    base, q, g = c1_small
    gg = _load(jasper, g, tmp_path)
    ids, d = _run(jasper, gg, q[:8], 80, 16)
    rid, rd = oracle.beam_search(g, q[:8], k=80, beam_width=16)
    msg = compare_search(ids, d, rid, rd)
    assert msg is None, msg
    assert (ids[:, 16:] == -1).all() and (d[:, 16:] == np.float32(1e30)).all()


def test_search_empty_query_batch(jasper, c1_small, tmp_path):
    base, q, g = c1_small
    gg = _load(jasper, g, tmp_path)
    ids, d = gg.search(torch.empty(0, 128, dtype=torch.float16, device="cuda"), k=10, beam_width=16)
    assert ids.shape == (0, 10)


def test_search_single_vertex_graph(jasper, oracle_lib, tmp_path):
    base = gaussian(1, 128, 9)
    g = oracle.build(base, R=32, distance="l2", alpha=1.2, max_batch=1)
    gg = _load(jasper, g, tmp_path)
    q = gaussian(3, 128, 10)
    ids, d = _run(jasper, gg, q, 5, 16)
    rid, rd = oracle.beam_search(g, q, k=5, beam_width=16)
    msg = compare_search(ids, d, rid, rd)
    assert msg is None, msg
    assert (ids[:, 0] == 0).all() and (ids[:, 1:] == -1).all()


def test_search_rejects_oversized_beam(jasper, c1_small, tmp_path):
    base, q, g = c1_small
    gg = _load(jasper, g, tmp_path)
    with pytest.raises(ValueError):
        gg.search(torch.from_numpy(q).cuda(), k=10, beam_width=1990)


def test_search_matches_oracle_subnormal_range(jasper, oracle_lib, tmp_path):
    """Values in the fp16 subnormal range exercise the in-instruction fp16
    conversion of the L2 scoring (and the oracle's exact conversions)."""
    base = gaussian(1500, 64, 50) * 3e-5
    q = gaussian(40, 64, 51) * 3e-5
    assert (np.abs(base.astype(np.float16)) < 6.1e-5).mean() > 0.5
    g = oracle.build(base, R=16, distance="l2", alpha=1.2)
    gg = _load(jasper, g, tmp_path)
    for bw in (16, 64):
        ids, d = _run(jasper, gg, q, 10, bw)
        rid, rd = oracle.beam_search(g, q, k=10, beam_width=bw)
        msg = compare_search(ids, d, rid, rd)
        assert msg is None, f"bw={bw}: {msg}"


@pytest.mark.parametrize("distance,dim,R", [("l2", 264, 32), ("l2", 960, 64), ("ip", 300, 32)])
def test_search_matches_oracle_long_rows(jasper, oracle_lib, tmp_path, distance, dim, R):
    """Rows longer than 32 chunks (dim > 256) are scored streamed from
    memory instead of from register fragments; same order, same bits."""
    from jasper_amd import datasets
    if distance == "ip":
        base, q = unit(1200, dim, 60), unit(32, dim, 61)
    else:
        base, q = datasets.sparse_abs(1200, dim, 60), datasets.sparse_abs(32, dim, 61)
    g = oracle.build(base, R=R, distance=distance, alpha=1.2)
    gg = _load(jasper, g, tmp_path)
    for bw in (16, 64):
        ids, d = _run(jasper, gg, q, 10, bw)
        rid, rd = oracle.beam_search(g, q, k=10, beam_width=bw)
        msg = compare_search(ids, d, rid, rd)
        assert msg is None, f"bw={bw}: {msg}"


@pytest.mark.parametrize("bw", [16, 64, 128])
def test_search_stats_match_oracle_counters(jasper, c1_small, tmp_path, bw):
    # the measurement run (exact seen set) walks the same traversal as the
    # reference: hops and degrees read equal the oracle's, vectors scored
    # equal the oracle's distinct scored ids; predicted hops are a subset
    base, q, g = c1_small
    gg = _load(jasper, g, tmp_path)
    st = gg.search_stats(torch.from_numpy(q).cuda(), k=10, beam_width=bw).astype(np.int64)
    _, _, ost = oracle.beam_search(g, q, k=10, beam_width=bw, stats=True)
    ost = ost.astype(np.int64)
    assert np.array_equal(st[:, 0], ost[:, 0])
    assert np.array_equal(st[:, 1], ost[:, 1])
    assert np.array_equal(st[:, 2], ost[:, 3])
    assert (st[:, 3] >= 0).all() and (st[:, 3] <= st[:, 0]).all()


_SMALL_CACHE_CHILD = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
import jasper_amd
g = jasper_amd.Graph.load(sys.argv[2], dim=int(sys.argv[3]), n_neighbors=int(sys.argv[4]), distance="l2")
q = torch.from_numpy(np.load(sys.argv[5])).cuda()
out = {}
for bw in (16, 48, 64):
    ids, d = g.search(q, k=10, beam_width=bw)
    torch.cuda.synchronize()
    out[f"ids{bw}"] = ids.cpu().numpy()
    out[f"d{bw}"] = d.cpu().numpy()
np.savez(sys.argv[6], **out)
print("child done", flush=True)
"""


def test_search_small_seen_cache_matches_oracle(jasper, oracle_lib, tmp_path):
    # a 256-entry seen cache forgets most of the ~1,000 vectors a query
    # scores, so members of the beam are re-scored and come back as
    # duplicates: the merge's general path (duplicates, members of B) runs
    # on many hops beside the register merge; results must not change
    import os
    import subprocess
    import sys
    from pathlib import Path
    base = integer_clustered(4000, 128, 3)
    q = integer_clustered(64, 128, 4)
    g = oracle.build(base, R=64, distance="l2", alpha=1.2)
    path = tmp_path / "g.bin"
    oracle.save_graph(g, path)
    np.save(tmp_path / "q.npy", q)
    env = dict(os.environ, JASPER_SEARCH_HASH_BITS="8")
    root = str(Path(__file__).resolve().parents[1])
    r = subprocess.run([sys.executable, "-c", _SMALL_CACHE_CHILD, root, str(path), "128", "64",
                        str(tmp_path / "q.npy"), str(tmp_path / "out.npz")],
                       env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    out = np.load(tmp_path / "out.npz")
    for bw in (16, 48, 64):
        rid, rd = oracle.beam_search(g, q, k=10, beam_width=bw)
        msg = compare_search(out[f"ids{bw}"], out[f"d{bw}"], rid, rd)
        assert msg is None, f"bw={bw}: {msg}"


def test_search_integer_queries_exact_span(jasper, oracle_lib, tmp_path):
    # rows are integers in [260, 299]; the packed form is taken per query
    # only when the query is integer-valued and the union of its values with
    # the rows' spans at most 362 (dim 128: 128 * 362^2 < 2^24). A query at
    # -100 spans 399: its partial sums pass 2^24 with odd terms, where the
    # fp32 chain rounds in order, so only the chain matches the oracle.
    rng = np.random.default_rng(21)
    base = rng.integers(260, 300, size=(2000, 128)).astype(np.float16)
    q = np.concatenate([
        rng.integers(260, 300, size=(16, 128)),
        np.full((4, 128), -63),                      # union span 362: packed form
        np.full((4, 128), -100),                     # span 399: fp32 chain
        rng.integers(-100, 300, size=(8, 128)),      # mixed spans
    ]).astype(np.float32)
    q = np.concatenate([q, q[:8] + 0.5]).astype(np.float16)  # non-integer queries
    g = oracle.build(base, R=32, distance="l2", alpha=1.2)
    gg = _load(jasper, g, tmp_path)
    # rows span 39 values: the search reads them as bytes (queries that take
    # the packed form), the other queries read the fp16 rows
    assert gg.row_format() == {"integer": True, "lo": 260, "hi": 299, "byte_rows": True}
    for bw in (16, 64, 128):
        ids, d = _run(jasper, gg, q, 10, bw)
        rid, rd = oracle.beam_search(g, q, k=10, beam_width=bw)
        msg = compare_search(ids, d, rid, rd)
        assert msg is None, f"bw={bw}: {msg}"


@pytest.mark.parametrize("dim,lo,hi,byte_rows", [(128, 0, 255, True), (128, 0, 256, False), (112, -40, 200, True),
                                                 (96, 0, 100, False)])
def test_search_byte_rows_match_oracle(jasper, oracle_lib, tmp_path, dim, lo, hi, byte_rows):
    """Byte rows are kept for integer rows spanning at most 255 values at
    dim 112 or 128; with and without them the results are the oracle's.
    Queries: in-range integers (bytes), integers up to the exact span's edge,
    and non-integers (fp16 rows)."""
    rng = np.random.default_rng(dim + hi)
    base = rng.integers(lo, hi + 1, size=(2500, dim))
    base[:, 0] = np.where(rng.random(2500) < 0.5, lo, hi)  # both ends present
    base = base.astype(np.float16)
    q = np.concatenate([rng.integers(lo, hi + 1, size=(24, dim)),
                        rng.integers(lo - 100, hi + 100, size=(8, dim))]).astype(np.float32)
    q = np.concatenate([q, q[:8] + 0.25]).astype(np.float16)
    g = oracle.build(base, R=32, distance="l2", alpha=1.2)
    gg = _load(jasper, g, tmp_path)
    assert gg.row_format()["byte_rows"] is byte_rows
    for bw in (24, 96):
        ids, d = _run(jasper, gg, q, 10, bw)
        rid, rd = oracle.beam_search(g, q, k=10, beam_width=bw)
        msg = compare_search(ids, d, rid, rd)
        assert msg is None, f"bw={bw}: {msg}"


def test_search_byte_rows_off_same_results(jasper, oracle_lib, tmp_path):
    """JASPER_SEARCH_BYTES=0 (read once per process, hence the child): no
    byte rows, and the same ids and distance bits as with them."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    base = integer_clustered(4000, 128, 71)
    q = integer_clustered(64, 128, 72)
    g = oracle.build(base, R=64, distance="l2", alpha=1.2)
    path = tmp_path / "g.bin"
    oracle.save_graph(g, path)
    np.save(tmp_path / "q.npy", q)
    code = f"""
import sys, numpy as np, torch
sys.path.insert(0, {str(Path(__file__).resolve().parents[1])!r})
import jasper_amd
gg = jasper_amd.Graph.load({str(path)!r}, dim=128, n_neighbors=64, distance='l2')
q = torch.from_numpy(np.load({str(tmp_path / 'q.npy')!r})).cuda()
ids, d = gg.search(q, k=10, beam_width=64)
np.savez({str(tmp_path / 'out.npz')!r}, ids=ids.cpu().numpy(), d=d.cpu().numpy(), b=gg.row_format()['byte_rows'])
"""
    r = subprocess.run([sys.executable, "-c", code], env=dict(os.environ, JASPER_SEARCH_BYTES="0"),
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    off = np.load(tmp_path / "out.npz")
    assert not bool(off["b"])
    gg = jasper.Graph.load(str(path), dim=128, n_neighbors=64, distance="l2")
    assert gg.row_format()["byte_rows"]
    ids, d = _run(jasper, gg, q, 10, 64)
    assert np.array_equal(ids, off["ids"])
    assert np.array_equal(d.view(np.uint32), off["d"].view(np.uint32))
    rid, rd = oracle.beam_search(g, q, k=10, beam_width=64)
    assert compare_search(ids, d, rid, rd) is None


def test_search_host_resident_graph_matches_oracle(jasper, oracle_lib, tmp_path):
    # on_host graphs live in pinned host memory and the kernels read them in
    # place over the host link (reference graph.cuh:140-147): same results
    base = integer_clustered(3000, 128, 51)
    q = integer_clustered(64, 128, 52)
    g = oracle.build(base, R=32, distance="l2", alpha=1.2)
    path = tmp_path / "g.bin"
    oracle.save_graph(g, path)
    gg = jasper.Graph.load(str(path), dim=128, n_neighbors=32, distance="l2", on_host=True)
    for bw in (16, 64):
        ids, d = _run(jasper, gg, q, 10, bw)
        rid, rd = oracle.beam_search(g, q, k=10, beam_width=bw)
        msg = compare_search(ids, d, rid, rd)
        assert msg is None, f"bw={bw}: {msg}"
