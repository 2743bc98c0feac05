"""GPU construction parity against the oracle build.

On inputs where the reverse-candidate cap cannot bind (batch <= 256, so no
target receives more than 256 + R candidates in one batch) the reference
build is deterministic up to its arithmetic, and the oracle restates that
arithmetic. The GPU graph must then equal the oracle graph: same edge counts,
same neighbour ids in the same slots, same bf16 edge distances. Where the cap
binds, the reference keeps an arrival-order subset; the oracle and the GPU
both keep the target's existing edges, then its sources in ascending id,
and the graphs must still be equal (test_build_matches_oracle_reverse_cap).
"""

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import gaussian, hub_mix, integer_clustered, unit

pytestmark = pytest.mark.gpu


def _gpu_build(jasper, base, R, distance):
    t = torch.from_numpy(np.ascontiguousarray(base)).cuda()
    g = jasper.Graph.build(t, n_neighbors=R, distance=distance, alpha=1.2)
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


@pytest.mark.parametrize("n,R", [(2000, 32), (3000, 16)])
def test_build_matches_oracle_gaussian(jasper, oracle_lib, n, R):
    base = gaussian(n, 128, 11)
    og = oracle.build(base, R=R, distance="l2", alpha=1.2)
    gg = _gpu_build(jasper, base, R, "l2")
    _compare(gg, og)


def test_build_matches_oracle_integer_r64(jasper, oracle_lib):
    base = integer_clustered(5000, 128, 12)
    og = oracle.build(base, R=64, distance="l2", alpha=1.2)
    gg = _gpu_build(jasper, base, 64, "l2")
    _compare(gg, og)


@pytest.mark.parametrize("hi", [255, 256, 362, 363])
def test_build_matches_oracle_integer_range_limit(jasper, oracle_lib, hi):
    # values {0, hi} at dim 128: hi = 362 keeps dim * hi^2 just under 2^24
    # (packed fp16 differences with v_dot2), 363 just over (fp32 chain);
    # hi = 255 is the widest span the reverse prune takes as bytes (int8
    # Gram), 256 the narrowest it takes as fp16; distances reach the limit,
    # and the many ties test the (dist, id) order
    rng = np.random.default_rng(14)
    base = (rng.integers(0, 2, size=(1500, 128)) * hi).astype(np.float16)
    base[:, :16] = rng.integers(0, hi + 1, size=(1500, 16)).astype(np.float16)
    og = oracle.build(base, R=32, distance="l2", alpha=1.2)
    gg = _gpu_build(jasper, base, 32, "l2")
    _compare(gg, og)


def test_build_matches_oracle_ip(jasper, oracle_lib):
    base = unit(2500, 96, 13)
    og = oracle.build(base, R=32, distance="ip", alpha=1.2)
    gg = _gpu_build(jasper, base, 32, "ip")
    _compare(gg, og)


@pytest.mark.parametrize("distance,dim,R", [("l2", 960, 32), ("ip", 264, 16)])
def test_build_matches_oracle_long_rows(jasper, oracle_lib, distance, dim, R):
    """dim > 256: search and prune distances stream the rows from memory."""
    from jasper_amd import datasets
    base = unit(1200, dim, 15) if distance == "ip" else datasets.sparse_abs(1500, dim, 15)
    og = oracle.build(base, R=R, distance=distance, alpha=1.2)
    gg = _gpu_build(jasper, base, R, distance)
    _compare(gg, og)


def test_build_tiny_inputs(jasper, oracle_lib):
    # n < 50 makes the reference's batch size 0 (an endless loop); both the
    # oracle and the GPU build clamp it to 1.
    for n in (1, 2, 7, 49):
        base = gaussian(n, 128, 14 + n)
        og = oracle.build(base, R=8, distance="l2", alpha=1.2)
        gg = _gpu_build(jasper, base, 8, "l2")
        _compare(gg, og)


@pytest.mark.parametrize("integer", [False, True])
def test_build_matches_oracle_reverse_cap(jasper, oracle_lib, integer):
    """Batches of 400 (n = 20000): row 0 is a hub that nearly every row of a
    batch links to, so its reverse candidates are cut at 256 + R (the cap of
    construct.cuh:642-658) in dozens of batches. Non-integer rows take the
    Gram prune with proof; integer rows (span 220) the exact integer paths."""
    base = hub_mix(20000, 64, 5, scale=32.0 if integer else 8.0, integer=integer)
    og = oracle.build(base, R=32, distance="l2", alpha=1.2)
    print(f"max batch {og.max_batch}, reverse groups cut at 256 + R: {og.capped_groups}")
    assert og.max_batch == 400 and og.capped_groups >= 20
    gg = _gpu_build(jasper, base, 32, "l2")
    _compare(gg, og)


def test_build_reverse_cap_byte_rows(jasper, oracle_lib):
    """The hub case at dim 128 on integer rows (span under 255): the graph
    keeps byte rows, so the reverse prune runs its byte mode, and the hub's
    groups of more than 96 candidates take that mode's u8 wave prune."""
    base = hub_mix(20000, 128, 6, scale=32.0, integer=True)
    og = oracle.build(base, R=32, distance="l2", alpha=1.2)
    assert og.max_batch == 400 and og.capped_groups >= 20
    gg = _gpu_build(jasper, base, 32, "l2")
    fmt = gg.row_format()
    print(f"row format {fmt}, reverse groups cut at 256 + R: {og.capped_groups}")
    assert fmt["byte_rows"]
    _compare(gg, og)


@pytest.mark.parametrize("gram8", ["0", "1"])
def test_build_byte_and_half_gram_agree(jasper, oracle_lib, gram8, tmp_path):
    """Integer rows of span 207 build the same graph with the reverse prune's
    Gram step on bytes (default) and on fp16 (JASPER_GRAM8=0, read once per
    process, hence the child process), both the oracle's."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    base = integer_clustered(6000, 128, 41)
    og = oracle.build(base, R=64, distance="l2", alpha=1.2)
    np.save(tmp_path / "base.npy", base)
    code = f"""
import sys, numpy as np, torch
sys.path.insert(0, {str(Path(__file__).resolve().parents[1])!r})
import jasper_amd
base = np.load({str(tmp_path / 'base.npy')!r})
g = jasper_amd.Graph.build(torch.from_numpy(base).cuda(), n_neighbors=64, distance='l2', alpha=1.2)
e, d, c = g.export_edges()
np.savez({str(tmp_path / 'out.npz')!r}, e=e, d=d, c=c)
"""
    env = dict(os.environ, JASPER_GRAM8=gram8)
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    out = np.load(tmp_path / "out.npz")
    assert np.array_equal(out["c"], og.counts)
    mask = np.arange(64)[None, :] < og.counts[:, None]
    assert np.array_equal(out["e"][mask], og.edges[mask])
    assert np.array_equal(out["d"][mask], og.edge_dist[mask])


@pytest.mark.parametrize("groups", ["3", "1"])
def test_build_reverse_grouping_several_tiles_per_group(jasper, oracle_lib, monkeypatch, groups):
    """The reverse pairs of a 400-row batch at R = 32 fill four 4,096-key
    sort tiles. With the sort's work-groups capped at 3 (tiles split 1, 1, 2)
    or 1 (one work-group walks all four), each work-group carries its digit
    offsets from tile to tile -- the path that otherwise runs only above
    8M keys -- and the graph must stay the oracle's."""
    monkeypatch.setenv("JASPER_SORT_GROUPS", groups)
    base = hub_mix(20000, 64, 5, scale=32.0, integer=True)
    og = oracle.build(base, R=32, distance="l2", alpha=1.2)
    assert og.max_batch == 400
    gg = _gpu_build(jasper, base, 32, "l2")
    _compare(gg, og)


def test_build_then_search_c1(jasper, oracle_lib):
    """Config 1 end to end: the GPU graph equals the oracle's bit for bit
    (batches of at most 200, so no cap binds) and the GPU search on it
    returns the oracle's ids and distances."""
    from jasper_amd import datasets
    base, q, p = datasets.config("c1")
    gg = _gpu_build(jasper, base, 32, "l2")
    og = oracle.build(base, R=32, distance="l2", alpha=1.2)
    assert og.max_batch == 200 and og.capped_groups == 0
    _compare(gg, og)
    gt, _ = oracle.bruteforce_exact(base, q, k=10)
    ids, d = gg.search(torch.from_numpy(q).cuda(), k=10, beam_width=64)
    rid, rd = oracle.beam_search(og, q, k=10, beam_width=64)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.array_equal(d.cpu().numpy().view(np.uint32), rd.view(np.uint32))
    r_gpu = oracle.recall(gt, ids.cpu().numpy(), 10)
    print(f"config 1 recall@10 at bw 64: {r_gpu:.3f}")   # 0.813: N(0,1) rows at d = 128
    assert r_gpu > 0.75


def test_build_host_resident_matches_oracle(jasper, oracle_lib):
    base = integer_clustered(2000, 128, 53)
    og = oracle.build(base, R=32, distance="l2", alpha=1.2)
    t = torch.from_numpy(np.ascontiguousarray(base)).cuda()
    gg = jasper.Graph.build(t, n_neighbors=32, distance="l2", alpha=1.2, on_host=True)
    torch.cuda.synchronize()
    _compare(gg, og)


_WIDE_MARGIN_CHILD = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
import jasper_amd
out = {}
for name in ("l2", "ip"):
    x = np.load(sys.argv[2] + f"/{name}.npy")
    g = jasper_amd.Graph.build(torch.from_numpy(x).cuda(), n_neighbors=32, distance=name, alpha=1.2)
    torch.cuda.synchronize()
    e, d, c = g.export_edges()
    out[name + "_e"], out[name + "_d"], out[name + "_c"] = e, d, c
np.savez(sys.argv[2] + "/out.npz", **out)
print("child done", flush=True)
"""


def test_build_gram_proof_path_matches_oracle(jasper, oracle_lib, tmp_path):
    # with the proof margin widened past every distance, no pair of the
    # non-integer Gram prune is decided by the matrix cores: each is settled
    # by the exact chain when its row comes up; the graphs must not change
    import os
    import subprocess
    import sys
    from pathlib import Path
    l2 = gaussian(2000, 128, 61)
    ip = unit(2000, 96, 62)
    np.save(tmp_path / "l2.npy", l2)
    np.save(tmp_path / "ip.npy", ip)
    env = dict(os.environ, JASPER_GRAM_MARGIN="1e30")
    root = str(Path(__file__).resolve().parents[1])
    r = subprocess.run([sys.executable, "-c", _WIDE_MARGIN_CHILD, root, str(tmp_path)], env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    out = np.load(tmp_path / "out.npz")
    for name, x in (("l2", l2), ("ip", ip)):
        og = oracle.build(x, R=32, distance=name, alpha=1.2)
        counts, edges, edist = out[name + "_c"], out[name + "_e"], out[name + "_d"]
        assert np.array_equal(counts, og.counts), name
        mask = np.arange(32)[None, :] < counts[:, None]
        assert np.array_equal(edges[mask], og.edges[mask]), name
        assert np.array_equal(edist[mask], og.edge_dist[mask]), name


def test_build_hand_computed_line(jasper, oracle_lib):
    """The six points of the hand-computed construction (test_oracle_build):
    n < 50 gives batches of one, and the device graph (R = 8, the smallest
    config) must be the one worked out by hand."""
    from tests.test_oracle_build import HAND_BATCH1, check_hand_graph, line_points
    g = _gpu_build(jasper, line_points().astype(np.float16), 8, "l2")
    edges, edist, counts = g.export_edges()
    check_hand_graph(edges, edist, counts, HAND_BATCH1)
    g.free()


@pytest.mark.parametrize("distance,dim,n", [("l2", 128, 6000), ("ip", 96, 4000)])
def test_build_rabitq_search_matches_oracle(jasper, oracle_lib, distance, dim, n):
    """build_search="rabitq": the RaBitQ codes of the stored (prerotated)
    rows, then construction whose search stage pops by their estimate; the
    graph equals the oracle's construction with the same codes (exported
    from the device), edges, order and bf16 distances."""
    x = integer_clustered(n, dim, 73) if distance == "l2" else unit(n, dim, 74)
    t = torch.from_numpy(np.ascontiguousarray(x.astype(np.float16))).cuda()
    g = jasper.Graph.build(t, n_neighbors=32, distance=distance, alpha=1.2, build_lsh=True, k_ranks=4,
                           prerotate=True, lsh_samples=2000, build_search="rabitq")
    torch.cuda.synchronize()
    assert g._has_rabitq
    rows = g.export_vectors().view(np.float16)[:, :dim]
    cent, nodes = g.export_rabitq()
    og = oracle.build(rows, R=32, distance=distance, alpha=1.2, rq=oracle.RqArtifacts(dim, nodes, cent))
    _compare(g, og)
    g.free()


@pytest.mark.parametrize("kind", ["integer", "gaussian"])
def test_build_work_counters_match_oracle(jasper, oracle_lib, kind):
    """Work counting (the build roofline's byte counts): the device build in
    counting mode makes the same graph, and its counters (search pops,
    adjacency entries, distinct vectors scored, popped keys; forward and
    reverse prune rows, existing edges, candidates, sources, edges written)
    equal the oracle's counts of the same build. Integer rows take the byte
    prunes, Gaussian rows the fp16 ones."""
    base = integer_clustered(3000, 128, 31) if kind == "integer" else gaussian(2500, 128, 32)
    og = oracle.build(base, R=32, distance="l2", alpha=1.2, count_work=True)
    jasper.set_build_work_counting(True)
    try:
        gg = _gpu_build(jasper, base, 32, "l2")
        work = jasper.last_build_work()
    finally:
        jasper.set_build_work_counting(False)
    _compare(gg, og)
    assert work == og.work, {k: (work[k], og.work[k]) for k in work if work[k] != og.work[k]}
    assert work["search_rows"] == work["forward_rows"] == len(base)
    assert work["reverse_sources"] == work["forward_selected"]
    gg.free()
    g2 = _gpu_build(jasper, base, 32, "l2")
    assert not any(jasper.last_build_work().values())  # counting off: nothing counted
    _compare(g2, og)
    g2.free()
