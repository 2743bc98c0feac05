"""GPU parity at the benchmark configurations' own parameter combinations.

The other GPU test files cover each kernel over many shapes; this file runs
the exact combinations the benchmark configurations name, on their own
generators, at row counts the oracle builds in seconds:

  * config 2: the 1,000-cluster integer mixture (`datasets.config("c2")`),
    R = 64, alpha = 1.2, plain search over the beam-width sweep 16..256;
  * config 5: the 10,000-cluster mixture, R = 64, prerotated, LSH with
    k_ranks = 16 (u8 words, 32,768 calibration samples) and the RaBitQ
    estimate driving the construction's search stage
    (`build_search="rabitq"`), then directional search at beam width 64.

Each asserts bit-identical graphs (counts, neighbour ids in slot order,
bf16 edge distances), artifacts and search results against the oracle.
"""

import numpy as np
import pytest
import torch

import oracle
from jasper_amd import datasets
from tests.helpers import compare_search
from tests.test_gpu_build import _compare

pytestmark = pytest.mark.gpu


def test_config2_generator_build_and_sweep(jasper, oracle_lib):
    """Config 2's generator (1,000 clusters, sigma 20, clipped to [0, 218],
    integers) at n = 20,000: the GPU build equals the oracle build, and
    the plain search equals the oracle's traversal at every beam width of
    the benchmark sweep (limit = 2 bw)."""
    base, queries, p = datasets.config("c2", n=20_000, nq=200)
    assert p["R"] == 64 and p["distance"] == "l2"
    print("[config2] n=20000 R=64 build", flush=True)
    og = oracle.build(base, R=64, distance="l2", alpha=1.2)
    t = torch.from_numpy(np.ascontiguousarray(base)).cuda()
    g = jasper.Graph.build(t, n_neighbors=64, distance="l2", alpha=p["alpha"])
    torch.cuda.synchronize()
    assert og.n_batches > 1
    _compare(g, og)
    qt = torch.from_numpy(np.ascontiguousarray(queries)).cuda()
    for bw in (16, 24, 32, 48, 64, 96, 128, 192, 256):
        print(f"[config2] search bw={bw}", flush=True)
        ids, d = g.search(qt, k=10, beam_width=bw)
        torch.cuda.synchronize()
        rid, rd = oracle.beam_search(og, queries, k=10, beam_width=bw, limit=2 * bw)
        msg = compare_search(ids.cpu().numpy(), d.cpu().numpy(), rid, rd)
        assert msg is None, f"bw={bw}: {msg}"
    g.free()


def test_config5_build_combination(jasper, oracle_lib):
    """Config 5's build at n = 8,000: 10,000-cluster integer mixture,
    R = 64, alpha = 1.2, prerotated, LSH k_ranks = 16 with u8 words and
    32,768 samples, and the construction's search stage popping by the
    RaBitQ one-bit estimate of the stored rows. The graph equals the
    oracle's construction with the same codes; the LSH constants and rows
    equal the oracle's on that graph; directional search at bw = 64 (the
    reference traversal and the distinct-results mode) equals the
    oracle's."""
    dim, R, K = 128, 64, 16
    x = datasets.clustered(8000, dim, 0, n_clusters=10_000)
    q = datasets.clustered(64, dim, 1, n_clusters=10_000)
    xt = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    print("[config5] n=8000 R=64 K=16 prerotate build_search=rabitq", flush=True)
    g = jasper.Graph.build(xt, n_neighbors=R, distance="l2", alpha=1.2, build_lsh=True, k_ranks=K,
                           prerotate=True, lsh_samples=32768, lsh_seed=7, build_search="rabitq")
    torch.cuda.synchronize()
    assert g._has_rabitq and g._has_lsh
    rows = g.export_vectors()
    stored = rows.view(np.float16)[:, :dim]
    cent, nodes = g.export_rabitq()
    og = oracle.build(stored, R=R, distance="l2", alpha=1.2, rq=oracle.RqArtifacts(dim, nodes, cent))
    _compare(g, og)

    c, nd, lrows = g.export_lsh()
    rc, rnd, nv = oracle.lsh_globals(og, K, n_samples=32768, seed=7)
    assert nv > 0
    assert np.array_equal(c.view(np.uint32), rc.view(np.uint32)), (c, rc)
    assert np.float32(nd).view(np.uint32) == np.float32(rnd).view(np.uint32)
    want = oracle.populate_lsh(og, K, 1)
    assert lrows.shape == want.shape == (8000, oracle.lsh_row_bytes(R, K, 1))
    assert np.array_equal(lrows, want), "LSH rows differ"

    art = oracle.LshArtifacts(K, 1, c, nd, lrows)
    q_rows = g.directional_query_rows(torch.from_numpy(q).cuda())
    qt = torch.from_numpy(np.ascontiguousarray(q)).cuda()
    for unique in (False, True):
        print(f"[config5] directional bw=64 unique={unique}", flush=True)
        ids, d = g.directional_search(qt, k=10, beam_width=64, unique=unique)
        torch.cuda.synchronize()
        rid, rd = oracle.directional_search(og, q_rows, lsh=art, k=10, beam_width=64, unique=unique)
        msg = compare_search(ids.cpu().numpy(), d.cpu().numpy(), rid, rd)
        assert msg is None, f"unique={unique}: {msg}"
    g.free()
