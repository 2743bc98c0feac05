"""GPU test of jasperx_directional_search_noalloc, the entry point that
allocates nothing (its scratch is a static device buffer of 64 MiB per GPU).

Called through the C ABI, it must return exactly what the allocating
jasperx_directional_search_ex returns for the same graph and queries: LSH, PQ
and RaBitQ estimators on a prerotated graph (so the rotated query rows live in the
scratch too), two calls in a row with the second on fewer queries (the
buffer keeps the first call's contents), and the unique flag. A call whose
scratch would exceed the buffer is rejected with a clear error.
"""

import ctypes

import numpy as np
import pytest
import torch

from tests.helpers import gaussian

pytestmark = pytest.mark.gpu


def _call(jasper, name, g, use_pq, q, k, bw, flags):
    from jasper_amd import _stream_ptr, _tensor_ptr
    nq = q.size(0)
    ids = torch.full((nq, k), -7, dtype=torch.int32, device="cuda")
    d = torch.full((nq, k), -7.0, dtype=torch.float32, device="cuda")
    jasper._agnostic(name)(g.handle, use_pq, _tensor_ptr(q), nq, q.size(1), _tensor_ptr(ids), _tensor_ptr(d), k,
                           bw, 2 * bw, flags, _stream_ptr(q.device))
    torch.cuda.synchronize()
    return ids.cpu().numpy(), d.cpu().numpy()


def test_noalloc_matches_allocating_search(jasper):
    dim = 120                                                   # padded to 120: rows need no padding kernel work
    x = gaussian(3000, dim, 91)
    g = jasper.Graph.build(torch.from_numpy(x).cuda(), n_neighbors=32, build_lsh=True, build_pq=True, k_ranks=4,
                           prerotate=True, lsh_samples=4000, pq_train=3000, pq_kmeans_iter=3, pq_m=24,
                           build_rabitq=True)
    for nq in (1500, 300):                                      # the second call is smaller
        q = torch.from_numpy(gaussian(nq, dim, 92 + nq)).cuda()
        for use_pq in (0, 1, 2):                                # estimators: LSH, PQ, RaBitQ
            for flags in (0, 1):
                want = _call(jasper, "jasperx_directional_search_ex", g, use_pq, q, 10, 48, flags)
                got = _call(jasper, "jasperx_directional_search_noalloc", g, use_pq, q, 10, 48, flags)
                assert np.array_equal(got[0], want[0]), (nq, use_pq, flags)
                assert np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32)), (nq, use_pq, flags)
                assert (got[0] != -7).all()
    g.free()


def test_noalloc_odd_dim_and_limit(jasper):
    dim = 61                                                    # rows padded to 64 by the pad kernel
    x = gaussian(2000, dim, 93)
    g = jasper.Graph.build(torch.from_numpy(x).cuda(), n_neighbors=32, build_lsh=True, build_pq=True, k_ranks=4,
                           prerotate=False, lsh_samples=3000, pq_train=2000, pq_kmeans_iter=2)
    q = torch.from_numpy(gaussian(700, dim, 94)).cuda()
    for use_pq in (0, 1):
        want = _call(jasper, "jasperx_directional_search_ex", g, use_pq, q, 10, 32, 0)
        got = _call(jasper, "jasperx_directional_search_noalloc", g, use_pq, q, 10, 32, 0)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32))
    # pq_search tables take m KB per query: 64 MiB hold about 16,000 queries at m = 4
    big = torch.from_numpy(gaussian(20000, dim, 95)).cuda()
    with pytest.raises(RuntimeError, match="scratch"):
        _call(jasper, "jasperx_directional_search_noalloc", g, 1, big, 10, 32, 0)
    small = q[:50]
    want = _call(jasper, "jasperx_directional_search_ex", g, 1, small, 10, 32, 0)
    got = _call(jasper, "jasperx_directional_search_noalloc", g, 1, small, 10, 32, 0)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32))
    g.free()


def test_noalloc_symbol_is_exported(jasper):
    lib = jasper._load_lib()
    assert isinstance(lib.jasperx_directional_search_noalloc, ctypes._CFuncPtr)
