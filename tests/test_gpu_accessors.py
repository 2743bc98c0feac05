"""GPU tests of the per-vector accessors.

get_vector (GetVector_, ffi/jasper_ffi_common.cuh:263-300) maps a stable id to
its slot (the identity with the reference's default build, labels off) and
copies the stored row; get_vector_directional (GetVectorDirectional_,
:735-763) copies the row at an index. A prerotated directional graph stores
rotated rows (the reference rotates the input before construction,
construct.cuh:1068-1107), so that is what both return.
"""

import numpy as np
import pytest
import torch

from tests.helpers import gaussian, integer_clustered

pytestmark = pytest.mark.gpu


def _rows(jasper_graph, ids):
    out = []
    for i in ids:
        v = jasper_graph.get_vector(int(i))
        torch.cuda.synchronize()
        assert v.dtype == torch.float16 and v.is_cuda
        out.append(v.cpu().numpy().view(np.uint16))
    return np.stack(out)


def test_get_vector_plain(jasper):
    x = integer_clustered(3000, 100, 81)        # dim 100: rows padded to 104 on the device
    g = jasper.Graph.build(torch.from_numpy(x).cuda(), n_neighbors=32)
    ids = [0, 1, 17, 1499, 2999]
    assert np.array_equal(_rows(g, ids), x[ids].view(np.uint16))
    with pytest.raises(ValueError, match="not found"):
        g.get_vector(3000)
    with pytest.raises(IndexError):
        g.get_vector(-1)
    g.free()


def test_get_vector_after_append(jasper):
    x = gaussian(2500, 64, 82)
    extra = gaussian(300, 64, 83)
    g = jasper.Graph.build(torch.from_numpy(x).cuda(), n_neighbors=32)
    new_ids = g.append(torch.from_numpy(extra).cuda())
    assert new_ids.tolist() == list(range(2500, 2800))
    got = _rows(g, [2500, 2650, 2799, 5])
    want = np.concatenate([extra[[0, 150, 299]], x[[5]]]).view(np.uint16)
    assert np.array_equal(got, want)
    g.free()


def test_get_vector_directional_prerotated(jasper):
    x = gaussian(2000, 96, 84)
    g = jasper.Graph.build(torch.from_numpy(x).cuda(), n_neighbors=32, build_lsh=True, k_ranks=4,
                           prerotate=True, lsh_samples=2000)
    stored = g.export_vectors()[:, :96]
    ids = [0, 999, 1999]
    assert np.array_equal(_rows(g, ids), stored[ids])
    assert not np.array_equal(stored[ids], x[ids].view(np.uint16))   # rows are rotated
    with pytest.raises(ValueError, match="not found"):
        g.get_vector(2000)
    g.free()
