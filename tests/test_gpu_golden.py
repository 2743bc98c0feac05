"""The HIP library against the committed golden fixtures (tests/golden):
fixed expected outputs, no oracle at run time. Plain search on the
fixture's file image, construction from the fixture's rows, a byte-exact
save of the loaded image, and the rotation matrix."""

from pathlib import Path

import numpy as np
import pytest
import torch

from tests.helpers import compare_search

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", ["plain_l2", "plain_ip"])
def test_search_on_fixture_image(jasper, tmp_path, name):
    f = _load(name)
    distance = "l2" if int(f["metric"]) == 0 else "ip"
    path = tmp_path / "g.bin"
    path.write_bytes(f["file_bytes"].tobytes())
    g = jasper.Graph.load(str(path), dim=f["base"].shape[1], n_neighbors=int(f["R"]), distance=distance)
    q = torch.from_numpy(f["queries"]).cuda()
    for bw in f["bws"].tolist():
        ids, d = g.search(q, k=5, beam_width=bw)
        msg = compare_search(ids.cpu().numpy(), d.cpu().numpy(), f[f"ids_bw{bw}"], f[f"dists_bw{bw}"])
        assert msg is None, f"{name} bw={bw}: {msg}"
    out = tmp_path / "again.bin"
    g.save(str(out))
    assert out.read_bytes() == f["file_bytes"].tobytes(), "save of a loaded image is not byte-identical"
    g.free()


@pytest.mark.parametrize("name", ["plain_l2", "plain_ip"])
def test_build_matches_fixture_graph(jasper, name):
    f = _load(name)
    distance = "l2" if int(f["metric"]) == 0 else "ip"
    g = jasper.Graph.build(torch.from_numpy(f["base"]).cuda(), n_neighbors=int(f["R"]), distance=distance,
                           alpha=1.2)
    edges, edist, counts = g.export_edges()
    assert np.array_equal(counts, f["counts"])
    mask = np.arange(edges.shape[1])[None, :] < counts[:, None]
    assert np.array_equal(edges[mask], f["edges"][mask])
    assert np.array_equal(edist[mask], f["edge_dist"][mask])
    g.free()


def test_rotation_matrix_matches_fixture(jasper):
    f = _load("rotation")
    m = jasper.rotation_matrix(int(f["dim"]), int(f["seed"]))
    assert np.array_equal(np.asarray(m, dtype=np.float32).view(np.uint32), f["matrix"].view(np.uint32))
