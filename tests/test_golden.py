"""The committed golden fixtures (tests/golden/*.npz) against the oracle.

The fixtures were written by tests/golden/make_golden.py from seeded inputs.
Regenerating them must give the same bytes: this freezes the oracle's
build, search, directional search, LSH / PQ artifacts, RaBitQ codes,
rotation matrix and file images, so an unintended change in the oracle
(which every GPU parity test relies on) fails here first.
"""

import tempfile
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def regenerated(oracle_lib):
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.make_all()


@pytest.mark.parametrize("name", ["plain_l2", "plain_ip", "directional_l2", "rabitq", "rotation"])
def test_oracle_reproduces_fixture(regenerated, name):
    want = _load(name)
    got = regenerated[name]
    assert set(got) == set(want), name
    for key, arr in want.items():
        g = np.asarray(got[key])
        assert g.dtype == arr.dtype and g.shape == arr.shape, f"{name}.{key}"
        assert g.tobytes() == arr.tobytes(), f"{name}.{key} differs"


@pytest.mark.parametrize("name", ["plain_l2", "plain_ip"])
def test_file_image_loads_to_fixture_graph(oracle_lib, name):
    f = _load(name)
    dim = f["base"].shape[1]
    distance = "l2" if int(f["metric"]) == 0 else "ip"
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "g.bin"
        path.write_bytes(f["file_bytes"].tobytes())
        g = oracle.load_graph(path, dim, int(f["R"]), distance)
    assert g.medoid == int(f["medoid"])
    assert np.array_equal(g.counts, f["counts"])
    mask = np.arange(g.R)[None, :] < g.counts[:, None]
    assert np.array_equal(g.edges[mask], f["edges"][mask])
    assert np.array_equal(g.edge_dist[mask], f["edge_dist"][mask])
    assert np.array_equal(g.vecs16[:, :dim], f["base"].view(np.uint16))
