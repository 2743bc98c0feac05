"""Host-side behaviour of the Python API (reference python/jasper/__init__.py)."""

import pytest
import torch

import jasper_amd
from jasper_amd import DataType, DistanceFunc


def test_storage_sizes_are_decimal():
    assert jasper_amd.parse_storage_size("10GB") == 10 ** 10      # __init__.py:152-171
    assert jasper_amd.parse_storage_size("1.5 MB") == 1_500_000
    assert jasper_amd.parse_storage_size("2GiB") == 2 * 2 ** 30
    with pytest.raises(ValueError):
        jasper_amd.parse_storage_size("ten gigabytes")


def test_plain_registry():
    assert len(jasper_amd._CONFIGS) == 8
    assert jasper_amd._resolve_config(DataType.FLOAT16, 64, DistanceFunc.L2) == "f16_r64_l2"
    with pytest.raises(ValueError, match="Unsupported config"):
        jasper_amd._resolve_config(DataType.FLOAT16, 48, DistanceFunc.L2)


def test_directional_registry():
    assert len(jasper_amd._DIRECTIONAL_CONFIGS) == 16
    r = jasper_amd._resolve_directional_config
    assert r(DataType.FLOAT16, 64, DistanceFunc.INNER_PRODUCT, 4, 96) == "f16_r64_ip_k4_d128"
    assert r(DataType.FLOAT16, 64, DistanceFunc.L2, 16, 960) == "f16_r64_l2_k16_d32678"
    with pytest.raises(ValueError, match="Unsupported directional config"):
        r(DataType.FLOAT16, 16, DistanceFunc.L2, 4, 128)
    with pytest.raises(ValueError):
        r(DataType.FLOAT16, 64, DistanceFunc.L2, 8, 128)


def test_build_argument_checks():
    with pytest.raises(ValueError, match="2D"):
        jasper_amd.Graph.build(torch.zeros(10, dtype=torch.float16))
    with pytest.raises(ValueError, match="dtype"):
        jasper_amd.Graph.build(torch.zeros(10, 8, dtype=torch.float32))
    with pytest.raises(ValueError, match="Unsupported config"):
        jasper_amd.Graph.build(torch.zeros(10, 8, dtype=torch.float16), n_neighbors=7)


def _fake_graph(directional=False):
    cfg = "f16_r64_ip_k4_d128" if directional else "f16_r32_l2"
    return jasper_amd.Graph(-1, cfg, DataType.FLOAT16, DistanceFunc.L2, 32, 16,
                            is_directional=directional, k_ranks=4 if directional else None)


def test_search_argument_checks():
    g = _fake_graph()
    with pytest.raises(ValueError, match="CUDA"):
        g.search(torch.zeros(2, 16, dtype=torch.float16))
    g._handle = None
    with pytest.raises(RuntimeError, match="freed"):
        g.search(torch.zeros(2, 16, dtype=torch.float16))


def test_directional_only_calls_are_rejected():
    g = _fake_graph()
    with pytest.raises(RuntimeError, match="build_lsh"):
        g.directional_search(torch.zeros(2, 16, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="build_pq"):
        g.pq_search(torch.zeros(2, 16, dtype=torch.float16))
    d = _fake_graph(directional=True)
    with pytest.raises(RuntimeError, match="directional graph"):
        d.search(torch.zeros(2, 16, dtype=torch.float16))
    g._handle = d._handle = None


def test_groundtruth_cpu_matches_oracle():
    import oracle
    from jasper_amd import datasets
    x = datasets.clustered(3000, 32, 0, n_clusters=10)
    q = datasets.clustered(20, 32, 1, n_clusters=10)
    ids, d = jasper_amd.generate_groundtruth(torch.from_numpy(x), torch.from_numpy(q), k=10, device="cpu")
    rid, rd = oracle.bruteforce_ref(x.astype("float32"), q.astype("float32"), k=10)
    # integer-valued data: distances are exact, ids agree up to ties
    assert (d.numpy() == rd).all()


def test_groundtruth_cpu_orders_by_distance_then_id():
    """The CPU path returns (distance, id) order: duplicated rows tie and
    must come out by id; IP distances are negative and zero rows give -0.0;
    k above n pads with (-1, FLT_MAX)."""
    import numpy as np
    rng = np.random.default_rng(5)
    base = rng.integers(-3, 4, size=(40, 8)).astype(np.float32)
    base[20:30] = base[0:10]          # exact ties
    base[35] = 0.0                    # IP distance -0.0 / 0.0
    q = rng.integers(-3, 4, size=(6, 8)).astype(np.float32)
    for dist in ("l2", "ip"):
        ids, d = jasper_amd.generate_groundtruth(torch.from_numpy(base), torch.from_numpy(q), k=12,
                                                 distance=dist, device="cpu", vector_batch_size=7)
        if dist == "l2":
            full = ((q[:, None, :] - base[None, :, :]) ** 2).sum(-1)
        else:
            full = -(q @ base.T)
        for i in range(len(q)):
            order = np.lexsort((np.arange(len(base)), full[i] + 0.0))[:12]
            assert ids[i].tolist() == order.tolist()
            assert np.array_equal(d[i].numpy(), full[i][order].astype(np.float32))
    ids, d = jasper_amd.generate_groundtruth(torch.from_numpy(base[:5]), torch.from_numpy(q), k=8, device="cpu")
    assert (ids[:, 5:] == -1).all() and (d[:, 5:] == np.finfo(np.float32).max).all()
    assert sorted(ids[0, :5].tolist()) == list(range(5))
