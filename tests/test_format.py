"""On-disk graph format (reference index/graph.cuh:1425-1788).

The oracle's writer/reader restate save_graph_to_file / load_graph_from_file;
they are pinned here by the byte offsets and sizes the reference format fixes
(bytes_per_node = 2*dim + 1 + 6R + 4; total = 32 + N*bpn + ceil(N/8) + 8),
and by the legacy per-node layouts the loader accepts.
"""

import struct

import numpy as np
import pytest

import oracle
from jasper_amd import datasets


@pytest.mark.parametrize("dim,R,bpn", [(128, 32, 453), (128, 64, 645), (96, 64, 581), (960, 64, 2309)])
def test_bytes_per_node(dim, R, bpn):
    assert oracle.bytes_per_node(dim, R) == bpn


def _small_graph(n=37, dim=16, R=8):
    x = datasets.gaussian(n, dim, 0)
    return oracle.build(x, R=R, max_batch=4)


def test_layout_offsets(tmp_path):
    g = _small_graph()
    g.deleted_bits[0] |= np.uint32(1 << 5)
    g.next_id = 41
    p = tmp_path / "g.bin"
    total = oracle.save_graph(g, p)
    raw = p.read_bytes()
    n, dim, R = g.n, g.dim, g.R
    bpn = 2 * dim + 1 + 6 * R + 4
    assert len(raw) == total == 32 + n * bpn + (n + 7) // 8 + 8
    assert struct.unpack_from("<QQQQ", raw, 0) == (total, n, 0, bpn)
    i = 3
    rec = raw[32 + i * bpn: 32 + (i + 1) * bpn]
    assert np.frombuffer(rec[:2 * dim], np.uint16).tolist() == g.vecs16[i, :dim].tolist()
    assert rec[2 * dim] == g.counts[i]
    o = 2 * dim + 1
    assert np.frombuffer(rec[o:o + 4 * R], np.uint32).tolist() == g.edges[i].tolist()
    o += 4 * R
    assert np.frombuffer(rec[o:o + 2 * R], np.uint16).tolist() == g.edge_dist[i].tolist()
    o += 2 * R
    assert struct.unpack_from("<I", rec, o)[0] == i
    dpos = 32 + n * bpn
    assert raw[dpos] == 1 << 5
    assert struct.unpack_from("<Q", raw, len(raw) - 8)[0] == 41


def test_round_trip(tmp_path):
    g = _small_graph()
    p = tmp_path / "g.bin"
    oracle.save_graph(g, p)
    h = oracle.load_graph(p, g.dim, g.R)
    assert np.array_equal(h.vecs16, g.vecs16)
    assert np.array_equal(h.edges, g.edges)
    assert np.array_equal(h.edge_dist, g.edge_dist)
    assert np.array_equal(h.counts, g.counts)
    assert h.medoid == g.medoid and h.next_id == g.next_id


@pytest.mark.parametrize("extra", [0, 1, 5])
def test_legacy_layouts(tmp_path, extra):
    # legacy (no deleted byte, no id), +deleted byte, +deleted byte + u32 id
    g = _small_graph(n=9)
    n, dim, R = g.n, g.dim, g.R
    bpn = 2 * dim + 1 + 6 * R + extra
    recs = []
    for i in range(n):
        r = g.vecs16[i, :dim].tobytes() + bytes([g.counts[i]]) + g.edges[i].tobytes() + g.edge_dist[i].tobytes()
        if extra >= 1:
            r += bytes([1 if i == 2 else 0])
        if extra == 5:
            r += struct.pack("<I", 100 + i)
        recs.append(r)
    body = b"".join(recs)
    tail = struct.pack("<Q", 77) if extra == 5 else b""
    p = tmp_path / "legacy.bin"
    p.write_bytes(struct.pack("<QQQQ", 32 + len(body), n, 0, bpn) + body + tail)
    h = oracle.load_graph(p, dim, R)
    assert np.array_equal(h.edges, g.edges) and np.array_equal(h.counts, g.counts)
    if extra >= 1:
        assert h.deleted_bits[0] == 1 << 2
    if extra == 5:
        assert h.slot_to_id.tolist() == [100 + i for i in range(n)] and h.next_id == 77
    else:
        assert h.slot_to_id.tolist() == list(range(n))


def test_unknown_layout_rejected(tmp_path):
    p = tmp_path / "bad.bin"
    p.write_bytes(struct.pack("<QQQQ", 40, 1, 0, 999) + b"\0" * 8)
    with pytest.raises(ValueError):
        oracle.load_graph(p, 16, 8)
