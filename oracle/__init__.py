"""CPU oracle for the Jasper query/build hot path -- TEST INFRASTRUCTURE ONLY.

This package is the parity checker. Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg may import it, and only to check or to
time the CPU baseline; the product (``jasper_amd``) never imports it.

The arithmetic lives in ``jasper_oracle.cpp`` (built by ``oracle/Makefile`` into
``oracle/build/liboracle.so``); this module binds it with ctypes and adds the
on-disk format restatement (reference ``include/jasper/index/graph.cuh``
:1425-1788, ``save_graph_to_file`` / ``load_graph_from_file``).

Pinning (what checks each function, see tests/test_oracle_*.py):
  * l2 / ip distance   -- reference KATs tests/test_distance.cu:32-136, exact
                          integer identities, brute-force fp64 comparison.
  * beam_search        -- brute-force equality when bw >= N on a connected
                          graph, complete-graph one-hop, hand-computed path
                          graph, invariants (sorted, unique, |B| <= bw).
  * build              -- invariants (degree <= R, no self loops, alpha-prune
                          dominance per row), recall against brute force.
  * rotation_matrix    -- reference tests tests/test_rotation.cu:56-185.
  * bruteforce_*       -- each other and a float64 numpy computation.
  * file format        -- byte offsets of graph.cuh:1653-1788, bpn values.
"""

from __future__ import annotations

import ctypes
import os
import struct
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "build" / "liboracle.so"
_lib = None

L2 = 0
IP = 1


def ensure_built(force: bool = False) -> Path:
    """Compile the oracle with its Makefile (g++ only; no GPU toolchain)."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            ensure_built()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        P = ctypes.c_void_p
        i32, i64, f32, u64 = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_uint64
        _lib.jo_build_work.restype = None
        _lib.jo_build_work.argtypes = [i32]
        _lib.jo_last_build_work.restype = None
        _lib.jo_last_build_work.argtypes = [P]
        _lib.jo_l2.restype = f32
        _lib.jo_l2.argtypes = [P, P, i32]
        _lib.jo_ip.restype = f32
        _lib.jo_ip.argtypes = [P, P, i32]
        _lib.jo_f2bf.restype = ctypes.c_uint16
        _lib.jo_f2bf.argtypes = [f32]
        _lib.jo_distance_pairs.restype = None
        _lib.jo_distance_pairs.argtypes = [i32, P, P, i64, i32, P, i32]
        _lib.jo_beam_search.restype = i32
        _lib.jo_beam_search.argtypes = [P, i64, i32, P, P, i32, P, P, i32, P, i64, ctypes.c_uint32,
                                        i32, i32, i32, i32, P, P, P, P, P, P, i32]
        _lib.jo_max_batch_size.restype = i64
        _lib.jo_max_batch_size.argtypes = [i64, i32, i64]
        _lib.jo_build.restype = i32
        _lib.jo_build.argtypes = [P, i64, i32, i32, i32, i32, f32, i64, P, P, P, i32, P]
        _lib.jo_build_scale.restype = i32
        _lib.jo_build_scale.argtypes = [P, i64, i32, i32, i32, i32, f32, i64, i64, i64, P, P, P, i32]
        _lib.jo_scale_merge_order.restype = i64
        _lib.jo_scale_merge_order.argtypes = [i64, P]
        _lib.jo_prune_scale.restype = i32
        _lib.jo_prune_scale.argtypes = [P, i32, i32, i32, f32, i32, i64, i64, i64, i64, ctypes.c_uint32, P, P,
                                        i32, P, P]
        _lib.jo_diskann_assign.restype = i32
        _lib.jo_diskann_assign.argtypes = [P, i64, i32, i32, i32, i32, u64, P, P]
        _lib.jo_build_diskann.restype = i32
        _lib.jo_build_diskann.argtypes = [P, i64, i32, i32, i32, i32, i32, f32, i32, i32, u64, i64, i64, P, P, P, P,
                                          i32]
        _lib.jo_build_rq.restype = i32
        _lib.jo_build_rq.argtypes = [P, i64, i32, i32, i32, i32, f32, i64, i32, P, P, P, P, P, i32, P]
        _lib.jo_last_capped_groups.restype = i64
        _lib.jo_last_capped_groups.argtypes = []
        _lib.jo_append.restype = i32
        _lib.jo_append.argtypes = [P, i64, i32, i32, i32, i32, f32, i64, i64, ctypes.c_uint32, P, P, P, P, i32, P]
        _lib.jo_consolidate.restype = i64
        _lib.jo_consolidate.argtypes = [P, i64, i32, i32, i32, i32, f32, P, P, P, P, i32]
        _lib.jo_bruteforce_exact.restype = None
        _lib.jo_bruteforce_exact.argtypes = [i32, P, i64, P, i64, i32, i32, P, P, i32]
        _lib.jo_bruteforce_ref.restype = None
        _lib.jo_bruteforce_ref.argtypes = [i32, P, i64, P, i64, i32, i32, P, P, i32, i32]
        _lib.jo_gaussian_matrix.restype = None
        _lib.jo_gaussian_matrix.argtypes = [i32, u64, P]
        _lib.jo_rotation_matrix.restype = None
        _lib.jo_rotation_matrix.argtypes = [i32, u64, P, P]
        u16, f64 = ctypes.c_uint16, ctypes.c_double
        _lib.jo_d2h.restype = u16
        _lib.jo_d2h.argtypes = [f64]
        _lib.jo_hsub.restype = u16
        _lib.jo_hsub.argtypes = [u16, u16]
        _lib.jo_hmul.restype = u16
        _lib.jo_hmul.argtypes = [u16, u16]
        _lib.jo_visit_exact.restype = f32
        _lib.jo_visit_exact.argtypes = [P, P, i32, i32, P]
        _lib.jo_vector_norms.restype = None
        _lib.jo_vector_norms.argtypes = [P, i64, i32, P, i32]
        _lib.jo_directional_search.restype = i32
        _lib.jo_directional_search.argtypes = [i32, P, i64, i32, P, P, i32, P, i32,
                                               i32, i32, P, f32, P,
                                               i32, i32, P, P, P,
                                               i32, P, P,
                                               P, i64, ctypes.c_uint32, i32, i32, i32, i32, P, P, P, P, P, P, i32, i32]
        _lib.jo_rq_estimates.restype = None
        _lib.jo_rq_estimates.argtypes = [P, i64, i32, P, i32, P, i64, i32, P, P, P, P]
        _lib.jo_populate_lsh.restype = None
        _lib.jo_populate_lsh.argtypes = [P, i64, i32, P, P, i32, i32, i32, P, i32]
        _lib.jo_lsh_globals.restype = i64
        _lib.jo_lsh_globals.argtypes = [P, i64, i32, P, P, i32, i32, i64, u64, P, P]
        _lib.jo_pq_train.restype = None
        _lib.jo_pq_train.argtypes = [P, i64, i32, P, P, i32, i32, i64, i32, u64, P, P, i32]
        _lib.jo_pq_hash.restype = u64
        _lib.jo_pq_hash.argtypes = [u64, u64]
        _lib.jo_splitmix.restype = u64
        _lib.jo_splitmix.argtypes = [u64]
        _lib.jo_sample_edge.restype = i32
        _lib.jo_sample_edge.argtypes = [P, P, i64, i32, u64, u64, P, P]
        _lib.jo_rabitq_code_bytes.restype = ctypes.c_uint32
        _lib.jo_rabitq_code_bytes.argtypes = [i32]
        _lib.jo_rabitq_quantize.restype = None
        _lib.jo_rabitq_quantize.argtypes = [P, i64, i32, P, P, i32, P, P, i32]
        _lib.jo_best_rescale_factor.restype = ctypes.c_double
        _lib.jo_best_rescale_factor.argtypes = [P, i64, i32]
        _lib.jo_const_scaling_factor.restype = ctypes.c_double
        _lib.jo_const_scaling_factor.argtypes = [P, i64, i64, i32]
        _lib.jo_frontier_insert_seq.restype = None
        _lib.jo_frontier_insert_seq.argtypes = [P, P, i32, i32, P, P, P]
        _lib.jo_pq_encode.restype = None
        _lib.jo_pq_encode.argtypes = [P, i64, i32, P, P, i32, i32, P, P, i32]
        _lib.jo_rotate_rows.restype = None
        _lib.jo_rotate_rows.argtypes = [P, i64, i32, i32, P, P, i32]
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def metric_code(distance: str) -> int:
    return L2 if distance in ("l2", L2) else IP


def pad_dim(dim: int) -> int:
    """vector_view::pad, reference include/jasper/index/vector.cuh:20-22."""
    return (dim + 7) // 8 * 8


def as_padded_f16(x: np.ndarray) -> np.ndarray:
    """[n, dim] float -> [n, pad(dim)] float16 bits (uint16), zero padded."""
    x = np.asarray(x)
    if x.dtype != np.float16:
        x = x.astype(np.float16)
    n, dim = x.shape
    dp = pad_dim(dim)
    out = np.zeros((n, dp), dtype=np.float16)
    out[:, :dim] = x
    return np.ascontiguousarray(out).view(np.uint16)


def f2bf(x: float) -> int:
    return int(lib().jo_f2bf(float(x)))


def distance(a: np.ndarray, b: np.ndarray, distance: str = "l2", dim: int | None = None) -> float:
    """Single distance between two fp16 vectors (reference distance/distance.cuh:33-106)."""
    pa = as_padded_f16(np.asarray(a).reshape(1, -1))
    pb = as_padded_f16(np.asarray(b).reshape(1, -1))
    d = pa.shape[1] if dim is None else dim
    f = lib().jo_l2 if metric_code(distance) == L2 else lib().jo_ip
    return float(f(_ptr(pa), _ptr(pb), d))


def distance_pairs(a16: np.ndarray, b16: np.ndarray, distance: str = "l2", nthreads: int = 0) -> np.ndarray:
    """Row-wise distances of two padded uint16 arrays of equal shape."""
    assert a16.shape == b16.shape and a16.dtype == np.uint16
    out = np.empty(a16.shape[0], dtype=np.float32)
    lib().jo_distance_pairs(metric_code(distance), _ptr(a16), _ptr(b16), a16.shape[0], a16.shape[1],
                            _ptr(out), nthreads)
    return out


class OracleGraph:
    """Host graph in the oracle's flat layout: vectors [n, dp] (fp16 bits),
    edges [n, R] u32, edge_dist [n, R] bf16 bits, counts [n] u8."""

    def __init__(self, vecs16, edges, edge_dist, counts, R, dim, distance="l2", medoid=0,
                 deleted_bits=None, slot_to_id=None, next_id=None):
        self.vecs16 = np.ascontiguousarray(vecs16, dtype=np.uint16)
        self.edges = np.ascontiguousarray(edges, dtype=np.uint32)
        self.edge_dist = np.ascontiguousarray(edge_dist, dtype=np.uint16)
        self.counts = np.ascontiguousarray(counts, dtype=np.uint8)
        self.R = int(R)
        self.dim = int(dim)
        self.distance = distance
        self.medoid = int(medoid)
        n = self.vecs16.shape[0]
        self.deleted_bits = (np.zeros((n + 31) // 32, dtype=np.uint32) if deleted_bits is None
                             else np.ascontiguousarray(deleted_bits, dtype=np.uint32))
        self.slot_to_id = (np.arange(n, dtype=np.uint32) if slot_to_id is None
                           else np.ascontiguousarray(slot_to_id, dtype=np.uint32))
        self.next_id = n if next_id is None else int(next_id)

    @property
    def n(self):
        return self.vecs16.shape[0]

    @property
    def dp(self):
        return self.vecs16.shape[1]


def max_batch_size(n: int, R: int, budget_bytes: int = 10 ** 10) -> int:
    return int(lib().jo_max_batch_size(n, R, budget_bytes))


BUILD_WORK_KEYS = ["search_rows", "search_hops", "search_adjacency", "search_scored", "search_visited",
                   "forward_rows", "forward_existing", "forward_visited", "forward_candidates", "forward_selected",
                   "reverse_targets", "reverse_existing", "reverse_sources", "reverse_selected"]


def build(vectors, R: int = 32, distance: str = "l2", alpha: float = 1.2,
          workspace_budget: int = 10 ** 10, max_batch: int | None = None,
          nthreads: int = 0, rq: "RqArtifacts | None" = None, count_work: bool = False) -> OracleGraph:
    """Vamana construction, reference index/construct.cuh:992-1160. With rq
    (this build's extension) the search stage pops by the RaBitQ estimate of
    those codes (rabitq_build_search) instead of the plain search.
    count_work: also count the build's work (g.work, a dict keyed by
    BUILD_WORK_KEYS: rows searched, pops, adjacency entries, distinct vectors
    scored and popped keys of the search stage; the forward and reverse
    prunes' rows, existing edges, visited keys / sources, candidates and
    edges written)."""
    vecs16 = as_padded_f16(vectors)
    n, dp = vecs16.shape
    dim = np.asarray(vectors).shape[1]
    if max_batch is None:
        max_batch = max(1, max_batch_size(n, R, workspace_budget))
    edges = np.empty((n, R), dtype=np.uint32)
    edist = np.empty((n, R), dtype=np.uint16)
    counts = np.empty(n, dtype=np.uint8)
    nb = ctypes.c_int64(0)
    lib().jo_build_work(1 if count_work else 0)
    if rq is None:
        rc = lib().jo_build(_ptr(vecs16), n, dp, dim, R, metric_code(distance), ctypes.c_float(alpha),
                            int(max_batch), _ptr(edges), _ptr(edist), _ptr(counts), nthreads,
                            ctypes.byref(nb))
    else:
        rc = lib().jo_build_rq(_ptr(vecs16), n, dp, dim, R, metric_code(distance), ctypes.c_float(alpha),
                               int(max_batch), rq.dim, _ptr(rq.nodes), _ptr(rq.centroid), _ptr(edges),
                               _ptr(edist), _ptr(counts), nthreads, ctypes.byref(nb))
    if rc != 0:
        raise RuntimeError(f"oracle build failed ({rc})")
    g = OracleGraph(vecs16, edges, edist, counts, R, dim, distance)
    g.n_batches = nb.value
    g.max_batch = max_batch
    if count_work:
        w = np.zeros(16, dtype=np.uint64)
        lib().jo_last_build_work(_ptr(w))
        lib().jo_build_work(0)
        g.work = {k: int(v) for k, v in zip(BUILD_WORK_KEYS, w.tolist())}
    # reverse-step groups cut at the 256 + R candidate cap (test counter)
    g.capped_groups = int(lib().jo_last_capped_groups())
    return g


def append(g: OracleGraph, vectors, alpha: float = 1.2, max_batch: int | None = None,
           nthreads: int = 0):
    """Live batch append, reference index/construct.cuh:1169-1265: the rows go
    to slots [n, n + count), are wired in by process_batch in batches of
    min(count, 100000), and get fresh stable ids from the monotonic counter.
    Returns (new graph, ids)."""
    new16 = as_padded_f16(vectors)
    assert new16.shape[1] == g.dp
    count = new16.shape[0]
    old_n = g.n
    n = old_n + count
    if max_batch is None:
        max_batch = min(count, 100000)
    vecs16 = np.concatenate([g.vecs16, new16])
    edges = np.concatenate([g.edges, np.full((count, g.R), 0xFFFFFFFF, dtype=np.uint32)])
    edist = np.concatenate([g.edge_dist, np.zeros((count, g.R), dtype=np.uint16)])
    counts = np.concatenate([g.counts, np.zeros(count, dtype=np.uint8)])
    bits = np.zeros((n + 31) // 32, dtype=np.uint32)
    bits[:g.deleted_bits.size] = g.deleted_bits
    nb = ctypes.c_int64(0)
    if count:
        rc = lib().jo_append(_ptr(vecs16), n, g.dp, g.dim, g.R, metric_code(g.distance), ctypes.c_float(alpha),
                             old_n, int(max_batch), g.medoid, _ptr(bits), _ptr(edges), _ptr(edist), _ptr(counts),
                             nthreads, ctypes.byref(nb))
        if rc != 0:
            raise RuntimeError(f"oracle append failed ({rc})")
    ids = np.arange(g.next_id, g.next_id + count, dtype=np.int64)
    slot_to_id = np.concatenate([g.slot_to_id, ids.astype(np.uint32)])
    out = OracleGraph(vecs16, edges, edist, counts, g.R, g.dim, g.distance, medoid=g.medoid,
                      deleted_bits=bits, slot_to_id=slot_to_id, next_id=g.next_id + count)
    out.n_deleted = getattr(g, "n_deleted", 0)
    out.n_batches = nb.value
    return out, ids.astype(np.int32)


def mark_deleted(g: OracleGraph, ids) -> int:
    """Soft delete by id (reference graph_ops.cuh:94-135 with stable-id labels
    off, the default: id == slot). Out-of-range ids are ignored; ids already
    deleted are counted once. A deleted medoid is replaced by its first live
    neighbour in edge order, else the lowest live vertex
    (find_new_medoid_kernel, deletion.cuh:245-266). Returns the number of
    newly deleted vertices."""
    newly = 0
    for x in np.asarray(ids, dtype=np.int64).ravel():
        v = int(x) & 0xFFFFFFFF
        if v >= g.n:
            continue
        w, b = v >> 5, np.uint32(1 << (v & 31))
        if not (g.deleted_bits[w] & b):
            g.deleted_bits[w] |= b
            newly += 1
    g.n_deleted = getattr(g, "n_deleted", 0) + newly

    def dead(v):
        return bool((g.deleted_bits[v >> 5] >> np.uint32(v & 31)) & np.uint32(1))

    if g.n and dead(g.medoid):
        new = None
        for e in range(int(g.counts[g.medoid])):
            nb = int(g.edges[g.medoid, e])
            if nb != 0xFFFFFFFF and nb < g.n and not dead(nb):
                new = nb
                break
        if new is None:
            for v in range(g.n):
                if not dead(v):
                    new = v
                    break
        if new is not None:
            g.medoid = new
    return newly


def consolidate(g: OracleGraph, alpha: float = 1.2, nthreads: int = 0) -> int:
    """Repair edges through deleted vertices and clear the tombstones
    (reference graph_ops.cuh:151-258); in place. Returns the number of repair
    candidates."""
    if getattr(g, "n_deleted", 0) == 0 and not g.deleted_bits.any():
        return 0
    n_rep = lib().jo_consolidate(_ptr(g.vecs16), g.n, g.dp, g.dim, g.R, metric_code(g.distance),
                                 ctypes.c_float(alpha), _ptr(g.deleted_bits), _ptr(g.edges), _ptr(g.edge_dist),
                                 _ptr(g.counts), nthreads)
    g.n_deleted = 0
    return int(n_rep)


def beam_search(g: OracleGraph, queries, k: int = 10, beam_width: int = 64,
                limit: int | None = None, max_result: int = 2048, get_visited: bool = False,
                stats: bool = False, nthreads: int = 0):
    """Plain beam search, reference beam_search/beam_search.cuh:27-225 with
    api.cuh defaults (limit = 2 * beam_width as python/jasper/__init__.py:501)."""
    q16 = queries if (isinstance(queries, np.ndarray) and queries.dtype == np.uint16) else as_padded_f16(queries)
    assert q16.shape[1] == g.dp
    nq = q16.shape[0]
    if limit is None:
        limit = 2 * beam_width
    ids = np.empty((nq, k), dtype=np.int32)
    dists = np.empty((nq, k), dtype=np.float32)
    vis_ids = vis_d = vis_c = None
    if get_visited:
        vis_ids = np.zeros((nq, max_result), dtype=np.uint32)
        vis_d = np.zeros((nq, max_result), dtype=np.float32)
        vis_c = np.zeros(nq, dtype=np.uint32)
    st = np.zeros((nq, 4), dtype=np.uint64) if stats else None
    lib().jo_beam_search(_ptr(g.vecs16), g.n, g.dp, _ptr(g.edges), _ptr(g.counts), g.R,
                         _ptr(g.deleted_bits), _ptr(g.slot_to_id), metric_code(g.distance),
                         _ptr(q16), nq, g.medoid, k, beam_width, limit, max_result,
                         _ptr(ids), _ptr(dists), _ptr(vis_ids), _ptr(vis_d), _ptr(vis_c),
                         _ptr(st), nthreads)
    out = [ids, dists]
    if get_visited:
        out += [vis_ids, vis_d, vis_c]
    if stats:
        out.append(st)
    return tuple(out)


def bruteforce_exact(vectors, queries, k: int = 10, distance: str = "l2", nthreads: int = 0):
    v16 = vectors if (isinstance(vectors, np.ndarray) and vectors.dtype == np.uint16) else as_padded_f16(vectors)
    q16 = queries if (isinstance(queries, np.ndarray) and queries.dtype == np.uint16) else as_padded_f16(queries)
    nq = q16.shape[0]
    ids = np.empty((nq, k), dtype=np.int32)
    d = np.empty((nq, k), dtype=np.float32)
    lib().jo_bruteforce_exact(metric_code(distance), _ptr(v16), v16.shape[0], _ptr(q16), nq,
                              v16.shape[1], k, _ptr(ids), _ptr(d), nthreads)
    return ids, d


def bruteforce_ref(vectors_f32, queries_f32, k: int = 10, distance: str = "l2", nthreads: int = 0,
                   ip_round_fp16: bool = False):
    """Reference ground-truth arithmetic (python/jasper/__init__.py:828-926);
    ip_round_fp16 models the fp16 matmul output of fp16 inputs under IP."""
    v = np.ascontiguousarray(vectors_f32, dtype=np.float32)
    q = np.ascontiguousarray(queries_f32, dtype=np.float32)
    nq = q.shape[0]
    ids = np.empty((nq, k), dtype=np.int32)
    d = np.empty((nq, k), dtype=np.float32)
    lib().jo_bruteforce_ref(metric_code(distance), _ptr(v), v.shape[0], _ptr(q), nq, v.shape[1], k,
                            _ptr(ids), _ptr(d), nthreads, 1 if ip_round_fp16 else 0)
    return ids, d


def rotation_matrix(d: int, seed: int = 42):
    """set_rotation_matrix, reference rotation/rotation.cuh:75-111. Returns
    (m, m_transpose) as column-major flat float32 arrays of length d*d."""
    m = np.empty(d * d, dtype=np.float32)
    mt = np.empty(d * d, dtype=np.float32)
    lib().jo_rotation_matrix(d, seed, _ptr(m), _ptr(mt))
    return m, mt


def gaussian_matrix(d: int, seed: int = 42) -> np.ndarray:
    """The N(0,1) matrix set_rotation_matrix factorises (column-major flat)."""
    a = np.empty(d * d, dtype=np.float32)
    lib().jo_gaussian_matrix(d, seed, _ptr(a))
    return a


# ------------------------------------------------------------- directional --
# Restatements of graph_beam_search_kernel (Appendix B) and its estimator
# artifacts; see directional_oracle.cpp.

def d2h(x: float) -> int:
    return int(lib().jo_d2h(float(x)))


def hsub(a: int, b: int) -> int:
    return int(lib().jo_hsub(a, b))


def hmul(a: int, b: int) -> int:
    return int(lib().jo_hmul(a, b))


def visit_exact(q16: np.ndarray, u16: np.ndarray, l2: bool = True):
    """compute_qu_diff_and_exact (beam_search_common.cuh:87-154): returns
    (exact, fp16 bits of q - u) for L2, (sum of fp16 products, None) for IP."""
    q16 = np.ascontiguousarray(q16, dtype=np.uint16)
    u16 = np.ascontiguousarray(u16, dtype=np.uint16)
    diff = np.zeros_like(q16) if l2 else None
    v = lib().jo_visit_exact(_ptr(q16), _ptr(u16), q16.shape[0], 1 if l2 else 0, _ptr(diff))
    return float(v), diff


def vector_norms(vecs16: np.ndarray, nthreads: int = 0) -> np.ndarray:
    out = np.empty(vecs16.shape[0], dtype=np.float32)
    lib().jo_vector_norms(_ptr(vecs16), vecs16.shape[0], vecs16.shape[1], _ptr(out), nthreads)
    return out


class LshArtifacts:
    def __init__(self, K, pbytes, c_per_rank, norm_denom, rows):
        self.K, self.pbytes = int(K), int(pbytes)
        self.c_per_rank = np.ascontiguousarray(c_per_rank, dtype=np.float32)
        self.norm_denom = float(np.float32(norm_denom))
        self.rows = np.ascontiguousarray(rows, dtype=np.uint8)


class PqArtifacts:
    def __init__(self, M, dsub, centroids, codes, norms):
        self.M, self.dsub = int(M), int(dsub)
        self.centroids = np.ascontiguousarray(centroids, dtype=np.float32)
        self.codes = np.ascontiguousarray(codes, dtype=np.uint8)
        self.norms = np.ascontiguousarray(norms, dtype=np.float32)


def lsh_row_bytes(R: int, K: int, pbytes: int) -> int:
    """sizeof(edge_lsh_list) (lsh/edge_lsh.cuh:9-27): packed[R*K] + bf16 mag[R]."""
    return R * K * pbytes + 2 * R


def populate_lsh(g: OracleGraph, K: int, pbytes: int, nthreads: int = 0) -> np.ndarray:
    rows = np.zeros((g.n, lsh_row_bytes(g.R, K, pbytes)), dtype=np.uint8)
    lib().jo_populate_lsh(_ptr(g.vecs16), g.n, g.dp, _ptr(g.edges), _ptr(g.counts), g.R, K, pbytes,
                          _ptr(rows), nthreads)
    return rows


def lsh_globals(g: OracleGraph, K: int, n_samples: int = 32768, seed: int = 42):
    c = np.zeros(K, dtype=np.float32)
    nd = ctypes.c_float(0.0)
    nv = lib().jo_lsh_globals(_ptr(g.vecs16), g.n, g.dp, _ptr(g.edges), _ptr(g.counts), g.R, K, n_samples,
                              seed, _ptr(c), ctypes.byref(nd))
    return c, float(nd.value), int(nv)


def build_lsh(g: OracleGraph, K: int, pbytes: int, n_samples: int = 32768, seed: int = 42,
              nthreads: int = 0) -> LshArtifacts:
    c, nd, _ = lsh_globals(g, K, n_samples, seed)
    return LshArtifacts(K, pbytes, c, nd, populate_lsh(g, K, pbytes, nthreads))


def pq_train(g: OracleGraph, M: int, n_train: int = 40000, iters: int = 12, seed: int = 123,
             nthreads: int = 0):
    """Codebook training (graph.cuh:1206-1273); returns (centroids
    [M*256*dsub], training residual rows [max(n_train, 256), dp] fp16 bits)."""
    dsub = g.dp // M
    nt = max(n_train, 256)
    cent = np.zeros(M * 256 * dsub, dtype=np.float32)
    X = np.zeros((nt, g.dp), dtype=np.uint16)
    lib().jo_pq_train(_ptr(g.vecs16), g.n, g.dp, _ptr(g.edges), _ptr(g.counts), g.R, M, n_train, iters, seed,
                      _ptr(cent), _ptr(X), nthreads)
    return cent, X


def pq_encode(g: OracleGraph, M: int, cent: np.ndarray, nthreads: int = 0) -> np.ndarray:
    codes = np.zeros((g.n, M * g.R), dtype=np.uint8)
    lib().jo_pq_encode(_ptr(g.vecs16), g.n, g.dp, _ptr(g.edges), _ptr(g.counts), g.R, M,
                       _ptr(np.ascontiguousarray(cent, dtype=np.float32)), _ptr(codes), nthreads)
    return codes


def pq_hash(x: int, seed: int) -> int:
    return int(lib().jo_pq_hash(x, seed))


def splitmix(x: int) -> int:
    return int(lib().jo_splitmix(x))


def sample_edge(g: OracleGraph, seed: int, s: int):
    u = ctypes.c_uint32(0)
    nb = ctypes.c_uint32(0)
    ok = lib().jo_sample_edge(_ptr(g.edges), _ptr(g.counts), g.n, g.R, seed, s, ctypes.byref(u), ctypes.byref(nb))
    return (int(u.value), int(nb.value)) if ok else None


def frontier_insert_seq(dists, ids, k: int):
    """frontier_insert_sorted (beam_search_common.cuh:156-185) applied to a
    sequence of (id, distance) visits; returns the frontier."""
    d = np.ascontiguousarray(dists, dtype=np.float32)
    i = np.ascontiguousarray(ids, dtype=np.uint32)
    od = np.zeros(max(k, 1), dtype=np.float32)
    oi = np.zeros(max(k, 1), dtype=np.uint32)
    cnt = ctypes.c_int(0)
    lib().jo_frontier_insert_seq(_ptr(d), _ptr(i), len(d), k, _ptr(od), _ptr(oi), ctypes.byref(cnt))
    return oi[:cnt.value].copy(), od[:cnt.value].copy()


def build_pq(g: OracleGraph, M: int, n_train: int = 40000, iters: int = 12, seed: int = 123,
             nthreads: int = 0) -> PqArtifacts:
    dsub = g.dp // M
    cent, _ = pq_train(g, M, n_train, iters, seed, nthreads)
    codes = np.zeros((g.n, M * g.R), dtype=np.uint8)
    lib().jo_pq_encode(_ptr(g.vecs16), g.n, g.dp, _ptr(g.edges), _ptr(g.counts), g.R, M, _ptr(cent),
                       _ptr(codes), nthreads)
    return PqArtifacts(M, dsub, cent, codes, vector_norms(g.vecs16, nthreads))


def directional_search(g: OracleGraph, queries, lsh: LshArtifacts | None = None, pq: PqArtifacts | None = None,
                       k: int = 10, beam_width: int = 64, limit: int | None = None, max_result: int = 2048,
                       get_visited: bool = False, unique: bool = False, nthreads: int = 0,
                       rq: "RqArtifacts | None" = None):
    """graph_beam_search_kernel (graph_beam_search.cuh:55-270) with the LSH,
    PQ or RaBitQ estimator; returns (ids, dists[, visited ids, visited dists,
    counts]). unique=True is this build's extension: pops of a node already
    in the frontier are skipped, so the results hold distinct ids. The
    RaBitQ estimator is this build's too (directional_oracle.cpp, rq_estimate)."""
    assert sum(a is not None for a in (lsh, pq, rq)) == 1
    mode = 0 if lsh is not None else (1 if pq is not None else 2)
    q16 = queries if (isinstance(queries, np.ndarray) and queries.dtype == np.uint16) else as_padded_f16(queries)
    nq = q16.shape[0]
    if limit is None:
        limit = 2 * beam_width
    ids = np.empty((nq, k), dtype=np.int32)
    d = np.empty((nq, k), dtype=np.float32)
    vi = vd = vc = None
    if get_visited:
        vi = np.zeros((nq, max_result), dtype=np.uint32)
        vd = np.zeros((nq, max_result), dtype=np.float32)
        vc = np.zeros(nq, dtype=np.uint32)
    L = lsh or LshArtifacts(0, 1, np.zeros(1, np.float32), 1.0, np.zeros(1, np.uint8))
    Q = pq or PqArtifacts(0, 0, np.zeros(1, np.float32), np.zeros(1, np.uint8), np.zeros(1, np.float32))
    Z = rq or RqArtifacts(0, np.zeros(1, np.uint8), np.zeros(1, np.float32))
    lib().jo_directional_search(mode, _ptr(g.vecs16), g.n, g.dp, _ptr(g.edges),
                                _ptr(g.counts), g.R, _ptr(g.deleted_bits), metric_code(g.distance),
                                L.K, L.pbytes, _ptr(L.c_per_rank), ctypes.c_float(L.norm_denom), _ptr(L.rows),
                                Q.M, Q.dsub, _ptr(Q.centroids), _ptr(Q.codes), _ptr(Q.norms),
                                Z.dim, _ptr(Z.nodes), _ptr(Z.centroid),
                                _ptr(q16), nq, g.medoid, k, beam_width, limit, max_result, _ptr(ids), _ptr(d),
                                _ptr(vi), _ptr(vd), _ptr(vc), None, 1 if unique else 0, nthreads)
    out = (ids, d)
    if get_visited:
        out += (vi, vd, vc)
    return out


def rotate_rows(vecs16: np.ndarray, dim: int, P16: np.ndarray, nthreads: int = 0) -> np.ndarray:
    """x' = P^T x per row, P column-major fp16 [dim*dim], fp32 accumulation."""
    out = np.zeros_like(vecs16)
    lib().jo_rotate_rows(_ptr(vecs16), vecs16.shape[0], dim, vecs16.shape[1],
                         _ptr(np.ascontiguousarray(P16, dtype=np.uint16)), _ptr(out), nthreads)
    return out


# ------------------------------------------------------------------ RaBitQ --
# rabitq_quantize<1> (rabitq/quantize.cuh:144-383); see rabitq_oracle.cpp.

def rabitq_code_bytes(dim: int) -> int:
    """rabitq_data_store::code_bytes (layout.cuh:57-63) at one bit per dim."""
    return int(lib().jo_rabitq_code_bytes(dim))


def rabitq_quantize(x, P, centroid=None, metric: str = "l2", nthreads: int = 0, return_residuals: bool = False):
    """One-bit RaBitQ codes of rows x [n, dim] (fp32) with rotation P
    (column-major [dim*dim]) and centroid c [dim] (None: zero). Returns
    (nodes u8 [n, code_bytes + 8], codes u8 [n, code_bytes], f_add f32 [n],
    f_rescale f32 [n][, residuals f32 [n, dim]])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, dim = x.shape
    P = np.ascontiguousarray(P, dtype=np.float32).ravel()
    c = None if centroid is None else np.ascontiguousarray(centroid, dtype=np.float32)
    cb = rabitq_code_bytes(dim)
    out = np.zeros((n, cb + 8), dtype=np.uint8)
    res = np.zeros((n, dim), dtype=np.float32) if return_residuals else None
    lib().jo_rabitq_quantize(_ptr(x), n, dim, _ptr(P), _ptr(c), 0 if metric == "l2" else 1, _ptr(out), _ptr(res),
                             nthreads)
    f_add = np.ascontiguousarray(out[:, cb:cb + 4]).view(np.float32).ravel()
    f_rescale = np.ascontiguousarray(out[:, cb + 4:cb + 8]).view(np.float32).ravel()
    r = (out, out[:, :cb].copy(), f_add, f_rescale)
    return r + (res,) if return_residuals else r


def best_rescale_factor(o_abs, ex_bits: int) -> float:
    """best_rescale_factor (reference quantize.cuh:22-82) of one row o = |x|."""
    o = np.ascontiguousarray(o_abs, dtype=np.float32).ravel()
    return float(lib().jo_best_rescale_factor(_ptr(o), o.shape[0], int(ex_bits)))


def const_scaling_factor(rows_abs, ex_bits: int) -> float:
    """Mean of best_rescale_factor over rows (get_const_scaling_factors'
    host loop, quantize.cuh:124-130)."""
    r = np.ascontiguousarray(rows_abs, dtype=np.float32)
    return float(lib().jo_const_scaling_factor(_ptr(r), r.shape[0], r.shape[1], int(ex_bits)))


def build_scale(vectors, R: int = 32, distance: str = "l2", alpha: float = 1.2, n_parts: int = 2,
                workspace_budget: int = 10 ** 10, part_batch: int | None = None,
                merge_batch: int | None = None, nthreads: int = 0) -> OracleGraph:
    """The partitioned build (reference index/construct_scale.cuh:68-450):
    n_parts contiguous partitions of ceil(n / n_parts) rows built on their own
    (batches doubling up to part_batch), their edges offset to global ids,
    then every pair of partitions merged once in the reference's cyclic order
    with B1 in batches of merge_batch. Defaults follow the reference
    (construct_scale.cuh:96-99 and 383-385, cmd/create_scale_index.cu:84):
    part_batch = min(budget batch, n / n_parts / 20), merge_batch = budget
    batch. Global ids; medoid 0."""
    v16 = as_padded_f16(vectors)
    n, dp = v16.shape
    dim = np.asarray(vectors).shape[1]
    # max_batch_size_for_budget (construct.cuh:238-262), without the FFI's n / 50 cap
    per_item = 8 * 64 + 8 * 256 + 4 + 8 * (256 + R) + 4 + 8 * R + 4 * R + 4 * R
    budget_batch = max(1, (workspace_budget - 4) // per_item)
    if part_batch is None:
        part_batch = max(1, min(budget_batch, n // n_parts // 20))
    if merge_batch is None:
        merge_batch = budget_batch
    edges = np.empty((n, R), dtype=np.uint32)
    edist = np.empty((n, R), dtype=np.uint16)
    counts = np.empty(n, dtype=np.uint8)
    rc = lib().jo_build_scale(_ptr(v16), n, dp, dim, R, metric_code(distance), float(alpha), n_parts,
                              part_batch, merge_batch, _ptr(edges), _ptr(edist), _ptr(counts), nthreads)
    if rc != 0:
        raise ValueError("build_scale: bad arguments (empty partition or batch < 1)")
    g = OracleGraph(v16, edges, edist, counts, R, dim, distance)
    g.n_parts = n_parts
    g.part_batch = part_batch
    g.merge_batch = merge_batch
    return g


def scale_merge_order(n_parts: int) -> list:
    """The (B1, B2) partition pairs in the order the partitioned build merges
    them (reference index/construct_scale.cuh:386-445)."""
    out = np.empty(max(1, n_parts * (n_parts - 1)), dtype=np.int64)
    m = int(lib().jo_scale_merge_order(n_parts, _ptr(out)))
    return [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(m)]


def prune_scale(vectors, b1: tuple, b2: tuple, self_id: int, cand_ids, cand_dists, R: int,
                alpha: float = 1.2, distance: str = "l2"):
    """The merge prune on one sorted candidate list (reference
    index/construct_scale_kernels.cuh:22-139): b1 / b2 are (first, count)
    row ranges whose vectors are resolvable. Returns (ids, dists)."""
    v16 = as_padded_f16(vectors)
    dim = np.asarray(vectors).shape[1]
    ids = np.ascontiguousarray(cand_ids, dtype=np.uint32)
    dists = np.ascontiguousarray(cand_dists, dtype=np.float32)
    out_i = np.empty(R, dtype=np.uint32)
    out_d = np.empty(R, dtype=np.float32)
    ns = lib().jo_prune_scale(_ptr(v16), v16.shape[1], dim, metric_code(distance), float(alpha), R, b1[0], b1[1],
                              b2[0], b2[1], self_id, _ptr(ids), _ptr(dists), len(ids), _ptr(out_i), _ptr(out_d))
    return out_i[:ns].copy(), out_d[:ns].copy()


def diskann_assign(vectors, n_parts: int, n_dup: int = 2, seed: int = 42):
    """Shard assignment of the DiskANN build (reference
    index/construct_diskann.cuh:104-276): per row, n_dup shards (INVALID =
    0xFFFFFFFF where a rank repeats a shard). Returns (shard_of [n, n_dup]
    uint32, mean [dim] fp16 bits)."""
    v16 = as_padded_f16(vectors)
    n, dp = v16.shape
    dim = np.asarray(vectors).shape[1]
    out = np.empty((n, n_dup), dtype=np.uint32)
    mean = np.empty(dim, dtype=np.uint16)
    rc = lib().jo_diskann_assign(_ptr(v16), n, dp, dim, n_parts, n_dup, seed, _ptr(out), _ptr(mean))
    if rc != 0:
        raise ValueError("diskann_assign: bad arguments")
    return out, mean


def diskann_batch_cap(n: int, R_int: int, n_parts: int, workspace_budget: int = 10 ** 10) -> int:
    """min(budget batch at R_int, max(1, n / n_parts / 20)) (construct_diskann.cuh:373-375,
    cmd/create_diskann_index.cu:84)."""
    per_item = 8 * 64 + 8 * 256 + 4 + 8 * (256 + R_int) + 4 + 8 * R_int + 4 * R_int + 4 * R_int
    budget_batch = (workspace_budget - 4) // per_item
    return max(1, min(budget_batch, max(1, n // n_parts // 20)))


def build_diskann(vectors, R_int: int = 32, R_fin: int = 32, distance: str = "l2", alpha: float = 1.2,
                  n_parts: int = 4, n_dup: int = 2, seed: int = 42, workspace_budget: int = 10 ** 10,
                  batch_cap: int | None = None, max_shard: int = 0, nthreads: int = 0) -> OracleGraph:
    """The DiskANN build (reference index/construct_diskann.cuh:328-613): LSH
    shards with duplication, one graph of degree R_int per shard (a shard
    above max_shard rows, when max_shard > 0, built as equal sub-shards),
    then the distance-only merge into rows of R_fin. Global ids; medoid 0."""
    v16 = as_padded_f16(vectors)
    n, dp = v16.shape
    dim = np.asarray(vectors).shape[1]
    if batch_cap is None:
        batch_cap = diskann_batch_cap(n, R_int, n_parts, workspace_budget)
    edges = np.empty((n, R_fin), dtype=np.uint32)
    edist = np.empty((n, R_fin), dtype=np.uint16)
    counts = np.empty(n, dtype=np.uint8)
    shard_of = np.empty((n, n_dup), dtype=np.uint32)
    rc = lib().jo_build_diskann(_ptr(v16), n, dp, dim, R_int, R_fin, metric_code(distance), float(alpha), n_parts,
                                n_dup, seed, batch_cap, int(max_shard), _ptr(edges), _ptr(edist), _ptr(counts),
                                _ptr(shard_of), nthreads)
    if rc != 0:
        raise ValueError("build_diskann: bad arguments")
    g = OracleGraph(v16, edges, edist, counts, R_fin, dim, distance)
    g.shard_of = shard_of
    g.batch_cap = batch_cap
    return g


class RqArtifacts:
    """RaBitQ one-bit codes of a graph's stored rows: nodes u8 [n,
    code_bytes + 8] (code, f_add, f_rescale) taken against centroid f32
    [dim]."""

    def __init__(self, dim, nodes, centroid):
        self.dim = int(dim)
        self.nodes = np.ascontiguousarray(nodes, dtype=np.uint8)
        self.centroid = np.ascontiguousarray(centroid, dtype=np.float32)


def rq_estimates(rq: RqArtifacts, queries16: np.ndarray, metric: str = "l2", with_factors: bool = False):
    """The RaBitQ estimate of every node for every query row (fp16 bits
    [nq, dp]): f32 [nq, n]; with_factors also returns each query's (sumq,
    (delta/2, lo/2, g_add), bit planes u32 [nq, 4, 8])."""
    q16 = np.ascontiguousarray(queries16, dtype=np.uint16)
    nq, dp = q16.shape
    n = rq.nodes.shape[0]
    out = np.zeros((nq, n), dtype=np.float32)
    sumq = np.zeros(nq, dtype=np.int32)
    hhg = np.zeros((nq, 3), dtype=np.float32)
    planes = np.zeros((nq, 4, 8), dtype=np.uint32)
    lib().jo_rq_estimates(_ptr(rq.nodes), n, rq.dim, _ptr(rq.centroid), metric_code(metric), _ptr(q16), nq, dp,
                          _ptr(out), _ptr(sumq), _ptr(hhg), _ptr(planes))
    return (out, sumq, hhg, planes) if with_factors else out


# ------------------------------------------------------------- file format --

def bytes_per_node(dim: int, R: int) -> int:
    """save_graph_to_file, graph.cuh:1676-1677: 2*dim + 1 + (4R + 2R) + 4."""
    return 2 * dim + 1 + 6 * R + 4


def save_graph(g: OracleGraph, path: str | os.PathLike) -> int:
    """Restates save_graph_to_file (graph.cuh:1653-1788) byte for byte."""
    n, dim, R = g.n, g.dim, g.R
    bpn = bytes_per_node(dim, R)
    deleted_bytes = (n + 7) // 8
    total = 32 + n * bpn + deleted_bytes + 8
    rec = np.zeros((n, bpn), dtype=np.uint8)
    off = 0
    rec[:, off:off + 2 * dim] = g.vecs16[:, :dim].view(np.uint8).reshape(n, -1)[:, :2 * dim]
    off += 2 * dim
    rec[:, off] = g.counts
    off += 1
    rec[:, off:off + 4 * R] = g.edges.view(np.uint8).reshape(n, 4 * R)
    off += 4 * R
    rec[:, off:off + 2 * R] = g.edge_dist.view(np.uint8).reshape(n, 2 * R)
    off += 2 * R
    rec[:, off:off + 4] = g.slot_to_id.view(np.uint8).reshape(n, 4)
    packed = np.zeros(deleted_bytes, dtype=np.uint8)
    bits = ((g.deleted_bits[np.arange(n) >> 5] >> (np.arange(n) & 31).astype(np.uint32)) & 1).astype(np.uint8)
    for b in range(8):
        sel = bits[b::8]
        packed[:len(sel)] |= (sel << b).astype(np.uint8)
    with open(path, "wb") as f:
        f.write(struct.pack("<QQQQ", total, n, g.medoid, bpn))
        f.write(rec.tobytes())
        f.write(packed.tobytes())
        f.write(struct.pack("<Q", g.next_id))
    return total


def load_graph(path: str | os.PathLike, dim: int, R: int, distance: str = "l2") -> OracleGraph:
    """Restates load_graph_from_file (graph.cuh:1425-1651) for the current
    bit-packed layout and the three legacy layouts it accepts."""
    data = Path(path).read_bytes()
    total, n, medoid, bpn = struct.unpack_from("<QQQQ", data, 0)
    base = 2 * dim + 1 + 6 * R
    if bpn not in (base, base + 1, base + 1 + 4, base + 4):
        raise ValueError(f"bytes_per_node {bpn} matches no known layout")
    rec = np.frombuffer(data, dtype=np.uint8, count=n * bpn, offset=32).reshape(n, bpn)
    dp = pad_dim(dim)
    vecs16 = np.zeros((n, dp), dtype=np.uint16)
    vecs16[:, :dim] = np.ascontiguousarray(rec[:, :2 * dim]).view(np.uint16)
    off = 2 * dim
    counts = rec[:, off].copy()
    off += 1
    edges = np.ascontiguousarray(rec[:, off:off + 4 * R]).view(np.uint32).reshape(n, R).copy()
    off += 4 * R
    edist = np.ascontiguousarray(rec[:, off:off + 2 * R]).view(np.uint16).reshape(n, R).copy()
    off += 2 * R
    deleted = np.zeros((n + 31) // 32, dtype=np.uint32)
    slot_to_id = np.arange(n, dtype=np.uint32)
    next_id = n
    if bpn in (base + 1, base + 5):
        dbytes = rec[:, off].astype(bool)
        off += 1
        for i in np.nonzero(dbytes)[0]:
            deleted[i >> 5] |= np.uint32(1 << (i & 31))
    if bpn in (base + 5, base + 4):
        slot_to_id = np.ascontiguousarray(rec[:, off:off + 4]).view(np.uint32).reshape(n).copy()
    pos = 32 + n * bpn
    if bpn == base + 4:
        nbytes = (n + 7) // 8
        packed = np.frombuffer(data, dtype=np.uint8, count=nbytes, offset=pos)
        pos += nbytes
        for i in range(n):
            if (packed[i >> 3] >> (i & 7)) & 1:
                deleted[i >> 5] |= np.uint32(1 << (i & 31))
    if bpn in (base + 5, base + 4):
        (next_id,) = struct.unpack_from("<Q", data, pos)
    return OracleGraph(vecs16, edges, edist, counts, R, dim, distance, medoid=medoid,
                       deleted_bits=deleted, slot_to_id=slot_to_id, next_id=next_id)


def recall(gt_ids: np.ndarray, ids: np.ndarray, k: int) -> float:
    """get_recall, python/jasper/__init__.py:819-826."""
    hit = 0
    for a, b in zip(gt_ids[:, :k], ids[:, :k]):
        hit += len(set(a.tolist()) & set(b.tolist()))
    return hit / (gt_ids.shape[0] * k)
