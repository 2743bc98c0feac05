"""jasper_amd -- MI355X-native Jasper query/build hot path.

Drop-in counterpart of the reference Python package (python/jasper/__init__.py):
the same ``Graph.build / load / save / search / directional_search /
pq_search`` API, config registries, argument checks and utilities, bound to
``lib/libjasper_amd.so`` (hand-written HIP for gfx950) through its C ABI
(``include/jasper_amd.h``) instead of TVM-FFI.

There is no CPU fallback: if the HIP library is missing every entry point
raises.
"""

from __future__ import annotations

import ctypes
import re
import struct
from enum import Enum
from pathlib import Path

import numpy as np
import torch

_LIB_PATH = Path(__file__).resolve().parent / "lib" / "libjasper_amd.so"
_lib = None


def _load_lib():
    """Load the HIP library (reference: tvm_ffi.load_module, __init__.py:13-14)."""
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise RuntimeError(
                f"jasper_amd HIP library not found at {_LIB_PATH}; build it with "
                "`python -m jasper_amd.build_lib` (there is no CPU fallback)")
        lib = ctypes.CDLL(str(_LIB_PATH))
        lib.jasper_last_error.restype = ctypes.c_char_p
        lib.jasper_last_error.argtypes = []
        lib.jasperx_version.restype = ctypes.c_char_p
        _lib = lib
    return _lib


def library_path() -> Path:
    return _LIB_PATH


_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p
_bool = ctypes.c_bool
_f64 = ctypes.c_double
_str = ctypes.c_char_p

# option flag of jasperx_directional_search_ex: distinct results
DIR_UNIQUE = 1

_SIGS = {
    "load": ([_str, _i64, _bool]),
    "construct": ([_ptr, _i64, _i64, _f64, _i64, _bool, _ptr]),
    "search": ([_i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _i64, _i64, _bool, _ptr]),
    "save": ([_i64, _str]),
    "get_vector": ([_i64, _i64, _ptr, _ptr]),
    "mark_deleted": ([_i64, _ptr, _i64]),
    "consolidate": ([_i64, _f64]),
    "compact": ([_i64]),
    "append": ([_i64, _ptr, _i64, _f64, _ptr, _ptr]),
    "construct_directional": ([_ptr, _i64, _i64, _f64, _i64, _bool, _bool, _i64, _ptr]),
    "build_lsh": ([_i64, _i64, _i64]),
    "build_pq": ([_i64, _i64, _i64, _i64]),
    "directional_search": ([_i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _i64, _i64, _bool, _ptr]),
    "pq_search": ([_i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _i64, _i64, _bool, _ptr]),
    "save_directional": ([_i64, _str]),
    "load_directional": ([_str, _i64, _bool, _bool, _i64]),
    "get_vector_directional": ([_i64, _i64, _ptr, _ptr]),
    "get_directional_flags": ([_i64]),
}

_AGNOSTIC = {
    "jasper_free_graph": [_i64],
    "jasper_get_n_vectors": [_i64],
    "jasper_get_n_tombstoned": [_i64],
    "jasper_get_n_live": [_i64],
    "jasper_reserve_ids": [_i64, _ptr, _i64],
    "jasper_get_dim": [_i64],
    "jasperx_export_graph": [_i64, _ptr, _ptr, _ptr],
    "jasperx_last_build_stats": [_ptr],
    "jasperx_build_work_counting": [_i64],
    "jasperx_last_build_work": [_ptr],
    "jasperx_prerotate_seed": [_i64],
    "jasperx_row_format": [_i64, _ptr],
    "jasperx_search_stats": [_i64, _ptr, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr],
    "jasperx_export_vectors": [_i64, _ptr],
    "jasperx_export_lsh": [_i64, _ptr, _ptr, _ptr],
    "jasperx_export_pq": [_i64, _ptr, _ptr, _ptr],
    "jasperx_rotation_matrix": [_i64, _i64, _ptr],
    "jasperx_directional_query_rows": [_i64, _ptr, _i64, _i64, _ptr, _ptr],
    "jasperx_rotate_rows": [_i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _ptr],
    "jasperx_rabitq_node_bytes": [_i64],
    "jasperx_directional_stats": [_i64, ctypes.c_int32, _ptr, _i64, _i64, _i64, _i64, _i64, ctypes.c_uint32,
                                  _ptr, _ptr],
    "jasperx_build_pq_m": [_i64, _i64, _i64, _i64, _i64],
    "jasperx_build_rabitq": [_i64],
    "jasperx_exact_search": [_i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _i64, _i64, _ptr],
    "jasperx_construct_directional_ex": [ctypes.c_char_p, _ptr, _i64, _i64, ctypes.c_double, _i64, ctypes.c_bool,
                                         ctypes.c_bool, _i64, ctypes.c_uint32, _ptr],
    "jasperx_export_rabitq": [_i64, _ptr, _ptr],
    "jasperx_construct_scale": [ctypes.c_char_p, _ptr, _i64, _i64, ctypes.c_double, _i64, _i64, _i64, _bool, _ptr],
    "jasperx_last_scale_stats": [_ptr],
    "jasperx_construct_diskann": [ctypes.c_char_p, _ptr, _i64, _i64, ctypes.c_double, _i64, _i64, _i64, _i64, _i64,
                                  _i64, _i64, _ptr],
    "jasperx_diskann_assign": [_ptr, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr, _ptr],
    "jasperx_last_diskann_stats": [_ptr],
    "jasperx_directional_search_noalloc": [_i64, ctypes.c_int32, _ptr, _i64, _i64, _ptr, _ptr, _i64, _i64,
                                           _i64, ctypes.c_uint32, _ptr],
    "jasperx_directional_search_ex": [_i64, ctypes.c_int32, _ptr, _i64, _i64, _ptr, _ptr, _i64, _i64, _i64,
                                      ctypes.c_uint32, _ptr],
    "jasperx_bruteforce_knn": [_ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, ctypes.c_int32, _ptr, _ptr, _ptr],
    "jasperx_rabitq_quantize": [_ptr, ctypes.c_int32, _i64, _i64, _i64, _ptr, _ptr, ctypes.c_int32, _ptr, _ptr],
}


class JasperError(RuntimeError):
    pass


def _bind(name: str, argtypes):
    lib = _load_lib()
    fn = getattr(lib, name)
    fn.restype = _i64
    fn.argtypes = argtypes

    def call(*args):
        r = fn(*args)
        if r < 0:
            msg = lib.jasper_last_error().decode(errors="replace")
            if msg.startswith("Invalid handle") or "different config" in msg:
                raise ValueError(msg)
            if "too large" in msg or "must be" in msg or "out of range" in msg or "not found" in msg:
                raise ValueError(msg)
            raise JasperError(msg)
        return r

    call.__name__ = name
    return call


def _op(op: str, config_id: str):
    return _bind(f"jasper_{op}_{config_id}", _SIGS[op])


def _agnostic(name: str):
    return _bind(name, _AGNOSTIC[name])


# ── Config enums (reference __init__.py:18-24) ────────────────────────
class DistanceFunc(str, Enum):
    L2 = "l2"
    INNER_PRODUCT = "ip"


class DataType(str, Enum):
    FLOAT16 = "f16"


# ── Config registry (reference __init__.py:29-38) ─────────────────────
_CONFIGS: dict[tuple[DataType, int, DistanceFunc], str] = {
    (DataType.FLOAT16, 8, DistanceFunc.L2): "f16_r8_l2",
    (DataType.FLOAT16, 16, DistanceFunc.L2): "f16_r16_l2",
    (DataType.FLOAT16, 32, DistanceFunc.L2): "f16_r32_l2",
    (DataType.FLOAT16, 64, DistanceFunc.L2): "f16_r64_l2",
    (DataType.FLOAT16, 8, DistanceFunc.INNER_PRODUCT): "f16_r8_ip",
    (DataType.FLOAT16, 16, DistanceFunc.INNER_PRODUCT): "f16_r16_ip",
    (DataType.FLOAT16, 32, DistanceFunc.INNER_PRODUCT): "f16_r32_ip",
    (DataType.FLOAT16, 64, DistanceFunc.INNER_PRODUCT): "f16_r64_ip",
}

_DTYPE_MAP = {DataType.FLOAT16: torch.float16}


def _resolve_config(data_type: DataType, n_neighbors: int, distance: DistanceFunc) -> str:
    key = (data_type, n_neighbors, distance)
    if key not in _CONFIGS:
        supported = "\n  ".join(f"({d.value}, R={r}, {f.value})" for (d, r, f) in _CONFIGS)
        raise ValueError(
            f"Unsupported config: data_type={data_type.value}, "
            f"n_neighbors={n_neighbors}, distance={distance.value}\n"
            f"Supported configs:\n  {supported}")
    return _CONFIGS[key]


# ── Directional registry (reference __init__.py:66-84) ────────────────
_DIRECTIONAL_CONFIGS: dict[tuple[DataType, int, DistanceFunc, int, bool], str] = {}
for _r in (32, 64):
    for _f in (DistanceFunc.L2, DistanceFunc.INNER_PRODUCT):
        for _k in (4, 16):
            for _small in (True, False):
                _DIRECTIONAL_CONFIGS[(DataType.FLOAT16, _r, _f, _k, _small)] = (
                    f"f16_r{_r}_{_f.value}_k{_k}_d{'128' if _small else '32678'}")


def _resolve_directional_config(data_type: DataType, n_neighbors: int, distance: DistanceFunc,
                                k_ranks: int, dim: int) -> str:
    key = (data_type, n_neighbors, distance, k_ranks, dim <= 128)
    if key not in _DIRECTIONAL_CONFIGS:
        supported = "\n  ".join(
            f"({d.value}, R={r}, {f.value}, k_ranks={kr}, dim<=128={le128})"
            for (d, r, f, kr, le128) in _DIRECTIONAL_CONFIGS)
        raise ValueError(
            f"Unsupported directional config: data_type={data_type.value}, "
            f"n_neighbors={n_neighbors}, distance={distance.value}, "
            f"k_ranks={k_ranks}, dim={dim}\n"
            f"Supported configs:\n  {supported}")
    return _DIRECTIONAL_CONFIGS[key]


# ── Storage sizes (reference __init__.py:152-171; decimal units) ──────
STORAGE_SIZE_RE = re.compile(r'^\s*([\d.]+)\s*([KMGTP]?i?B)\s*$', re.IGNORECASE)
STORAGE_UNITS = {
    "B": 1, "KB": 10 ** 3, "MB": 10 ** 6, "GB": 10 ** 9, "TB": 10 ** 12,
    "KIB": 2 ** 10, "MIB": 2 ** 20, "GIB": 2 ** 30, "TIB": 2 ** 40,
}


def parse_storage_size(s: str) -> int:
    m = STORAGE_SIZE_RE.match(s)
    if not m:
        raise ValueError(f"Invalid storage size: {s}")
    value, unit = m.groups()
    if unit.upper() not in STORAGE_UNITS:
        raise ValueError(f"Invalid storage size: {s}")
    return int(float(value) * STORAGE_UNITS[unit.upper()])


def _stream_ptr(device=None) -> int:
    if not torch.cuda.is_available():
        return 0
    return torch.cuda.current_stream(device).cuda_stream


def _tensor_ptr(t: torch.Tensor):
    return ctypes.c_void_p(t.data_ptr())


# ── Graph (reference __init__.py:174-766) ─────────────────────────────
class Graph:
    """A GPU-resident Vamana graph index (see the reference class docstring)."""

    def __init__(self, handle: int, config_id: str, data_type: DataType, distance: DistanceFunc,
                 n_neighbors: int, dim: int, *, is_directional: bool = False,
                 k_ranks: int | None = None, has_lsh: bool = False, has_pq: bool = False,
                 prerotate: bool = False, prerotate_seed: int = 42, has_rabitq: bool = False):
        self._handle = handle
        self._config_id = config_id
        self._data_type = data_type
        self._distance = distance
        self._n_neighbors = n_neighbors
        self._dim = dim
        self._torch_dtype = _DTYPE_MAP[data_type]
        self._is_directional = is_directional
        self._k_ranks = k_ranks
        self._has_lsh = has_lsh
        self._has_pq = has_pq
        self._has_rabitq = has_rabitq
        self._prerotate = prerotate
        self._prerotate_seed = prerotate_seed
        if is_directional:
            self._save_fn = _op("save_directional", config_id)
            self._get_vector_fn = _op("get_vector_directional", config_id)
            self._directional_search_fn = _op("directional_search", config_id)
            self._pq_search_fn = _op("pq_search", config_id)
            self._get_flags_fn = _op("get_directional_flags", config_id)
            self._build_lsh_fn = _op("build_lsh", config_id)
            self._build_pq_fn = _op("build_pq", config_id)
            self._search_fn = None
            self._mark_deleted_fn = self._consolidate_fn = self._compact_fn = self._append_fn = None
        else:
            self._search_fn = _op("search", config_id)
            self._save_fn = _op("save", config_id)
            self._get_vector_fn = _op("get_vector", config_id)
            self._mark_deleted_fn = _op("mark_deleted", config_id)
            self._consolidate_fn = _op("consolidate", config_id)
            self._compact_fn = _op("compact", config_id)
            self._append_fn = _op("append", config_id)

    # -- construction -------------------------------------------------------
    @classmethod
    def load(cls, path: str, dim: int, n_neighbors: int = 32,
             data_type: DataType | str = DataType.FLOAT16,
             distance: DistanceFunc | str = DistanceFunc.L2, on_host: bool = False,
             k_ranks: int | None = None, prerotate: bool = False,
             prerotate_seed: int = 42) -> "Graph":
        """Load a graph file (reference __init__.py:238-320)."""
        if isinstance(data_type, str):
            data_type = DataType(data_type)
        if isinstance(distance, str):
            distance = DistanceFunc(distance)
        if k_ranks is None:
            config_id = _resolve_config(data_type, n_neighbors, distance)
            handle = _op("load", config_id)(str(path).encode(), dim, on_host)
            return cls(handle, config_id, data_type, distance, n_neighbors, dim)
        config_id = _resolve_directional_config(data_type, n_neighbors, distance, k_ranks, dim)
        handle = _op("load_directional", config_id)(str(path).encode(), dim, on_host, prerotate,
                                                    prerotate_seed)
        flags = _op("get_directional_flags", config_id)(handle)
        if flags & 8:  # the file records its prerotation; it wins over the arguments
            prerotate, prerotate_seed = True, int(_agnostic("jasperx_prerotate_seed")(handle))
        return cls(handle, config_id, data_type, distance, n_neighbors, dim,
                   is_directional=True, k_ranks=k_ranks, has_lsh=bool(flags & 1),
                   has_pq=bool(flags & 2), prerotate=prerotate, prerotate_seed=prerotate_seed,
                   has_rabitq=bool(flags & 16))

    def save(self, path: str) -> None:
        """Save to the reference's binary format (reference __init__.py:307-320)."""
        self._check_alive()
        self._save_fn(self._handle, str(path).encode())

    @classmethod
    def build(cls, vectors: torch.Tensor, n_neighbors: int = 32,
              distance: DistanceFunc | str = DistanceFunc.L2, alpha: float = 1.2,
              workspace_budget: str = "10GB", on_host: bool = False, build_lsh: bool = False,
              build_pq: bool = False, k_ranks: int = 4, prerotate: bool | None = None,
              prerotate_seed: int = 42, lsh_samples: int = 32768, lsh_seed: int = 42,
              pq_train: int = 40000, pq_kmeans_iter: int = 12, pq_seed: int = 123,
              pq_m: int | None = None, build_rabitq: bool = False,
              build_search: str = "exact") -> "Graph":
        """Construct a Vamana graph on the GPU (reference __init__.py:322-428).

        pq_m (an extension, no reference counterpart) sets the number of PQ
        subspaces; None keeps the reference's pq_m = k_ranks. Any value that
        divides the padded dim, up to 128, e.g. 120 for one subspace per 8
        dims at d = 960. build_rabitq (an extension) adds one-bit RaBitQ codes
        of the stored rows for rabitq_search; it makes the graph directional
        like build_lsh / build_pq. build_search="rabitq" (an extension) makes
        the construction's search stage pop by the RaBitQ estimate of the
        stored rows (their codes are computed first and kept) instead of the
        exact plain search; "exact" is the reference construction."""
        if build_search not in ("exact", "rabitq"):
            raise ValueError(f"build_search must be 'exact' or 'rabitq', got {build_search!r}")
        if isinstance(distance, str):
            distance = DistanceFunc(distance)
        workspace_budget_bytes = parse_storage_size(workspace_budget)
        if vectors.ndim != 2:
            raise ValueError(f"vectors must be 2D, got {vectors.ndim}D")
        vectors = vectors.contiguous()
        dim = vectors.size(1)
        if vectors.dtype == torch.float16:
            data_type = DataType.FLOAT16
        else:
            raise ValueError(f"Unsupported tensor dtype: {vectors.dtype}. Use torch.float16.")
        n = vectors.size(0)
        stream = _stream_ptr(vectors.device if vectors.is_cuda else None)
        if build_search == "rabitq":
            build_rabitq = True
        if not (build_lsh or build_pq or build_rabitq):
            config_id = _resolve_config(data_type, n_neighbors, distance)
            handle = _op("construct", config_id)(_tensor_ptr(vectors), n, dim, float(alpha),
                                                 workspace_budget_bytes, on_host, stream)
            return cls(handle, config_id, data_type, distance, n_neighbors, dim)
        config_id = _resolve_directional_config(data_type, n_neighbors, distance, k_ranks, dim)
        resolved_prerotate = prerotate if prerotate is not None else True
        if build_search == "rabitq":
            handle = _agnostic("jasperx_construct_directional_ex")(
                config_id.encode(), _tensor_ptr(vectors), n, dim, float(alpha), workspace_budget_bytes, on_host,
                resolved_prerotate, prerotate_seed, 1, stream)
        else:
            handle = _op("construct_directional", config_id)(
                _tensor_ptr(vectors), n, dim, float(alpha), workspace_budget_bytes, on_host,
                resolved_prerotate, prerotate_seed, stream)
        if build_lsh:
            _op("build_lsh", config_id)(handle, lsh_samples, lsh_seed)
        if build_pq:
            if pq_m is None or pq_m == k_ranks:
                _op("build_pq", config_id)(handle, pq_train, pq_kmeans_iter, pq_seed)
            else:
                _agnostic("jasperx_build_pq_m")(handle, pq_m, pq_train, pq_kmeans_iter, pq_seed)
        if build_rabitq and build_search != "rabitq":
            _agnostic("jasperx_build_rabitq")(handle)
        return cls(handle, config_id, data_type, distance, n_neighbors, dim,
                   is_directional=True, k_ranks=k_ranks, has_lsh=build_lsh, has_pq=build_pq,
                   has_rabitq=build_rabitq,
                   prerotate=resolved_prerotate, prerotate_seed=prerotate_seed)

    @classmethod
    def build_scale(cls, vectors: torch.Tensor, n_neighbors: int = 32,
                    distance: DistanceFunc | str = DistanceFunc.L2, alpha: float = 1.2, n_parts: int = 2,
                    workspace_budget: str = "10GB", max_batch_size: int | None = None,
                    on_host: bool = False) -> "Graph":
        """The partitioned build of the reference's create_scale_index command
        (cmd/create_scale_index.cu:57-98; include/jasper/index/
        construct_scale.cuh): n_parts partitions built on their own, then
        every pair merged. max_batch_size caps the partitions' batches (None:
        n / n_parts / 20, as the command sets it); merges use the workspace
        budget's batch. on_host: the graph lives in pinned host memory and
        partitions are staged through the device two at a time (indexes
        larger than HBM); the same graph. Returns a plain graph (search,
        save, updates)."""
        if isinstance(distance, str):
            distance = DistanceFunc(distance)
        if vectors.ndim != 2:
            raise ValueError(f"vectors must be 2D, got {vectors.ndim}D")
        if vectors.dtype != torch.float16:
            raise ValueError(f"Unsupported tensor dtype: {vectors.dtype}. Use torch.float16.")
        vectors = vectors.contiguous()
        n, dim = vectors.shape
        config_id = _resolve_config(DataType.FLOAT16, n_neighbors, distance)
        stream = _stream_ptr(vectors.device if vectors.is_cuda else None)
        handle = _agnostic("jasperx_construct_scale")(
            config_id.encode(), _tensor_ptr(vectors), n, dim, float(alpha), int(n_parts),
            parse_storage_size(workspace_budget), int(max_batch_size or 0), bool(on_host), stream)
        return cls(handle, config_id, DataType.FLOAT16, distance, n_neighbors, dim)

    @classmethod
    def build_diskann(cls, vectors: torch.Tensor, n_neighbors: int = 32, r_int: int = 32,
                      distance: DistanceFunc | str = DistanceFunc.L2, alpha: float = 1.2, n_parts: int = 4,
                      n_dup: int = 2, workspace_budget: str = "10GB", max_batch_size: int | None = None,
                      seed: int = 42, max_shard: int | None = None) -> "Graph":
        """The DiskANN build of the reference's create_diskann_index command
        (cmd/create_diskann_index.cu:59-103; include/jasper/index/
        construct_diskann.cuh): rows sharded by cross-polytope LSH into n_dup
        of n_parts shards, each shard built at degree r_int, rows merged by
        stored distance into n_neighbors (the final degree). A shard of more
        than max_shard rows is built as equal sub-shards (None: the largest
        shard graph the free device memory holds). Returns a plain graph
        (search, save, updates)."""
        if isinstance(distance, str):
            distance = DistanceFunc(distance)
        if vectors.ndim != 2:
            raise ValueError(f"vectors must be 2D, got {vectors.ndim}D")
        if vectors.dtype != torch.float16:
            raise ValueError(f"Unsupported tensor dtype: {vectors.dtype}. Use torch.float16.")
        vectors = vectors.contiguous()
        n, dim = vectors.shape
        config_id = _resolve_config(DataType.FLOAT16, n_neighbors, distance)
        stream = _stream_ptr(vectors.device if vectors.is_cuda else None)
        handle = _agnostic("jasperx_construct_diskann")(
            config_id.encode(), _tensor_ptr(vectors), n, dim, float(alpha), int(r_int), int(n_parts), int(n_dup),
            parse_storage_size(workspace_budget), int(max_batch_size or 0), int(seed), int(max_shard or 0), stream)
        return cls(handle, config_id, DataType.FLOAT16, distance, n_neighbors, dim)

    # -- properties ---------------------------------------------------------
    @property
    def dim(self) -> int:
        return self._dim

    @property
    def n_vectors(self) -> int:
        self._check_alive()
        return _agnostic("jasper_get_n_vectors")(self._handle)

    @property
    def n_neighbors(self) -> int:
        return self._n_neighbors

    @property
    def data_type(self) -> DataType:
        return self._data_type

    @property
    def distance(self) -> DistanceFunc:
        return self._distance

    @property
    def handle(self) -> int:
        return self._handle

    # -- search -------------------------------------------------------------
    def _query_check(self, queries: torch.Tensor) -> torch.Tensor:
        if not queries.is_cuda:
            raise ValueError("queries must be a CUDA tensor")
        if queries.dtype != self._torch_dtype:
            raise ValueError(f"queries must be {self._torch_dtype}, got {queries.dtype}")
        if queries.ndim != 2:
            raise ValueError(f"queries must be 2D, got {queries.ndim}D")
        if queries.size(1) != self._dim:
            raise ValueError(f"query dim ({queries.size(1)}) != graph dim ({self._dim})")
        return queries.contiguous()

    def _run_search(self, fn, queries, k, beam_width, limit, print_throughput):
        n_queries = queries.size(0)
        out_indices = torch.empty(n_queries, k, dtype=torch.int32, device=queries.device)
        out_distances = torch.empty(n_queries, k, dtype=torch.float32, device=queries.device)
        fn(self._handle, _tensor_ptr(queries), n_queries, self._dim, _tensor_ptr(out_indices),
           _tensor_ptr(out_distances), k, beam_width, limit, print_throughput,
           _stream_ptr(queries.device))
        return out_indices, out_distances

    def search(self, queries: torch.Tensor, k: int = 10, beam_width: int = 64,
               print_throughput: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
        """Plain beam search (reference __init__.py:451-508); limit = 2 * beam_width."""
        self._check_alive()
        if self._is_directional:
            raise RuntimeError(
                "search() is not available on a directional graph "
                "(built with build_lsh=True/build_pq=True) — use "
                "directional_search() or pq_search() instead")
        queries = self._query_check(queries)
        return self._run_search(self._search_fn, queries, k, beam_width, beam_width * 2,
                                print_throughput)

    def _run_ex(self, estimator, queries, k, beam_width, limit, unique):
        n_queries = queries.size(0)
        out_indices = torch.empty(n_queries, k, dtype=torch.int32, device=queries.device)
        out_distances = torch.empty(n_queries, k, dtype=torch.float32, device=queries.device)
        _agnostic("jasperx_directional_search_ex")(
            self._handle, estimator, _tensor_ptr(queries), n_queries, self._dim,
            _tensor_ptr(out_indices), _tensor_ptr(out_distances), k, beam_width, limit,
            DIR_UNIQUE if unique else 0, _stream_ptr(queries.device))
        return out_indices, out_distances

    def _run_unique(self, use_pq, queries, k, beam_width, limit):
        return self._run_ex(1 if use_pq else 0, queries, k, beam_width, limit, True)

    def directional_search(self, queries: torch.Tensor, k: int = 10, beam_width: int = 64,
                           limit: int | None = None, print_throughput: bool = False,
                           unique: bool = False):
        """LSH-estimated beam search (reference __init__.py:525-572).

        unique=True (an extension, no reference counterpart) skips every pop
        of a node already among the k exact results, so the results are
        distinct ids; the default keeps the reference's traversal, which can
        return one id in several slots."""
        self._check_alive()
        if not self._is_directional or not self._has_lsh:
            raise RuntimeError(
                "directional_search() requires a graph built with "
                "build_lsh=True (or loaded with LSH artifacts present)")
        queries = self._query_check(queries)
        resolved_limit = limit if limit is not None else beam_width * 2
        if unique:
            return self._run_unique(False, queries, k, beam_width, resolved_limit)
        return self._run_search(self._directional_search_fn, queries, k, beam_width,
                                resolved_limit, print_throughput)

    def pq_search(self, queries: torch.Tensor, k: int = 10, beam_width: int = 64,
                  limit: int | None = None, print_throughput: bool = False,
                  unique: bool = False):
        """PQ-ADC-estimated beam search (reference __init__.py:574-621);
        unique as for directional_search."""
        self._check_alive()
        if not self._is_directional or not self._has_pq:
            raise RuntimeError(
                "pq_search() requires a graph built with build_pq=True "
                "(or loaded with PQ artifacts present)")
        queries = self._query_check(queries)
        resolved_limit = limit if limit is not None else beam_width * 2
        if unique:
            return self._run_unique(True, queries, k, beam_width, resolved_limit)
        return self._run_search(self._pq_search_fn, queries, k, beam_width, resolved_limit,
                                print_throughput)

    def exact_search(self, queries: torch.Tensor, k: int = 10, beam_width: int = 64,
                     limit: int | None = None):
        """The plain beam search with exact distances on any graph,
        directional ones included (an extension: the reference's search()
        refuses directional graphs); queries are rotated as for
        directional_search on a prerotated graph. Shows what the graph
        itself allows, without an estimator."""
        self._check_alive()
        queries = self._query_check(queries)
        nq = queries.size(0)
        out_indices = torch.empty(nq, k, dtype=torch.int32, device=queries.device)
        out_distances = torch.empty(nq, k, dtype=torch.float32, device=queries.device)
        lim = limit if limit is not None else 2 * beam_width
        _agnostic("jasperx_exact_search")(self._handle, _tensor_ptr(queries), nq, self._dim,
                                          _tensor_ptr(out_indices), _tensor_ptr(out_distances), k, beam_width,
                                          lim, _stream_ptr(queries.device))
        return out_indices, out_distances

    def rabitq_search(self, queries: torch.Tensor, k: int = 10, beam_width: int = 64,
                      limit: int | None = None, unique: bool = False):
        """Directional search with the one-bit RaBitQ estimator (an
        extension, no reference counterpart): the traversal of
        directional_search, with each neighbour estimated from its RaBitQ
        code (built with build_rabitq=True) and the query quantized to 4 bits;
        unique as for directional_search."""
        self._check_alive()
        if not self._is_directional or not self._has_rabitq:
            raise RuntimeError(
                "rabitq_search() requires a graph built with build_rabitq=True "
                "(or loaded with RaBitQ codes present)")
        queries = self._query_check(queries)
        resolved_limit = limit if limit is not None else beam_width * 2
        return self._run_ex(2, queries, k, beam_width, resolved_limit, unique)

    # -- misc (reference __init__.py:623-766) -------------------------------
    def get_vector(self, stable_id: int) -> torch.Tensor:
        self._check_alive()
        if stable_id < 0:
            raise IndexError(f"stable_id must be non-negative, got {stable_id}")
        out = torch.empty(self._dim, dtype=self._torch_dtype, device="cuda")
        self._get_vector_fn(self._handle, stable_id, _tensor_ptr(out), _stream_ptr(out.device))
        return out

    @property
    def n_tombstoned(self) -> int:
        self._check_alive()
        return _agnostic("jasper_get_n_tombstoned")(self._handle)

    @property
    def n_live(self) -> int:
        self._check_alive()
        return _agnostic("jasper_get_n_live")(self._handle)

    def reserve_ids(self, count: int) -> torch.Tensor:
        self._check_alive()
        if count <= 0:
            return torch.empty(0, dtype=torch.int32)
        out = torch.empty(count, dtype=torch.int32)
        _agnostic("jasper_reserve_ids")(self._handle, _tensor_ptr(out), count)
        return out

    def append(self, vectors: torch.Tensor, alpha: float = 1.2) -> torch.Tensor:
        self._check_alive()
        if self._append_fn is None:
            raise RuntimeError("append() is not available on a directional graph")
        if not vectors.is_cuda:
            raise ValueError("vectors must be a CUDA tensor")
        if vectors.dtype != self._torch_dtype:
            raise ValueError(f"vectors must be {self._torch_dtype}, got {vectors.dtype}")
        if vectors.ndim != 2 or vectors.size(1) != self._dim:
            raise ValueError(f"vectors must be [n, {self._dim}]")
        vectors = vectors.contiguous()
        out_ids = torch.empty(vectors.size(0), dtype=torch.int32)
        self._append_fn(self._handle, _tensor_ptr(vectors), vectors.size(0), float(alpha),
                        _tensor_ptr(out_ids), _stream_ptr(vectors.device))
        return out_ids

    def mark_deleted(self, ids: torch.Tensor) -> None:
        self._check_alive()
        if self._mark_deleted_fn is None:
            raise RuntimeError("mark_deleted() is not available on a directional graph")
        if ids.ndim != 1:
            raise ValueError(f"ids must be 1D, got {ids.ndim}D")
        ids = ids.detach().to(device="cpu", dtype=torch.int32).contiguous()
        if ids.numel() == 0:
            return
        self._mark_deleted_fn(self._handle, _tensor_ptr(ids), ids.numel())

    def consolidate(self, alpha: float = 1.2) -> None:
        self._check_alive()
        if self._consolidate_fn is None:
            raise RuntimeError("consolidate() is not available on a directional graph")
        self._consolidate_fn(self._handle, float(alpha))

    def compact(self) -> None:
        self._check_alive()
        if self._compact_fn is None:
            raise RuntimeError("compact() is not available on a directional graph")
        self._compact_fn(self._handle)

    def export_edges(self):
        """Host copies (edges u32 [n,R], edge distances bf16 bits [n,R],
        counts u8 [n]); an extension used by parity tests."""
        self._check_alive()
        n = self.n_vectors
        R = self._n_neighbors
        edges = np.empty((n, R), dtype=np.uint32)
        edist = np.empty((n, R), dtype=np.uint16)
        counts = np.empty(n, dtype=np.uint8)
        _agnostic("jasperx_export_graph")(self._handle, edges.ctypes.data_as(_ptr),
                                          edist.ctypes.data_as(_ptr), counts.ctypes.data_as(_ptr))
        return edges, edist, counts

    def export_vectors(self) -> np.ndarray:
        """Host copy of the stored rows [n, padded_dim] as fp16 bits (after
        prerotation when the graph was prerotated); a test extension."""
        self._check_alive()
        dp = _agnostic("jasperx_export_vectors")(self._handle, None)
        out = np.empty((self.n_vectors, dp), dtype=np.uint16)
        _agnostic("jasperx_export_vectors")(self._handle, out.ctypes.data_as(_ptr))
        return out

    def directional_query_rows(self, queries: torch.Tensor) -> np.ndarray:
        """The rows a directional search reads for these queries [nq,
        padded_dim] fp16 bits (rotated when prerotated); a test extension."""
        self._check_alive()
        queries = self._query_check(queries)
        nq = queries.size(0)
        dp = (self._dim + 7) // 8 * 8
        out = np.zeros((nq, dp), dtype=np.uint16)
        _agnostic("jasperx_directional_query_rows")(self._handle, _tensor_ptr(queries), nq, self._dim,
                                                    out.ctypes.data_as(_ptr), _stream_ptr(queries.device))
        return out

    def directional_stats(self, queries: torch.Tensor, k: int = 10, beam_width: int = 64,
                          limit: int | None = None, pq: bool = False, unique: bool = False,
                          estimator: int | None = None) -> np.ndarray:
        """Per-query work counters of directional_search (pq=False),
        pq_search (pq=True) or another estimator (estimator = 0 LSH, 1 PQ,
        2 RaBitQ) [n_queries, 3]: visits, hops expanded, adjacency entries
        read. A measurement extension."""
        self._check_alive()
        queries = self._query_check(queries)
        nq = queries.size(0)
        out = np.zeros((nq, 3), dtype=np.uint32)
        lim = limit if limit is not None else 2 * beam_width
        est = estimator if estimator is not None else (1 if pq else 0)
        _agnostic("jasperx_directional_stats")(self._handle, est, _tensor_ptr(queries), nq, self._dim,
                                               k, beam_width, lim, DIR_UNIQUE if unique else 0,
                                               out.ctypes.data_as(_ptr),
                                               _stream_ptr(queries.device))
        return out

    def export_rabitq(self):
        """(centroid f32 [dim], nodes u8 [n, node_bytes]); a test extension."""
        self._check_alive()
        fn = _agnostic("jasperx_export_rabitq")
        nb = fn(self._handle, None, None)
        c = np.empty(self._dim, dtype=np.float32)
        nodes = np.empty((self.n_vectors, nb), dtype=np.uint8)
        fn(self._handle, c.ctypes.data_as(_ptr), nodes.ctypes.data_as(_ptr))
        return c, nodes

    def export_lsh(self):
        """(c_per_rank f32 [k_ranks], norm_denom, rows u8 [n, row_bytes]); a
        test extension."""
        self._check_alive()
        fn = _agnostic("jasperx_export_lsh")
        row_bytes = fn(self._handle, None, None, None)
        c = np.empty(self._k_ranks, dtype=np.float32)
        nd = np.empty(1, dtype=np.float32)
        rows = np.empty((self.n_vectors, row_bytes), dtype=np.uint8)
        fn(self._handle, c.ctypes.data_as(_ptr), nd.ctypes.data_as(_ptr), rows.ctypes.data_as(_ptr))
        return c, float(nd[0]), rows

    def export_pq(self):
        """(centroids f32 [M*256*dsub], codes u8 [n, M*R], vector norms f32
        [n]); a test extension."""
        self._check_alive()
        fn = _agnostic("jasperx_export_pq")
        dsub = fn(self._handle, None, None, None)
        M = ((self._dim + 7) // 8 * 8) // dsub
        cent = np.empty(M * 256 * dsub, dtype=np.float32)
        codes = np.empty((self.n_vectors, M * self._n_neighbors), dtype=np.uint8)
        norms = np.empty(self.n_vectors, dtype=np.float32)
        fn(self._handle, cent.ctypes.data_as(_ptr), codes.ctypes.data_as(_ptr), norms.ctypes.data_as(_ptr))
        return cent, codes, norms

    def search_stats(self, queries: torch.Tensor, k: int = 10, beam_width: int = 64,
                     limit: int | None = None) -> np.ndarray:
        """Per-query work counters of the plain search [n_queries, 4]:
        hops, adjacency entries read, vectors scored (exact distinct count),
        hops whose adjacency row was read one hop ahead (predicted pop). A
        measurement extension used for algorithmic-bytes accounting."""
        self._check_alive()
        queries = self._query_check(queries)
        nq = queries.size(0)
        out = np.zeros((nq, 4), dtype=np.uint32)
        lim = limit if limit is not None else 2 * beam_width
        _agnostic("jasperx_search_stats")(self._handle, _tensor_ptr(queries), nq, self._dim, k,
                                          beam_width, lim, out.ctypes.data_as(_ptr),
                                          _stream_ptr(queries.device))
        return out

    def free(self):
        if getattr(self, "_handle", None) is not None:
            try:
                _agnostic("jasper_free_graph")(self._handle)
            finally:
                self._handle = None

    def _check_alive(self):
        if self._handle is None:
            raise RuntimeError("Graph has been freed")

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def row_format(self) -> dict:
        """The row formats the graph keeps (jasperx_row_format): whether all
        values are integers, their range, and whether the search reads the
        rows as bytes."""
        out = np.zeros(4, dtype=np.int64)
        _agnostic("jasperx_row_format")(self._handle, out.ctypes.data_as(_ptr))
        return {"integer": int(out[0]) == 1, "lo": int(out[1]), "hi": int(out[2]), "byte_rows": bool(out[3])}

    def __repr__(self) -> str:
        if self._handle is None:
            return "Graph(freed)"
        extra = ""
        if self._is_directional:
            extra = (f", k_ranks={self._k_ranks}, lsh={self._has_lsh}, "
                     f"pq={self._has_pq}, rabitq={self._has_rabitq}, prerotate={self._prerotate}")
        return (f"Graph(n_vectors={self.n_vectors}, dim={self.dim}, "
                f"R={self._n_neighbors}, dtype={self._data_type.value}, "
                f"dist={self._distance.value}{extra})")


def last_build_stats() -> dict:
    """Per-stage times of the last construction (set JASPER_BUILD_TIMING=1
    before building to get stage times; the total is always recorded)."""
    out = np.zeros(7, dtype=np.float64)
    _agnostic("jasperx_last_build_stats")(out.ctypes.data_as(_ptr))
    keys = ["search_ms", "prune_ms", "group_ms", "reverse_ms", "total_ms", "batches", "max_batch"]
    return dict(zip(keys, out.tolist()))


BUILD_WORK_KEYS = ["search_rows", "search_hops", "search_adjacency", "search_scored", "search_visited",
                   "forward_rows", "forward_existing", "forward_visited", "forward_candidates", "forward_selected",
                   "reverse_targets", "reverse_existing", "reverse_sources", "reverse_selected"]


def set_build_work_counting(on: bool) -> None:
    """Count the work of the following constructions (measurement mode: the
    search stage runs with an exact per-query seen bitmap; same graph)."""
    _agnostic("jasperx_build_work_counting")(ctypes.c_int64(1 if on else 0))


def last_build_work() -> dict:
    """Work counters of the last construction made with counting on."""
    out = np.zeros(16, dtype=np.uint64)
    _agnostic("jasperx_last_build_work")(out.ctypes.data_as(_ptr))
    return {k: int(v) for k, v in zip(BUILD_WORK_KEYS, out.tolist())}


def last_scale_stats() -> dict:
    """Times and batch counts of the last partitioned build (Graph.build_scale)."""
    out = np.zeros(7, dtype=np.float64)
    _agnostic("jasperx_last_scale_stats")(out.ctypes.data_as(_ptr))
    keys = ["partition_ms", "merge_ms", "total_ms", "merges", "merge_batches", "part_batch", "merge_batch"]
    return dict(zip(keys, out.tolist()))


def last_diskann_stats() -> dict:
    """Times of the last DiskANN build (Graph.build_diskann)."""
    out = np.zeros(6, dtype=np.float64)
    _agnostic("jasperx_last_diskann_stats")(out.ctypes.data_as(_ptr))
    keys = ["assign_ms", "build_ms", "merge_ms", "total_ms", "shards", "max_shard"]
    return dict(zip(keys, out.tolist()))


def diskann_assign(vectors: torch.Tensor, n_parts: int, n_dup: int = 2, seed: int = 42):
    """Shard assignment of the DiskANN build on the GPU: (shard_of [n, n_dup]
    uint32 with 0xFFFFFFFF for repeated shards, mean [dim] fp16 bits)."""
    vectors = vectors.contiguous()
    n, dim = vectors.shape
    so = np.empty((n, n_dup), dtype=np.uint32)
    mean = np.empty(dim, dtype=np.uint16)
    _agnostic("jasperx_diskann_assign")(_tensor_ptr(vectors), n, dim, int(n_parts), int(n_dup), int(seed),
                                        so.ctypes.data_as(_ptr), mean.ctypes.data_as(_ptr),
                                        _stream_ptr(vectors.device if vectors.is_cuda else None))
    return so, mean


# ── Utilities (reference __init__.py:770-946) ─────────────────────────

def read_bin(path: str, dtype: str = "f32", max_vectors: int = 0) -> torch.Tensor:
    """Read an [n, dim] .bin file (f32 or u8) as a float16 tensor."""
    if dtype == "f32":
        np_dtype = np.float32
    elif dtype == "u8":
        np_dtype = np.uint8
    else:
        raise ValueError(f"Unsupported dtype: {dtype!r}. Expected 'f32' or 'u8'.")
    with open(path, "rb") as f:
        n_vectors, dim = struct.unpack("II", f.read(8))
        if max_vectors > 0:
            n_vectors = min(n_vectors, max_vectors)
        nbytes = n_vectors * dim * np.dtype(np_dtype).itemsize
        data = np.frombuffer(f.read(nbytes), dtype=np_dtype).reshape(n_vectors, dim).copy()
    t = torch.from_numpy(data).to(torch.float16)
    return t.pin_memory() if torch.cuda.is_available() else t


def read_groundtruth(path: str, k: int = 10) -> tuple[torch.Tensor, torch.Tensor]:
    with open(path, "rb") as f:
        n_queries, gt_k = struct.unpack("II", f.read(8))
        if gt_k < k:
            raise ValueError(f"Requested k={k} but ground truth only has k={gt_k}")
        ids = np.frombuffer(f.read(n_queries * gt_k * 4), dtype=np.uint32).reshape(n_queries, gt_k)
        distances = np.frombuffer(f.read(n_queries * gt_k * 4), dtype=np.float32).reshape(n_queries, gt_k)
    return (torch.from_numpy(ids[:, :k].copy()).to(dtype=torch.int32),
            torch.from_numpy(distances[:, :k].copy()))


def get_recall(gt, result_indices, k, n_queries, verbose: bool = True):
    count = sum(len(set(result_indices[i].tolist()) & set(gt[i].tolist())) for i in range(n_queries))
    recall = count / (n_queries * k)
    if verbose:
        print(f"Recall@{k}: {recall:.3f} ({count}/{(n_queries * k)})")
    return recall


def save_groundtruth(path: str, indices: torch.Tensor, distances: torch.Tensor):
    ids_np = indices.cpu().numpy().astype(np.uint32)
    dists_np = distances.cpu().numpy().astype(np.float32)
    nq, k = ids_np.shape
    with open(path, "wb") as f:
        f.write(struct.pack("II", nq, k))
        f.write(ids_np.tobytes())
        f.write(dists_np.tobytes())


from .groundtruth import bruteforce_knn, generate_groundtruth  # noqa: E402

__all__ = [
    "Graph", "DistanceFunc", "DataType", "JasperError", "read_bin", "read_groundtruth",
    "get_recall", "generate_groundtruth", "bruteforce_knn", "save_groundtruth", "parse_storage_size",
    "last_build_stats", "last_scale_stats", "last_diskann_stats", "diskann_assign", "library_path",
]


def rotation_matrix(dim: int, seed: int = 42) -> np.ndarray:
    """The prerotation matrix for (dim, seed), column-major f32 [dim*dim]
    (reference include/jasper/rotation/rotation.cuh:71-111)."""
    out = np.empty(dim * dim, dtype=np.float32)
    _agnostic("jasperx_rotation_matrix")(dim, seed, out.ctypes.data_as(_ptr))
    return out


def rotate(vectors: torch.Tensor, seed: int = 42) -> torch.Tensor:
    """Rows x -> P^T x with the prerotation matrix of (dim, seed) on the
    matrix cores (fp16 in and out, fp32 accumulation)."""
    if vectors.ndim != 2 or vectors.dtype != torch.float16:
        raise ValueError("vectors must be a 2D float16 tensor")
    vectors = vectors.contiguous()
    n, dim = vectors.shape
    dev = vectors.device if vectors.is_cuda else torch.device("cuda")
    out = torch.empty((n, dim), dtype=torch.float16, device=dev)
    if n:
        _agnostic("jasperx_rotate_rows")(dim, seed, _tensor_ptr(vectors), n, dim, _tensor_ptr(out), dim,
                                         _stream_ptr(dev))
    return out


class RabitqCodes:
    """One-bit RaBitQ store (reference rabitq/layout.cuh:43-117): `nodes` is
    a device uint8 tensor [n, node_bytes] of code bytes (LSB-first) followed
    by f_add and f_rescale (fp32)."""

    def __init__(self, nodes: torch.Tensor, dim: int):
        self.nodes = nodes
        self.dim = dim
        self.node_bytes = nodes.size(1)
        self.code_bytes = self.node_bytes - 8

    @property
    def codes(self) -> torch.Tensor:
        return self.nodes[:, :self.code_bytes]

    @property
    def f_add(self) -> torch.Tensor:
        return self.nodes[:, self.code_bytes:self.code_bytes + 4].contiguous().view(torch.float32).view(-1)

    @property
    def f_rescale(self) -> torch.Tensor:
        return self.nodes[:, self.code_bytes + 4:].contiguous().view(torch.float32).view(-1)

    def bits(self) -> torch.Tensor:
        """Unpacked codes [n, dim] as uint8 0/1."""
        b = self.codes.to(torch.int32)
        shifts = torch.arange(8, device=b.device, dtype=torch.int32)
        out = (b.unsqueeze(-1) >> shifts) & 1
        return out.reshape(b.size(0), -1)[:, :self.dim].to(torch.uint8)


def rabitq_quantize(vectors: torch.Tensor, rotation: torch.Tensor | None = None,
                    centroid: torch.Tensor | None = None, distance: DistanceFunc | str = DistanceFunc.L2,
                    seed: int = 42) -> RabitqCodes:
    """One-bit RaBitQ codes of `vectors` [n, dim] (fp16 or fp32, CUDA)
    (reference rabitq_quantize<1>, rabitq/quantize.cuh:322-383). `rotation`
    is a column-major fp32 [dim, dim] matrix (default: the prerotation matrix
    of `seed`); `centroid` defaults to zero."""
    if isinstance(distance, str):
        distance = DistanceFunc(distance)
    if vectors.ndim != 2 or not vectors.is_cuda:
        raise ValueError("vectors must be a 2D CUDA tensor")
    if vectors.dtype not in (torch.float16, torch.float32):
        raise ValueError("vectors must be float16 or float32")
    n, dim = vectors.shape
    dev = vectors.device
    if rotation is None:
        rotation = torch.from_numpy(rotation_matrix(dim, seed)).to(dev)
    rotation = rotation.to(device=dev, dtype=torch.float32).contiguous()
    if rotation.numel() != dim * dim:
        raise ValueError(f"rotation must hold {dim}x{dim} values")
    if centroid is not None:
        centroid = centroid.to(device=dev, dtype=torch.float32).contiguous()
        if centroid.numel() != dim:
            raise ValueError(f"centroid must hold {dim} values")
    if vectors.dtype == torch.float16 and (dim % 8 != 0 or vectors.data_ptr() % 16 != 0):
        stride = (dim + 7) // 8 * 8
        padded = torch.zeros((n, stride), dtype=torch.float16, device=dev)
        padded[:, :dim] = vectors
        vectors = padded
    else:
        vectors = vectors.contiguous()
        stride = dim
    node_bytes = _agnostic("jasperx_rabitq_node_bytes")(dim)
    nodes = torch.empty((n, node_bytes), dtype=torch.uint8, device=dev)
    if n:
        _agnostic("jasperx_rabitq_quantize")(
            _tensor_ptr(vectors), 0 if vectors.dtype == torch.float16 else 1, n, dim, stride,
            _tensor_ptr(rotation), None if centroid is None else _tensor_ptr(centroid),
            0 if distance == DistanceFunc.L2 else 1, _tensor_ptr(nodes), _stream_ptr(dev))
    return RabitqCodes(nodes, dim)
