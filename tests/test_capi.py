"""The C-ABI library: exported symbols and host-side conventions (no GPU work).

Every function include/jasper_amd.h declares must be exported by
libjasper_amd.so; the reference's 222 TVM-FFI export names must all be
present (8 plain configs x 9 ops + 16 directional configs x 9 ops + 6
config-agnostic ops, reference ffi/jasper_ffi_common.cuh:787-807 and
ffi/jasper_ffi_plain.cu:123-131). Calls that only touch the handle table run
without a GPU and must follow the error convention (negative return +
jasper_last_error()).
"""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "jasper_amd.h"


@pytest.fixture(scope="module")
def lib():
    from jasper_amd import build_lib
    if not build_lib.LIB.exists():
        build_lib.build(verbose=False)
    return ctypes.CDLL(str(build_lib.LIB))


def declared_functions():
    out = subprocess.run(["gcc", "-E", "-P", "-x", "c", str(HEADER)], capture_output=True, text=True, check=True)
    return sorted(set(re.findall(r"\b(jasperx?_\w+)\s*\(", out.stdout)))


def reference_export_names():
    plain = [f"f16_r{r}_{m}" for m in ("l2", "ip") for r in (8, 16, 32, 64)]
    directional = [f"f16_r{r}_{m}_k{k}_d{d}" for m in ("l2", "ip") for k in (4, 16) for r in (32, 64)
                   for d in ("128", "32678")]
    ops = ["load", "construct", "search", "save", "get_vector", "mark_deleted", "consolidate", "compact",
           "append"]
    dops = ["construct_directional", "build_lsh", "build_pq", "directional_search", "pq_search",
            "save_directional", "load_directional", "get_vector_directional", "get_directional_flags"]
    names = [f"jasper_{o}_{c}" for c in plain for o in ops]
    names += [f"jasper_{o}_{c}" for c in directional for o in dops]
    names += ["jasper_free_graph", "jasper_get_n_vectors", "jasper_get_n_tombstoned", "jasper_get_n_live",
              "jasper_reserve_ids", "jasper_get_dim"]
    return names


def test_header_declares_every_reference_export():
    names = reference_export_names()
    assert len(names) == 222 and len(set(names)) == 222
    missing = sorted(set(names) - set(declared_functions()))
    assert not missing, missing[:10]


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing[:10]


def test_invalid_handle_error_convention(lib):
    lib.jasper_get_dim.restype = ctypes.c_int64
    lib.jasper_get_dim.argtypes = [ctypes.c_int64]
    lib.jasper_last_error.restype = ctypes.c_char_p
    assert lib.jasper_get_dim(987654) < 0
    assert lib.jasper_last_error().decode().startswith("Invalid handle: 987654")
    lib.jasper_free_graph.restype = ctypes.c_int64
    lib.jasper_free_graph.argtypes = [ctypes.c_int64]
    assert lib.jasper_free_graph(-3) < 0


def test_python_invalid_handle_raises():
    import jasper_amd
    with pytest.raises(ValueError, match="Invalid handle"):
        jasper_amd._agnostic("jasper_get_n_vectors")(123456)


def test_load_missing_file_raises():
    import jasper_amd
    with pytest.raises(jasper_amd.JasperError, match="failed to open"):
        jasper_amd.Graph.load("/nonexistent/graph.bin", dim=128, n_neighbors=32)


@pytest.mark.parametrize("dim", [1, 8, 96, 128, 200])
def test_rotation_matrix_matches_oracle(lib, oracle_lib, dim):
    """The library's prerotation matrix (host code, no GPU) is bit-identical
    to the oracle's restatement of set_rotation_matrix."""
    import numpy as np
    import oracle
    fn = lib.jasperx_rotation_matrix
    fn.restype = ctypes.c_int64
    fn.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
    for seed in (42, 7):
        out = np.zeros(dim * dim, dtype=np.float32)
        assert fn(dim, seed, out.ctypes.data_as(ctypes.c_void_p)) == 0
        m, _ = oracle.rotation_matrix(dim, seed)
        assert np.array_equal(out.view(np.uint32), np.asarray(m, dtype=np.float32).view(np.uint32))
