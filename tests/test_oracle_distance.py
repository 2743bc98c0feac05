"""Oracle distance arithmetic (reference include/jasper/distance/distance.cuh).

Pinned by the reference's own known-answer tests (tests/test_distance.cu:
32-136), by exactness on integer-valued data (every partial sum is an exact
integer below 2^24, so any accumulation order gives the same bits), and by a
float64 computation on Gaussian data. The 4-lane combine order
(l0+l2)+(l1+l3) is not fixed by the reference source (cg::reduce); it is
documented as parity unpinned for non-integer data.
"""

import numpy as np
import pytest

import oracle


def d(a, b, metric="l2"):
    return oracle.distance(np.asarray(a, dtype=np.float32), np.asarray(b, dtype=np.float32), metric)


# --- reference KATs, tests/test_distance.cu ---------------------------------

def test_kat_l2_identical_is_zero():          # :32-43
    assert d([1, 2, 3, 4], [1, 2, 3, 4]) == 0.0


def test_kat_l2_known_distance():             # :45-58
    assert d([0, 0, 0, 0], [3, 4, 0, 0]) == 25.0


def test_kat_l2_larger_dim():                 # :60-74
    assert d(np.ones(16), np.zeros(16)) == 16.0


def test_kat_l2_symmetric():                  # :76-91
    a, b = [1, 2, 3, 4], [5, 6, 7, 8]
    assert d(a, b) == d(b, a) == 64.0


def test_kat_ip_orthogonal_zero():            # :95-108
    assert d([1, 0, 0, 0], [0, 1, 0, 0], "ip") == 0.0


def test_kat_ip_known_value():                # :110-123
    assert d([1, 2, 3, 4], [2, 3, 4, 5], "ip") == -40.0


def test_kat_ip_self_dot_negative():          # :125-137
    assert d([3, 4, 0, 0], [3, 4, 0, 0], "ip") == -25.0


# --- closed forms -------------------------------------------------------------

@pytest.mark.parametrize("dim", [8, 96, 128, 200, 960])
def test_l2_exact_on_integer_data(dim):
    rng = np.random.default_rng(dim)
    a = rng.integers(0, 219, size=(64, dim)).astype(np.float16)
    b = rng.integers(0, 219, size=(64, dim)).astype(np.float16)
    got = oracle.distance_pairs(oracle.as_padded_f16(a), oracle.as_padded_f16(b), "l2")
    exact = ((a.astype(np.int64) - b.astype(np.int64)) ** 2).sum(axis=1)
    assert np.array_equal(got.astype(np.int64), exact)


@pytest.mark.parametrize("dim", [8, 96, 128])
def test_ip_exact_on_integer_data(dim):
    rng = np.random.default_rng(dim + 1)
    a = rng.integers(-40, 41, size=(64, dim)).astype(np.float16)
    b = rng.integers(-40, 41, size=(64, dim)).astype(np.float16)
    got = oracle.distance_pairs(oracle.as_padded_f16(a), oracle.as_padded_f16(b), "ip")
    exact = -(a.astype(np.int64) * b.astype(np.int64)).sum(axis=1)
    assert np.array_equal(got.astype(np.int64), exact)


@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_gaussian_close_to_float64(metric):
    rng = np.random.default_rng(7)
    a = rng.standard_normal((256, 128)).astype(np.float16)
    b = rng.standard_normal((256, 128)).astype(np.float16)
    got = oracle.distance_pairs(oracle.as_padded_f16(a), oracle.as_padded_f16(b), metric)
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    ref = ((a64 - b64) ** 2).sum(1) if metric == "l2" else -(a64 * b64).sum(1)
    scale = np.abs(ref).max()
    assert np.max(np.abs(got - ref)) <= 1e-5 * scale


def test_l2_uses_only_whole_chunks_of_dim():
    # The reference prunes with `dim` (construct.cuh:437-448) and its L2 loop
    # covers dim/8 whole 16-byte chunks: a tail of dim % 8 elements is ignored.
    a = np.zeros(12, dtype=np.float32)
    b = np.zeros(12, dtype=np.float32)
    b[9] = 3.0
    assert oracle.distance(a, b, "l2", dim=12) == 0.0   # element 9 lies past chunk 0
    assert oracle.distance(a, b, "l2", dim=16) == 9.0   # padded dim covers it


def test_bf16_rounding_is_nearest_even():
    assert oracle.f2bf(1.0) == 0x3F80
    # 1 + 2^-8 is exactly halfway between bf16 1.0 and 1.0078125 -> even (1.0)
    assert oracle.f2bf(1.0 + 2 ** -8) == 0x3F80
    # 1 + 3*2^-8 is halfway between 1.0078125 (odd) and 1.015625 (even)
    assert oracle.f2bf(1.0 + 3 * 2 ** -8) == 0x3F82
    assert oracle.f2bf(1.0 + 2 ** -8 + 2 ** -20) == 0x3F81
