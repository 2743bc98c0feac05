"""Oracle rotation matrix (reference rotation/rotation.cuh:28-111).

The reference's own tests (tests/test_rotation.cu:50-185) plus an
independent check: Q must be the orthogonal factor of the QR decomposition
of the seeded Gaussian matrix with a positive diagonal R, which a float64
LAPACK QR with the same sign convention reproduces.
"""

import numpy as np
import pytest

import oracle


def colmajor(flat, d):
    return np.asarray(flat, dtype=np.float64).reshape(d, d).T  # [i, j] = flat[i + j*d]


def test_qtq_identity():                           # :52-60
    q, qt = oracle.rotation_matrix(16, 42)
    Q, Qt = colmajor(q, 16), colmajor(qt, 16)
    assert np.abs(Qt @ Q - np.eye(16)).max() < 1e-5


def test_qqt_identity():                           # :62-70
    q, qt = oracle.rotation_matrix(16, 42)
    Q, Qt = colmajor(q, 16), colmajor(qt, 16)
    assert np.abs(Q @ Qt - np.eye(16)).max() < 1e-5


def test_qt_is_transpose():                        # :72-84
    q, qt = oracle.rotation_matrix(8, 123)
    assert np.array_equal(colmajor(q, 8).T, colmajor(qt, 8))


def test_determinant_unit():                       # :86-94
    q, _ = oracle.rotation_matrix(16, 42)
    assert abs(abs(np.linalg.det(colmajor(q, 16))) - 1.0) < 1e-4


def test_preserves_norm():                         # :96-118
    q, _ = oracle.rotation_matrix(8, 99)
    x = np.arange(1, 9, dtype=np.float64)
    assert abs(np.sum((colmajor(q, 8) @ x) ** 2) - np.sum(x ** 2)) < 1e-4


def test_same_seed_same_matrix():                  # :120-133
    a, _ = oracle.rotation_matrix(8, 77)
    b, _ = oracle.rotation_matrix(8, 77)
    assert np.array_equal(a, b)


def test_different_seed_different_matrix():        # :135-148
    a, _ = oracle.rotation_matrix(8, 1)
    b, _ = oracle.rotation_matrix(8, 2)
    assert np.abs(a - b).max() > 1e-6


def test_d128_orthogonal():                        # :150-164
    q, qt = oracle.rotation_matrix(128, 42)
    Q, Qt = colmajor(q, 128), colmajor(qt, 128)
    assert np.abs(Qt @ Q - np.eye(128)).max() < 1e-3


def test_d1_edge_case():                           # :166-177
    q, qt = oracle.rotation_matrix(1, 42)
    assert abs(abs(q[0]) - 1.0) < 1e-6 and q[0] == qt[0]


@pytest.mark.parametrize("d", [8, 96, 128])
def test_matches_independent_qr(d):
    """The reference loop (rotation.cuh:28-69) accumulates the Householder
    product H = H_{d-1}...H_0 (so H A = R, i.e. H is the transposed Q factor)
    and then flips *columns* i of H where R_ii < 0 (rotation.cuh:94-101).
    With a float64 LAPACK QR A = Qn Rn this means m^T = D Qn S for sign
    matrices D (rows) and S (columns), with D_i S_i = sign(Rn_ii)."""
    A = colmajor(oracle.gaussian_matrix(d, 42), d)
    q, _ = oracle.rotation_matrix(d, 42)
    M = colmajor(q, d)
    Qn, Rn = np.linalg.qr(A)
    assert np.abs(np.abs(M.T) - np.abs(Qn)).max() < 2e-4 * d ** 0.5
    sig = np.sign(M.T * Qn)
    big = np.abs(Qn) > 1e-3
    # rank-one sign pattern D_i * S_j
    D = sig[:, 0] * sig[0, 0]
    S = sig[0, :] * sig[0, 0]
    assert np.all((sig == np.outer(D, S) * sig[0, 0])[big])
    assert np.all(np.diag(sig) == np.sign(np.diag(Rn)))
