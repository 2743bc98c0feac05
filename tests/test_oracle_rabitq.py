"""Oracle of the one-bit RaBitQ quantizer (reference rabitq/quantize.cuh:
144-383, rabitq/layout.cuh:43-143).

Pinned by the reference's own tests (tests/test_rabitq.cu: node sizes
:103-145, bit extraction :20-95, quantizer properties :264-440) and by the
closed form at one bit per dimension, checked in float64 with numpy.
"""

import numpy as np
import pytest

import oracle


def colmajor_to_P(flat, d):
    return np.asarray(flat, dtype=np.float64).reshape(d, d).T   # P[i, j] = flat[i + j*d]


def extract_1bit(code, i):            # layout.cuh:134-136, the reference's decode
    return (int(code[i >> 3]) >> (i & 7)) & 1


@pytest.mark.parametrize("dim,code,node", [(128, 16, 24), (97, 16, 24), (8, 4, 12), (33, 8, 16), (256, 32, 40)])
def test_node_sizes(dim, code, node):        # test_rabitq.cu:103-145 (1-bit cases)
    assert oracle.rabitq_code_bytes(dim) == code
    x = np.ones((3, dim), np.float32)
    nodes, *_ = oracle.rabitq_quantize(x, np.eye(dim, dtype=np.float32).ravel())
    assert nodes.shape == (3, node)


def test_total_bytes():                      # test_rabitq.cu:138-144
    assert 1000 * (oracle.rabitq_code_bytes(128) + 8) == 24000


def test_bit_order_lsb_first():
    # signs -,+,-,+,... -> bits 1,3,5,7 -> 0xAA (test_rabitq.cu:36-47 decodes 0xAA this way)
    x = np.array([[-1, 1] * 8], dtype=np.float32)
    _, codes, _, _ = oracle.rabitq_quantize(x, np.eye(16, dtype=np.float32).ravel())
    assert codes[0, 0] == 0xAA and codes[0, 1] == 0xAA
    assert [extract_1bit(codes[0], i) for i in range(8)] == [0, 1, 0, 1, 0, 1, 0, 1]
    _, codes, _, _ = oracle.rabitq_quantize(np.ones((1, 20), np.float32), np.eye(20, dtype=np.float32).ravel())
    assert codes[0].tolist() == [0xFF, 0xFF, 0x0F, 0x00]        # zero padding past dim
    _, codes, _, _ = oracle.rabitq_quantize(-np.ones((1, 20), np.float32), np.eye(20, dtype=np.float32).ravel())
    assert not codes.any()


@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_identity_closed_form(metric):
    rng = np.random.default_rng(0)
    x = rng.normal(size=(50, 64)).astype(np.float32)
    _, codes, f_add, f_rescale = oracle.rabitq_quantize(x, np.eye(64, dtype=np.float32).ravel(), metric=metric)
    xd = x.astype(np.float64)
    sq = (xd ** 2).sum(1)
    l1 = np.abs(xd).sum(1)
    if metric == "l2":
        np.testing.assert_allclose(f_add, sq, rtol=1e-5)
        np.testing.assert_allclose(f_rescale, -4 * sq / l1, rtol=1e-5)
    else:
        np.testing.assert_allclose(f_add, 1.0, rtol=1e-6)
        np.testing.assert_allclose(f_rescale, -2 * sq / l1, rtol=1e-5)
    bits = np.array([[extract_1bit(c, i) for i in range(64)] for c in codes])
    assert np.array_equal(bits, (x >= 0).astype(int))


@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_general_formula_float64(metric):
    d = 48
    rng = np.random.default_rng(1)
    x = rng.normal(size=(40, d)).astype(np.float32)
    c = rng.normal(size=d).astype(np.float32) * 0.3
    m, _ = oracle.rotation_matrix(d, 5)
    _, codes, f_add, f_rescale = oracle.rabitq_quantize(x, m, c, metric=metric)
    P = colmajor_to_P(m, d)
    rc = P @ c.astype(np.float64)                  # centroid through P (CUBLAS_OP_N)
    r = x.astype(np.float64) @ P - rc              # data through P^T (CUBLAS_OP_T)
    nrm2 = (r ** 2).sum(1)
    b = (r >= 0)
    xucb = np.where(b, 0.5, -0.5)
    ipn = 0.5 * np.abs(r).sum(1) / np.sqrt(nrm2)
    s_rx = (r * xucb).sum(1)
    s_cx = (rc[None] * xucb).sum(1)
    s_rc = (r * rc[None]).sum(1)
    if metric == "l2":
        want_add = nrm2 + 2 * nrm2 * s_cx / s_rx
        want_res = -2 * np.sqrt(nrm2) / ipn
    else:
        want_add = 1 - s_rc + nrm2 * s_cx / s_rx
        want_res = -np.sqrt(nrm2) / ipn
    scale = np.abs(nrm2) + np.abs(2 * nrm2 * s_cx / s_rx) + np.abs(s_rc) + 1
    assert np.all(np.abs(f_add - want_add) <= 1e-5 * scale)
    np.testing.assert_allclose(f_rescale, want_res, rtol=1e-5)
    bits = np.array([[extract_1bit(cc, i) for i in range(d)] for cc in codes]).astype(bool)
    clear = np.abs(r) > 1e-5 * np.sqrt(nrm2)[:, None]
    assert np.array_equal(bits[clear], b[clear])


def test_centroid_goes_through_P_not_PT():
    d = 16
    m, _ = oracle.rotation_matrix(d, 9)
    P = colmajor_to_P(m, d)
    c = np.arange(1, d + 1, dtype=np.float32)
    _, codes, _, _ = oracle.rabitq_quantize(np.zeros((1, d), np.float32), m, c)
    bits = np.array([extract_1bit(codes[0], i) for i in range(d)])
    assert np.array_equal(bits, (-(P @ c) >= 0).astype(int))
    assert not np.array_equal(bits, (-(P.T @ c) >= 0).astype(int))


def test_reference_quantizer_properties():       # test_rabitq.cu:264-440
    rng = np.random.default_rng(42)
    x = rng.normal(size=(8, 32)).astype(np.float32)
    eye = np.eye(32, dtype=np.float32).ravel()
    _, codes, f_add, f_rescale = oracle.rabitq_quantize(x, eye)
    assert np.all(f_rescale < 0) and np.all(np.isfinite(f_add))
    same = np.tile(np.arange(1, 17, dtype=np.float32), (4, 1))
    nodes, *_ = oracle.rabitq_quantize(same, np.eye(16, dtype=np.float32).ravel())
    assert all(np.array_equal(nodes[0], nodes[i]) for i in range(4))
    m, _ = oracle.rotation_matrix(32, 42)
    _, _, fa, fr = oracle.rabitq_quantize(x, m)
    assert np.all(np.isfinite(fa)) and np.all(np.isfinite(fr)) and np.all(fr != 0)
    _, _, fa_l2, _ = oracle.rabitq_quantize(x, eye, metric="l2")
    _, _, fa_ip, _ = oracle.rabitq_quantize(x, eye, metric="ip")
    assert np.any(np.abs(fa_l2 - fa_ip) > 1e-6)
