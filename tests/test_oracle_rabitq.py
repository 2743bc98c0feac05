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


# ------------------------------------------------ the one-bit RaBitQ estimator
# (this build's; the reference stops at the quantizer). Pinned by closed
# forms where every step is exact, by properties of the 4-bit query, and by
# its statistics against exact distances.

def _sign_case(dim, metric, seed):
    rng = np.random.default_rng(seed)
    x = rng.choice([-1.0, 1.0], size=(300, dim)).astype(np.float32)
    nodes, codes, f_add, f_rescale = oracle.rabitq_quantize(x, np.eye(dim, dtype=np.float32).ravel(),
                                                             metric=metric)
    # integer queries spanning exactly [-7, 8]: delta = 1, lo = -7, qbar = q + 7
    q = rng.integers(-7, 9, size=(12, dim)).astype(np.float32)
    q[:, 0], q[:, 1] = -7.0, 8.0
    rq = oracle.RqArtifacts(dim, nodes, np.zeros(dim, np.float32))
    return x, q, rq, f_add, f_rescale


@pytest.mark.parametrize("metric", ["l2", "ip"])
@pytest.mark.parametrize("dim", [16, 64, 256])
def test_estimate_exact_on_sign_vectors(metric, dim):
    """x in {-1, +1}^dim, zero centroid, dim a perfect square: f_add = dim
    (L2) or 1 (IP), f_rescale = -4 (L2) or -2 (IP) exactly; integer queries
    in [-7, 8] are exact at 4 bits; every term of the estimate is then an
    exact fp32 value and it equals the exact distance: ||x - q||^2 (L2),
    -<x, q> (IP)."""
    x, q, rq, f_add, f_rescale = _sign_case(dim, metric, dim)
    if metric == "l2":
        assert (f_add == dim).all() and (f_rescale == -4.0).all()
    else:
        assert (f_add == 1.0).all() and (f_rescale == -2.0).all()
    est, sumq, hhg, planes = oracle.rq_estimates(rq, oracle.as_padded_f16(q), metric, with_factors=True)
    assert (hhg[:, 0] == 0.5).all() and (hhg[:, 1] == -3.5).all()
    assert np.array_equal(sumq, (q + 7).sum(1).astype(np.int32))
    xd, qd = x.astype(np.float64), q.astype(np.float64)
    exact = ((qd[:, None, :] - xd[None]) ** 2).sum(-1) if metric == "l2" else -(qd @ xd.T)
    assert np.array_equal(est.astype(np.float64), exact)


def test_query_bit_planes():
    """Plane j holds bit j of qbar_i at dword i // 32, bit i % 32."""
    x, q, rq, _, _ = _sign_case(64, "l2", 3)
    _, _, _, planes = oracle.rq_estimates(rq, oracle.as_padded_f16(q), "l2", with_factors=True)
    qbar = (q + 7).astype(np.int64)
    for r in range(len(q)):
        for j in range(4):
            for i in range(64):
                assert ((int(planes[r, j, i // 32]) >> (i % 32)) & 1) == ((qbar[r, i] >> j) & 1)
        assert not planes[r, :, 2:].any()


def test_query_quantization_properties():
    """Real-valued queries: qbar in [0, 15] with lo + delta * qbar within
    delta / 2 (plus rounding) of q; sumq = sum qbar; g_add = ||q - c||^2 to
    fp32 accuracy."""
    rng = np.random.default_rng(4)
    dim = 100
    q = rng.standard_normal((20, dim)).astype(np.float16).astype(np.float32)
    c = rng.standard_normal(dim).astype(np.float32)
    nodes, *_ = oracle.rabitq_quantize(rng.standard_normal((5, dim)).astype(np.float32),
                                       np.eye(dim, dtype=np.float32).ravel())
    rq = oracle.RqArtifacts(dim, nodes, c)
    _, sumq, hhg, planes = oracle.rq_estimates(rq, oracle.as_padded_f16(q), "l2", with_factors=True)
    for r in range(len(q)):
        qbar = np.zeros(dim, np.int64)
        for j in range(4):
            bits = np.array([(int(planes[r, j, i // 32]) >> (i % 32)) & 1 for i in range(dim)])
            qbar |= bits << j
        delta, lo = 2.0 * hhg[r, 0], 2.0 * hhg[r, 1]
        assert lo == q[r].min() and abs(delta - (q[r].max() - lo) / 15) <= 1e-6 * abs(delta)
        assert qbar.min() == 0 and qbar.max() == 15 and sumq[r] == qbar.sum()
        assert np.abs(lo + delta * qbar - q[r]).max() <= 0.5 * delta * (1 + 1e-5)
        g = ((q[r].astype(np.float64) - c) ** 2).sum()
        assert abs(hhg[r, 2] - g) <= 1e-5 * g


@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_estimate_tracks_exact_distance(metric):
    """On rotated Gaussian data with the data mean as centroid the estimate
    is unbiased and its error has the one-bit estimator's known scale: the
    estimate of <r^, q^> has standard deviation sqrt(1 - a^2) / a / sqrt(dim)
    with a = <x_bar, r^> ~ 0.8 (about 0.75 / sqrt(dim)), so in units of
    ||x - c|| ||q - c|| / sqrt(dim) the error of -2<r, q_r> (L2) is ~1.5 and
    of -<r, q'> (IP) ~0.75. A lost rescale factor or a wrong sign fails it."""
    rng = np.random.default_rng(5)
    dim = 128
    P = oracle.rotation_matrix(dim, 42)[0]
    x = rng.standard_normal((2000, dim)).astype(np.float32)
    q = rng.standard_normal((40, dim)).astype(np.float32)
    Pm = colmajor_to_P(P, dim)
    xr = (x.astype(np.float64) @ Pm).astype(np.float16).astype(np.float32)    # rows P^T x
    qr = (q.astype(np.float64) @ Pm).astype(np.float16).astype(np.float32)
    if metric == "ip":
        xr /= np.linalg.norm(xr, axis=1, keepdims=True)
        qr /= np.linalg.norm(qr, axis=1, keepdims=True)
        xr, qr = xr.astype(np.float16).astype(np.float32), qr.astype(np.float16).astype(np.float32)
    c = xr.mean(0).astype(np.float32)
    nodes, *_ = oracle.rabitq_quantize(xr, np.eye(dim, dtype=np.float32).ravel(), centroid=c, metric=metric)
    est = oracle.rq_estimates(oracle.RqArtifacts(dim, nodes, c), oracle.as_padded_f16(qr), metric).astype(np.float64)
    xd, qd = xr.astype(np.float64), qr.astype(np.float64)
    exact = ((qd[:, None, :] - xd[None]) ** 2).sum(-1) if metric == "l2" else -(qd @ xd.T)
    err = est - exact
    scale = (np.linalg.norm(qd - c, axis=1)[:, None] * np.linalg.norm(xd - c, axis=1)[None]) / np.sqrt(dim)
    f = 2.0 if metric == "l2" else 1.0
    assert abs(err.mean()) < 0.02 * scale.mean()
    assert 0.6 * f < np.sqrt((err ** 2).mean()) / scale.mean() < 0.9 * f
    assert np.corrcoef(est.ravel(), exact.ravel())[0, 1] > 0.75


# ------------------------------------------------ best_rescale_factor (host) --
# The reference's host routine behind get_const_scaling_factors
# (quantize.cuh:22-131). Pinned by a closed form and by an independent
# restatement: a binary heap of step thresholds (the reference's structure)
# with the ratio recomputed from scratch at every step.

def _rescale_by_heap(o, ex_bits):
    import heapq
    tight = [0, 0.15, 0.20, 0.52, 0.59, 0.71, 0.75, 0.77, 0.81]
    top = (1 << ex_bits) - 1
    o = [float(v) for v in np.asarray(o, dtype=np.float32)]
    t_end = (top + 10) / max(o)
    t0 = t_end * tight[ex_bits]
    bar = [int(t0 * v + 1e-5) for v in o]
    heap = [((b + 1) / v, i) for i, (b, v) in enumerate(zip(bar, o))]
    heapq.heapify(heap)
    best, best_t = 0.0, 0.0
    while heap:
        t, i = heapq.heappop(heap)
        bar[i] += 1
        num = sum((b + 0.5) * v for b, v in zip(bar, o))
        den = sum((b + 0.5) ** 2 for b in bar)
        ip = num / np.sqrt(den)
        if ip > best:
            best, best_t = ip, t
        if bar[i] < top:
            tn = (bar[i] + 1) / o[i]
            if tn < t_end:
                heapq.heappush(heap, (tn, i))
    return best_t


def test_best_rescale_factor_one_dim_closed_form(oracle_lib):
    # dim 1, one bit: t_end = 11 / x, the counter starts at floor(1.65) = 1
    # and its one step (threshold 2 / x) raises the ratio from 0 to x
    for x in (0.7, 0.05, 1.0):
        xf = float(np.float32(x))
        assert oracle.best_rescale_factor(np.array([x], np.float32), 1) == pytest.approx(2.0 / xf, rel=1e-15)


@pytest.mark.parametrize("dim,ex_bits", [(8, 1), (16, 2), (32, 3), (24, 4), (128, 1)])
def test_best_rescale_factor_matches_heap_restatement(oracle_lib, dim, ex_bits):
    rng = np.random.default_rng(dim * 10 + ex_bits)
    for _ in range(5):
        x = rng.standard_normal(dim).astype(np.float32)
        o = np.abs(x / np.linalg.norm(x)).astype(np.float32)
        got = oracle.best_rescale_factor(o, ex_bits)
        want = _rescale_by_heap(o, ex_bits)
        assert got == pytest.approx(want, rel=1e-12), (got, want)


def test_const_scaling_factor_is_the_mean(oracle_lib):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((20, 64)).astype(np.float32)
    o = np.abs(x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)
    want = np.mean([oracle.best_rescale_factor(r, 1) for r in o])
    assert oracle.const_scaling_factor(o, 1) == pytest.approx(want, rel=1e-12)
