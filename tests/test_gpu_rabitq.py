"""GPU parity of the one-bit RaBitQ quantizer against the oracle.

The device computes P^T x on the matrix cores in fp32 with a different
summation order than the oracle (the reference's cuBLAS order is
unspecified as well), so:
  * a code bit must match wherever |r_i| > 1e-5 * ||r|| (a sign can only
    differ where rounding moves r_i across zero);
  * f_rescale within 2e-5 relative; f_add within 2e-5 of the magnitude of
    its terms (||r||^2, 2||r||^2 s_cx / s_rx, <r, c'>, 1).
"""

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _check(jasper, x, m, c, metric, f16):
    n, dim = x.shape
    xt = torch.from_numpy(x.astype(np.float16 if f16 else np.float32)).cuda()
    rot = torch.from_numpy(np.asarray(m, dtype=np.float32)).cuda()
    cen = None if c is None else torch.from_numpy(c).cuda()
    got = jasper.rabitq_quantize(xt, rotation=rot, centroid=cen, distance=metric)
    torch.cuda.synchronize()
    nodes = got.nodes.cpu().numpy()
    xin = x.astype(np.float16).astype(np.float32) if f16 else x.astype(np.float32)
    ref, codes, f_add, f_rescale, r = oracle.rabitq_quantize(xin, m, c, metric=metric, return_residuals=True)
    assert nodes.shape == ref.shape
    cb = codes.shape[1]
    gb = np.unpackbits(nodes[:, :cb], axis=1, bitorder="little")[:, :dim]
    rb = np.unpackbits(codes, axis=1, bitorder="little")[:, :dim]
    nrm = np.sqrt((r.astype(np.float64) ** 2).sum(1))
    clear = np.abs(r) > 1e-5 * nrm[:, None]
    assert np.array_equal(gb[clear], rb[clear]), f"{(gb != rb)[clear].sum()} clear bits differ"
    assert not np.unpackbits(nodes[:, :cb], axis=1, bitorder="little")[:, dim:].any()
    ga = nodes[:, cb:cb + 4].copy().view(np.float32).ravel()
    gr = nodes[:, cb + 4:].copy().view(np.float32).ravel()
    np.testing.assert_allclose(gr, f_rescale, rtol=2e-5)
    rc = np.zeros(dim) if c is None else (np.asarray(m, np.float64).reshape(dim, dim).T @ c)
    s_cx = np.abs(rc).sum() * 0.5
    scale = nrm ** 2 * (1 + 2 * s_cx / np.maximum(0.5 * np.abs(r).sum(1), 1e-30)) + nrm * np.abs(rc).sum() + 1
    assert np.all(np.abs(ga - f_add) <= 2e-5 * scale), np.abs(ga - f_add).max()
    return got


@pytest.mark.parametrize("dim", [8, 32, 96, 100, 128, 200, 256])
@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_rabitq_matches_oracle(jasper, oracle_lib, dim, metric):
    rng = np.random.default_rng(dim)
    n = 1000 + dim
    x = (rng.normal(size=(n, dim)) * 3).astype(np.float32)
    m, _ = oracle.rotation_matrix(dim, 42)
    c = (rng.normal(size=dim) * 0.5).astype(np.float32)
    _check(jasper, x, m, c, metric, f16=True)
    _check(jasper, x, m, None, metric, f16=False)


def test_rabitq_identity_closed_form(jasper, oracle_lib):
    rng = np.random.default_rng(7)
    x = rng.normal(size=(333, 64)).astype(np.float32)
    got = _check(jasper, x, np.eye(64, dtype=np.float32).ravel(), None, "l2", f16=False)
    sq = (x.astype(np.float64) ** 2).sum(1)
    np.testing.assert_allclose(got.f_add.cpu().numpy(), sq, rtol=1e-5)
    assert torch.equal(got.bits().cpu(), torch.from_numpy((x >= 0).astype(np.uint8)))


def test_rabitq_default_rotation_and_sizes(jasper, oracle_lib):
    x = torch.randn(5, 97, device="cuda", dtype=torch.float16)
    got = jasper.rabitq_quantize(x)
    assert got.nodes.shape == (5, 24) and got.code_bytes == 16
    assert torch.isfinite(got.f_add).all() and (got.f_rescale < 0).all()
    empty = jasper.rabitq_quantize(x[:0])
    assert empty.nodes.shape == (0, 24)
