"""The whole-output GPU reference GEMM (qgemm_reference_gemm, the role of
the reference's gemm_ref_gpu, MX4 gemm_a4w4_mxfp4_4wave_host.cc:66-94)
pinned before the full-size tests trust it:

* MXFP4 and E8M0 block scales: every product and every partial sum is exact
  in fp64 at these K, so the fp32 results are bit-identical to the oracle's
  fp64-accumulating restatements (MX4 gemm_ref_gpu, SNAP gemm_ref);
* MXFP8: bit-identical to an fp64 numpy brute force (exact products and
  sums), and within the oracle's own fp32 bound of the oracle;
* fp32 block scales: within 1e-12 of the summed magnitudes of an fp64 numpy
  brute force (a product of two fp32-scaled codes has 56 bits), and within
  the oracle's fp32 bound of the oracle, for both SFA layouts;
* ragged M and N (1, 37, 130, 7 ... columns) and tile-crossing K.

A planted mistake (a dropped scale, a transposed operand, a wrong nibble)
moves these results far past the bounds (test_oracle.py pins the oracle the
same way).
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import make_bs, make_mx4, make_mx8

pytestmark = pytest.mark.gpu

E2M1_GRID = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
SHAPES = [(1, 7, 256), (37, 100, 512), (130, 260, 1024), (64, 64, 2048)]


def _dec8(q):
    return torch.from_numpy(np.ascontiguousarray(q)).view(torch.float8_e4m3fn).double().numpy()


def _dec4(q):
    codes = np.stack([q & 15, q >> 4], -1).reshape(q.shape[0], -1)
    grid = np.array(E2M1_GRID + [-v for v in E2M1_GRID], np.float64)
    return grid[codes]


def _e8(e):
    return np.ldexp(1.0, e.astype(np.int64) - 127)


def _dev(x, gpu):
    return torch.from_numpy(np.ascontiguousarray(x)).to(gpu)


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_reference_mxfp4_equals_oracle(qgemm, gpu, m, n, k):
    qa, qb, ea, eb = make_mx4(m, n, k, seed=m + k)
    got = qgemm.reference_gemm("mxfp4", _dev(qa, gpu), _dev(qb, gpu), _dev(ea, gpu), _dev(eb, gpu)).cpu().numpy()
    assert np.array_equal(got, O.gemm_mx4(qa, qb, ea, eb)), (m, n, k)
    A = _dec4(qa) * np.repeat(_e8(ea), 32, 1)
    B = _dec4(qb) * np.repeat(_e8(eb), 32, 1)
    assert np.array_equal(got, (A @ B.T).astype(np.float32))


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_reference_mxfp8_equals_fp64(qgemm, gpu, m, n, k):
    qa, qb, ea, eb = make_mx8(m, n, k, seed=m + k)
    got = qgemm.reference_gemm("mxfp8", _dev(qa, gpu).view(torch.float8_e4m3fn), _dev(qb, gpu).view(torch.float8_e4m3fn),
                               _dev(ea, gpu), _dev(eb, gpu)).cpu().numpy()
    A = _dec8(qa) * np.repeat(_e8(ea), 32, 1)
    B = _dec8(qb) * np.repeat(_e8(eb), 32, 1)
    assert np.array_equal(got, (A @ B.T).astype(np.float32)), (m, n, k)
    mag = np.abs(A) @ np.abs(B).T
    assert np.all(np.abs(got - O.gemm_mx8(qa, qb, ea, eb)) <= 1e-5 * mag + 1e-30)


@pytest.mark.parametrize("m,n,k", SHAPES[1:])
def test_reference_bs_e8m0_equals_oracle(qgemm, gpu, m, n, k):
    a, b = O.randn((m, k), m, 0), O.randn((n, k), m, 1)
    qa, ea = O.quant_bs_e8m0_act(a)                  # ea [M, K/128]
    qb, eb = O.quant_bs_e8m0_wgt(b)                  # eb [ceil(N/128), K/128]
    sfa_km = np.ascontiguousarray(ea.T)
    A_scale = _dev(sfa_km, gpu).t()                  # the (1, M)-strided view of [K/128][M]
    got = qgemm.reference_gemm("bs_e8m0", _dev(qa, gpu).view(torch.float8_e4m3fn),
                               _dev(qb, gpu).view(torch.float8_e4m3fn), A_scale, _dev(eb, gpu)).cpu().numpy()
    assert np.array_equal(got, O.gemm_bs_e8m0(qa, qb, sfa_km, eb)), (m, n, k)


@pytest.mark.parametrize("m,n,k", SHAPES[1:])
@pytest.mark.parametrize("sfa_layout", ["mk", "km"])
def test_reference_bs_fp32_vs_fp64(qgemm, gpu, m, n, k, sfa_layout):
    qa, qb, sa, sb = make_bs(m, n, k, seed=m + k)
    if sfa_layout == "mk":
        A_scale = _dev(sa, gpu)
    else:
        A_scale = _dev(np.ascontiguousarray(sa.T), gpu).t()
    got = qgemm.reference_gemm("bs_fp32", _dev(qa, gpu).view(torch.float8_e4m3fn),
                               _dev(qb, gpu).view(torch.float8_e4m3fn), A_scale, _dev(sb, gpu)).cpu().numpy()
    A = _dec8(qa) * np.repeat(sa.astype(np.float64), 128, 1)
    B = _dec8(qb) * np.repeat(np.repeat(sb.astype(np.float64), 128, 0), 128, 1)[:n]
    mag = np.abs(A) @ np.abs(B).T
    assert np.all(np.abs(got - A @ B.T) <= 2.0 ** -24 * np.abs(A @ B.T) + 1e-12 * mag + 1e-30), (m, n, k)
    assert np.all(np.abs(got - O.gemm_bs_fp32(qa, qb, sa, sb)) <= 1e-5 * mag + 1e-30)
