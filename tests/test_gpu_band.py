"""GPU parity of the band kernel (band_gemm.hpp: MX decode shapes, M <= 64,
row-major B; a workgroup owns 128 or 256 output columns and a K slice with
A's slice in LDS) through the MX entries' kernel id QGEMM_KID_BAND, against
the oracle's MXFP8 / MXFP4 GEMMs.

Shapes cover every (mb, cb) instantiation the plan takes (16-, 32- and
64-row A images; 128- and 256-column bands), K unsplit and split over 2-16
slices, M / N tails (M not a multiple of 16, N not a multiple of 16 or 4),
batch 2, bf16 and fp32 output, the configs[4] cells M = 16 / 32 / 64
(N = 7168, K = 16384), determinism over two calls and the workspace
counters re-armed; without its workspace a split plan is refused.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, make_mx4, make_mx8, out_to_f32

pytestmark = pytest.mark.gpu

KID_BAND = 7


def _problem(m, n, k, fp4, seed, batch=1):
    make = make_mx4 if fp4 else make_mx8
    return [make(m, n, k, seed=seed + i) for i in range(batch)]


def _ref(d, fp4):
    return O.gemm_mx4(*d) if fp4 else O.gemm_mx8(*d)


def _call(qgemm, gpu, data, fp4, out_dtype, workspace=True):
    batch = len(data)
    qa, qb = data[0][0], data[0][1]
    m, kb, n = qa.shape[0], qa.shape[1], qb.shape[0]
    k = 2 * kb if fp4 else kb
    kg = k // 32
    st = lambda i: torch.stack([torch.from_numpy(np.ascontiguousarray(d[i])) for d in data]).to(gpu)
    A, B, SA, SB = st(0), st(1), st(2), st(3)
    C = torch.full((batch, m, n), float("nan"), dtype=out_dtype, device=gpu)
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, batch, kb, kb, n, m * kb, n * kb, m * n,
                       SA.data_ptr(), SB.data_ptr(), kg, kg, m * kg, n * kg)
    L = qgemm.lib()
    name = "gemm_a4w4_mxfp4_kid" if fp4 else "gemm_a8w8_mxfp8_kid"
    need = getattr(L, name + "_workspace_bytes")(ctypes.byref(args), KID_BAND)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=gpu) if workspace and need else None
    rc = getattr(L, name)(ctypes.byref(args), 1 if out_dtype == torch.bfloat16 else 0, KID_BAND,
                          ws.data_ptr() if ws is not None else None, need if ws is not None else 0,
                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    kern = qgemm.last_launch()
    torch.cuda.synchronize()
    return rc, C, kern, ws


# (M, N, K): mb 1 / 2 / 4; unsplit (K <= 16 or 8 K-tiles) and split; tails
BAND_SHAPES = [(1, 520, 2048), (16, 1000, 4096), (9, 7168, 16384), (17, 300, 1536), (32, 2112, 7168),
               (33, 4096, 2048), (48, 520, 1024), (64, 2048, 4096), (64, 1030, 8192)]


@pytest.mark.parametrize("m,n,k", BAND_SHAPES)
@pytest.mark.parametrize("fp4", [False, True])
def test_band(qgemm, gpu, m, n, k, fp4):
    data = _problem(m, n, k, fp4, seed=5 * m + n)
    ref = _ref(data[0], fp4)
    for dtype in (torch.bfloat16, torch.float32):
        rc, C, kern, ws = _call(qgemm, gpu, data, fp4, dtype)
        assert rc == 0
        assert kern.startswith(f"band_gemm<{'fp4' if fp4 else 'fp8'},"), kern
        assert_close(ref, out_to_f32(C[0]), f"band {m}x{n}x{k} {dtype} ({kern})")
        if ws is not None:
            assert int(ws[:2048].to(torch.int32).sum()) == 0, "band counters not re-armed"
            rc2, C2, _, _ = _call(qgemm, gpu, data, fp4, dtype)
            assert rc2 == 0
            same = torch.equal(C.view(torch.int16), C2.view(torch.int16)) if dtype == torch.bfloat16 \
                else torch.equal(C, C2)
            assert same, "band split-K not deterministic"


@pytest.mark.parametrize("fp4", [False, True])
def test_band_batched(qgemm, gpu, fp4):
    data = _problem(40, 700, 4096, fp4, seed=77, batch=2)
    rc, C, kern, _ = _call(qgemm, gpu, data, fp4, torch.bfloat16)
    assert rc == 0, kern
    for i, d in enumerate(data):
        assert_close(_ref(d, fp4), out_to_f32(C[i]), f"band batch {i} ({kern})")


@pytest.mark.parametrize("m", [16, 32, 64])
def test_band_configs4(qgemm, gpu, m):
    """configs[4] cells: MXFP4 N = 7168, K = 16384 (sampled points)."""
    n, k = 7168, 16384
    qa, qb, ea, eb = make_mx4(m, n, k, seed=m)
    rc, C, kern, _ = _call(qgemm, gpu, [(qa, qb, ea, eb)], True, torch.bfloat16)
    assert rc == 0 and kern.startswith("band_gemm<fp4,"), kern
    rng = np.random.default_rng(m)
    rows = rng.integers(0, m, 4096).astype(np.int32)
    cols = rng.integers(0, n, 4096).astype(np.int32)
    ref = O.gemm_mx4_points(qa, qb, ea, eb, rows, cols)
    assert_close(ref, C[0].float().cpu().numpy()[rows, cols], f"band configs[4] M={m} ({kern})")


def test_band_needs_its_workspace(qgemm, gpu):
    data = _problem(32, 2112, 7168, True, seed=3)
    rc, _, _, _ = _call(qgemm, gpu, data, True, torch.bfloat16, workspace=False)
    assert rc == 1, "a split band plan without its workspace must be refused"
    # N = 32768: 256 bands of 128 columns fill the CUs unsplit
    data = _problem(32, 32768, 1024, True, seed=4)
    rc, C, kern, _ = _call(qgemm, gpu, data, True, torch.bfloat16, workspace=False)
    assert rc == 0 and kern.endswith("splitk1>"), kern
    assert_close(_ref(data[0], True), out_to_f32(C[0]), f"band unsplit ({kern})")


@pytest.mark.parametrize("fp4", [False, True])
def test_band_auto_route(qgemm, gpu, fp4):
    """AUTO takes the band kernel when one unsplit round of bands covers
    three quarters of the CUs (M = 40, N = 24576: 192 bands of 128 columns,
    K = 1024 within one slice)."""
    m, n, k = 40, 24576, 1024
    qa, qb, ea, eb = (make_mx4 if fp4 else make_mx8)(m, n, k, seed=12)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)
    fn = qgemm.gemm_a4w4_mxfp4 if fp4 else qgemm.gemm_a8w8_mxfp8
    y = fn(dev(qa), dev(qb), dev(ea), dev(eb), dtype=torch.bfloat16)
    kern = qgemm.last_launch()
    torch.cuda.synchronize()
    if torch.cuda.get_device_properties(gpu).multi_processor_count == 256:
        assert kern.startswith("band_gemm<") and kern.endswith("splitk1>"), kern
    rng = np.random.default_rng(1)
    rows = rng.integers(0, m, 4096).astype(np.int32)
    cols = rng.integers(0, n, 4096).astype(np.int32)
    pts = O.gemm_mx4_points if fp4 else O.gemm_mx8_points
    assert_close(pts(qa, qb, ea, eb, rows, cols), y.float().cpu().numpy()[rows, cols], f"AUTO band ({kern})")
