"""GPU parity of the 128 x 128 kernel on MXFP8 and MXFP4 (row-major B, E8M0
scales applied by the MFMA) against the CPU oracle.  The MX entries route
here when M > 64 and the 256 x 256 kernel would have fewer than 128 tiles:
M and N tails, K split on and off, per-K-group scale patterns, batched calls
with padded pitches through the C ABI, and the workspace re-armed across
calls."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, make_mx4, make_mx8, out_to_f32, to_dev

pytestmark = pytest.mark.gpu


def _fp8(x, dev):
    return to_dev(x, None, dev).view(torch.float8_e4m3fn)


def _run(qgemm, gpu, fp4, qa, qb, ea, eb, dtype=torch.bfloat16, workspace=None):
    if fp4:
        return qgemm.gemm_a4w4_mxfp4(to_dev(qa, None, gpu), to_dev(qb, None, gpu), to_dev(ea, None, gpu),
                                     to_dev(eb, None, gpu), dtype=dtype, workspace=workspace)
    return qgemm.gemm_a8w8_mxfp8(_fp8(qa, gpu), _fp8(qb, gpu), to_dev(ea, None, gpu), to_dev(eb, None, gpu),
                                 dtype=dtype, workspace=workspace)


# (m, n, k): every shape has M > 64 and < 128 256 x 256 tiles; (128, 7168,
# 16384) is configs[4] at M = 128; 65, 130, 300, 1500 and N = 1000, 700 end
# in partial tiles
MID_SHAPES = [(128, 7168, 16384), (65, 1000, 1024), (200, 2112, 7168), (256, 4096, 2048), (300, 1536, 4096),
              (520, 2112, 2048), (1000, 2112, 1024), (1500, 640, 3072)]
# one K-tile for fp4 (two for fp8: the prologue's empty-range DMAs and the
# tail loop alone), N below one tile, 129-row / 129-column tails
EDGE_SHAPES = [(100, 50, 256), (70, 130, 512), (129, 129, 1024), (80, 16, 768)]


@pytest.mark.parametrize("m,n,k", MID_SHAPES)
@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("fp4", [False, True])
def test_mx_mid(qgemm, gpu, fp4, m, n, k, split):
    make, gemm = (make_mx4, O.gemm_mx4) if fp4 else (make_mx8, O.gemm_mx8)
    qa, qb, ea, eb = make(m, n, k, seed=7 * m + n + k + fp4)
    y = _run(qgemm, gpu, fp4, qa, qb, ea, eb, workspace=None if split else False)
    assert_close(gemm(qa, qb, ea, eb), out_to_f32(y), f"{'mxfp4' if fp4 else 'mxfp8'} mid {m}x{n}x{k} split={split}")


@pytest.mark.parametrize("m,n,k", EDGE_SHAPES)
@pytest.mark.parametrize("fp4", [False, True])
def test_mx_mid_edges(qgemm, gpu, fp4, m, n, k):
    make, gemm = (make_mx4, O.gemm_mx4) if fp4 else (make_mx8, O.gemm_mx8)
    qa, qb, ea, eb = make(m, n, k, seed=3 * m + n + k + fp4)
    for dtype in (torch.bfloat16, torch.float32):
        y = _run(qgemm, gpu, fp4, qa, qb, ea, eb, dtype=dtype)
        assert_close(gemm(qa, qb, ea, eb), out_to_f32(y), f"mid edge {m}x{n}x{k} {dtype}")


@pytest.mark.parametrize("fp4", [False, True])
def test_mx_mid_k_pattern_scales(qgemm, gpu, fp4):
    """Distinct E8M0 per K group on both operands, fp32 output: a lane whose
    data and scale byte come from different groups scales products by the
    wrong power of two, far outside the tolerance."""
    m, n, k = 130, 500, 4096
    make, gemm = (make_mx4, O.gemm_mx4) if fp4 else (make_mx8, O.gemm_mx8)
    qa, qb, ea, eb = make(m, n, k, seed=41 + fp4)
    g = np.arange(k // 32)
    ea = np.broadcast_to((116 + g % 19).astype(np.uint8), ea.shape).copy()
    eb = np.broadcast_to((120 + (7 * g) % 13).astype(np.uint8), eb.shape).copy()
    y = _run(qgemm, gpu, fp4, qa, qb, ea, eb, dtype=torch.float32)
    assert_close(gemm(qa, qb, ea, eb), out_to_f32(y), "mid K-pattern")


def _padded(rows, cols, pitch, batch, fill, arrays):
    out = np.full((batch, rows, pitch), fill, dtype=np.uint8)
    for i, a in enumerate(arrays):
        out[i, :, :cols] = a
    return out


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("fp4", [False, True])
def test_mx_mid_batched_strided(qgemm, gpu, fp4, split):
    """Batch of 2 through the C ABI with padded row pitches on A, B, both
    scale arrays and C (padding bytes are NaN codes / 0xFF scales that must
    never be read; C's padding must stay zero)."""
    m, n, k, batch = 150, 700, 8192, 2
    make, gemm = (make_mx4, O.gemm_mx4) if fp4 else (make_mx8, O.gemm_mx8)
    data = [make(m, n, k, seed=600 + i + 10 * fp4) for i in range(batch)]
    kb = k // 2 if fp4 else k
    kg = k // 32
    lda, ldb, lsa, lsb, ldc = kb + 48, kb + 128, kg + 12, kg + 8, n + 24
    A = torch.from_numpy(_padded(m, kb, lda, batch, 0xFF, [d[0] for d in data])).to(gpu)
    B = torch.from_numpy(_padded(n, kb, ldb, batch, 0xFF, [d[1] for d in data])).to(gpu)
    SA = torch.from_numpy(_padded(m, kg, lsa, batch, 0xFF, [d[2] for d in data])).to(gpu)
    SB = torch.from_numpy(_padded(n, kg, lsb, batch, 0xFF, [d[3] for d in data])).to(gpu)
    C = torch.zeros(batch, m, ldc, dtype=torch.float32, device=gpu)
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, batch, lda, ldb, ldc, m * lda, n * ldb,
                       m * ldc, SA.data_ptr(), SB.data_ptr(), lsa, lsb, m * lsa, n * lsb)
    name = "gemm_a4w4_mxfp4" if fp4 else "gemm_a8w8_mxfp8"
    L = qgemm.lib()
    nbytes = getattr(L, name + "_workspace_bytes")(ctypes.byref(args)) if split else 0
    if split:
        assert nbytes > 2048, "expected a K split for this shape"
    ws = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=gpu)
    st = getattr(L, name)(ctypes.byref(args), qgemm.OUT_FP32, ctypes.c_void_p(ws.data_ptr() if split else 0),
                          nbytes, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, f"{name} returned {st}"
    torch.cuda.synchronize()
    Cc = C.cpu().numpy()
    for i, d in enumerate(data):
        assert_close(gemm(*d), Cc[i, :, :n], f"batch {i}")
        assert not Cc[i, :, n:].any(), "wrote past N"
    if split:
        assert int(ws[:2048].to(torch.int32).sum()) == 0, "split-K counters not re-armed"


def test_mx_mid_rearms_workspace(qgemm, gpu):
    """Calls sharing one workspace, the second smaller, the last a repeat of
    the first: within tolerance, the repeat bit-identical, counters zero."""
    shapes = [(False, 200, 2112, 7168), (True, 96, 1000, 4096), (False, 200, 2112, 7168)]
    ws = torch.zeros(1 << 24, dtype=torch.uint8, device=gpu)
    outs = []
    for i, (fp4, m, n, k) in enumerate(shapes):
        make, gemm = (make_mx4, O.gemm_mx4) if fp4 else (make_mx8, O.gemm_mx8)
        qa, qb, ea, eb = make(m, n, k, seed=900 + m)
        y = _run(qgemm, gpu, fp4, qa, qb, ea, eb, dtype=torch.float32, workspace=ws)
        torch.cuda.synchronize()
        assert_close(gemm(qa, qb, ea, eb), out_to_f32(y), f"call {i}")
        outs.append(y.cpu())
    assert torch.equal(outs[0], outs[2])
    assert int(ws[:2048].to(torch.int32).sum()) == 0, "split-K counters not re-armed"
