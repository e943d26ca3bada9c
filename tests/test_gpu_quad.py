"""GPU parity of the one-by-four wave MXFP4 kernel (quad_gemm, kernel id
QGEMM_KID_QUAD): each wave holds all 256 rows of A from LDS and loads its own
64 rows of B straight into registers.

* row-major operands through gemm_a4w4_mxfp4_kid (both scale tensors first
  shuffled into the workspace): one K-tile, odd and even K-tile counts,
  ragged M and N, a single row, batch 2, bf16 and fp32 output;
* aiter's bpreshuffle operands (B shuffle_weight(16,16), e8m0_shuffle
  scales) through gemm_a4w4_mxfp4_bpreshuffle_kid, against the oracle;
* configs[3] (8192^3) in aiter's formats, every output against the GPU
  reference GEMM, and two calls giving the same bits.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, assert_close_all, make_mx4, out_to_f32

pytestmark = pytest.mark.gpu

KID_QUAD = 8

ROW_MAJOR = [(256, 256, 256), (256, 256, 512), (512, 768, 768), (300, 200, 1280), (1, 64, 256),
             (513, 1000, 2048), (257, 520, 3584)]


def _row_major(qgemm, gpu, m, n, k, batch, dtype, seed):
    data = [make_mx4(m, n, k, seed=seed + i) for i in range(batch)]
    st = lambda i: torch.stack([torch.from_numpy(np.ascontiguousarray(d[i])) for d in data]).to(gpu)
    A, B, SA, SB = st(0), st(1), st(2), st(3)
    kb, kg = k // 2, k // 32
    C = torch.full((batch, m, n), float("nan"), dtype=dtype, device=gpu)
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, batch, kb, kb, n, m * kb, n * kb, m * n,
                       SA.data_ptr(), SB.data_ptr(), kg, kg, m * kg, n * kg)
    L = qgemm.lib()
    need = L.gemm_a4w4_mxfp4_kid_workspace_bytes(ctypes.byref(args), KID_QUAD)
    assert need > 0
    # no workspace: refused (the shuffled scales live there)
    st0 = L.gemm_a4w4_mxfp4_kid(ctypes.byref(args), 1 if dtype == torch.bfloat16 else 0, KID_QUAD, None, 0,
                                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st0 == 1
    ws = torch.full((need,), 0xAB, dtype=torch.uint8, device=gpu)
    stc = L.gemm_a4w4_mxfp4_kid(ctypes.byref(args), 1 if dtype == torch.bfloat16 else 0, KID_QUAD, ws.data_ptr(),
                                need, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert stc == 0, f"error {stc}"
    trace = qgemm.last_launch()
    torch.cuda.synchronize()
    return data, C, trace


@pytest.mark.parametrize("m,n,k", ROW_MAJOR)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_quad_row_major(qgemm, gpu, m, n, k, dtype):
    data, C, trace = _row_major(qgemm, gpu, m, n, k, 1, dtype, seed=m + 5 * n + k)
    f = "bf16" if dtype == torch.bfloat16 else "fp32"
    assert trace == f"e8m0_shuffle_blocks<2>+quad_gemm<fp4,MXS,RAW,{f}>", trace
    assert_close(O.gemm_mx4(*data[0]), out_to_f32(C[0]), f"quad row-major {m}x{n}x{k} {f}")


def test_quad_row_major_batch2(qgemm, gpu):
    m, n, k = 192, 320, 1024
    data, C, trace = _row_major(qgemm, gpu, m, n, k, 2, torch.bfloat16, seed=11)
    for i in range(2):
        assert_close(O.gemm_mx4(*data[i]), out_to_f32(C[i]), f"quad batch {i} {m}x{n}x{k} ({trace})")


def _aiter_operands(qa, qb, ea, eb, gpu):
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)
    return dev(qa), dev(O.shuffle_weight_16x16(qb)), dev(O.e8m0_shuffle(ea)), dev(O.e8m0_shuffle(eb))


@pytest.mark.parametrize("m,n,k", [(256, 256, 512), (300, 272, 2048), (33, 4096, 256), (1024, 2048, 7168),
                                   (768, 1280, 1536)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_quad_bpreshuffle(qgemm, gpu, m, n, k, dtype):
    qa, qb, ea, eb = make_mx4(m, n, k, seed=m + 3 * n + k)
    A, B, SA, SB = _aiter_operands(qa, qb, ea, eb, gpu)
    y = qgemm.gemm_a4w4(A, B, SA, SB, dtype=dtype, kernel_id=KID_QUAD)
    f = "bf16" if dtype == torch.bfloat16 else "fp32"
    assert qgemm.last_launch() == f"quad_gemm<fp4,MXS,W16,{f}>", qgemm.last_launch()
    assert_close(O.gemm_mx4(qa, qb, ea, eb), out_to_f32(y), f"quad bpreshuffle {m}x{n}x{k} {f}")
    with pytest.raises(RuntimeError):    # one tile per workgroup: no persistent grid
        qgemm.gemm_a4w4(A, B, SA, SB, dtype=dtype, kernel_id=KID_QUAD, grid_blocks=8)


def test_quad_full_size_every_output(qgemm, gpu):
    """configs[3] in aiter's formats on the one-by-four wave kernel."""
    m = n = k = 8192
    qa, sa = O.quant_mx4(O.randn((m, k), 0, 0))
    qb, sb = O.quant_mx4(O.randn((n, k), 0, 1))
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)
    A, B, SA, SB = dev(qa), dev(O.shuffle_weight_16x16(qb)), dev(O.e8m0_shuffle(sa)), dev(O.e8m0_shuffle(sb))
    y = qgemm.gemm_a4w4(A, B, SA, SB, kernel_id=KID_QUAD)
    assert qgemm.last_launch() == "quad_gemm<fp4,MXS,W16,bf16>"
    y2 = qgemm.gemm_a4w4(A, B, SA, SB, kernel_id=KID_QUAD)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), "two calls differ"
    ref = qgemm.reference_gemm("mxfp4", dev(qa), dev(qb), dev(sa), dev(sb))
    assert_close_all(ref, y, f"quad mxfp4 aiter {m}x{n}x{k}, every output")
