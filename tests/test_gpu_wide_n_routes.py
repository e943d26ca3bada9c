"""GPU routes of the library plan for M = 17-64 at wide N (the decode-sized
batches of the reference's traced weight shapes, N = 8192 - 32768): which
kernel AUTO runs, and its outputs at 4096 sampled points against the
oracle.

* fp32 block scales, M = 33-64 with 128 x 128 tiles filling 3/4 of the CUs
  (N = 24576): the 128 x 128 kernel;
* fp32 block scales, M = 17-32 on K-panel B at the same N (N = 32768,
  K = 2048): the decode kernel;
* fp32 block scales, N = 8192, K = 7168, M = 32 / 64: the decode kernel
  (M = 32: not the 16-wave burst plan);
* MXFP8 M = 64 (K = 2048) and MXFP4 M = 48 (K = 4096) at N = 24576: the
  slice kernel (one round of 192 workgroups, one K slice each).

The expected kernel names assume the 256 CUs of an MI355X.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close

pytestmark = pytest.mark.gpu


def _cus(gpu):
    return torch.cuda.get_device_properties(gpu).multi_processor_count


def _points(m, n, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, m, 4096).astype(np.int32), rng.integers(0, n, 4096).astype(np.int32)


@pytest.mark.parametrize("m,n,k,expect", [
    (48, 24576, 2048, "mid_gemm<fp8,BSF32,KPANEL"),
    (32, 32768, 2048, "decode_gemm<fp8,BSF32,KPANEL,mb2"),
    (32, 8192, 7168, "decode_gemm<fp8,BSF32,KPANEL,mb2"),
    (64, 8192, 7168, "decode_gemm<fp8,BSF32,KPANEL,mb4"),
])
def test_bs_fp32_wide_n_route(qgemm, gpu, m, n, k, expect):
    a, b = O.randn((m, k), 21, 0), O.randn((n, k), 21, 1)
    qa, sa = O.quant_bs_act(a)
    qb, sb = O.quant_bs_wgt(b)
    del a, b
    dev = lambda x: torch.from_numpy(x).to(gpu)
    bk = qgemm.shuffle_b_kpanel(dev(qb)).view(torch.float8_e4m3fn)
    y = qgemm.gemm_a8w8_bpreshuffle(dev(qa).view(torch.float8_e4m3fn), bk, dev(sa), dev(sb), dtype=torch.bfloat16)
    trace = qgemm.last_launch()
    torch.cuda.synchronize()
    if _cus(gpu) == 256:
        assert trace.startswith(expect), trace
    rows, cols = _points(m, n, m + n + k)
    ref = O.gemm_bs_fp32_points(qa, qb, sa, sb, rows, cols)
    assert_close(ref, y.float().cpu().numpy()[rows, cols], f"{m}x{n}x{k} ({trace})")


@pytest.mark.parametrize("fp4,m,n,k", [(False, 64, 24576, 2048), (True, 48, 24576, 4096)])
def test_mx_wide_n_route(qgemm, gpu, fp4, m, n, k):
    a, b = O.randn((m, k), 22, 0), O.randn((n, k), 22, 1)
    quant = O.quant_mx4 if fp4 else O.quant_mx8
    (qa, ea), (qb, eb) = quant(a), quant(b)
    del a, b
    dev = lambda x: torch.from_numpy(x).to(gpu)
    if fp4:
        y = qgemm.gemm_a4w4_mxfp4(dev(qa), dev(qb), dev(ea), dev(eb), dtype=torch.bfloat16)
    else:
        y = qgemm.gemm_a8w8_mxfp8(dev(qa).view(torch.float8_e4m3fn), dev(qb).view(torch.float8_e4m3fn), dev(ea),
                                  dev(eb), dtype=torch.bfloat16)
    trace = qgemm.last_launch()
    torch.cuda.synchronize()
    if _cus(gpu) == 256:
        assert trace.startswith("slice_gemm<fp4" if fp4 else "slice_gemm<fp8"), trace
    rows, cols = _points(m, n, m + n + k)
    ref = (O.gemm_mx4_points if fp4 else O.gemm_mx8_points)(qa, qb, ea, eb, rows, cols)
    assert_close(ref, y.float().cpu().numpy()[rows, cols], f"{'mx4' if fp4 else 'mx8'} {m}x{n}x{k} ({trace})")
