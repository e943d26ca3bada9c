"""GPU routes of the library plan where the 128 x 128 kernel's separate
split-K reduce moved the boundaries between kernels: which kernel AUTO
runs, and its outputs at 4096 sampled points against the oracle.

* MX, M > 256: 256 x 256 tiles from 96 tiles with long K, their K split
  into batch-strided slices of whole scale panels summed by
  splitk_reduce_kernel while the tiles leave half of the CUs idle (also
  with N % 4 != 0), and for M > 128 in place of a 128 x 128 plan where the
  slices fill 9/16 of the CUs; the 128 x 128 kernel at exactly 128 tiles
  with short K;
* MX, M <= 64 from N = 12288: the 128 x 128 kernel (M = 33-64, and M = 17-32
  where the skinny plan spills into a second round), split band plans;
* fp32 block scales: the 128 x 128 kernel with a deep split where one round
  of skinny workgroups would stream > 512 KB each, at exactly 128 tiles
  with >= 12 K-tiles (not at K = 512), and at M = 17-64 where the skinny
  plan spills 1 to 1.5 rounds.

Operands are drawn on the GPU and quantized by the library's quantizers
(bit-exact to the host recipes, test_gpu_quant.py); the oracle reads the
quantized bytes.  The expected kernels assume the 256 CUs of an MI355X.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close

pytestmark = pytest.mark.gpu


def _cus(gpu):
    return torch.cuda.get_device_properties(gpu).multi_processor_count


def _randn(shape, seed, gpu):
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    return torch.randn(shape, generator=g, device=gpu, dtype=torch.float32)


def _points(m, n, seed):
    rng = np.random.default_rng(seed)
    rows = np.concatenate([rng.integers(0, m, 4092), [0, m - 1, 0, m - 1]]).astype(np.int32)
    cols = np.concatenate([rng.integers(0, n, 4092), [0, 0, n - 1, n - 1]]).astype(np.int32)
    return rows, cols


def _host(t):
    return t.contiguous().view(torch.uint8).cpu().numpy() if t.element_size() == 1 else t.contiguous().cpu().numpy()


@pytest.mark.parametrize("fam,m,n,k,expect", [
    ("mx8", 512, 12288, 7168, "mx_scale_panels<pb16>+wide_gemm<fp8,MX,RAW,fp32,pb16>+splitk_reduce<bf16,x4,splitk2>"),
    ("mx8", 768, 8192, 16384, "mx_scale_panels<pb16>+wide_gemm<fp8,MX,RAW,fp32,pb16>+splitk_reduce<bf16,x4,splitk2>"),
    ("mx4", 768, 8192, 16384, "mx_scale_panels<pb32>+wide_gemm<fp4,MX,RAW,fp32,pb32>+splitk_reduce<bf16,x4,splitk2>"),
    ("mx8", 600, 10002, 7168, "mx_scale_panels<pb16>+wide_gemm<fp8,MX,RAW,fp32,pb16>+splitk_reduce<bf16,x1,splitk2>"),
    ("mx8", 768, 6144, 12288, "mx_scale_panels<pb16>+wide_gemm<fp8,MX,RAW,fp32,pb16>+splitk_reduce<bf16,x4,splitk3>"),
    ("mx4", 768, 6144, 7168, "mid_gemm<fp4,MX"),
    ("mx8", 192, 24576, 7168, "mx_scale_panels<pb16>+wide_gemm<fp8,MX,RAW,fp32,pb16>+splitk_reduce<bf16,x4,splitk2>"),
    ("mx8", 4096, 2048, 1536, "mid_gemm<fp8,MX"),
    ("mx4", 4096, 2048, 1536, "mid_gemm<fp4,MX"),
    ("mx4", 1024, 6144, 4096, "mx_scale_panels<pb32>+wide_gemm<fp4"),
    ("mx8", 64, 16384, 16384, "mid_gemm<fp8,MX,RAW,bf16,st4,ntb,splitk2>+splitk_reduce"),
    ("mx4", 32, 20480, 16384, "mid_gemm<fp4,MX"),
    ("mx4", 64, 16384, 7168, "band_gemm<fp4,mb4"),
    ("mx8", 32, 12288, 4096, "slice_gemm<fp8,MX,RAW,mb2"),
])
def test_mx_plan_route(qgemm, gpu, fam, m, n, k, expect):
    fp4 = fam == "mx4"
    quant = qgemm.quant_mxfp4 if fp4 else qgemm.quant_mxfp8
    A, SA = quant(_randn((m, k), m + n, gpu))
    B, SB = quant(_randn((n, k), m + n + 1, gpu))
    if fp4:
        y = qgemm.gemm_a4w4_mxfp4(A, B, SA, SB, dtype=torch.bfloat16)
    else:
        y = qgemm.gemm_a8w8_mxfp8(A, B, SA, SB, dtype=torch.bfloat16)
    trace = qgemm.last_launch()
    torch.cuda.synchronize()
    if _cus(gpu) == 256:
        assert trace.startswith(expect), trace
    rows, cols = _points(m, n, m + n + k)
    ref = (O.gemm_mx4_points if fp4 else O.gemm_mx8_points)(_host(A), _host(B), _host(SA), _host(SB), rows, cols)
    assert_close(ref, y.float().cpu().numpy()[rows, cols], f"{fam} {m}x{n}x{k} ({trace})")


@pytest.mark.parametrize("m,n,k,expect", [
    (192, 1536, 7168, "mid_gemm<fp8,BSF32,KPANEL,bf16,st4,splitk7>+splitk_reduce<bf16,x4,splitk7>"),
    (4096, 2048, 7168, "mid_gemm<fp8,BSF32,KPANEL"),
    (256, 32768, 512, "bsf32_gemm<fp8,BSF32,KPANEL"),
    (48, 20480, 7168, "mid_gemm<fp8,BSF32,KPANEL"),
])
def test_bs_plan_route(qgemm, gpu, m, n, k, expect):
    A, SA = qgemm.quant_fp8_blockscale(_randn((m, k), m + n, gpu), "1x128")
    B, SB = qgemm.quant_fp8_blockscale(_randn((n, k), m + n + 1, gpu), "128x128")
    Bk = qgemm.shuffle_b_kpanel(B)
    y = qgemm.gemm_a8w8_bpreshuffle(A, Bk, SA, SB, dtype=torch.bfloat16)
    trace = qgemm.last_launch()
    torch.cuda.synchronize()
    if _cus(gpu) == 256:
        assert trace.startswith(expect), trace
    rows, cols = _points(m, n, m + n + k)
    ref = O.gemm_bs_fp32_points(_host(A), _host(B), _host(SA), _host(SB), rows, cols)
    assert_close(ref, y.float().cpu().numpy()[rows, cols], f"bs {m}x{n}x{k} ({trace})")


def _panel_bytes(m, n, k):
    r256 = lambda b: (b + 255) // 256 * 256
    return 2048 + r256(m * (k // 32)) + r256(n * (k // 32))


@pytest.mark.parametrize("case", ["rowmajor_bf16", "rowmajor_fp32", "panels_only_ws"])
def test_mx8_wide_split_variants(qgemm, gpu, case):
    """The four-wave kernel's K split on row-major scales (K % 512 != 0, so
    no panel copy: 50 K-tiles in two 25-K-tile slices, pb4), with bf16 and
    fp32 output, and a caller workspace of exactly the scale-panel bytes,
    where the split's planes do not fit and the kernel runs unsplit."""
    m, n, k = (512, 12288, 6400) if case.startswith("rowmajor") else (512, 12288, 7168)
    dtype = torch.float32 if case == "rowmajor_fp32" else torch.bfloat16
    A, SA = qgemm.quant_mxfp8(_randn((m, k), m + k, gpu))
    B, SB = qgemm.quant_mxfp8(_randn((n, k), m + k + 1, gpu))
    ws = None
    if case == "panels_only_ws":
        ws = torch.zeros(_panel_bytes(m, n, k), dtype=torch.uint8, device=gpu)
    y = qgemm.gemm_a8w8_mxfp8(A, B, SA, SB, dtype=dtype, workspace=ws)
    trace = qgemm.last_launch()
    torch.cuda.synchronize()
    expect = {
        "rowmajor_bf16": "wide_gemm<fp8,MX,RAW,fp32,pb4>+splitk_reduce<bf16,x4,splitk2>",
        "rowmajor_fp32": "wide_gemm<fp8,MX,RAW,fp32,pb4>+splitk_reduce<fp32,x4,splitk2>",
        "panels_only_ws": "mx_scale_panels<pb16>+wide_gemm<fp8,MX,RAW,bf16,pb16>",
    }[case]
    if _cus(gpu) == 256:
        assert trace == expect, trace
    rows, cols = _points(m, n, m + n + k)
    ref = O.gemm_mx8_points(_host(A), _host(B), _host(SA), _host(SB), rows, cols)
    assert_close(ref, y.float().cpu().numpy()[rows, cols], f"mx8 {m}x{n}x{k} {case} ({trace})")
