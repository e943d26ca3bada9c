"""Full-size parity of the exact kernels bench.py times.

Each test builds the benchmark's own inputs (BASELINE recipe: N(0,1) from
seed 0, stream 0 for A and 1 for B, quantized on the host), calls the entry
point the way bench.py does (bf16 output, the queried workspace), asserts
which kernel instantiations ran (qgemm_last_launch) and checks the output
two ways: against the CPU oracle at 4096 random points plus one whole band
of rows that straddles a 256-row tile boundary, and -- the way the
reference verifies its full-size runs (MX4
gemm_a4w4_mxfp4_4wave_host.cc:219-257 compares every 8192^3 output with
gemm_ref_gpu) -- every output element against the whole-output GPU
reference GEMM (qgemm_reference_gemm, pinned to the oracle in
test_gpu_reference.py).  Tolerance: |y - y_ref| <= 2^-7 |y_ref| + 1e-3
rms(y_ref), rms over the checked elements (the sampled check) or over the
whole output (the full check).
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, assert_close_all

pytestmark = pytest.mark.gpu

N_POINTS = 4096


def _points(m, n, seed):
    rng = np.random.default_rng(seed)
    rows = rng.integers(0, m, N_POINTS).astype(np.int32)
    cols = rng.integers(0, n, N_POINTS).astype(np.int32)
    # corners and tile edges
    rows[:4] = [0, m - 1, 0, m - 1]
    cols[:4] = [0, 0, n - 1, n - 1]
    return rows, cols


def _band(m, rows):
    r0 = max(0, min(m - rows, m // 2 - rows // 2))
    return slice(r0, r0 + rows)


def _check(y, ref_points_fn, ref_band_fn, m, n, band_rows, what, seed=1):
    got = y.float().cpu().numpy()
    rows, cols = _points(m, n, seed)
    band = _band(m, band_rows)
    ref_p = ref_points_fn(rows, cols)
    ref_b = ref_band_fn(band)
    ref = np.concatenate([ref_p, ref_b.reshape(-1)])
    out = np.concatenate([got[rows, cols], got[band].reshape(-1)])
    assert_close(ref, out, what)


def _bench_inputs(m, n, k):
    return O.randn((m, k), 0, 0), O.randn((n, k), 0, 1)


@pytest.mark.parametrize("m,n,k,kernel", [
    (8192, 8192, 8192, "mx_scale_panels<pb16>+wide_gemm<fp8,MX,RAW,bf16,pb16>"),      # configs[1]
])
def test_mxfp8_bench_kernel_full_size(qgemm, gpu, m, n, k, kernel):
    a, b = _bench_inputs(m, n, k)
    qa, sa = O.quant_mx8(a)
    qb, sb = O.quant_mx8(b)
    del a, b
    dev = lambda x: torch.from_numpy(x).to(gpu)
    y = qgemm.gemm_a8w8_mxfp8(dev(qa).view(torch.float8_e4m3fn), dev(qb).view(torch.float8_e4m3fn), dev(sa), dev(sb),
                              dtype=torch.bfloat16)
    assert qgemm.last_launch() == kernel
    torch.cuda.synchronize()
    _check(y, lambda r, c: O.gemm_mx8_points(qa, qb, sa, sb, r, c),
           lambda band: O.gemm_mx8(qa[band], qb, sa[band], sb), m, n, 256, f"mxfp8 {m}x{n}x{k}")
    ref = qgemm.reference_gemm("mxfp8", dev(qa).view(torch.float8_e4m3fn), dev(qb).view(torch.float8_e4m3fn), dev(sa),
                               dev(sb))
    assert_close_all(ref, y, f"mxfp8 {m}x{n}x{k}, every output")


@pytest.mark.parametrize("m,n,k,kernel", [
    (8192, 8192, 8192, "mx_scale_panels<pb32>+wide_gemm<fp4,MX,RAW,bf16,pb32>"),      # configs[3]
    (16384, 7168, 2048, "mx_scale_panels<pb32>+wide_gemm<fp4,MX,RAW,bf16,pb32>"),     # configs[4] large M
])
def test_mxfp4_bench_kernel_full_size(qgemm, gpu, m, n, k, kernel):
    a, b = _bench_inputs(m, n, k)
    qa, sa = O.quant_mx4(a)
    qb, sb = O.quant_mx4(b)
    del a, b
    dev = lambda x: torch.from_numpy(x).to(gpu)
    y = qgemm.gemm_a4w4_mxfp4(dev(qa), dev(qb), dev(sa), dev(sb), dtype=torch.bfloat16)
    assert qgemm.last_launch() == kernel
    torch.cuda.synchronize()
    _check(y, lambda r, c: O.gemm_mx4_points(qa, qb, sa, sb, r, c),
           lambda band: O.gemm_mx4(qa[band], qb, sa[band], sb), m, n, 256, f"mxfp4 {m}x{n}x{k}")
    ref = qgemm.reference_gemm("mxfp4", dev(qa), dev(qb), dev(sa), dev(sb))
    assert_close_all(ref, y, f"mxfp4 {m}x{n}x{k}, every output")


@pytest.mark.parametrize("grid_blocks,kernel", [
    (0, "quad_gemm<fp4,MXS,W16,bf16>"),
    (256, "wide_gemm<fp4,MXS,W16,bf16,pb32,persist256>"),
])
def test_mxfp4_aiter_bench_kernel_full_size(qgemm, gpu, grid_blocks, kernel):
    """configs[3] in aiter's gemm_a4w4(bpreshuffle=True) formats (bench.py
    workload mxfp4_8192_aiter): B shuffle_weight(16,16), e8m0_shuffle scales."""
    m = n = k = 8192
    a, b = _bench_inputs(m, n, k)
    qa, sa = O.quant_mx4(a)
    qb, sb = O.quant_mx4(b)
    del a, b
    dev = lambda x: torch.from_numpy(x).to(gpu)
    y = qgemm.gemm_a4w4(dev(qa), dev(O.shuffle_weight_16x16(qb)), dev(O.e8m0_shuffle(sa)), dev(O.e8m0_shuffle(sb)),
                        grid_blocks=grid_blocks)
    assert qgemm.last_launch() == kernel
    torch.cuda.synchronize()
    _check(y, lambda r, c: O.gemm_mx4_points(qa, qb, sa, sb, r, c),
           lambda band: O.gemm_mx4(qa[band], qb, sa[band], sb), m, n, 256, f"mxfp4 aiter {m}x{n}x{k}")
    ref = qgemm.reference_gemm("mxfp4", dev(qa), dev(qb), dev(sa), dev(sb))
    assert_close_all(ref, y, f"mxfp4 aiter {m}x{n}x{k}, every output")


def test_blockscale_fp32_bench_kernel_full_size(qgemm, gpu):
    """bench.py --workload bs_fp32_8192: fp32 1x128 / 128x128 scales, K-panel B."""
    m = n = k = 8192
    a, b = _bench_inputs(m, n, k)
    qa, sa = O.quant_bs_act(a)
    qb, sb = O.quant_bs_wgt(b)
    del a, b
    dev = lambda x: torch.from_numpy(x).to(gpu)
    bk = qgemm.shuffle_b_kpanel(dev(qb)).view(torch.float8_e4m3fn)
    y = qgemm.gemm_a8w8_bpreshuffle(dev(qa).view(torch.float8_e4m3fn), bk, dev(sa), dev(sb), dtype=torch.bfloat16)
    assert qgemm.last_launch() == "bsf32_gemm<fp8,BSF32,KPANEL,bf16>"
    torch.cuda.synchronize()
    _check(y, lambda r, c: O.gemm_bs_fp32_points(qa, qb, sa, sb, r, c),
           lambda band: O.gemm_bs_fp32(qa[band], qb, sa[band], sb), m, n, 128, "bs-fp32 8192^3")
    ref = qgemm.reference_gemm("bs_fp32", dev(qa).view(torch.float8_e4m3fn), dev(qb).view(torch.float8_e4m3fn),
                               dev(sa), dev(sb))
    assert_close_all(ref, y, "bs-fp32 8192^3, every output")


def test_blockscale_e8m0_bench_kernel_full_size(qgemm, gpu):
    """bench.py --workload bs_e8m0_8192: the reference's headline kernel
    (E8M0 1x128 / 128x128 scales, shuffle_weight(16,16) B) through the
    reference adapter."""
    m = n = k = 8192
    a, b = _bench_inputs(m, n, k)
    qa, ea = O.quant_bs_e8m0_act(a)
    qb, eb = O.quant_bs_e8m0_wgt(b)
    del a, b
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)
    sfa_km = np.ascontiguousarray(ea.T)                 # physical [K/128][M]
    A_scale = dev(sfa_km).t()                            # logical [M, K/128], strides (1, M)
    y = qgemm.blockscale_bpreshuffle.gemm_a8w8_blockscale_bpreshuffle(
        dev(qa).view(torch.float8_e4m3fn), dev(O.shuffle_weight_16x16(qb)), A_scale, dev(eb), dtype=torch.bfloat16)
    assert qgemm.last_launch() == "wide_gemm<fp8,BS8,W16,bf16,pb16>"
    torch.cuda.synchronize()
    _check(y, lambda r, c: O.gemm_bs_e8m0_points(qa, qb, sfa_km, eb, r, c),
           lambda band: O.gemm_bs_e8m0(qa[band], qb, np.ascontiguousarray(sfa_km[:, band]), eb),
           m, n, 64, "bs-e8m0 8192^3")
    ref = qgemm.reference_gemm("bs_e8m0", dev(qa).view(torch.float8_e4m3fn), dev(qb).view(torch.float8_e4m3fn),
                               A_scale, dev(eb))
    assert_close_all(ref, y, "bs-e8m0 8192^3, every output")

    # the same GEMM in the NN / TT / TN layouts (bench.py --workload
    # bs_e8m0_8192_{nn,tt,tn}): the K-major operands feed the same MFMAs in
    # the same K order, so every output equals the NT result bit for bit
    A_km = dev(qa).t().contiguous().view(torch.float8_e4m3fn)          # [K, M]
    B_kn = dev(qb).t().contiguous().view(torch.float8_e4m3fn)          # [K, N]
    B_nk = dev(qb).view(torch.float8_e4m3fn)                           # [N, K]
    for layout, A_op, B_op, kern in (("nn", dev(qa).view(torch.float8_e4m3fn), B_kn, "wide_gemm<fp8,BS8,KN,bf16,pb16>"),
                                     ("tt", A_km, B_nk, "wide_gemm<fp8,BS8,RAW,bf16,pb16,akm>"),
                                     ("tn", A_km, B_kn, "wide_gemm<fp8,BS8,KN,bf16,pb16,akm>")):
        out = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
        getattr(qgemm, f"opus_gemm_mxfp8_{layout}")(A_op, B_op, A_scale, dev(eb), out)
        assert qgemm.last_launch() == kern, (layout, qgemm.last_launch())
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), y.view(torch.int16)), f"{layout.upper()} 8192^3 differs from NT"


SWEEP_NK = [(24576, 1536), (32768, 512), (7168, 16384), (4096, 7168), (7168, 2048), (2112, 7168)]
SWEEP_M = [1, 16, 64, 256, 1024, 4096, 16384]


@pytest.mark.parametrize("m", SWEEP_M)
@pytest.mark.parametrize("n,k", SWEEP_NK)
@pytest.mark.parametrize("variant", ["bpreshuffle", "ldsbypass"])
def test_blockscale_sweep_cell(qgemm, gpu, m, n, k, variant):
    """Every configs[2] cell (bench.py --sweep), both B layouts, through the
    entry and plan the sweep times, with its workspace: 4096 sampled points
    (every output when M*N is smaller) against the oracle."""
    a, b = O.randn((m, k), 2, 0), O.randn((n, k), 2, 1)
    qa, sa = O.quant_bs_act(a)
    qb, sb = O.quant_bs_wgt(b)
    del a, b
    dev = lambda x: torch.from_numpy(x).to(gpu)
    bk = qgemm.shuffle_b_kpanel(dev(qb))
    A = dev(qa).view(torch.float8_e4m3fn)
    if variant == "bpreshuffle":
        y = qgemm.gemm_a8w8_bpreshuffle(A, bk.view(torch.float8_e4m3fn), dev(sa), dev(sb), dtype=torch.bfloat16)
    else:
        y = qgemm.gemm_a8w8_ldsbypass(A, qgemm.ldsbypass_repack(bk), dev(sa), dev(sb), n, dtype=torch.bfloat16)
    kernel = qgemm.last_launch()
    torch.cuda.synchronize()
    if m * n <= N_POINTS:
        rows, cols = (x.reshape(-1).astype(np.int32) for x in np.meshgrid(np.arange(m), np.arange(n), indexing="ij"))
    else:
        rows, cols = _points(m, n, 3)
    ref = O.gemm_bs_fp32_points(qa, qb, sa, sb, rows, cols)
    assert_close(ref, y.float().cpu().numpy()[rows, cols], f"bs {variant} {m}x{n}x{k} ({kernel})")
