"""GPU parity of the row-run decode kernel (runs_gemm, kernel id
QGEMM_KID_RUNS): MXFP8 / MXFP4 with row-major B, M <= 64, B rows read in
512-byte runs through LDS.

* against the oracle: M 1-64 (one, two and four 16-row A blocks, ragged
  rows), ragged N, K of 1-64 K-tiles including slices that end inside a
  4-K-tile stage (those K-tiles are zeroed), bf16 and fp32 output;
* the K split over workgroups (narrow N) with a workspace of garbage
  counters, two calls giving the same bits; the unsplit plan without a
  workspace, and the refusal where K needs a split;
* batch 2 through the batch strides;
* configs[4] (M = 32 / 64, N = 7168, K = 16384) against the GPU reference
  GEMM, every output;
* operands the kernel cannot take (scale rows not 16-byte aligned) are
  refused with hipErrorInvalidValue.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, assert_close_all, make_mx4, make_mx8, out_to_f32

pytestmark = pytest.mark.gpu

KID_RUNS = 9
HIP_INVALID_VALUE = 1


def _operands(fp4, m, n, k, batch, seed):
    make = make_mx4 if fp4 else make_mx8
    data = [make(m, n, k, seed=seed + i) for i in range(batch)]
    return data, [torch.stack([torch.from_numpy(np.ascontiguousarray(d[j])) for d in data]) for j in range(4)]


def _call(qgemm, gpu, fp4, m, n, k, batch, dtype, ops, ws="query", C=None):
    A, B, SA, SB = [t.to(gpu) for t in ops]
    kb, kg = (k // 2 if fp4 else k), k // 32
    if C is None:
        C = torch.full((batch, m, n), float("nan"), dtype=dtype, device=gpu)
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, batch, kb, kb, n, m * kb, n * kb, m * n,
                       SA.data_ptr(), SB.data_ptr(), kg, kg, m * kg, n * kg)
    L = qgemm.lib()
    name = "gemm_a4w4_mxfp4_kid" if fp4 else "gemm_a8w8_mxfp8_kid"
    need = getattr(L, name + "_workspace_bytes")(ctypes.byref(args), KID_RUNS)
    buf = None
    if ws == "query" and need:
        buf = torch.full((need,), 0x5A, dtype=torch.uint8, device=gpu)    # garbage counters and planes
    st = getattr(L, name)(ctypes.byref(args), 1 if dtype == torch.bfloat16 else 0, KID_RUNS,
                          buf.data_ptr() if buf is not None else None, need if buf is not None else 0,
                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    trace = qgemm.last_launch() if st == 0 else None
    torch.cuda.synchronize()
    return st, C, trace, need


CASES = [(17, 100, 512), (32, 1000, 2048), (33, 64, 1536), (64, 520, 4096), (1, 300, 1024), (16, 33, 8192),
         (48, 2000, 16384), (64, 7, 512)]


@pytest.mark.parametrize("fmt", ["mx4", "mx8"])
@pytest.mark.parametrize("m,n,k", CASES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_runs_parity(qgemm, gpu, fmt, m, n, k, dtype):
    fp4 = fmt == "mx4"
    data, ops = _operands(fp4, m, n, k, 1, seed=m * 3 + n + k)
    st, C, trace, _ = _call(qgemm, gpu, fp4, m, n, k, 1, dtype, ops)
    assert st == 0, f"error {st}"
    assert trace.startswith(f"runs_gemm<{'fp4' if fp4 else 'fp8'},MX,RAW,mb"), trace
    ref = (O.gemm_mx4 if fp4 else O.gemm_mx8)(*data[0])
    assert_close(ref, out_to_f32(C[0]), f"runs {fmt} {m}x{n}x{k} ({trace})")


@pytest.mark.parametrize("fmt", ["mx4", "mx8"])
def test_runs_split(qgemm, gpu, fmt):
    """N = 256: eight tiles, K split over workgroups (fp4: 66 K-tiles in
    slices of 20, the last of 6 ends inside a stage) with garbage in the
    workspace's counters; two calls give the same bits."""
    fp4 = fmt == "mx4"
    m, n, k = 40, 256, 16896 if fp4 else 8192
    data, ops = _operands(fp4, m, n, k, 1, seed=5)
    ref = (O.gemm_mx4 if fp4 else O.gemm_mx8)(*data[0])
    st, C, trace, need = _call(qgemm, gpu, fp4, m, n, k, 1, torch.bfloat16, ops)
    assert st == 0 and need > 0 and "splitk1>" not in trace, (st, trace)
    assert_close(ref, out_to_f32(C[0]), f"runs split {fmt} ({trace})")
    st2, C2, trace2, _ = _call(qgemm, gpu, fp4, m, n, k, 1, torch.bfloat16, ops)
    assert st2 == 0 and trace2 == trace
    assert torch.equal(C.view(torch.int16), C2.view(torch.int16)), "two calls differ"


@pytest.mark.parametrize("fmt", ["mx4", "mx8"])
def test_runs_no_workspace(qgemm, gpu, fmt):
    """Without a workspace: K of at most 64 K-tiles runs unsplit; more is refused."""
    fp4 = fmt == "mx4"
    m, n, k = 40, 256, 16384 if fp4 else 8192
    data, ops = _operands(fp4, m, n, k, 1, seed=7)
    st, C, trace, _ = _call(qgemm, gpu, fp4, m, n, k, 1, torch.bfloat16, ops, ws=None)
    assert st == 0 and trace.endswith("splitk1>"), (st, trace)
    assert_close((O.gemm_mx4 if fp4 else O.gemm_mx8)(*data[0]), out_to_f32(C[0]), f"runs unsplit {fmt} ({trace})")
    kl = 32768 if fp4 else 16384    # 128 K-tiles: two slices at least
    _, ops_l = _operands(fp4, 8, 64, kl, 1, seed=6)
    st2, _, _, _ = _call(qgemm, gpu, fp4, 8, 64, kl, 1, torch.bfloat16, ops_l, ws=None)
    assert st2 == HIP_INVALID_VALUE


@pytest.mark.parametrize("fmt", ["mx4", "mx8"])
def test_runs_batch2(qgemm, gpu, fmt):
    fp4 = fmt == "mx4"
    m, n, k = 24, 200, 2048
    data, ops = _operands(fp4, m, n, k, 2, seed=17)
    st, C, trace, _ = _call(qgemm, gpu, fp4, m, n, k, 2, torch.float32, ops)
    assert st == 0, f"error {st}"
    for i in range(2):
        ref = (O.gemm_mx4 if fp4 else O.gemm_mx8)(*data[i])
        assert_close(ref, out_to_f32(C[i]), f"runs batch {i} {fmt} ({trace})")


def test_runs_refuses_unaligned_scales(qgemm, gpu):
    """K = 256 (fp4): 8-byte scale rows, which the 16-byte scale loads cannot take."""
    data, ops = _operands(True, 32, 64, 256, 1, seed=1)
    st, _, _, _ = _call(qgemm, gpu, True, 32, 64, 256, 1, torch.bfloat16, ops)
    assert st == HIP_INVALID_VALUE


@pytest.mark.parametrize("m", [32, 64])
def test_runs_configs4_every_output(qgemm, gpu, m):
    """configs[4] decode shapes, every output against the GPU reference GEMM."""
    n, k = 7168, 16384
    qa, sa = O.quant_mx4(O.randn((m, k), 0, 0))
    qb, sb = O.quant_mx4(O.randn((n, k), 0, 1))
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)
    ops = [torch.from_numpy(np.ascontiguousarray(x))[None] for x in (qa, qb, sa, sb)]
    st, C, trace, _ = _call(qgemm, gpu, True, m, n, k, 1, torch.bfloat16, ops)
    assert st == 0 and trace.startswith("runs_gemm<fp4,MX,RAW"), (st, trace)
    ref = qgemm.reference_gemm("mxfp4", dev(qa), dev(qb), dev(sa), dev(sb))
    assert_close_all(ref, C[0], f"runs configs[4] M={m} ({trace})")


@pytest.mark.parametrize("fmt,m,n,k", [("mx4", 64, 2112, 16384), ("mx8", 48, 4096, 8192)])
def test_runs_auto_route(qgemm, gpu, fmt, m, n, k):
    """AUTO takes the row-run kernel at M = 41-64, N <= 4096 and >= 64
    K-tiles when it has the workspace (and another kernel without one)."""
    fp4 = fmt == "mx4"
    data, ops = _operands(fp4, m, n, k, 1, seed=9)
    A, B, SA, SB = [t.to(gpu) for t in ops]
    kb, kg = (k // 2 if fp4 else k), k // 32
    C = torch.full((1, m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, 1, kb, kb, n, m * kb, n * kb, m * n,
                       SA.data_ptr(), SB.data_ptr(), kg, kg, m * kg, n * kg)
    L = qgemm.lib()
    name = "gemm_a4w4_mxfp4_kid" if fp4 else "gemm_a8w8_mxfp8_kid"
    need = getattr(L, name + "_workspace_bytes")(ctypes.byref(args), 0)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=gpu)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert getattr(L, name)(ctypes.byref(args), 1, 0, ws.data_ptr(), need, s) == 0
    trace = qgemm.last_launch()
    assert trace.startswith(f"runs_gemm<{'fp4' if fp4 else 'fp8'},MX,RAW,mb"), trace
    torch.cuda.synchronize()
    ref = (O.gemm_mx4 if fp4 else O.gemm_mx8)(*data[0])
    assert_close(ref, out_to_f32(C[0]), f"AUTO {fmt} {m}x{n}x{k} ({trace})")
    assert getattr(L, name)(ctypes.byref(args), 1, 0, None, 0, s) == 0
    assert not qgemm.last_launch().startswith("runs_gemm"), qgemm.last_launch()
