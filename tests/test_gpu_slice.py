"""GPU parity of the slice decode kernel (slice_gemm, kernel id
QGEMM_KID_SLICE): MXFP8 / MXFP4 with row-major B, M <= 64, A's K slice in LDS,
B fragments straight from memory, 32 / 64 / 128 columns per workgroup.

* against the oracle: M 1-64 (one, two and four 16-row A blocks, ragged
  rows), ragged N (a last tile of 7-127 columns, waves past N), K of 1-64
  K-tiles including slices shorter than a wave's 16 K-tiles and K parts wholly
  past the end (their loads are empty, their K-tiles zeroed), bf16 and fp32
  output;
* the K split over workgroups with a workspace of garbage counters, two calls
  giving the same bits; the unsplit plan without a workspace where K fits one
  slice, and the refusal where K needs a split;
* batch 2 through the batch strides;
* configs[4] (M = 16 / 32 / 64, N = 7168, K = 16384) against the GPU
  reference GEMM, every output;
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

KID_SLICE = 10
HIP_INVALID_VALUE = 1


def _operands(fp4, m, n, k, batch, seed):
    make = make_mx4 if fp4 else make_mx8
    data = [make(m, n, k, seed=seed + i) for i in range(batch)]
    return data, [torch.stack([torch.from_numpy(np.ascontiguousarray(d[j])) for d in data]) for j in range(4)]


def _call(qgemm, gpu, fp4, m, n, k, batch, dtype, ops, ws="query"):
    A, B, SA, SB = [t.to(gpu) for t in ops]
    kb, kg = (k // 2 if fp4 else k), k // 32
    C = torch.full((batch, m, n), float("nan"), dtype=dtype, device=gpu)
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, batch, kb, kb, n, m * kb, n * kb, m * n,
                       SA.data_ptr(), SB.data_ptr(), kg, kg, m * kg, n * kg)
    L = qgemm.lib()
    name = "gemm_a4w4_mxfp4_kid" if fp4 else "gemm_a8w8_mxfp8_kid"
    need = getattr(L, name + "_workspace_bytes")(ctypes.byref(args), KID_SLICE)
    buf = None
    if ws == "query" and need:
        buf = torch.full((need,), 0x5A, dtype=torch.uint8, device=gpu)    # garbage counters and planes
    st = getattr(L, name)(ctypes.byref(args), 1 if dtype == torch.bfloat16 else 0, KID_SLICE,
                          buf.data_ptr() if buf is not None else None, need if buf is not None else 0,
                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    trace = qgemm.last_launch() if st == 0 else None
    torch.cuda.synchronize()
    return st, C, trace, need


CASES = [(17, 100, 512), (32, 1000, 2048), (33, 64, 1536), (64, 520, 4096), (1, 300, 1024), (16, 33, 8192),
         (48, 2000, 16384), (64, 7, 512), (8, 2112, 16384), (24, 135, 3072), (12, 700, 14336)]


@pytest.mark.parametrize("fmt", ["mx4", "mx8"])
@pytest.mark.parametrize("m,n,k", CASES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_slice_parity(qgemm, gpu, fmt, m, n, k, dtype):
    fp4 = fmt == "mx4"
    data, ops = _operands(fp4, m, n, k, 1, seed=m * 7 + n + k)
    st, C, trace, _ = _call(qgemm, gpu, fp4, m, n, k, 1, dtype, ops)
    assert st == 0, f"error {st}"
    assert trace.startswith(f"slice_gemm<{'fp4' if fp4 else 'fp8'},MX,RAW,mb"), trace
    ref = (O.gemm_mx4 if fp4 else O.gemm_mx8)(*data[0])
    assert_close(ref, out_to_f32(C[0]), f"slice {fmt} {m}x{n}x{k} ({trace})")


@pytest.mark.parametrize("fmt", ["mx4", "mx8"])
def test_slice_split(qgemm, gpu, fmt):
    """M = 40 (slices of 16 K-tiles), N = 256: K split over workgroups (fp4: 66
    K-tiles in 5 slices, the last of 2) with garbage in the workspace's
    counters; two calls give the same bits."""
    fp4 = fmt == "mx4"
    m, n, k = 40, 256, 16896 if fp4 else 8192
    data, ops = _operands(fp4, m, n, k, 1, seed=5)
    ref = (O.gemm_mx4 if fp4 else O.gemm_mx8)(*data[0])
    st, C, trace, need = _call(qgemm, gpu, fp4, m, n, k, 1, torch.bfloat16, ops)
    assert st == 0 and need > 0 and "splitk1>" not in trace, (st, trace)
    assert_close(ref, out_to_f32(C[0]), f"slice split {fmt} ({trace})")
    st2, C2, trace2, _ = _call(qgemm, gpu, fp4, m, n, k, 1, torch.bfloat16, ops)
    assert st2 == 0 and trace2 == trace
    assert torch.equal(C.view(torch.int16), C2.view(torch.int16)), "two calls differ"


@pytest.mark.parametrize("fmt", ["mx4", "mx8"])
def test_slice_no_workspace(qgemm, gpu, fmt):
    """Without a workspace: K within one slice (M <= 16: 64 K-tiles) runs
    unsplit; more is refused."""
    fp4 = fmt == "mx4"
    m, n, k = 16, 384, 16384 if fp4 else 8192
    data, ops = _operands(fp4, m, n, k, 1, seed=7)
    st, C, trace, _ = _call(qgemm, gpu, fp4, m, n, k, 1, torch.bfloat16, ops, ws=None)
    assert st == 0 and trace.endswith("splitk1>"), (st, trace)
    assert_close((O.gemm_mx4 if fp4 else O.gemm_mx8)(*data[0]), out_to_f32(C[0]), f"slice unsplit {fmt} ({trace})")
    kl = 8192 if fp4 else 4096    # M = 40: 32 K-tiles, two slices of 16
    _, ops_l = _operands(fp4, 40, 64, kl, 1, seed=6)
    st2, _, _, _ = _call(qgemm, gpu, fp4, 40, 64, kl, 1, torch.bfloat16, ops_l, ws=None)
    assert st2 == HIP_INVALID_VALUE


@pytest.mark.parametrize("fmt", ["mx4", "mx8"])
def test_slice_batch2(qgemm, gpu, fmt):
    fp4 = fmt == "mx4"
    m, n, k = 24, 200, 2048
    data, ops = _operands(fp4, m, n, k, 2, seed=17)
    st, C, trace, _ = _call(qgemm, gpu, fp4, m, n, k, 2, torch.float32, ops)
    assert st == 0, f"error {st}"
    for i in range(2):
        ref = (O.gemm_mx4 if fp4 else O.gemm_mx8)(*data[i])
        assert_close(ref, out_to_f32(C[i]), f"slice batch {i} {fmt} ({trace})")


def test_slice_refuses_unaligned_scales(qgemm, gpu):
    """K = 256 (fp4): 8-byte scale rows, which the 16-byte scale loads cannot take."""
    data, ops = _operands(True, 32, 64, 256, 1, seed=1)
    st, _, _, _ = _call(qgemm, gpu, True, 32, 64, 256, 1, torch.bfloat16, ops)
    assert st == HIP_INVALID_VALUE


@pytest.mark.parametrize("fmt,m", [("mx4", 16), ("mx4", 32), ("mx4", 64), ("mx8", 32)])
def test_slice_configs4_every_output(qgemm, gpu, fmt, m):
    """configs[4] decode shapes, every output against the GPU reference GEMM."""
    fp4 = fmt == "mx4"
    n, k = 7168, 16384
    quant = O.quant_mx4 if fp4 else O.quant_mx8
    qa, sa = quant(O.randn((m, k), 0, 0))
    qb, sb = quant(O.randn((n, k), 0, 1))
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)
    ops = [torch.from_numpy(np.ascontiguousarray(x))[None] for x in (qa, qb, sa, sb)]
    st, C, trace, _ = _call(qgemm, gpu, fp4, m, n, k, 1, torch.bfloat16, ops)
    assert st == 0 and trace.startswith(f"slice_gemm<{'fp4' if fp4 else 'fp8'},MX,RAW"), (st, trace)
    ref = qgemm.reference_gemm("mxfp4" if fp4 else "mxfp8", dev(qa), dev(qb), dev(sa), dev(sb))
    assert_close_all(ref, C[0], f"slice configs[4] {fmt} M={m} ({trace})")
