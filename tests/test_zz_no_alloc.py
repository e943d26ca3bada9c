"""gemm_a4w4_mxfp4_noalloc (the allocation-free MXFP4 entry, static
per-device scratch) against gemm_a4w4_mxfp4 with a caller workspace of the
queried size: bit-identical outputs on consecutive calls -- the second with
a smaller problem, so the scratch keeps the first call's contents -- and
within tolerance of the oracle."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, make_mx4

pytestmark = pytest.mark.gpu

# each shape uses the scratch, largest first: the 128 x 128 kernel's 4-way K
# split (14.7 MB of partials), the skinny kernel's K split, the row-streaming
# kernel's K split, the wide kernel's panel-major scale copy
SHAPES = [(128, 7168, 16384), (32, 1024, 8192), (4, 7168, 32768), (2304, 3600, 2048)]


def _kargs(qgemm, A, B, C, SA, SB, m, n, k):
    kb, kg = k // 2, k // 32
    return qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, 1, kb, kb, n, m * kb, n * kb, m * n,
                       SA.data_ptr(), SB.data_ptr(), kg, kg, m * kg, n * kg)


def test_noalloc_matches_workspace_entry(qgemm, gpu):
    L = qgemm.lib()
    assert L.gemm_a4w4_mxfp4_noalloc_max_workspace_bytes() == 32 << 20
    stream = torch.cuda.current_stream()
    sptr = ctypes.c_void_p(stream.cuda_stream)
    for m, n, k in SHAPES:
        qa, qb, ea, eb = make_mx4(m, n, k, seed=m + n)
        A, B = torch.from_numpy(qa).to(gpu), torch.from_numpy(qb).to(gpu)
        SA, SB = torch.from_numpy(ea).to(gpu), torch.from_numpy(eb).to(gpu)
        outs = []
        for noalloc in (True, False):
            C = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
            args = _kargs(qgemm, A, B, C, SA, SB, m, n, k)
            need = L.gemm_a4w4_mxfp4_workspace_bytes(ctypes.byref(args))
            assert 0 < need <= 32 << 20, (m, n, k, need)
            if noalloc:
                st = L.gemm_a4w4_mxfp4_noalloc(ctypes.byref(args), qgemm.OUT_BF16, sptr)
            else:
                ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
                st = L.gemm_a4w4_mxfp4(ctypes.byref(args), qgemm.OUT_BF16, ws.data_ptr(), need, sptr)
            assert st == 0
            torch.cuda.synchronize()
            outs.append(C.float().cpu())
        assert torch.equal(outs[0], outs[1]), (m, n, k)
        assert_close(O.gemm_mx4(qa, qb, ea, eb), outs[0].numpy(), f"noalloc {m}x{n}x{k}")


def test_noalloc_rejects_beyond_the_scratch(qgemm, gpu):
    """A call whose workspace query exceeds the static array is refused."""
    L = qgemm.lib()
    m, n, k = 8192, 8192, 65536               # panel-major scale copy of 32 MiB + counters
    base = [(1 << 44) + (i << 38) for i in range(5)]
    kb, kg = k // 2, k // 32
    args = qgemm.Kargs(base[0], base[1], base[2], m, n, k, 1, kb, kb, n, m * kb, n * kb, m * n, base[3], base[4],
                       kg, kg, m * kg, n * kg)
    assert L.gemm_a4w4_mxfp4_workspace_bytes(ctypes.byref(args)) > 32 << 20
    assert L.gemm_a4w4_mxfp4_noalloc(ctypes.byref(args), 1, None) == 1


def test_noalloc_split_within_the_scratch(qgemm, gpu):
    """A four-wave K split whose planes fit the 32 MiB scratch (M = 129:
    two 129 x 18432 fp32 planes + the scale panels): the allocation-free
    entry runs the same split as the workspace entry with the queried
    bytes, bit for bit, and matches the oracle at 4096 sampled points."""
    L = qgemm.lib()
    m, n, k = 129, 18432, 16384
    g = torch.Generator(device=gpu)
    g.manual_seed(129)
    A, SA = qgemm.quant_mxfp4(torch.randn((m, k), generator=g, device=gpu))
    B, SB = qgemm.quant_mxfp4(torch.randn((n, k), generator=g, device=gpu))
    stream = torch.cuda.current_stream()
    sptr = ctypes.c_void_p(stream.cuda_stream)
    outs, traces = [], []
    for noalloc in (True, False):
        C = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
        args = _kargs(qgemm, A, B, C, SA, SB, m, n, k)
        need = L.gemm_a4w4_mxfp4_workspace_bytes(ctypes.byref(args))
        assert 2 * m * n * 4 < need <= 32 << 20, need
        if noalloc:
            st = L.gemm_a4w4_mxfp4_noalloc(ctypes.byref(args), qgemm.OUT_BF16, sptr)
        else:
            ws = torch.empty(need, dtype=torch.uint8, device=gpu)
            st = L.gemm_a4w4_mxfp4(ctypes.byref(args), qgemm.OUT_BF16, ws.data_ptr(), need, sptr)
        assert st == 0
        traces.append(qgemm.last_launch())
        torch.cuda.synchronize()
        outs.append(C)
    assert traces[0] == traces[1] and "splitk_reduce" in traces[0], traces
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    rng = np.random.default_rng(5)
    rows = rng.integers(0, m, 4096).astype(np.int32)
    cols = rng.integers(0, n, 4096).astype(np.int32)
    host = lambda t: t.contiguous().view(torch.uint8).cpu().numpy()
    ref = O.gemm_mx4_points(host(A), host(B), host(SA), host(SB), rows, cols)
    assert_close(ref, outs[0].float().cpu().numpy()[rows, cols], f"noalloc split {m}x{n}x{k} ({traces[0]})")
