"""Seeded random shapes through every kernel id of the MXFP8, MXFP4 and
fp32-block-scale (bpreshuffle and LDS-bypass) entries, against the oracle.

The hand-picked shape lists of the other GPU tests follow the planner's
regions; these draws (M 1-200 weighted to decode sizes, N 1-1100 with any
tail, K up to 2048, batch 1 or 2, bf16 or fp32 output) reach the tails and
tile counts in between.  Each id is forced through the `*_kid` C ABI with
its queried workspace; an id whose kernel cannot take the shape must answer
hipErrorInvalidValue, every launch must match the oracle (BASELINE
tolerance) and leave the workspace's split-K counters at zero.
"""
import ctypes
import random

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, make_bs, make_mx4, make_mx8, out_to_f32

pytestmark = pytest.mark.gpu

HIP_INVALID_VALUE = 1


def _draws(family, count, seed):
    rng = random.Random(seed)
    kq = 256 if family == "mx4" else 128
    out = []
    for _ in range(count):
        m = rng.choice([1, 2, 3, 5, 8, 13, 16, 17, 31, 32, 33, 48, 64, rng.randint(65, 200)])
        n = rng.choice([rng.randint(1, 64), rng.randint(65, 1100)])
        k = kq * rng.randint(1, 2048 // kq)
        out.append((m, n, k, rng.choice([1, 1, 2]), rng.choice([True, False])))
    return out


def _run_ids(qgemm, gpu, name, args, kids, out_dtype, m, n, batch):
    """Yields (kid, C, trace) for every id that launched."""
    L = qgemm.lib()
    for kid in kids:
        C = torch.full((batch, m, n), float("nan"), dtype=out_dtype, device=gpu)
        args.ptr_c = C.data_ptr()
        need = getattr(L, name + "_workspace_bytes")(ctypes.byref(args), kid)
        ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=gpu)
        st = getattr(L, name)(ctypes.byref(args), 1 if out_dtype == torch.bfloat16 else 0, kid,
                              ws.data_ptr() if need else None, need,
                              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if st != 0:
            assert st == HIP_INVALID_VALUE, f"{name} kid {kid}: error {st}"
            continue
        trace = qgemm.last_launch()
        torch.cuda.synchronize()
        if need and "quad_gemm" not in trace:    # (the one-by-four wave kernel's workspace holds scales)
            assert int(ws[:2048].sum()) == 0, f"{name} kid {kid} ({trace}): split-K counters not re-armed"
        yield kid, C, trace


@pytest.mark.parametrize("family", ["mx8", "mx4"])
@pytest.mark.parametrize("case", range(24))
def test_mx_random_shapes(qgemm, gpu, family, case):
    fp4 = family == "mx4"
    m, n, k, batch, bf16 = _draws(family, 24, 1000 + int(fp4))[case]
    make = make_mx4 if fp4 else make_mx8
    data = [make(m, n, k, seed=case * 7 + i) for i in range(batch)]
    refs = [(O.gemm_mx4 if fp4 else O.gemm_mx8)(*d) for d in data]
    st = lambda i: torch.stack([torch.from_numpy(np.ascontiguousarray(d[i])) for d in data]).to(gpu)
    A, B, SA, SB = st(0), st(1), st(2), st(3)
    kb, kg = (k // 2 if fp4 else k), k // 32
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), 0, m, n, k, batch, kb, kb, n, m * kb, n * kb, m * n,
                       SA.data_ptr(), SB.data_ptr(), kg, kg, m * kg, n * kg)
    name = "gemm_a4w4_mxfp4_kid" if fp4 else "gemm_a8w8_mxfp8_kid"
    dt = torch.bfloat16 if bf16 else torch.float32
    launched = 0
    for kid, C, trace in _run_ids(qgemm, gpu, name, args, range(10), dt, m, n, batch):
        launched += 1
        for i in range(batch):
            assert_close(refs[i], out_to_f32(C[i]), f"{family} {m}x{n}x{k} b{i} kid {kid} ({trace})")
    assert launched >= 2    # AUTO and at least the kernel it chose


@pytest.mark.parametrize("case", range(24))
def test_bs_random_shapes(qgemm, gpu, case):
    m, n, k, batch, bf16 = _draws("bs", 24, 2000)[case]
    data = [make_bs(m, n, k, seed=case * 5 + i) for i in range(batch)]
    refs = [O.gemm_bs_fp32(*d) for d in data]
    kg, nbk = k // 128, (n + 127) // 128
    A = torch.stack([torch.from_numpy(d[0]) for d in data]).to(gpu)
    SA = torch.stack([torch.from_numpy(d[2]) for d in data]).to(gpu)
    SB = torch.stack([torch.from_numpy(d[3]) for d in data]).to(gpu)
    Bk = torch.stack([qgemm.shuffle_b_kpanel(torch.from_numpy(d[1])) for d in data]).to(gpu)
    args = qgemm.Kargs(A.data_ptr(), Bk.data_ptr(), 0, m, n, k, batch, k, 128, n, m * k, n * k, m * n,
                       SA.data_ptr(), SB.data_ptr(), 1, kg, m * kg, nbk * kg)
    dt = torch.bfloat16 if bf16 else torch.float32
    launched = 0
    for kid, C, trace in _run_ids(qgemm, gpu, "gemm_a8w8_blockscale_bpreshuffle_kid", args, range(6), dt, m, n,
                                  batch):
        launched += 1
        for i in range(batch):
            assert_close(refs[i], out_to_f32(C[i]), f"bs {m}x{n}x{k} b{i} kid {kid} ({trace})")
    assert launched >= 2


@pytest.mark.parametrize("case", range(24))
def test_ldsbypass_random_shapes(qgemm, gpu, case):
    """The LDS-bypass entry (B'' packed on the GPU from B) over the same kind
    of draws."""
    m, n, k, batch, bf16 = _draws("bs", 24, 3000)[case]
    data = [make_bs(m, n, k, seed=case * 3 + i) for i in range(batch)]
    refs = [O.gemm_bs_fp32(*d) for d in data]
    kg, nbk = k // 128, (n + 127) // 128
    A = torch.stack([torch.from_numpy(d[0]) for d in data]).to(gpu)
    SA = torch.stack([torch.from_numpy(d[2]) for d in data]).to(gpu)
    SB = torch.stack([torch.from_numpy(d[3]) for d in data]).to(gpu)
    Bp = torch.stack([qgemm.ldsbypass_pack_b(torch.from_numpy(d[1]).to(gpu)) for d in data])
    args = qgemm.LdsBypassKargs(A.data_ptr(), None, Bp.data_ptr(), 0, m, n, k, batch, k, 128, n, m * k,
                                Bp[0].numel(), m * n, SA.data_ptr(), SB.data_ptr(), 1, kg, m * kg, nbk * kg,
                                Bp[0].numel())
    dt = torch.bfloat16 if bf16 else torch.float32
    launched = 0
    for kid, C, trace in _run_ids(qgemm, gpu, "gemm_a8w8_blockscale_ldsbypass_kid", args, range(6), dt, m, n,
                                  batch):
        launched += 1
        for i in range(batch):
            assert_close(refs[i], out_to_f32(C[i]), f"ldsbypass {m}x{n}x{k} b{i} kid {kid} ({trace})")
    assert launched >= 2
