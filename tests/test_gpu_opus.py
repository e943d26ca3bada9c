"""GPU parity of the aiter-facing wrappers (355_1_trans_amd/opus.py) and the
C entries behind them against the CPU oracle:

* every kernel id of the fp32 block-scale entries (bpreshuffle and
  LDS-bypass), forced, on shapes each family takes; ids a shape cannot take
  are rejected (opus_a8w8_bpreshuffle_integration_and_benchmark.md 3-4);
* gemm_a8w8_bpreshuffle_opus batched and with a pre-shuffled B;
* gemm_a8w8_mxfp8_opus batched with fp32 output;
* the E8M0 block-scale GEMM in the NT / NN / TT / TN physical layouts
  (opus_mxfp8_layouts_trace_8192_20261027T005846Z/capture.py:42-62): the
  same logical GEMM fed as [M,K] or [K,M] A and [N,K] or [K,N] B matches
  the oracle on the logical operands.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, make_bs, make_mx8, out_to_f32, to_dev

pytestmark = pytest.mark.gpu

KIDS = {"auto": 0, "tile256": 1, "mid128": 2, "skinny": 3, "decode": 4, "burst": 5}


def _fp8(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev).view(torch.float8_e4m3fn)


@pytest.mark.parametrize("m,n,k", [(1, 1536, 7168), (32, 1536, 7168), (64, 2112, 1024), (200, 1000, 2048),
                                   (300, 520, 384)])
@pytest.mark.parametrize("kid", list(KIDS))
def test_bpreshuffle_kernel_ids(qgemm, gpu, m, n, k, kid):
    qa, qb, sa, sb = make_bs(m, n, k, seed=m + 2 * n + k)
    ref = O.gemm_bs_fp32(qa, qb, sa, sb)
    run = lambda: qgemm.gemm_a8w8_bpreshuffle_opus(_fp8(qa, gpu), _fp8(qb, gpu), to_dev(sa, None, gpu),
                                                   to_dev(sb, None, gpu), kernelId=KIDS[kid])
    if kid in ("decode", "burst") and m > 64:
        with pytest.raises(RuntimeError):
            run()
        return
    y = run()
    launched = qgemm.last_launch()
    expect = {"tile256": "bsf32_gemm", "mid128": "mid_gemm", "skinny": "skinny_gemm", "decode": "decode_gemm",
              "burst": "burst_gemm"}.get(kid)
    assert expect is None or expect in launched, launched
    assert_close(ref, out_to_f32(y), f"kid {kid} {m}x{n}x{k} ({launched})")


@pytest.mark.parametrize("m,n,k", [(16, 2048, 4096), (96, 512, 1536)])
@pytest.mark.parametrize("kid", ["auto", "tile256", "mid128", "skinny", "burst"])
def test_ldsbypass_kernel_ids(qgemm, gpu, m, n, k, kid):
    qa, qb, sa, sb = make_bs(m, n, k, seed=5 * m + n)
    bpp = qgemm.ldsbypass_pack_b(torch.from_numpy(qb)).to(gpu)
    A, SA, SB = _fp8(qa, gpu), to_dev(sa, None, gpu), to_dev(sb, None, gpu)
    C = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    kg = k // 128
    args = qgemm.LdsBypassKargs(A.data_ptr(), None, bpp.data_ptr(), C.data_ptr(), m, n, k, 1, k, 128, n, m * k,
                                n * k, m * n, SA.data_ptr(), SB.data_ptr(), 1, kg, m * kg, SB.numel(), bpp.numel())
    L = qgemm.lib()
    need = L.gemm_a8w8_blockscale_ldsbypass_kid_workspace_bytes(ctypes.byref(args), KIDS[kid])
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=gpu)
    st = L.gemm_a8w8_blockscale_ldsbypass_kid(ctypes.byref(args), 1, KIDS[kid], ws.data_ptr() if need else None,
                                              need, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    if kid == "burst" and m > 64:
        assert st == 1
        return
    assert st == 0
    torch.cuda.synchronize()
    assert_close(O.gemm_bs_fp32(qa, qb, sa, sb), out_to_f32(C), f"ldsbypass kid {kid} ({qgemm.last_launch()})")
    assert int(ws[:2048].sum()) == 0, "split-K counters not re-armed"


def test_bpreshuffle_opus_batched_and_preshuffled(qgemm, gpu):
    batch, m, n, k = 2, 96, 640, 1024
    data = [make_bs(m, n, k, seed=70 + i) for i in range(batch)]
    A = torch.stack([_fp8(d[0], gpu) for d in data])
    B = torch.stack([_fp8(d[1], gpu) for d in data])
    xs = torch.stack([to_dev(d[2], None, gpu) for d in data])
    ws = torch.stack([to_dev(d[3], None, gpu) for d in data])
    for out_dtype in (torch.bfloat16, torch.float32):
        y = qgemm.gemm_a8w8_bpreshuffle_opus(A, B, xs, ws, out_dtype=out_dtype)
        assert y.shape == (batch, m, n) and y.dtype == out_dtype
        for i, d in enumerate(data):
            assert_close(O.gemm_bs_fp32(*d), out_to_f32(y[i]), f"batch {i} {out_dtype}")
    Bk = torch.stack([qgemm.shuffle_b_kpanel(B[i].view(torch.uint8)) for i in range(batch)])
    y = qgemm.gemm_a8w8_bpreshuffle_opus(A, Bk, xs, ws, preshuffled=True)
    for i, d in enumerate(data):
        assert_close(O.gemm_bs_fp32(*d), out_to_f32(y[i]), f"preshuffled batch {i}")


def test_mxfp8_opus_batched(qgemm, gpu):
    batch, m, n, k = 2, 300, 512, 1024
    data = [make_mx8(m, n, k, seed=90 + i) for i in range(batch)]
    A = torch.stack([_fp8(d[0], gpu) for d in data])
    B = torch.stack([_fp8(d[1], gpu) for d in data])
    xs = torch.stack([to_dev(d[2], None, gpu) for d in data])
    ws = torch.stack([to_dev(d[3], None, gpu) for d in data])
    y = qgemm.gemm_a8w8_mxfp8_opus(A, B, xs, ws)
    assert y.shape == (batch, m, n) and y.dtype == torch.float32
    for i, d in enumerate(data):
        assert_close(O.gemm_mx8(*d), out_to_f32(y[i]), f"mxfp8 opus batch {i}")


def _e8m0_inputs(m, n, k, seed):
    rng = np.random.default_rng(seed)
    a = O.e4m3_encode(rng.uniform(-1, 1, (m, k)).astype(np.float32))
    b = O.e4m3_encode(rng.uniform(-1, 1, (n, k)).astype(np.float32))
    sfa_km = rng.integers(124, 131, (k // 128, m)).astype(np.uint8)
    sfb = rng.integers(124, 131, (n // 128, k // 128)).astype(np.uint8)
    return a, b, sfa_km, sfb


@pytest.mark.parametrize("m,n,k", [(256, 512, 384), (512, 256, 1024), (768, 512, 2048), (256, 256, 128),
                                   (512, 768, 640), (1024, 1280, 256)])
@pytest.mark.parametrize("layout", ["nt", "nn", "tt", "tn"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_e8m0_layouts(qgemm, gpu, m, n, k, layout, dtype):
    a, b, sfa_km, sfb = _e8m0_inputs(m, n, k, seed=m + n + k)
    ref = O.gemm_bs_e8m0(a, b, sfa_km, sfb)
    A = _fp8(a.T if layout[0] == "t" else a, gpu)                       # [K, M] or [M, K]
    if layout == "nt":
        B = qgemm.shuffle_weight_16x16(torch.from_numpy(b)).to(gpu).view(torch.float8_e4m3fn)
    else:
        B = _fp8(b.T if layout[1] == "n" else b, gpu)                   # [K, N] or [N, K]
    sfa = torch.from_numpy(sfa_km).to(gpu).t()                          # [M, K/128] view of [K/128, M]
    out = torch.empty(m, n, dtype=dtype, device=gpu)
    getattr(qgemm, f"opus_gemm_mxfp8_{layout}")(A, B, sfa, torch.from_numpy(sfb).to(gpu), out)
    launched = qgemm.last_launch()
    f = "bf16" if dtype == torch.bfloat16 else "fp32"
    # NN / TT / TN: the M- or N-contiguous operands go through the kernel's
    # K-major LDS stages (transposing LDS reads), no transpose pass
    want = {"nt": f"wide_gemm<fp8,BS8,W16,{f},pb16>", "nn": f"wide_gemm<fp8,BS8,KN,{f},pb16>",
            "tt": f"wide_gemm<fp8,BS8,RAW,{f},pb16,akm>", "tn": f"wide_gemm<fp8,BS8,KN,{f},pb16,akm>"}
    assert launched == want[layout], launched
    assert_close(ref, out_to_f32(out), f"{layout} {m}x{n}x{k}")


def test_layout_entry_rejects(qgemm, gpu):
    m, n, k = 256, 512, 384
    a, b, sfa_km, sfb = _e8m0_inputs(m, n, k, seed=3)
    A, B = _fp8(a, gpu), _fp8(b.T, gpu)
    SA, SB = torch.from_numpy(sfa_km).to(gpu), torch.from_numpy(sfb).to(gpu)
    C = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    L = qgemm.lib()
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, 1, k, n, n, m * k, n * k, m * n,
                       SA.data_ptr(), SB.data_ptr(), m, k // 128, m * (k // 128), SB.numel())
    assert L.gemm_a8w8_blockscale_layout_workspace_bytes(ctypes.byref(args), 1) == 0   # no copies
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.gemm_a8w8_blockscale_layout(ctypes.byref(args), 4, 1, None, 0, s) == 1   # layout code
    assert L.gemm_a8w8_blockscale_layout(ctypes.byref(args), 2, 1, None, 0, s) == 1   # TT strides
    bad = qgemm.Kargs(*[getattr(args, f) for f, _ in qgemm.Kargs._fields_])
    bad.n = 384                                                                         # N % 256
    assert L.gemm_a8w8_blockscale_layout(ctypes.byref(bad), 1, 1, None, 0, s) == 1
    assert L.gemm_a8w8_blockscale_layout(ctypes.byref(args), 1, 1, None, 0, s) == 0
    assert qgemm.last_launch() == "wide_gemm<fp8,BS8,KN,bf16,pb16>"
    torch.cuda.synchronize()
    assert_close(O.gemm_bs_e8m0(a, b, sfa_km, sfb), out_to_f32(C), "NN through the C ABI")


@pytest.mark.parametrize("layout", [1, 2, 3])
def test_layout_entry_batch2(qgemm, gpu, layout):
    """Batched K-major operands through the C ABI: each batch entry of A
    [K][M] (TT, TN) and B [K][N] (NN, TN) at its dense batch stride."""
    m, n, k, batch = 512, 256, 768, 2
    at, bn = layout in (2, 3), layout in (1, 3)
    data = [_e8m0_inputs(m, n, k, seed=40 + i) for i in range(batch)]
    A = _fp8(np.stack([d[0].T if at else d[0] for d in data]), gpu)
    B = _fp8(np.stack([d[1].T if bn else d[1] for d in data]), gpu)
    SA = torch.from_numpy(np.stack([d[2] for d in data])).to(gpu)
    SB = torch.from_numpy(np.stack([d[3] for d in data])).to(gpu)
    C = torch.full((batch, m, n), float("nan"), dtype=torch.float32, device=gpu)
    kg = k // 128
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, batch, m if at else k, n if bn else k, n,
                       m * k, n * k, m * n, SA.data_ptr(), SB.data_ptr(), m, kg, m * kg, (n // 128) * kg)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert qgemm.lib().gemm_a8w8_blockscale_layout(ctypes.byref(args), layout, 0, None, 0, s) == 0
    torch.cuda.synchronize()
    for i, d in enumerate(data):
        assert_close(O.gemm_bs_e8m0(*d), out_to_f32(C[i]), f"layout {layout} batch {i}")
