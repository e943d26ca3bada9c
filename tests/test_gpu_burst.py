"""GPU parity of the burst kernel (fp8, fp32 block scales, M <= 64, K <=
8192; burst_gemm.hpp) against the CPU oracle: every tile shape the planner
picks (16/32/64 rows, 16/32 columns), K split over workgroups and not, both
B layouts (K-panel B' through the LDS slot, fragment-order B'' straight
into registers), both SFA layouts, bf16 and fp32 output, M and N tails,
batched calls through the C ABI, and the no-workspace fallback."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, make_bs, make_mx4, make_mx8, out_to_f32, to_dev

pytestmark = pytest.mark.gpu

# (M, N, K) -> the burst plan the library picks (mb, nb, split)
SHAPES = [(1, 2112, 7168), (5, 1000, 2048), (17, 1000, 4096), (24, 1536, 7168), (32, 1536, 7168),
          (40, 300, 1024), (48, 7168, 2048), (64, 1536, 7168), (2, 200, 3072), (16, 24576, 1536),
          (64, 7168, 512), (30, 520, 8192), (3, 1000, 256)]


def _fp8(x, dev):
    return to_dev(x, None, dev).view(torch.float8_e4m3fn)


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("layout", ["kpanel", "frag"])
def test_burst(qgemm, gpu, m, n, k, layout):
    qa, qb, sa, sb = make_bs(m, n, k, seed=9 * m + n + k)
    ref = O.gemm_bs_fp32(qa, qb, sa, sb)
    bk = qgemm.shuffle_b_kpanel(to_dev(qb, None, gpu))
    for dtype, sfa_layout in ((torch.bfloat16, "mk"), (torch.float32, "km")):
        A_scale = to_dev(sa, None, gpu) if sfa_layout == "mk" else to_dev(np.ascontiguousarray(sa.T), None, gpu).t()
        if layout == "kpanel":
            y = qgemm.gemm_a8w8_bpreshuffle(_fp8(qa, gpu), bk.view(torch.float8_e4m3fn), A_scale,
                                            to_dev(sb, None, gpu), dtype=dtype)
        else:
            y = qgemm.gemm_a8w8_ldsbypass(_fp8(qa, gpu), qgemm.ldsbypass_repack(bk), A_scale, to_dev(sb, None, gpu),
                                          n, dtype=dtype)
        kern = qgemm.last_launch()
        assert kern.startswith(f"burst_gemm<fp8,BSF32,{'KPANEL' if layout == 'kpanel' else 'FRAG'},"), kern
        assert_close(ref, out_to_f32(y), f"burst {m}x{n}x{k} {layout} {dtype} {sfa_layout} ({kern})")


@pytest.mark.parametrize("m,n,k", [(32, 1536, 7168), (64, 1536, 7168)])
def test_burst_plan_without_workspace(qgemm, gpu, m, n, k):
    """A split burst plan needs the workspace; without one the call runs an
    unsplit kernel and still matches the oracle."""
    qa, qb, sa, sb = make_bs(m, n, k, seed=m + 5)
    bk = qgemm.shuffle_b_kpanel(to_dev(qb, None, gpu)).view(torch.float8_e4m3fn)
    y = qgemm.gemm_a8w8_bpreshuffle(_fp8(qa, gpu), bk, to_dev(sa, None, gpu), to_dev(sb, None, gpu),
                                    dtype=torch.bfloat16, workspace=False)
    assert not qgemm.last_launch().startswith("burst_gemm"), qgemm.last_launch()
    assert_close(O.gemm_bs_fp32(qa, qb, sa, sb), out_to_f32(y), "unsplit fallback")


@pytest.mark.parametrize("m,n,k", [(2, 2112, 2048), (32, 1536, 7168)])
def test_burst_batched_c_abi(qgemm, gpu, m, n, k):
    """Batch 2 through the C ABI (per-batch A, B', scales and C; the split
    plan's counters cover every batch's tiles)."""
    batch = 2
    data = [make_bs(m, n, k, seed=300 + i) for i in range(batch)]
    kg, nbk = k // 128, (n + 127) // 128
    A = torch.stack([torch.from_numpy(d[0]) for d in data]).to(gpu)
    Bk = torch.stack([qgemm.shuffle_b_kpanel(torch.from_numpy(d[1])) for d in data]).to(gpu)
    SA = torch.stack([torch.from_numpy(d[2]) for d in data]).to(gpu)
    SB = torch.stack([torch.from_numpy(d[3]) for d in data]).to(gpu)
    C = torch.empty(batch, m, n, dtype=torch.bfloat16, device=gpu)
    args = qgemm.Kargs(A.data_ptr(), Bk.data_ptr(), C.data_ptr(), m, n, k, batch, k, 128, n, m * k, n * k, m * n,
                       SA.data_ptr(), SB.data_ptr(), 1 if m > 1 else m, kg, m * kg, nbk * kg)
    L = qgemm.lib()
    need = L.gemm_a8w8_blockscale_bpreshuffle_workspace_bytes(ctypes.byref(args))
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=gpu)
    st = L.gemm_a8w8_blockscale_bpreshuffle(ctypes.byref(args), 1, ws.data_ptr() if need else None, need,
                                            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0
    assert qgemm.last_launch().startswith("burst_gemm"), qgemm.last_launch()
    torch.cuda.synchronize()
    for i, d in enumerate(data):
        assert_close(O.gemm_bs_fp32(*d), C[i].float().cpu().numpy(), f"batch {i}")
    assert int(ws[:2048].to(torch.int32).sum()) == 0, "split-K counters not re-armed"


# ----------------------------------------------------------------- MX burst
MX_KIDS = {"auto": 0, "tile256": 1, "mid128": 2, "skinny": 3, "decode": 4, "burst": 5, "stream": 6, "band": 7}


def _mx_call(qgemm, gpu, fp4, qa, qb, ea, eb, kid, out_dtype=torch.bfloat16, batch_data=None):
    m, n = qa.shape[0], qb.shape[0]
    kb = qa.shape[1]
    k = 2 * kb if fp4 else kb
    A, B = to_dev(qa, None, gpu), to_dev(qb, None, gpu)
    SA, SB = to_dev(ea, None, gpu), to_dev(eb, None, gpu)
    C = torch.empty(m, n, dtype=out_dtype, device=gpu)
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, 1, kb, kb, n, m * kb, n * kb, m * n,
                       SA.data_ptr(), SB.data_ptr(), k // 32, k // 32, m * (k // 32), n * (k // 32))
    L = qgemm.lib()
    name = "gemm_a4w4_mxfp4_kid" if fp4 else "gemm_a8w8_mxfp8_kid"
    need = getattr(L, name + "_workspace_bytes")(ctypes.byref(args), kid)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=gpu)
    st = getattr(L, name)(ctypes.byref(args), 1 if out_dtype == torch.bfloat16 else 0, kid,
                          ws.data_ptr() if need else None, need,
                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    kern = qgemm.last_launch()
    torch.cuda.synchronize()
    if need:
        assert int(ws[:2048].sum()) == 0, "split-K counters not re-armed"
    return st, C, kern


# (M, N, K): tile shapes 16/32/64 rows x 16/32 columns, M and N tails, K
# split over workgroups and not, configs[4] M = 32 (N = 7168, K = 16384)
MX_BURST_SHAPES = [(1, 1000, 2048), (9, 2112, 7168), (17, 520, 4096), (32, 7168, 16384), (33, 1536, 2048),
                   (48, 300, 1024), (64, 4096, 7168), (24, 7168, 16384)]


@pytest.mark.parametrize("m,n,k", MX_BURST_SHAPES)
@pytest.mark.parametrize("fp4", [False, True])
def test_mx_burst(qgemm, gpu, m, n, k, fp4):
    if fp4:
        qa, qb, ea, eb = make_mx4(m, n, k, seed=3 * m + n)
        ref = O.gemm_mx4(qa, qb, ea, eb)
    else:
        qa, qb, ea, eb = make_mx8(m, n, k, seed=3 * m + n)
        ref = O.gemm_mx8(qa, qb, ea, eb)
    for dtype in (torch.bfloat16, torch.float32):
        st, C, kern = _mx_call(qgemm, gpu, fp4, qa, qb, ea, eb, MX_KIDS["burst"], dtype)
        if k // (256 if fp4 else 128) > 64:      # more K-tiles than the burst plan takes
            assert st == 1
            return
        assert st == 0
        assert kern.startswith(f"burst_gemm<{'fp4' if fp4 else 'fp8'},MX,RAW,"), kern
        assert_close(ref, out_to_f32(C), f"mx burst {m}x{n}x{k} {dtype} ({kern})")


@pytest.mark.parametrize("m,n,k", [(4, 2112, 7168), (24, 1536, 4096), (100, 1024, 2048)])
@pytest.mark.parametrize("fp4", [False, True])
@pytest.mark.parametrize("kid", list(MX_KIDS))
def test_mx_kernel_ids(qgemm, gpu, m, n, k, fp4, kid):
    """Every kernel id of the MX entries against the oracle, or a clean
    rejection where the family cannot take the shape."""
    if fp4:
        qa, qb, ea, eb = make_mx4(m, n, k, seed=m + n)
        ref = O.gemm_mx4(qa, qb, ea, eb)
    else:
        qa, qb, ea, eb = make_mx8(m, n, k, seed=m + n)
        ref = O.gemm_mx8(qa, qb, ea, eb)
    st, C, kern = _mx_call(qgemm, gpu, fp4, qa, qb, ea, eb, MX_KIDS[kid])
    if (kid in ("decode", "burst", "band") and m > 64) or (kid == "stream" and m > 8):
        assert st == 1
        return
    assert st == 0
    want = {"tile256": "wide_gemm", "mid128": "mid_gemm", "skinny": "skinny_gemm", "decode": "decode_gemm",
            "burst": "burst_gemm", "stream": "stream_gemm", "band": "band_gemm"}.get(kid)
    assert want is None or want in kern, kern
    assert_close(ref, out_to_f32(C), f"mx kid {kid} {m}x{n}x{k} ({kern})")
