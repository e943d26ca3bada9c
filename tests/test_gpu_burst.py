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
from helpers import assert_close, make_bs, out_to_f32, to_dev

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
