"""GPU parity of the tail split of the 256 x 256 fp32-block-scale kernel
(bsf32_gemm.hpp): the tiles past the last whole round of one workgroup per CU
are cut into K slices whose fp32 partial images the last slice sums in slice
order (the data-parallel + split-K form of stream-K that
opus_gemm_splitk_and_interface_refactor.md:41-45 names next to the fused
split-K reduce).

The 256 x 256 kernel id runs its own plan: with fewer tiles than CUs every
tile is in the tail, so small shapes reach the split (edge tiles, batch 2,
both B layouts, bf16 and fp32 output) and are checked in full against the
oracle; without a workspace the same call runs unsplit.  One AUTO shape
with one whole round and a tail of 16 tiles (16384 sampled points).
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, make_bs, out_to_f32

pytestmark = pytest.mark.gpu

KID_TILE256 = 1


def _call(qgemm, gpu, data, variant, out_dtype, kid, workspace=True):
    """C ABI call of the fp32-block-scale entry over a batch of make_bs
    problems; returns (C, trace, workspace tensor or None)."""
    batch = len(data)
    qa, qb = data[0][0], data[0][1]
    m, k, n = qa.shape[0], qa.shape[1], qb.shape[0]
    kg, nbk = k // 128, (n + 127) // 128
    A = torch.stack([torch.from_numpy(d[0]) for d in data]).to(gpu)
    SA = torch.stack([torch.from_numpy(d[2]) for d in data]).to(gpu)
    SB = torch.stack([torch.from_numpy(d[3]) for d in data]).to(gpu)
    Bk = torch.stack([qgemm.shuffle_b_kpanel(torch.from_numpy(d[1])) for d in data]).to(gpu)
    C = torch.full((batch, m, n), float("nan"), dtype=out_dtype, device=gpu)
    L = qgemm.lib()
    if variant == "bpreshuffle":
        args = qgemm.Kargs(A.data_ptr(), Bk.data_ptr(), C.data_ptr(), m, n, k, batch, k, 128, n, m * k, n * k, m * n,
                           SA.data_ptr(), SB.data_ptr(), 1, kg, m * kg, nbk * kg)
        entry, query = L.gemm_a8w8_blockscale_bpreshuffle_kid, L.gemm_a8w8_blockscale_bpreshuffle_kid_workspace_bytes
    else:
        Bp = torch.stack([qgemm.ldsbypass_repack(Bk[i]) for i in range(batch)])
        args = qgemm.LdsBypassKargs(A.data_ptr(), None, Bp.data_ptr(), C.data_ptr(), m, n, k, batch, k, 128, n,
                                    m * k, Bp[0].numel(), m * n, SA.data_ptr(), SB.data_ptr(), 1, kg, m * kg,
                                    nbk * kg, Bp[0].numel())
        entry, query = L.gemm_a8w8_blockscale_ldsbypass_kid, L.gemm_a8w8_blockscale_ldsbypass_kid_workspace_bytes
    need = query(ctypes.byref(args), kid)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=gpu) if workspace and need else None
    st = entry(ctypes.byref(args), 1 if out_dtype == torch.bfloat16 else 0, kid,
               ws.data_ptr() if ws is not None else None, need if ws is not None else 0,
               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0
    trace = qgemm.last_launch()
    torch.cuda.synchronize()
    return C, trace, ws


@pytest.mark.parametrize("variant", ["bpreshuffle", "ldsbypass"])
@pytest.mark.parametrize("m,n,k,batch", [(700, 600, 6144, 1), (300, 520, 1536, 1), (512, 768, 3072, 2),
                                         (256, 256, 7168, 1)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_tail_split_tile256(qgemm, gpu, variant, m, n, k, batch, out_dtype):
    data = [make_bs(m, n, k, seed=11 * m + n + i) for i in range(batch)]
    C, trace, ws = _call(qgemm, gpu, data, variant, out_dtype, KID_TILE256)
    assert ",tail" in trace, trace
    for i, d in enumerate(data):
        assert_close(O.gemm_bs_fp32(*d), out_to_f32(C[i]), f"{variant} {m}x{n}x{k} batch {i} ({trace})")
    assert int(ws[:2048].to(torch.int32).sum()) == 0, "tail counters not re-armed"
    # a second call on the same workspace (counters re-armed, images rewritten)
    C2, trace2, _ = _call(qgemm, gpu, data, variant, out_dtype, KID_TILE256)
    assert trace2 == trace
    assert torch.equal(C.view(torch.uint8) if out_dtype == torch.bfloat16 else C,
                       C2.view(torch.uint8) if out_dtype == torch.bfloat16 else C2), "tail split not deterministic"


@pytest.mark.parametrize("variant", ["bpreshuffle", "ldsbypass"])
def test_tail_split_needs_its_workspace(qgemm, gpu, variant):
    """Without a workspace the 256 x 256 kernel runs every tile unsplit."""
    data = [make_bs(300, 520, 1536, seed=4)]
    C, trace, _ = _call(qgemm, gpu, data, variant, torch.bfloat16, KID_TILE256, workspace=False)
    assert ",tail" not in trace and trace.startswith("bsf32_gemm"), trace
    assert_close(O.gemm_bs_fp32(*data[0]), out_to_f32(C[0]), f"{variant} unsplit ({trace})")


def test_tail_split_auto(qgemm, gpu):
    """M = 4352, N = 4096, K = 7168: 272 tiles of 256 x 256 on 256 CUs --
    AUTO runs one whole round and splits the 16 tail tiles four ways."""
    m, n, k = 4352, 4096, 7168
    a, b = O.randn((m, k), 6, 0), O.randn((n, k), 6, 1)
    qa, sa = O.quant_bs_act(a)
    qb, sb = O.quant_bs_wgt(b)
    del a, b
    dev = lambda x: torch.from_numpy(x).to(gpu)
    bk = qgemm.shuffle_b_kpanel(dev(qb)).view(torch.float8_e4m3fn)
    y = qgemm.gemm_a8w8_bpreshuffle(dev(qa).view(torch.float8_e4m3fn), bk, dev(sa), dev(sb), dtype=torch.bfloat16)
    trace = qgemm.last_launch()
    torch.cuda.synchronize()
    if torch.cuda.get_device_properties(gpu).multi_processor_count == 256:
        assert trace == "bsf32_gemm<fp8,BSF32,KPANEL,bf16,tail16x4>", trace
    # 16384 points: about 960 of them in the 16 tail tiles
    rng = np.random.default_rng(8)
    rows = rng.integers(0, m, 16384).astype(np.int32)
    cols = rng.integers(0, n, 16384).astype(np.int32)
    ref = O.gemm_bs_fp32_points(qa, qb, sa, sb, rows, cols)
    assert_close(ref, y.float().cpu().numpy()[rows, cols], f"AUTO {m}x{n}x{k} ({trace})")
