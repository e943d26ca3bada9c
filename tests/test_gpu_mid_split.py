"""The 128 x 128 kernel's K split and its reduce: each workgroup stores its
slice's fp32 partial plane and splitk_reduce_kernel, launched next on the
stream, sums the slices in slice order into C.

* AUTO at the shapes whose split is deepest (8-K-tile slices while one
  workgroup per CU holds them): fp32 block scales M = 128, N = 2112,
  K = 7168 (7 slices) and MXFP4 M = 256, N = 1536, K = 7168 (3 slices);
* the 128 x 128 id forced at N % 4 != 0 (the per-element reduce), batch 2,
  fp32 output;
* outputs against the oracle (BASELINE tolerance), two calls bit-equal, the
  workspace's counter block left at zero.

The expected split counts assume the 256 CUs of an MI355X.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, make_bs, make_mx4, make_mx8, out_to_f32

pytestmark = pytest.mark.gpu

KID_AUTO, KID_MID = 0, 2


def _cus(gpu):
    return torch.cuda.get_device_properties(gpu).multi_processor_count


def _launch(qgemm, gpu, name, args, kid, out_dtype, m, n, batch):
    L = qgemm.lib()
    need = getattr(L, name + "_workspace_bytes")(ctypes.byref(args), kid)
    assert need > 2048, f"{name} kid {kid}: expected a K split, workspace {need}"
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
    outs = []
    for _ in range(2):
        C = torch.full((batch, m, n), float("nan"), dtype=out_dtype, device=gpu)
        args.ptr_c = C.data_ptr()
        st = getattr(L, name)(ctypes.byref(args), 1 if out_dtype == torch.bfloat16 else 0, kid, ws.data_ptr(), need,
                              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert st == 0, f"{name} kid {kid}: error {st}"
        trace = qgemm.last_launch()
        torch.cuda.synchronize()
        outs.append(C)
    assert int(ws[:2048].sum()) == 0, f"{name}: counter block not zero"
    assert torch.equal(outs[0].view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32),
                       outs[1].view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32)), \
        f"{name} ({trace}): two calls differ"
    return outs[0], trace


def _mx_args(qgemm, data, fp4, m, n, k, batch, gpu):
    st = lambda i: torch.stack([torch.from_numpy(np.ascontiguousarray(d[i])) for d in data]).to(gpu)
    A, B, SA, SB = st(0), st(1), st(2), st(3)
    kb, kg = (k // 2 if fp4 else k), k // 32
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), 0, m, n, k, batch, kb, kb, n, m * kb, n * kb, m * n,
                       SA.data_ptr(), SB.data_ptr(), kg, kg, m * kg, n * kg)
    return args, (A, B, SA, SB)


def test_bs_auto_deep_split(qgemm, gpu):
    m, n, k = 128, 2112, 7168
    qa, qb, sa, sb = make_bs(m, n, k, seed=41)
    A, SA, SB = (torch.from_numpy(x).to(gpu) for x in (qa, sa, sb))
    Bk = qgemm.shuffle_b_kpanel(torch.from_numpy(qb)).to(gpu)
    kg = k // 128
    args = qgemm.Kargs(A.data_ptr(), Bk.data_ptr(), 0, m, n, k, 1, k, 128, n, m * k, n * k, m * n,
                       SA.data_ptr(), SB.data_ptr(), 1, kg, m * kg, ((n + 127) // 128) * kg)
    C, trace = _launch(qgemm, gpu, "gemm_a8w8_blockscale_bpreshuffle_kid", args, KID_AUTO, torch.bfloat16, m, n, 1)
    if _cus(gpu) == 256:
        assert trace == "mid_gemm<fp8,BSF32,KPANEL,bf16,st4,splitk7>+splitk_reduce<bf16,x4,splitk7>", trace
    assert_close(O.gemm_bs_fp32(qa, qb, sa, sb), out_to_f32(C[0]), f"bs {m}x{n}x{k} ({trace})")


def test_mx4_auto_deep_split(qgemm, gpu):
    m, n, k = 256, 1536, 7168
    data = [make_mx4(m, n, k, seed=42)]
    args, keep = _mx_args(qgemm, data, True, m, n, k, 1, gpu)
    C, trace = _launch(qgemm, gpu, "gemm_a4w4_mxfp4_kid", args, KID_AUTO, torch.bfloat16, m, n, 1)
    if _cus(gpu) == 256:
        assert trace == "mid_gemm<fp4,MX,RAW,bf16,st4,splitk3>+splitk_reduce<bf16,x4,splitk3>", trace
    assert_close(O.gemm_mx4(*data[0]), out_to_f32(C[0]), f"mx4 {m}x{n}x{k} ({trace})")


@pytest.mark.parametrize("fp4", [False, True])
def test_mx_forced_mid_ragged_batch(qgemm, gpu, fp4):
    """N % 4 != 0: the per-element reduce; batch 2 planes; fp32 output."""
    m, n, batch = 200, 1003, 2
    k = 8192 if fp4 else 4096    # 32 K-tiles either way: four slices of 8
    data = [(make_mx4 if fp4 else make_mx8)(m, n, k, seed=43 + i) for i in range(batch)]
    args, keep = _mx_args(qgemm, data, fp4, m, n, k, batch, gpu)
    name = "gemm_a4w4_mxfp4_kid" if fp4 else "gemm_a8w8_mxfp8_kid"
    C, trace = _launch(qgemm, gpu, name, args, KID_MID, torch.float32, m, n, batch)
    if _cus(gpu) == 256:
        assert trace.endswith("splitk4>+splitk_reduce<fp32,x1,splitk4>"), trace
    for i in range(batch):
        ref = (O.gemm_mx4 if fp4 else O.gemm_mx8)(*data[i])
        assert_close(ref, out_to_f32(C[i]), f"{'mx4' if fp4 else 'mx8'} {m}x{n}x{k} b{i} ({trace})")
