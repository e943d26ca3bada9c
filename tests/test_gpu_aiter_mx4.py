"""GPU parity of the MXFP4 entry that takes aiter's gemm_a4w4(bpreshuffle=True)
operands (gemm_a4w4_mxfp4_bpreshuffle; MX4 candidate_m10/
gemm_a4w4_mxfp4_4wave_host.cc:194-250): B in shuffle_weight(16,16) order, both
scale tensors in e8m0_shuffle order, optional persistent grid.

Operands are the oracle's quantized row-major codes, laid out by the oracle's
own shuffle_weight_16x16 / e8m0_shuffle (pinned against aiter's view/permute
forms in test_oracle.py); the expected output is the oracle's MXFP4 GEMM of
the row-major codes.  One case takes the device quantizer's shuffled output
instead, the way a serving caller would.  The persistent-grid cases use the
block counts the reference verifies with (default = one per CU, 37, 1).
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, make_mx4, out_to_f32

pytestmark = pytest.mark.gpu


def _aiter_operands(qa, qb, ea, eb, gpu):
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)
    return dev(qa), dev(O.shuffle_weight_16x16(qb)), dev(O.e8m0_shuffle(ea)), dev(O.e8m0_shuffle(eb))


# K % 1024 == 0 takes the 4-K-tile scale DMAs, K % 1024 == 512 one K-tile;
# M and N tails (N % 16 == 0), one 32-row scale block, several tiles
SHAPES = [(256, 256, 512), (512, 512, 1024), (300, 272, 2048), (1, 1024, 1024), (64, 7168, 2048),
          (768, 1280, 1536), (33, 4096, 256), (1024, 2048, 7168)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("kernel_id", [0, 1])
def test_gemm_a4w4_bpreshuffle(qgemm, gpu, m, n, k, dtype, kernel_id):
    """kernel_id 0: the library's choice, the one-by-four wave kernel;
    1: the two-by-two wave kernel."""
    qa, qb, ea, eb = make_mx4(m, n, k, seed=m + 3 * n + k)
    A, B, SA, SB = _aiter_operands(qa, qb, ea, eb, gpu)
    y = qgemm.gemm_a4w4(A, B, SA, SB, dtype=dtype, kernel_id=kernel_id)
    pb = 32 if k % 1024 == 0 else 8
    f = "bf16" if dtype == torch.bfloat16 else "fp32"
    want = f"quad_gemm<fp4,MXS,W16,{f}>" if kernel_id == 0 else f"wide_gemm<fp4,MXS,W16,{f},pb{pb}>"
    assert qgemm.last_launch() == want, qgemm.last_launch()
    assert_close(O.gemm_mx4(qa, qb, ea, eb), out_to_f32(y), f"a4w4 bpreshuffle {m}x{n}x{k} ({want})")


@pytest.mark.parametrize("m,n,k", [(768, 1280, 1536), (1024, 1024, 2048), (2048, 1024, 7168)])
@pytest.mark.parametrize("grid_blocks", [256, 37, 1])
def test_gemm_a4w4_persistent(qgemm, gpu, m, n, k, grid_blocks):
    qa, qb, ea, eb = make_mx4(m, n, k, seed=7 * m + n)
    A, B, SA, SB = _aiter_operands(qa, qb, ea, eb, gpu)
    y = qgemm.gemm_a4w4(A, B, SA, SB, grid_blocks=grid_blocks)
    tiles = ((m + 255) // 256) * ((n + 255) // 256)
    assert qgemm.last_launch().endswith(f"persist{min(grid_blocks, tiles)}>"), qgemm.last_launch()
    assert_close(O.gemm_mx4(qa, qb, ea, eb), out_to_f32(y), f"a4w4 persistent {grid_blocks} {m}x{n}x{k}")


def test_gemm_a4w4_device_quantizer(qgemm, gpu):
    """quant_mxfp4(x, shuffle=True) + shuffle_weight_16x16 on the GPU feed the
    entry directly; the codes are the oracle's, byte for byte."""
    m, n, k = 320, 512, 2048
    a, b = O.randn((m, k), 4, 0), O.randn((n, k), 4, 1)
    qa, ea = O.quant_mx4(a)
    qb, eb = O.quant_mx4(b)
    A, SA = qgemm.quant_mxfp4(torch.from_numpy(a).to(gpu), shuffle=True)
    Bq, SB = qgemm.quant_mxfp4(torch.from_numpy(b).to(gpu), shuffle=True)
    assert np.array_equal(A.cpu().numpy(), qa) and np.array_equal(SA.cpu().numpy(), O.e8m0_shuffle(ea))
    y = qgemm.gemm_a4w4(A, qgemm.shuffle_weight_16x16(Bq), SA, SB)
    assert_close(O.gemm_mx4(qa, qb, ea, eb), out_to_f32(y), "a4w4 from the device quantizer")


def test_gemm_a4w4_batched_c_abi(qgemm, gpu):
    """Batch 3 through the C ABI with padded scale batch strides, one- and
    multi-tile persistent grids over the batch x tiles list."""
    batch, m, n, k = 3, 384, 512, 1024
    data = [make_mx4(m, n, k, seed=50 + i) for i in range(batch)]
    kb, kg = k // 2, k // 32
    A = torch.stack([torch.from_numpy(d[0]) for d in data]).to(gpu)
    B = torch.stack([torch.from_numpy(O.shuffle_weight_16x16(d[1])) for d in data]).to(gpu)
    sa_rows, sb_rows = (m + 31) // 32 * 32 + 64, (n + 31) // 32 * 32    # SFA batches padded by two blocks
    SA = torch.full((batch, sa_rows * kg), 0x7F, dtype=torch.uint8)
    SB = torch.empty((batch, sb_rows * kg), dtype=torch.uint8)
    for i, d in enumerate(data):
        sa = O.e8m0_shuffle(d[2]).reshape(-1)
        SA[i, :sa.size] = torch.from_numpy(sa)
        SB[i] = torch.from_numpy(O.e8m0_shuffle(d[3]).reshape(-1))
    SA, SB = SA.to(gpu), SB.to(gpu)
    L = qgemm.lib()
    for grid_blocks in (0, 5, 1):
        C = torch.full((batch, m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
        args = qgemm.Mxfp4Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, batch, kb, kb, n, m * kb,
                                n * kb, m * n, SA.data_ptr(), SB.data_ptr(), 32 * kg, 32 * kg, sa_rows * kg,
                                sb_rows * kg, grid_blocks)
        st = L.gemm_a4w4_mxfp4_bpreshuffle(ctypes.byref(args), 1, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert st == 0
        torch.cuda.synchronize()
        for i, d in enumerate(data):
            assert_close(O.gemm_mx4(*d), C[i].float().cpu().numpy(), f"batch {i} grid {grid_blocks}")


def test_gemm_a4w4_rejects(qgemm, gpu):
    qa, qb, ea, eb = make_mx4(64, 256, 512, seed=1)
    A, B, SA, SB = _aiter_operands(qa, qb, ea, eb, gpu)
    with pytest.raises(ValueError):
        qgemm.gemm_a4w4(A, B[:250], SA, SB)                  # N % 16
    with pytest.raises(ValueError):
        qgemm.gemm_a4w4(A, B, SA[: SA.numel() // 2], SB)     # short scale tensor
    with pytest.raises(NotImplementedError):
        qgemm.gemm_a4w4(A, B, SA, SB, bias=torch.zeros(256, device=gpu))
    L = qgemm.lib()
    C = torch.empty(64, 256, dtype=torch.bfloat16, device=gpu)
    base = dict(m=64, n=256, k=512)
    def call(**kw):
        f = dict(base, **kw)
        args = qgemm.Mxfp4Kargs(A.data_ptr(), B.data_ptr(), kw.get("c", C.data_ptr()), f["m"], f["n"], f["k"], 1,
                                256, kw.get("stride_b", 256), 256, 0, 0, 0, SA.data_ptr(), SB.data_ptr(),
                                kw.get("stride_sf", 512), kw.get("stride_sf", 512), 0, 0, kw.get("grid", 0))
        return L.gemm_a4w4_mxfp4_bpreshuffle(ctypes.byref(args), 1, None)
    assert call() == 0
    torch.cuda.synchronize()
    assert call(k=384) == 1              # K % 256
    assert call(stride_b=512) == 1       # W16 B: stride_b must be K/2
    assert call(stride_sf=256) == 1      # scale block smaller than 32 rows x K/32
    assert call(grid=-1) == 1
    assert call(c=A.data_ptr()) == 1     # C overlapping A
