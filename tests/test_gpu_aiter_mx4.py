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
    """kernel_id 0: the library's choice (the burst kernel for decode M,
    else the one-by-four wave kernel); 1: the two-by-two wave kernel."""
    qa, qb, ea, eb = make_mx4(m, n, k, seed=m + 3 * n + k)
    A, B, SA, SB = _aiter_operands(qa, qb, ea, eb, gpu)
    y = qgemm.gemm_a4w4(A, B, SA, SB, dtype=dtype, kernel_id=kernel_id)
    pb = 32 if k % 1024 == 0 else 8
    f = "bf16" if dtype == torch.bfloat16 else "fp32"
    trace = qgemm.last_launch()
    if kernel_id == 1:
        assert trace == f"wide_gemm<fp4,MXS,W16,{f},pb{pb}>", trace
    elif m <= 64:
        assert trace.startswith(("burst_gemm<fp4,MXS,FRAG,", "quad_gemm<fp4,MXS,W16,", "slice_gemm<fp4,MXS,W16,")), \
            trace
    else:    # (split over K into fp32 planes where the tiles leave most CUs idle)
        assert trace == f"quad_gemm<fp4,MXS,W16,{f}>" or \
            trace.startswith(f"quad_gemm<fp4,MXS,W16,fp32>+splitk_reduce<{f},"), trace
    assert_close(O.gemm_mx4(qa, qb, ea, eb), out_to_f32(y), f"a4w4 bpreshuffle {m}x{n}x{k} ({trace})")


# decode shapes on the burst kernel (W16 B streamed as the 16x16x128 MFMA's
# 1 KB operands, e8m0_shuffle scales picked by byte): row counts across the
# 16 / 32 / 64-row tiles, unsplit and K split over workgroups (configs[4]'s
# N = 7168, K = 16384), a workspace of garbage, and no workspace
DECODE = [(1, 1024, 1024), (8, 512, 8192), (16, 7168, 2048), (17, 2112, 7168), (32, 4096, 4096),
          (33, 4096, 256), (48, 1536, 7168), (64, 7168, 2048), (32, 7168, 16384), (1, 7168, 16384)]


@pytest.mark.parametrize("m,n,k", DECODE)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gemm_a4w4_decode_burst(qgemm, gpu, m, n, k, dtype):
    qa, qb, ea, eb = make_mx4(m, n, k, seed=5 * m + n + k)
    A, B, SA, SB = _aiter_operands(qa, qb, ea, eb, gpu)
    ref = O.gemm_mx4(qa, qb, ea, eb)
    args = qgemm.Mxfp4Kargs(A.data_ptr(), B.data_ptr(), 0, m, n, k, 1, k // 2, k // 2, n, 0, 0, 0, SA.data_ptr(),
                            SB.data_ptr(), k, k, 0, 0, 0)
    need = qgemm.lib().gemm_a4w4_mxfp4_bpreshuffle_kid_workspace_bytes(ctypes.byref(args), 5)
    junk = torch.full((max(need, 256),), 0xFF, dtype=torch.uint8, device=gpu)
    y = qgemm.gemm_a4w4(A, B, SA, SB, dtype=dtype, kernel_id=5, workspace=junk)
    trace = qgemm.last_launch()
    assert trace.startswith("burst_gemm<fp4,MXS,FRAG,"), trace
    assert_close(ref, out_to_f32(y), f"a4w4 decode {m}x{n}x{k} ({trace})")
    y2 = qgemm.gemm_a4w4(A, B, SA, SB, dtype=dtype, kernel_id=5, workspace=junk)
    torch.cuda.synchronize()
    assert torch.equal(y, y2), f"two calls differ ({trace})"
    # the library's choice: the slice kernel where its plan fills the CUs in
    # one round, else the burst kernel where its plan gate accepts the shape
    y0 = qgemm.gemm_a4w4(A, B, SA, SB, dtype=dtype)
    trace0 = qgemm.last_launch()
    assert trace0.startswith(("burst_gemm<fp4,MXS,FRAG,", "quad_gemm<fp4,MXS,W16,", "slice_gemm<fp4,MXS,W16,")), \
        trace0
    assert_close(ref, out_to_f32(y0), f"a4w4 decode auto {m}x{n}x{k} ({trace0})")
    # no workspace: an unsplit plan, or refused when K needs a split
    try:
        yn = qgemm.gemm_a4w4(A, B, SA, SB, dtype=dtype, kernel_id=5, workspace=False)
    except RuntimeError as e:
        assert "HIP error 1" in str(e) and need > 0, (trace, str(e))
    else:
        tn = qgemm.last_launch()
        assert tn.endswith(",splitk1>"), tn
        assert_close(ref, out_to_f32(yn), f"a4w4 decode unsplit {m}x{n}x{k} ({tn})")
    # the plain entry (no workspace) always answers: burst unsplit or the tile kernel
    yp = torch.empty_like(y)
    st = qgemm.lib().gemm_a4w4_mxfp4_bpreshuffle(ctypes.byref(qgemm.Mxfp4Kargs(
        A.data_ptr(), B.data_ptr(), yp.data_ptr(), m, n, k, 1, k // 2, k // 2, n, 0, 0, 0, SA.data_ptr(),
        SB.data_ptr(), k, k, 0, 0, 0)), 1 if dtype == torch.bfloat16 else 0,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0
    torch.cuda.synchronize()
    assert_close(ref, out_to_f32(yp), f"a4w4 decode plain entry {m}x{n}x{k} ({qgemm.last_launch()})")


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


# middle M: the one-by-four wave kernel split over K (slices as batch
# entries into fp32 partial planes, summed by the split-K reduce) where its
# 256 x 256 tiles would leave most CUs idle
MIDDLE = [(128, 7168, 16384), (96, 2112, 7168), (256, 4096, 7168), (200, 1536, 2048), (256, 2112, 4096)]


@pytest.mark.parametrize("m,n,k", MIDDLE)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gemm_a4w4_middle_m_split(qgemm, gpu, m, n, k, dtype):
    qa, qb, ea, eb = make_mx4(m, n, k, seed=3 * m + n + 7 * k)
    A, B, SA, SB = _aiter_operands(qa, qb, ea, eb, gpu)
    ref = O.gemm_mx4(qa, qb, ea, eb)
    y = qgemm.gemm_a4w4(A, B, SA, SB, dtype=dtype)
    trace = qgemm.last_launch()
    assert trace.startswith("quad_gemm<fp4,MXS,W16,fp32>+splitk_reduce"), trace
    assert_close(ref, out_to_f32(y), f"a4w4 middle {m}x{n}x{k} ({trace})")
    # without a workspace the unsplit kernel, the same sums in another order
    y0 = qgemm.gemm_a4w4(A, B, SA, SB, dtype=dtype, workspace=False)
    t0 = qgemm.last_launch()
    assert t0.startswith("quad_gemm<fp4,MXS,W16,") and "splitk" not in t0, t0
    assert_close(ref, out_to_f32(y0), f"a4w4 middle unsplit {m}x{n}x{k} ({t0})")


# the slice kernel on aiter's operands (W16 B: each fragment load one 1 KB
# run; e8m0_shuffle scales: A's slice of them in LDS as they lie, B's dword
# per K-tile with its fragments): row counts across its 16 / 32 / 64-row
# plans and 32-row scale-block halves, N % 32 == 16 (a 16-row block whose
# 32-row scale block is half used), K slices past the end, K split over
# workgroups with a workspace of garbage, and configs[4]'s shapes
SLICE = [(9, 4096, 4096), (16, 7168, 16384), (17, 2064, 8192), (32, 7168, 16384), (33, 1040, 4096),
         (48, 4096, 6144), (64, 7168, 16384), (64, 3088, 2304), (12, 700 - 700 % 16, 14336)]


_SLICE_REF = {}


@pytest.mark.parametrize("m,n,k", SLICE)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gemm_a4w4_slice(qgemm, gpu, m, n, k, dtype):
    qa, qb, ea, eb = make_mx4(m, n, k, seed=11 * m + n + k)
    A, B, SA, SB = _aiter_operands(qa, qb, ea, eb, gpu)
    if (m, n, k) not in _SLICE_REF:    # the oracle once per shape (both output types)
        _SLICE_REF[(m, n, k)] = O.gemm_mx4(qa, qb, ea, eb)
    ref = _SLICE_REF[(m, n, k)]
    args = qgemm.Mxfp4Kargs(A.data_ptr(), B.data_ptr(), 0, m, n, k, 1, k // 2, k // 2, n, 0, 0, 0, SA.data_ptr(),
                            SB.data_ptr(), k, k, 0, 0, 0)
    need = qgemm.lib().gemm_a4w4_mxfp4_bpreshuffle_kid_workspace_bytes(ctypes.byref(args), 10)
    junk = torch.full((max(need, 256),), 0xFF, dtype=torch.uint8, device=gpu)
    y = qgemm.gemm_a4w4(A, B, SA, SB, dtype=dtype, kernel_id=10, workspace=junk)
    trace = qgemm.last_launch()
    assert trace.startswith("slice_gemm<fp4,MXS,W16,"), trace
    assert (need > 0) == (not trace.endswith(",splitk1>")), (need, trace)
    assert_close(ref, out_to_f32(y), f"a4w4 slice {m}x{n}x{k} ({trace})")
    y2 = qgemm.gemm_a4w4(A, B, SA, SB, dtype=dtype, kernel_id=10, workspace=junk)
    torch.cuda.synchronize()
    assert torch.equal(y, y2), f"two calls differ ({trace})"
    if need:    # the plan's counter words (one per 16 * nbw-column tile) re-armed to zero
        nbw = 2 if m <= 16 else (4 if m <= 32 else 8)
        tiles = -(-n // (16 * nbw))
        assert int(junk[:4 * tiles].to(torch.int32).sum()) == 0, "split-K counters not re-armed"
    # no workspace: refused when K needs a split
    try:
        yn = qgemm.gemm_a4w4(A, B, SA, SB, dtype=dtype, kernel_id=10, workspace=False)
    except RuntimeError as e:
        assert "HIP error 1" in str(e) and need > 0, (trace, str(e))
    else:
        assert need == 0 and torch.equal(yn, y), trace


def test_gemm_a4w4_slice_matches_row_major(qgemm, gpu):
    """configs[4] M = 64 on both MXFP4 entries' slice kernels: the same bits
    (same products, same order of sums)."""
    m, n, k = 64, 7168, 16384
    qa, qb, ea, eb = make_mx4(m, n, k, seed=99)
    A, B, SA, SB = _aiter_operands(qa, qb, ea, eb, gpu)
    ya = qgemm.gemm_a4w4(A, B, SA, SB, kernel_id=10)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)
    yr = qgemm.gemm_a4w4_mxfp4(dev(qa), dev(qb), dev(ea), dev(eb))
    assert qgemm.last_launch().startswith("slice_gemm<fp4,MX,RAW,mb4"), qgemm.last_launch()
    assert torch.equal(ya, yr)


@pytest.mark.parametrize("m,n,k", [(32, 2064, 4096), (48, 1024, 6144)])
def test_gemm_a4w4_slice_batched_c_abi(qgemm, gpu, m, n, k):
    """Batch 2 on the slice kernel (kernel id 10) through the C ABI, padded
    A-scale batch strides; (48, 1024, 6144) splits K in two (a workspace of
    garbage), (32, 2064, 4096) runs unsplit with a half-used last scale
    block."""
    batch = 2
    data = [make_mx4(m, n, k, seed=70 + i + m) for i in range(batch)]
    kb, kg = k // 2, k // 32
    A = torch.stack([torch.from_numpy(d[0]) for d in data]).to(gpu)
    B = torch.stack([torch.from_numpy(O.shuffle_weight_16x16(d[1])) for d in data]).to(gpu)
    sa_rows, sb_rows = (m + 31) // 32 * 32 + 32, (n + 31) // 32 * 32
    SA = torch.full((batch, sa_rows * kg), 0x7F, dtype=torch.uint8)
    SB = torch.empty((batch, sb_rows * kg), dtype=torch.uint8)
    for i, d in enumerate(data):
        sa = O.e8m0_shuffle(d[2]).reshape(-1)
        SA[i, :sa.size] = torch.from_numpy(sa)
        SB[i] = torch.from_numpy(O.e8m0_shuffle(d[3]).reshape(-1))
    SA, SB = SA.to(gpu), SB.to(gpu)
    L = qgemm.lib()
    C = torch.full((batch, m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
    args = qgemm.Mxfp4Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, batch, kb, kb, n, m * kb, n * kb,
                            m * n, SA.data_ptr(), SB.data_ptr(), 32 * kg, 32 * kg, sa_rows * kg, sb_rows * kg, 0)
    need = L.gemm_a4w4_mxfp4_bpreshuffle_kid_workspace_bytes(ctypes.byref(args), 10)
    junk = torch.full((max(need, 256),), 0xA5, dtype=torch.uint8, device=gpu)
    st = L.gemm_a4w4_mxfp4_bpreshuffle_kid(ctypes.byref(args), 1, 10, ctypes.c_void_p(junk.data_ptr()), junk.numel(),
                                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0
    torch.cuda.synchronize()
    trace = qgemm.last_launch()
    assert trace.startswith("slice_gemm<fp4,MXS,W16,"), trace
    assert (need > 0) == (not trace.endswith(",splitk1>")), (need, trace)
    for i, d in enumerate(data):
        assert_close(O.gemm_mx4(*d), C[i].float().cpu().numpy(), f"slice batch {i} {m}x{n}x{k} ({trace})")
