"""GPU parity of the row-streaming decode kernel (MXFP8 / MXFP4 with M <= 8,
row-major B) against the CPU oracle: partial last pieces (K not a multiple
of the segment), the largest K the kernel holds in LDS, N tails that cut a
workgroup's last group of 2 or 4 rows, every M from 1 to 8 (1, 2 or 4 rows
of B per MFMA), per-K-group scale patterns on both operands (which pin the
lane -> E8M0 group routing of both formats), padded strides with batching
through the C ABI, fp32 and bf16 outputs, and bit-identical repeated
calls."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, make_mx4, make_mx8, out_to_f32, to_dev

pytestmark = pytest.mark.gpu


def _fp8(x, dev):
    return to_dev(x, None, dev).view(torch.float8_e4m3fn)


# (m, n, k): K = 16384 is configs[4] and the largest K the kernel holds in LDS
# without a K split; 7168 and 2304 end in a partial segment, 256 / 128 are a
# single partial segment
MX4_STREAM = [(1, 7168, 16384), (8, 7168, 16384), (3, 1000, 7168), (5, 4100, 256), (2, 512, 32768),
              (7, 257, 2304), (4, 2048, 4096), (6, 300, 1024)]
MX8_STREAM = [(1, 7168, 16384), (8, 2112, 7168), (6, 300, 128), (1, 4096, 2048), (2, 1536, 7168),
              (3, 777, 640), (5, 7168, 2048), (4, 2560, 16384)]


@pytest.mark.parametrize("m,n,k", MX4_STREAM)
def test_mxfp4_stream(qgemm, gpu, m, n, k):
    qa, qb, ea, eb = make_mx4(m, n, k, seed=7 * m + n + k)
    ref = O.gemm_mx4(qa, qb, ea, eb)
    y = qgemm.gemm_a4w4_mxfp4(to_dev(qa, None, gpu), to_dev(qb, None, gpu), to_dev(ea, None, gpu),
                              to_dev(eb, None, gpu), dtype=torch.bfloat16)
    assert_close(ref, out_to_f32(y), f"mxfp4 stream {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", MX8_STREAM)
def test_mxfp8_stream(qgemm, gpu, m, n, k):
    qa, qb, ea, eb = make_mx8(m, n, k, seed=5 * m + n + k)
    ref = O.gemm_mx8(qa, qb, ea, eb)
    y = qgemm.gemm_a8w8_mxfp8(_fp8(qa, gpu), _fp8(qb, gpu), to_dev(ea, None, gpu), to_dev(eb, None, gpu),
                              dtype=torch.bfloat16)
    assert_close(ref, out_to_f32(y), f"mxfp8 stream {m}x{n}x{k}")


@pytest.mark.parametrize("m", range(1, 9))
def test_stream_every_m(qgemm, gpu, m):
    n, k = 640, 6144
    qa, qb, ea, eb = make_mx4(m, n, k, seed=90 + m)
    y = qgemm.gemm_a4w4_mxfp4(to_dev(qa, None, gpu), to_dev(qb, None, gpu), to_dev(ea, None, gpu),
                              to_dev(eb, None, gpu), dtype=torch.float32)
    assert_close(O.gemm_mx4(qa, qb, ea, eb), out_to_f32(y), f"mxfp4 stream m={m}")
    qa, qb, ea, eb = make_mx8(m, n, k, seed=190 + m)
    y = qgemm.gemm_a8w8_mxfp8(_fp8(qa, gpu), _fp8(qb, gpu), to_dev(ea, None, gpu), to_dev(eb, None, gpu),
                              dtype=torch.float32)
    assert_close(O.gemm_mx8(qa, qb, ea, eb), out_to_f32(y), f"mxfp8 stream m={m}")


def _k_pattern(ea, eb):
    g = np.arange(ea.shape[1])
    ea = np.broadcast_to((116 + g % 19).astype(np.uint8), ea.shape).copy()
    eb = np.broadcast_to((120 + (7 * g) % 13).astype(np.uint8), eb.shape).copy()
    return ea, eb


@pytest.mark.parametrize("k", [4096, 7168])
@pytest.mark.parametrize("m", [1, 2, 3])
def test_stream_k_pattern_scales(qgemm, gpu, m, k):
    """Distinct E8M0 per K group on both operands, for 1, 2 and 4 rows of B
    per MFMA: a lane whose data and scale byte come from different groups
    scales products by the wrong power of two, far outside the tolerance."""
    n = 768
    qa, qb, ea, eb = make_mx4(m, n, k, seed=k + 1)
    ea, eb = _k_pattern(ea, eb)
    y = qgemm.gemm_a4w4_mxfp4(to_dev(qa, None, gpu), to_dev(qb, None, gpu), to_dev(ea, None, gpu),
                              to_dev(eb, None, gpu), dtype=torch.float32)
    assert_close(O.gemm_mx4(qa, qb, ea, eb), out_to_f32(y), "mxfp4 stream K-pattern")
    qa, qb, ea, eb = make_mx8(m, n, k, seed=k + 2)
    ea, eb = _k_pattern(ea, eb)
    y = qgemm.gemm_a8w8_mxfp8(_fp8(qa, gpu), _fp8(qb, gpu), to_dev(ea, None, gpu), to_dev(eb, None, gpu),
                              dtype=torch.float32)
    assert_close(O.gemm_mx8(qa, qb, ea, eb), out_to_f32(y), "mxfp8 stream K-pattern")


def _padded(rows, cols, pitch, batch, fill, arrays):
    out = np.full((batch, rows, pitch), fill, dtype=np.uint8)
    for i, a in enumerate(arrays):
        out[i, :, :cols] = a
    return out


@pytest.mark.parametrize("fp4", [True, False])
def test_stream_batched_strided(qgemm, gpu, fp4):
    """Batch of 2 through the C ABI with padded row pitches on A, B, both
    scale arrays and C (padding bytes are NaN codes / 0xFF scales that must
    never be read)."""
    m, n, k, batch = 5, 1100, 5120, 2
    make = make_mx4 if fp4 else make_mx8
    data = [make(m, n, k, seed=300 + i + 10 * fp4) for i in range(batch)]
    kb = k // 2 if fp4 else k
    kg = k // 32
    lda, ldb, lsa, lsb, ldc = kb + 48, kb + 128, kg + 12, kg + 8, n + 24    # scale pitches: multiples of 4
    A = torch.from_numpy(_padded(m, kb, lda, batch, 0xFF, [d[0] for d in data])).to(gpu)
    B = torch.from_numpy(_padded(n, kb, ldb, batch, 0xFF, [d[1] for d in data])).to(gpu)
    SA = torch.from_numpy(_padded(m, kg, lsa, batch, 0xFF, [d[2] for d in data])).to(gpu)
    SB = torch.from_numpy(_padded(n, kg, lsb, batch, 0xFF, [d[3] for d in data])).to(gpu)
    C = torch.zeros(batch, m, ldc, dtype=torch.float32, device=gpu)
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, batch, lda, ldb, ldc, m * lda, n * ldb,
                       m * ldc, SA.data_ptr(), SB.data_ptr(), lsa, lsb, m * lsa, n * lsb)
    name = "gemm_a4w4_mxfp4" if fp4 else "gemm_a8w8_mxfp8"
    L = qgemm.lib()
    st = getattr(L, name)(ctypes.byref(args), qgemm.OUT_FP32, None, 0,
                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, f"{name} returned {st}"
    torch.cuda.synchronize()
    gemm = O.gemm_mx4 if fp4 else O.gemm_mx8
    Cc = C.cpu().numpy()
    for i, d in enumerate(data):
        assert_close(gemm(*d), Cc[i, :, :n], f"batch {i}")
        assert not Cc[i, :, n:].any(), "wrote past N"


def test_stream_deterministic(qgemm, gpu):
    m, n, k = 8, 7168, 16384
    qa, qb, ea, eb = make_mx4(m, n, k, seed=5)
    args = [to_dev(x, None, gpu) for x in (qa, qb, ea, eb)]
    y0 = qgemm.gemm_a4w4_mxfp4(*args, dtype=torch.float32)
    y1 = qgemm.gemm_a4w4_mxfp4(*args, dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)


# K split over workgroups: A's LDS image holds 16384 K elements per row;
# longer K (uneven last slices, partial segments)
MX4_SPLIT = [(1, 512, 32768), (8, 2048, 32768), (5, 1000, 24576), (2, 3000, 40960), (3, 777, 17152)]
MX8_SPLIT = [(3, 1024, 24576), (8, 2560, 32768), (1, 1536, 20480), (6, 777, 17408)]


@pytest.mark.parametrize("m,n,k", MX4_SPLIT)
def test_mxfp4_stream_split(qgemm, gpu, m, n, k):
    qa, qb, ea, eb = make_mx4(m, n, k, seed=3 * m + n + k)
    y = qgemm.gemm_a4w4_mxfp4(to_dev(qa, None, gpu), to_dev(qb, None, gpu), to_dev(ea, None, gpu),
                              to_dev(eb, None, gpu), dtype=torch.bfloat16)
    assert_close(O.gemm_mx4(qa, qb, ea, eb), out_to_f32(y), f"mxfp4 stream split {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", MX8_SPLIT)
def test_mxfp8_stream_split(qgemm, gpu, m, n, k):
    qa, qb, ea, eb = make_mx8(m, n, k, seed=9 * m + n + k)
    y = qgemm.gemm_a8w8_mxfp8(_fp8(qa, gpu), _fp8(qb, gpu), to_dev(ea, None, gpu), to_dev(eb, None, gpu),
                              dtype=torch.float32)
    assert_close(O.gemm_mx8(qa, qb, ea, eb), out_to_f32(y), f"mxfp8 stream split {m}x{n}x{k}")


def test_stream_split_without_workspace(qgemm, gpu):
    """No workspace: the call runs the skinny kernel without a K split."""
    m, n, k = 4, 2048, 32768
    qa, qb, ea, eb = make_mx4(m, n, k, seed=77)
    y = qgemm.gemm_a4w4_mxfp4(to_dev(qa, None, gpu), to_dev(qb, None, gpu), to_dev(ea, None, gpu),
                              to_dev(eb, None, gpu), dtype=torch.float32, workspace=False)
    assert_close(O.gemm_mx4(qa, qb, ea, eb), out_to_f32(y), "no workspace")


def test_stream_split_rearms_workspace(qgemm, gpu):
    """Calls sharing one workspace, the second with a smaller problem and a
    batch of 2: results within tolerance, the repeat bit-identical, the
    counters back at zero."""
    ws = torch.zeros(1 << 24, dtype=torch.uint8, device=gpu)
    outs = []
    for i, (m, n, k) in enumerate([(8, 4096, 32768), (5, 1024, 24576), (8, 4096, 32768)]):
        qa, qb, ea, eb = make_mx4(m, n, k, seed=400 + m)
        y = qgemm.gemm_a4w4_mxfp4(to_dev(qa, None, gpu), to_dev(qb, None, gpu), to_dev(ea, None, gpu),
                                  to_dev(eb, None, gpu), dtype=torch.float32, workspace=ws)
        torch.cuda.synchronize()
        assert_close(O.gemm_mx4(qa, qb, ea, eb), out_to_f32(y), f"call {i}")
        outs.append(y.cpu())
    assert torch.equal(outs[0], outs[2])
    assert int(ws[:2048].to(torch.int32).sum()) == 0, "stream split counters not re-armed"

    m, n, k, batch = 6, 1100, 32768, 2
    data = [make_mx4(m, n, k, seed=500 + i) for i in range(batch)]
    A = torch.stack([torch.from_numpy(d[0]) for d in data]).to(gpu)
    B = torch.stack([torch.from_numpy(d[1]) for d in data]).to(gpu)
    SA = torch.stack([torch.from_numpy(d[2]) for d in data]).to(gpu)
    SB = torch.stack([torch.from_numpy(d[3]) for d in data]).to(gpu)
    C = torch.empty(batch, m, n, dtype=torch.bfloat16, device=gpu)
    kb, kg = k // 2, k // 32
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, batch, kb, kb, n, m * kb, n * kb, m * n,
                       SA.data_ptr(), SB.data_ptr(), kg, kg, m * kg, n * kg)
    L = qgemm.lib()
    need = L.gemm_a4w4_mxfp4_workspace_bytes(ctypes.byref(args))
    assert 0 < need <= ws.numel()
    st = L.gemm_a4w4_mxfp4(ctypes.byref(args), qgemm.OUT_BF16, ws.data_ptr(), ws.numel(),
                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0
    torch.cuda.synchronize()
    for i, d in enumerate(data):
        assert_close(O.gemm_mx4(*d), out_to_f32(C[i]), f"batched split {i}")
    assert int(ws[:2048].to(torch.int32).sum()) == 0


@pytest.mark.parametrize("m,n", [(8, 256), (8, 255), (9, 256), (1, 255)])
def test_stream_routing_boundaries(qgemm, gpu, m, n):
    """Both sides of the stream kernel's limits (M <= 8, N >= 256) give the
    oracle's result."""
    k = 4096
    qa, qb, ea, eb = make_mx4(m, n, k, seed=m * 1000 + n)
    y = qgemm.gemm_a4w4_mxfp4(to_dev(qa, None, gpu), to_dev(qb, None, gpu), to_dev(ea, None, gpu),
                              to_dev(eb, None, gpu), dtype=torch.float32)
    assert_close(O.gemm_mx4(qa, qb, ea, eb), out_to_f32(y), f"mxfp4 {m}x{n}x{k}")
    qa, qb, ea, eb = make_mx8(m, n, k, seed=m * 1000 + n + 1)
    y = qgemm.gemm_a8w8_mxfp8(_fp8(qa, gpu), _fp8(qb, gpu), to_dev(ea, None, gpu), to_dev(eb, None, gpu),
                              dtype=torch.float32)
    assert_close(O.gemm_mx8(qa, qb, ea, eb), out_to_f32(y), f"mxfp8 {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,workspace,expect", [
    (4, 7168, None, "stream_gemm<fp4,wr4,mb4,fp32,splitk2>"),
    (4, 7168, False, "skinny_gemm<fp4"),
    (4, 32768, None, "skinny_gemm<fp4"),
    (16, 32768, None, "skinny_gemm<fp4"),
])
def test_long_k_routes(qgemm, gpu, m, n, workspace, expect):
    """K = 16640: 65 fp4 K-tiles (past the burst kernel's 32) and 8320 bytes
    per row (past the 8 KB of a row the row-streaming kernel's LDS holds).
    M = 4, N = 7168: the row-streaming kernel splits K in two with a
    workspace, and without one the skinny kernel runs unsplit.  N = 32768
    (128 tiles of 256 x 256): the streaming split would need more counters
    than it has, and M <= 16 runs the skinny kernel, not 256-row tiles.
    Random fp4 codes and E8M0 bytes keep the host arrays small; 4096
    sampled outputs against the oracle."""
    k = 16640
    rng = np.random.default_rng(5 + m + n)
    qa = rng.integers(0, 256, (m, k // 2), dtype=np.uint8)
    qb = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    ea = rng.integers(120, 135, (m, k // 32), dtype=np.uint8)
    eb = rng.integers(120, 135, (n, k // 32), dtype=np.uint8)
    dev = lambda x: torch.from_numpy(x).to(gpu)
    y = qgemm.gemm_a4w4_mxfp4(dev(qa), dev(qb), dev(ea), dev(eb), dtype=torch.float32, workspace=workspace)
    assert qgemm.last_launch().startswith(expect), qgemm.last_launch()
    torch.cuda.synchronize()
    rows = rng.integers(0, m, 4096).astype(np.int32)
    cols = rng.integers(0, n, 4096).astype(np.int32)
    ref = O.gemm_mx4_points(qa, qb, ea, eb, rows, cols)
    assert_close(ref, y.cpu().numpy()[rows, cols], f"M={m} N={n} K={k} workspace={workspace}")
