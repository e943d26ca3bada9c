"""GPU parity of the skinny-M / split-K kernel and the LDS-bypass entry
against the CPU oracle: decode shapes (M = 1 .. 256), N and M tails,
split-K on and off, batched calls through the C ABI, workspace re-arming
across calls, and B'' built on the host and on the GPU."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, make_bs, make_mx4, make_mx8, out_to_f32, to_dev

pytestmark = pytest.mark.gpu


def _fp8(x, dev):
    return to_dev(x, None, dev).view(torch.float8_e4m3fn)


# ----------------------------------------------------------------- MXFP8
# M <= 64 with too few N tiles for the skinny kernel runs the decode kernel
# (rows 1..64 in 1, 2 or 4 blocks; 64- or 128-column workgroups; split-K),
# the rest the skinny kernel
MX8_DECODE = [(1, 2112, 7168), (8, 1024, 2048), (16, 7168, 512), (17, 1000, 1024), (33, 4096, 1024),
              (64, 2112, 7168), (128, 1536, 2048), (256, 512, 1024),
              (1, 1536, 7168), (40, 1200, 4096), (64, 1536, 7168), (5, 300, 26624),
              (16, 24576, 1536), (40, 32768, 512)]


@pytest.mark.parametrize("m,n,k", MX8_DECODE)
@pytest.mark.parametrize("split", [True, False])
def test_mxfp8_skinny(qgemm, gpu, m, n, k, split):
    qa, qb, ea, eb = make_mx8(m, n, k, seed=11 * m + n + k)
    ref = O.gemm_mx8(qa, qb, ea, eb)
    y = qgemm.gemm_a8w8_mxfp8(_fp8(qa, gpu), _fp8(qb, gpu), to_dev(ea, None, gpu), to_dev(eb, None, gpu),
                              dtype=torch.bfloat16, workspace=None if split else False)
    assert_close(ref, out_to_f32(y), f"mxfp8 skinny {m}x{n}x{k} split={split}")


def test_mxfp8_skinny_k_pattern_fp32(qgemm, gpu):
    """Distinct per-K-group scales on both operands, fp32 output."""
    m, n, k = 8, 512, 2048
    qa, qb, ea, eb = make_mx8(m, n, k, seed=3)
    g = np.arange(k // 32)
    ea = np.broadcast_to((118 + g % 17).astype(np.uint8), ea.shape).copy()
    eb = np.broadcast_to((121 + (5 * g) % 11).astype(np.uint8), eb.shape).copy()
    ref = O.gemm_mx8(qa, qb, ea, eb)
    y = qgemm.gemm_a8w8_mxfp8(_fp8(qa, gpu), _fp8(qb, gpu), to_dev(ea, None, gpu), to_dev(eb, None, gpu),
                              dtype=torch.float32)
    assert_close(ref, out_to_f32(y), "mxfp8 skinny K-pattern")


def test_splitk_rearms_workspace(qgemm, gpu):
    """Three calls sharing one workspace (the counters must return to zero),
    the second with a smaller problem; results are bit-identical to a
    fresh run and within tolerance of the oracle."""
    shapes = [(4, 2048, 4096), (2, 1024, 2048), (1, 7168, 2048), (4, 2048, 4096)]
    ws = torch.zeros(1 << 22, dtype=torch.uint8, device=gpu)
    outs = []
    for i, (m, n, k) in enumerate(shapes):
        qa, qb, ea, eb = make_mx8(m, n, k, seed=100 + m)
        ref = O.gemm_mx8(qa, qb, ea, eb)
        y = qgemm.gemm_a8w8_mxfp8(_fp8(qa, gpu), _fp8(qb, gpu), to_dev(ea, None, gpu), to_dev(eb, None, gpu),
                                  dtype=torch.float32, workspace=ws)
        torch.cuda.synchronize()
        assert_close(ref, out_to_f32(y), f"call {i}")
        outs.append(y.cpu())
    assert torch.equal(outs[0], outs[3])
    # counters: the first 2048 bytes of the workspace
    assert int(ws[:2048].to(torch.int32).sum()) == 0, "split-K counters not re-armed"


# ----------------------------------------------------------------- MXFP4
# (16, 24576, 3072), (40, 16384, 2048): short K with >= 256 skinny tiles -> decode kernel
# (32, 7168, 16384), (64, 7168, 16384): configs[4] as benched (skinny MB2/NB2
# and MB4/NB2 with per-wave scale panels and nontemporal B)
MX4_DECODE = [(1, 2112, 7168), (4, 1000, 2048), (16, 4096, 512), (31, 512, 4096), (64, 7168, 1024),
              (200, 768, 1536), (8, 7168, 16384), (32, 2048, 16384), (16, 24576, 3072), (40, 16384, 2048),
              (32, 7168, 16384), (64, 7168, 16384), (128, 7168, 16384)]


@pytest.mark.parametrize("m,n,k", MX4_DECODE)
@pytest.mark.parametrize("split", [True, False])
def test_mxfp4_skinny(qgemm, gpu, m, n, k, split):
    qa, qb, ea, eb = make_mx4(m, n, k, seed=7 * m + k)
    ref = O.gemm_mx4(qa, qb, ea, eb)
    y = qgemm.gemm_a4w4_mxfp4(to_dev(qa, None, gpu), to_dev(qb, None, gpu), to_dev(ea, None, gpu),
                              to_dev(eb, None, gpu), dtype=torch.bfloat16, workspace=None if split else False)
    assert_close(ref, out_to_f32(y), f"mxfp4 skinny {m}x{n}x{k} split={split}")


@pytest.mark.parametrize("m,n,k", [(16, 2112, 7168), (5, 4096, 16384), (32, 1000, 4096)])
def test_mxfp4_skinny_k_pattern(qgemm, gpu, m, n, k):
    """Distinct per-K-group scales on both operands through the skinny
    kernel (per-wave scale panels and the interleaved path)."""
    qa, qb, ea, eb = make_mx4(m, n, k, seed=13)
    g = np.arange(k // 32)
    ea = np.broadcast_to((119 + g % 15).astype(np.uint8), ea.shape).copy()
    eb = np.broadcast_to((122 + (7 * g) % 9).astype(np.uint8), eb.shape).copy()
    ref = O.gemm_mx4(qa, qb, ea, eb)
    y = qgemm.gemm_a4w4_mxfp4(to_dev(qa, None, gpu), to_dev(qb, None, gpu), to_dev(ea, None, gpu),
                              to_dev(eb, None, gpu), dtype=torch.float32)
    assert_close(ref, out_to_f32(y), f"mxfp4 skinny K-pattern {m}x{n}x{k}")


# ----------------------------------------------- block-scale, fp32 scales
BS_DECODE = [(1, 2112, 7168), (1, 7168, 2048), (4, 24576, 1536), (32, 2112, 7168), (48, 300, 1024),
             (32, 1536, 7168), (64, 1536, 7168), (17, 1000, 4096), (2, 200, 26624),
             (64, 7168, 512), (128, 4096, 1024), (48, 7168, 8192)]


@pytest.mark.parametrize("m,n,k", BS_DECODE)
@pytest.mark.parametrize("sfa_layout", ["mk", "km"])
def test_blockscale_fp32_skinny(qgemm, gpu, m, n, k, sfa_layout):
    qa, qb, sa, sb = make_bs(m, n, k, seed=5 * m + n)
    ref = O.gemm_bs_fp32(qa, qb, sa, sb)
    Bk = qgemm.shuffle_b_kpanel(to_dev(qb, None, gpu)).view(torch.float8_e4m3fn)
    A_scale = to_dev(sa, None, gpu) if sfa_layout == "mk" else to_dev(np.ascontiguousarray(sa.T), None, gpu).t()
    y = qgemm.gemm_a8w8_bpreshuffle(_fp8(qa, gpu), Bk, A_scale, to_dev(sb, None, gpu), dtype=torch.bfloat16)
    assert_close(ref, out_to_f32(y), f"bs-fp32 skinny {m}x{n}x{k} {sfa_layout}")


# ----------------------------------------------- LDS bypass (B'')
def test_ldsbypass_repack_matches_host_pack(qgemm, gpu):
    for n, k in [(2112, 1024), (100, 256), (16, 128), (7168, 512)]:
        b = np.random.default_rng(n + k).integers(0, 256, (n, k), dtype=np.uint8)
        host = qgemm.ldsbypass_pack_b(torch.from_numpy(b))
        Bk = qgemm.shuffle_b_kpanel(to_dev(b, None, gpu))
        dev = qgemm.ldsbypass_repack(Bk)
        torch.cuda.synchronize()
        assert torch.equal(host, dev.cpu()), f"repack != host pack for N={n} K={k}"


# (32, 1536, 7168): configs[0] as the ldsbypass_c0 bench workload runs it
LBP_SHAPES = [(1, 2112, 7168), (16, 1536, 1024), (37, 100, 512), (64, 7168, 1024), (256, 512, 768),
              (300, 520, 384), (600, 384, 256), (32, 1536, 7168), (24, 1536, 7168)]


@pytest.mark.parametrize("m,n,k", LBP_SHAPES)
@pytest.mark.parametrize("sfa_layout", ["mk", "km"])
@pytest.mark.parametrize("split", [True, False])
def test_ldsbypass(qgemm, gpu, m, n, k, sfa_layout, split):
    qa, qb, sa, sb = make_bs(m, n, k, seed=m + 3 * n + k)
    ref = O.gemm_bs_fp32(qa, qb, sa, sb)
    Bpp = qgemm.ldsbypass_repack(qgemm.shuffle_b_kpanel(to_dev(qb, None, gpu)))
    A_scale = to_dev(sa, None, gpu) if sfa_layout == "mk" else to_dev(np.ascontiguousarray(sa.T), None, gpu).t()
    y = qgemm.gemm_a8w8_ldsbypass(_fp8(qa, gpu), Bpp, A_scale, to_dev(sb, None, gpu), n, dtype=torch.bfloat16,
                                  workspace=None if split else False)
    assert_close(ref, out_to_f32(y), f"ldsbypass {m}x{n}x{k} {sfa_layout} split={split}")


# tile-kernel cases of the LDS-bypass entry (M > 256: B'' blocks staged
# through LDS): one K-tile, odd K-tile counts, ragged tiles, fp32 output
@pytest.mark.parametrize("m,n,k", [(520, 300, 128), (264, 1000, 640), (512, 512, 1408), (768, 256, 256),
                                   (130, 1000, 7168), (4096, 4096, 384)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_ldsbypass_tile(qgemm, gpu, m, n, k, dtype):
    qa, qb, sa, sb = make_bs(m, n, k, seed=5 * m + n + k)
    ref = O.gemm_bs_fp32(qa, qb, sa, sb)
    Bpp = qgemm.ldsbypass_repack(qgemm.shuffle_b_kpanel(to_dev(qb, None, gpu)))
    y = qgemm.gemm_a8w8_ldsbypass(_fp8(qa, gpu), Bpp, to_dev(sa, None, gpu), to_dev(sb, None, gpu), n, dtype=dtype)
    assert_close(ref, out_to_f32(y), f"ldsbypass tile {m}x{n}x{k} {dtype}")


# ----------------------------------------------- batched calls (C ABI)
def _call(qgemm, name, args, out_code, ws):
    L = qgemm.lib()
    need = getattr(L, name + "_workspace_bytes")(ctypes.byref(args))
    ws_ptr = ws.data_ptr() if (ws is not None and need) else None
    st = getattr(L, name)(ctypes.byref(args), out_code, ws_ptr, ws.numel() if ws_ptr else 0,
                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, f"{name} returned {st}"
    torch.cuda.synchronize()


@pytest.mark.parametrize("m,n,k", [(3, 1000, 1024), (40, 512, 2048), (300, 300, 256)])
def test_mxfp8_batched(qgemm, gpu, m, n, k):
    batch = 3
    data = [make_mx8(m, n, k, seed=50 + i) for i in range(batch)]
    A = torch.stack([torch.from_numpy(d[0]) for d in data]).to(gpu)
    B = torch.stack([torch.from_numpy(d[1]) for d in data]).to(gpu)
    SA = torch.stack([torch.from_numpy(d[2]) for d in data]).to(gpu)
    SB = torch.stack([torch.from_numpy(d[3]) for d in data]).to(gpu)
    C = torch.empty(batch, m, n, dtype=torch.float32, device=gpu)
    kg = k // 32
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, batch, k, k, n, m * k, n * k, m * n,
                       SA.data_ptr(), SB.data_ptr(), kg, kg, m * kg, n * kg)
    ws = torch.zeros(1 << 24, dtype=torch.uint8, device=gpu)
    _call(qgemm, "gemm_a8w8_mxfp8", args, qgemm.OUT_FP32, ws)
    for i, d in enumerate(data):
        assert_close(O.gemm_mx8(*d), C[i].cpu().numpy(), f"batch {i}")


@pytest.mark.parametrize("m,n,k", [(1, 2112, 2048), (24, 640, 1024), (300, 520, 384), (300, 520, 2048)])
def test_blockscale_fp32_batched(qgemm, gpu, m, n, k):
    batch = 2
    data = [make_bs(m, n, k, seed=70 + i) for i in range(batch)]
    kg, nbk = k // 128, (n + 127) // 128
    A = torch.stack([torch.from_numpy(d[0]) for d in data]).to(gpu)
    Bk = torch.stack([qgemm.shuffle_b_kpanel(torch.from_numpy(d[1])) for d in data]).to(gpu)
    SA = torch.stack([torch.from_numpy(d[2]) for d in data]).to(gpu)        # row-major [M][K/128]
    SB = torch.stack([torch.from_numpy(d[3]) for d in data]).to(gpu)
    C = torch.empty(batch, m, n, dtype=torch.bfloat16, device=gpu)
    args = qgemm.Kargs(A.data_ptr(), Bk.data_ptr(), C.data_ptr(), m, n, k, batch, k, 128, n, m * k, n * k, m * n,
                       SA.data_ptr(), SB.data_ptr(), 1 if m > 1 else m, kg, m * kg, nbk * kg)
    ws = torch.zeros(1 << 24, dtype=torch.uint8, device=gpu)
    _call(qgemm, "gemm_a8w8_blockscale_bpreshuffle", args, qgemm.OUT_BF16, ws)
    for i, d in enumerate(data):
        assert_close(O.gemm_bs_fp32(*d), C[i].float().cpu().numpy(), f"batch {i}")
