"""GPU parity of every entry point against the CPU oracle (seeded inputs,
BASELINE tolerance |y-y_ref| <= 2^-7|y_ref| + 1e-3 rms(y_ref))."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, make_bs, make_mx4, make_mx8, out_to_f32, to_dev

pytestmark = pytest.mark.gpu


# ----------------------------------------------------------------- probes
def test_probe_known_answers(qgemm, gpu):
    w = qgemm.probe_mfma_layout(gpu).numpy()
    lanes = np.arange(64)
    # srcA row index i and srcB column index j of every (lane, reg) output.
    i_of = w[0:256].reshape(64, 4) - 1
    j_of = w[256:512].reshape(64, 4) - 1
    exp_i = (4 * (lanes // 16))[:, None] + np.arange(4)[None, :]
    exp_j = np.repeat((lanes % 16)[:, None], 4, axis=1)
    assert np.array_equal(i_of, exp_i), f"srcA-row map {i_of}"
    assert np.array_equal(j_of, exp_j), f"srcB-col map {j_of}"
    # reference known answers: 480 (per-K-block scales), 128 (op_sel byte 1)
    assert np.all(w[512:768] == 480)
    assert np.all(w[768:1024] == 128)
    # single-lane scale boost: +32 on exactly the boosted srcA row (BLOCK model)
    d = w[1024:1280].reshape(64, 4)
    assert np.all(d[i_of == 5] == 160) and np.all(d[i_of != 5] == 128)
    assert np.all(w[1280:1536] == 128)
    d4 = w[1536:1792].reshape(64, 4)
    assert np.all(d4[i_of == 5] == 160) and np.all(d4[i_of != 5] == 128)
    # LDS DMA: lane L's 16 bytes land at LDS offset 16*L
    img = w[1792:2048].astype(np.int64).astype(np.uint32).view(np.uint8).reshape(64, 16)
    pattern = ((7 * np.arange(1024) + 3) & 255).astype(np.uint8).reshape(64, 16)
    src = (5 * lanes + 3) & 63
    assert np.array_equal(img, pattern[src])
    # fp8 register -> scale-block map: dwords 0-3 of lane group q carry K
    # [16q, 16q+16), dwords 4-7 carry K [64+16q, 64+16q+16); scale block = K/32.
    q0, d0 = np.arange(32) // 8, np.arange(32) % 8
    exp8 = 2 ** np.where(d0 < 4, q0 // 2, 2 + q0 // 2)
    assert np.array_equal(w[2048:2080], exp8), w[2048:2080]
    # fp4: dwords 0-3 of lane group q carry K [32q, 32q+32) -> block q
    assert np.array_equal(w[2080:2096], 2 ** (np.arange(16) // 4)), w[2080:2096]

    # 32x32x64: accumulator register r of lane L holds D[i][j] with srcA row
    # i = 8*(r//4) + 4*(L//32) + r%4 and srcB row j = L%32; srcA / srcB lanes
    # t and t+32 feed the same row (two halves of K)
    r = np.arange(16)[None, :]
    lane = np.arange(64)[:, None]
    rows_a = np.broadcast_to(8 * (r // 4) + 4 * (lane // 32) + r % 4, (64, 16))
    rows_b = np.broadcast_to(lane % 32, (64, 16))
    for base, expect in [(2096, rows_a), (3120, rows_a), (4144, rows_b), (5168, rows_b),
                         (6192, rows_a), (7216, rows_b)]:
        got = w[base:base + 1024].reshape(64, 16)
        assert np.array_equal(got, expect), f"32x32x64 map at word {base}:\n{got}"
    # scale blocks of K=64: fp8 dwords 0-3 of either lane group are block 0
    # (lane group 0's scale), dwords 4-7 block 1; fp4 lane group g is block g
    assert w[8240:8256].tolist() == [0, 0, 0, 0, 1, 1, 1, 1] * 2, w[8240:8256]
    assert w[8256:8264].tolist() == [0, 0, 0, 0, 1, 1, 1, 1], w[8256:8264]


# ----------------------------------------------------------------- MXFP8
# M <= 64 runs the stream / skinny / decode kernels; larger M the 256 x 256
# tile kernel with >= 128 of its tiles ((2100, 4100, 256): 153, tails in M
# and N), else the 128 x 128 kernel
MX8_SHAPES = [(256, 256, 128), (256, 512, 1024), (300, 520, 384), (1, 1536, 7168), (32, 1536, 7168),
              (513, 272, 256), (512, 512, 2048), (768, 1024, 512), (2100, 4100, 256)]


@pytest.mark.parametrize("m,n,k", MX8_SHAPES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_mxfp8(qgemm, gpu, m, n, k, dtype):
    qa, qb, ea, eb = make_mx8(m, n, k, seed=m + n + k)
    ref = O.gemm_mx8(qa, qb, ea, eb)
    y = qgemm.gemm_a8w8_mxfp8(to_dev(qa, None, gpu).view(torch.float8_e4m3fn),
                              to_dev(qb, None, gpu).view(torch.float8_e4m3fn),
                              to_dev(ea, None, gpu), to_dev(eb, None, gpu), dtype=dtype)
    assert_close(ref, out_to_f32(y), f"mxfp8 {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(512, 256, 1024), (512, 512, 4096), (300, 520, 1536), (2304, 3600, 1536)])
def test_mxfp8_k_pattern_scales(qgemm, gpu, m, n, k):
    """Distinct per-K-group scales catch K-group and scale panel misrouting
    (MX4 host.cc:185-187; 32- and 16-byte panels)."""
    qa, qb, ea, eb = make_mx8(m, n, k, seed=7)
    ea = np.broadcast_to((120 + (np.arange(k // 32) % 13)).astype(np.uint8), ea.shape).copy()
    ref = O.gemm_mx8(qa, qb, ea, eb)
    y = qgemm.gemm_a8w8_mxfp8(to_dev(qa, None, gpu).view(torch.float8_e4m3fn),
                              to_dev(qb, None, gpu).view(torch.float8_e4m3fn),
                              to_dev(ea, None, gpu), to_dev(eb, None, gpu), dtype=torch.float32)
    assert_close(ref, out_to_f32(y), "mxfp8 K-pattern")


# ----------------------------------------------------------------- MXFP4
MX4_SHAPES = [(256, 256, 256), (256, 512, 1024), (100, 300, 512), (1, 512, 2048), (257, 256, 768),
              (512, 512, 2048), (384, 1024, 512), (300, 520, 3072), (512, 768, 4096), (2100, 4100, 512)]


@pytest.mark.parametrize("m,n,k", MX4_SHAPES)
def test_mxfp4(qgemm, gpu, m, n, k):
    qa, qb, ea, eb = make_mx4(m, n, k, seed=m * 3 + k)
    ref = O.gemm_mx4(qa, qb, ea, eb)
    y = qgemm.gemm_a4w4_mxfp4(to_dev(qa, None, gpu), to_dev(qb, None, gpu), to_dev(ea, None, gpu),
                              to_dev(eb, None, gpu), dtype=torch.bfloat16)
    assert_close(ref, out_to_f32(y), f"mxfp4 {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(512, 256, 4096), (300, 520, 3072), (512, 512, 1536), (2304, 3600, 2048),
                                   (2304, 3600, 1536)])
def test_mxfp4_k_pattern_scales(qgemm, gpu, m, n, k):
    """Distinct per-K-group scales on both operands catch K-group and scale
    panel misrouting (32-, 16- and 8-byte panels)."""
    qa, qb, ea, eb = make_mx4(m, n, k, seed=11)
    g = np.arange(k // 32)
    ea = np.broadcast_to((122 + (g % 11)).astype(np.uint8), ea.shape).copy()
    eb = np.broadcast_to((121 + ((3 * g) % 13)).astype(np.uint8), eb.shape).copy()
    ref = O.gemm_mx4(qa, qb, ea, eb)
    y = qgemm.gemm_a4w4_mxfp4(to_dev(qa, None, gpu), to_dev(qb, None, gpu), to_dev(ea, None, gpu),
                              to_dev(eb, None, gpu), dtype=torch.float32)
    assert_close(ref, out_to_f32(y), f"mxfp4 K-pattern {m}x{n}x{k}")


# ----------------------------------------------- block-scale, E8M0 (SNAP ABI)
def _snap_inputs(m, n, k, seed):
    rng = np.random.default_rng(seed)
    a = O.e4m3_encode(rng.uniform(-1, 1, (m, k)).astype(np.float32))
    b = O.e4m3_encode(rng.uniform(-1, 1, (n, k)).astype(np.float32))
    sfa_km = rng.integers(124, 131, (k // 128, m)).astype(np.uint8)  # physical [K/128][M]
    sfb = rng.integers(124, 131, (n // 128, k // 128)).astype(np.uint8)
    return a, b, sfa_km, sfb


@pytest.mark.parametrize("m,n,k", [(256, 256, 256), (512, 256, 1152), (256, 768, 640)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_blockscale_e8m0(qgemm, gpu, m, n, k, dtype):
    a, b, sfa_km, sfb = _snap_inputs(m, n, k, seed=m + k)
    ref = O.gemm_bs_e8m0(a, b, sfa_km, sfb)
    bp = O.shuffle_weight_16x16(b)
    A = to_dev(a, None, gpu).view(torch.float8_e4m3fn)
    Bp = to_dev(bp, None, gpu)
    A_scale = to_dev(sfa_km, None, gpu).t()          # logical [M, K/128], strides (1, M)
    y = qgemm.blockscale_bpreshuffle.gemm_a8w8_blockscale_bpreshuffle(A, Bp, A_scale, to_dev(sfb, None, gpu),
                                                                      dtype=dtype)
    assert_close(ref, out_to_f32(y), f"bs-e8m0 {m}x{n}x{k}")


def test_blockscale_e8m0_batch2_c_abi(qgemm, gpu):
    """The drop-in launcher at batch 2, as the reference's own `make verify`
    runs it (SNAP Makefile:51): dense batch strides, per-batch scales."""
    m, n, k, batch = 512, 256, 1152, 2
    data = [_snap_inputs(m, n, k, seed=90 + i) for i in range(batch)]
    A = torch.stack([torch.from_numpy(d[0]) for d in data]).to(gpu)
    B = torch.stack([torch.from_numpy(O.shuffle_weight_16x16(d[1])) for d in data]).to(gpu)
    SA = torch.stack([torch.from_numpy(d[2]) for d in data]).to(gpu)           # [b][K/128][M]
    SB = torch.stack([torch.from_numpy(d[3]) for d in data]).to(gpu)
    kg = k // 128
    for out_code, odt in ((1, torch.bfloat16), (0, torch.float32)):
        C = torch.empty(batch, m, n, dtype=odt, device=gpu)
        args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, batch, k, k, n, m * k, n * k, m * n,
                           SA.data_ptr(), SB.data_ptr(), m, kg, m * kg, (n // 128) * kg)
        st = qgemm.lib().launch_blockscale_bpreshuffle(ctypes.byref(args), out_code, 0,
                                                       ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert st == 0
        torch.cuda.synchronize()
        for i, d in enumerate(data):
            assert_close(O.gemm_bs_e8m0(*d), C[i].float().cpu().numpy(), f"bs-e8m0 batch {i} out={out_code}")


def test_blockscale_e8m0_adapter_contract(qgemm, gpu):
    """The Python adapter raises ValueError where the launcher's contract is
    broken (SNAP blockscale_bpreshuffle.py:37-97 behaviour), before launching."""
    f = qgemm.blockscale_bpreshuffle.gemm_a8w8_blockscale_bpreshuffle
    m, n, k = 256, 256, 256
    A = torch.zeros(m, k, dtype=torch.uint8, device=gpu).view(torch.float8_e4m3fn)
    B = torch.zeros(n, k, dtype=torch.uint8, device=gpu)
    sa = torch.full((k // 128, m), 127, dtype=torch.uint8, device=gpu).t()
    sb = torch.full((n // 128, k // 128), 127, dtype=torch.uint8, device=gpu)
    assert torch.count_nonzero(f(A, B, sa, sb).float()) == 0
    bad = [
        dict(A=A[:, :128].contiguous()),                                # K mismatch
        dict(A=torch.zeros(128, k, dtype=torch.uint8, device=gpu).view(torch.float8_e4m3fn)),   # M % 256
        dict(A_scale=torch.ones(m, k // 128, dtype=torch.float32, device=gpu)),                  # fp32 scales
        dict(A_scale=torch.full((m, 4), 127, dtype=torch.uint8, device=gpu)[:, :2]),             # strided scales
        dict(B_scale=sb[:1]),                                            # wrong scale shape
        dict(dtype=torch.float16),
        dict(tiles=2),
        dict(A=A.view(torch.uint8)),                                     # A not e4m3
    ]
    for change in bad:
        kw = dict(A=A, B=B, A_scale=sa, B_scale=sb)
        kw.update(change)
        with pytest.raises(ValueError):
            f(**kw)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        f(A, B, sa, sb, out=out.view(torch.float32))                    # wrong out dtype
    alias = torch.empty(m * n * 2, dtype=torch.uint8, device=gpu)
    with pytest.raises(ValueError):                                     # out overlapping B
        f(A, alias[:n * k].view(n, k), sa, sb, out=alias.view(torch.bfloat16).view(m, n))


# ----------------------------------------------- block-scale, fp32 scales
BS_SHAPES = [(32, 1536, 7168), (256, 256, 128), (300, 520, 384), (1, 2112, 7168), (16, 4096, 1024),
             (600, 384, 256), (512, 768, 1024)]


@pytest.mark.parametrize("m,n,k", BS_SHAPES)
@pytest.mark.parametrize("sfa_layout", ["mk", "km"])
def test_blockscale_fp32(qgemm, gpu, m, n, k, sfa_layout):
    qa, qb, sa, sb = make_bs(m, n, k, seed=m + 2 * n + k)
    ref = O.gemm_bs_fp32(qa, qb, sa, sb)
    A = to_dev(qa, None, gpu).view(torch.float8_e4m3fn)
    Bk = qgemm.shuffle_b_kpanel(to_dev(qb, None, gpu)).view(torch.float8_e4m3fn)
    if sfa_layout == "mk":
        A_scale = to_dev(sa, None, gpu)
    else:
        A_scale = to_dev(np.ascontiguousarray(sa.T), None, gpu).t()
    y = qgemm.gemm_a8w8_bpreshuffle(A, Bk, A_scale, to_dev(sb, None, gpu), dtype=torch.bfloat16)
    assert_close(ref, out_to_f32(y), f"bs-fp32 {m}x{n}x{k} {sfa_layout}")


# tile-kernel cases: one K-tile, odd K-tile counts (the loops run two and
# four half-steps per iteration), whole and ragged tiles, fp32 output; the
# 128 x 128 kernel with K split 2, 3 and 7 ways (ragged last slice) and
# without a split; the 256 x 256 kernel at 4096 x 4096
@pytest.mark.parametrize("m,n,k", [(520, 300, 128), (264, 1000, 640), (512, 512, 1408), (768, 256, 256),
                                   (300, 520, 2048), (130, 1000, 7168), (1024, 2112, 7168), (4096, 4096, 384)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_blockscale_fp32_tile(qgemm, gpu, m, n, k, dtype):
    qa, qb, sa, sb = make_bs(m, n, k, seed=3 * m + n + k)
    ref = O.gemm_bs_fp32(qa, qb, sa, sb)
    A = to_dev(qa, None, gpu).view(torch.float8_e4m3fn)
    Bk = qgemm.shuffle_b_kpanel(to_dev(qb, None, gpu)).view(torch.float8_e4m3fn)
    y = qgemm.gemm_a8w8_bpreshuffle(A, Bk, to_dev(sa, None, gpu), to_dev(sb, None, gpu), dtype=dtype)
    assert_close(ref, out_to_f32(y), f"bs-fp32 tile {m}x{n}x{k} {dtype}")


# ------------------------------------- wide MX kernels: scale-panel copy
@pytest.mark.parametrize("fp4,k", [(False, 2048), (True, 2048), (True, 1536), (False, 1536)])
@pytest.mark.parametrize("out_code", [0, 1])
def test_mx_wide_scale_panels(qgemm, gpu, fp4, k, out_code):
    """Batched wide-kernel call through the C ABI with the queried workspace
    (E8M0 scales copied panel-major first: 32-byte panels for fp4 with
    K % 1024 == 0, else 16-byte) against the oracle, and bit-equal to the
    same call without a workspace (row-major scales read directly); padded
    scale row pitches and batch strides, M and N tails; 144 256 x 256 tiles
    keep the shape on the wide kernel (below 128 it runs 128 x 128 tiles)."""
    m, n, batch = 1300, 3000, 2
    make = make_mx4 if fp4 else make_mx8
    data = [make(m, n, k, seed=600 + i + 10 * fp4) for i in range(batch)]
    kb, kg = (k // 2 if fp4 else k), k // 32
    lsa, lsb = kg + 16, kg + 32
    A = torch.stack([torch.from_numpy(d[0]) for d in data]).to(gpu)
    B = torch.stack([torch.from_numpy(d[1]) for d in data]).to(gpu)
    SA = torch.full((batch, m, lsa), 0xFF, dtype=torch.uint8)
    SB = torch.full((batch, n, lsb), 0xFF, dtype=torch.uint8)
    for i, d in enumerate(data):
        SA[i, :, :kg] = torch.from_numpy(d[2])
        SB[i, :, :kg] = torch.from_numpy(d[3])
    SA, SB = SA.to(gpu), SB.to(gpu)
    name = "gemm_a4w4_mxfp4" if fp4 else "gemm_a8w8_mxfp8"
    L = qgemm.lib()
    outs = []
    pb = 32 if fp4 and k % 1024 == 0 else 16
    odt, otag = (torch.float32, "fp32") if out_code == 0 else (torch.bfloat16, "bf16")
    for use_ws in (True, False):
        C = torch.empty(batch, m, n, dtype=odt, device=gpu)
        args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, batch, kb, kb, n, m * kb, n * kb,
                           m * n, SA.data_ptr(), SB.data_ptr(), lsa, lsb, m * lsa, n * lsb)
        need = getattr(L, name + "_workspace_bytes")(ctypes.byref(args))
        ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=gpu)
        if use_ws:
            assert need >= batch * (m + n) * kg, "query must cover the scale panels"
        st = getattr(L, name)(ctypes.byref(args), out_code, ws.data_ptr() if use_ws else None,
                              need if use_ws else 0, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert st == 0, f"{name} returned {st}"
        # the instantiations bench.py times at 8192^3 (bf16, 16-byte fp8 /
        # 32-byte fp4 panels after the copy) and their no-workspace twins
        fmt = "fp4" if fp4 else "fp8"
        # (without a workspace the same panel width reads the row-major scales)
        want = (f"mx_scale_panels<pb{pb}>+wide_gemm<{fmt},MX,RAW,{otag},pb{pb}>" if use_ws
                else f"wide_gemm<{fmt},MX,RAW,{otag},pb{pb}>")
        assert qgemm.last_launch() == want
        torch.cuda.synchronize()
        outs.append(C.float().cpu())
    gemm = O.gemm_mx4 if fp4 else O.gemm_mx8
    for i, d in enumerate(data):
        assert_close(gemm(*d), outs[0][i].numpy(), f"batch {i}")
    assert torch.equal(outs[0], outs[1]), "panel-major and row-major scale paths differ"
