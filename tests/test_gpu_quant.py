"""Device-side quantizers and layout kernels against the CPU oracle, byte for
byte: the BASELINE recipes (fp32 1x128 / 128x128 block scales, E8M0 block
scales, MXFP8, MXFP4, e8m0_shuffle) on seeded N(0,1) data, bf16 sources,
tail blocks, all-zero groups, and hand-placed values on every rounding tie
and saturation edge of e4m3 / e2m1; then device-quantized operands through
the GEMM."""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close

pytestmark = pytest.mark.gpu


def _data(rows, k, seed):
    x = O.randn((rows, k), seed, 0)
    x *= np.float32(np.logspace(-3, 3, rows))[:, None]          # scales spread over six decades
    x[rows // 2, : min(k, 256)] = 0.0                             # all-zero groups / blocks
    return x


def _bf16_round(x):
    return torch.from_numpy(x).bfloat16().float().numpy()


def _src(x, dtype, gpu):
    return torch.from_numpy(x).to(gpu).to(dtype)


@pytest.mark.parametrize("rows,k", [(300, 4096), (1, 7168), (33, 128), (64, 1536)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("layout", ["mk", "km"])
def test_quant_fp8_blockscale_act(qgemm, gpu, rows, k, dtype, layout):
    x = _data(rows, k, rows + k)
    ref_x = x if dtype == torch.float32 else _bf16_round(x)
    qr, sr = O.quant_bs_act(ref_x)
    q, s = qgemm.quant_fp8_blockscale(_src(x, dtype, gpu), "1x128", layout)
    assert qgemm.last_launch() == f"quant_rows<e4m3,fp32,g128,{'bf16' if dtype == torch.bfloat16 else 'fp32'}>"
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), qr)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), sr.view(np.uint32))
    if layout == "km":
        assert s.stride() == (1, rows)


@pytest.mark.parametrize("n,k", [(1000, 2048), (256, 128), (7168, 512), (130, 384)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_quant_fp8_blockscale_wgt(qgemm, gpu, n, k, dtype):
    x = O.randn((n, k), n + k, 1)
    x[128:256 if n >= 256 else n, :128] *= 1000.0
    ref_x = x if dtype == torch.float32 else _bf16_round(x)
    qr, sr = O.quant_bs_wgt(ref_x)
    q, s = qgemm.quant_fp8_blockscale(_src(x, dtype, gpu), "128x128")
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), qr)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), sr.view(np.uint32))


@pytest.mark.parametrize("rows,k", [(300, 4096), (8, 1024)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_quant_fp8_e8m0(qgemm, gpu, rows, k, dtype):
    x = _data(rows, k, 5)
    ref_x = x if dtype == torch.float32 else _bf16_round(x)
    qr, er = O.quant_bs_e8m0_act(ref_x)
    q, e = qgemm.quant_fp8_e8m0_blockscale(_src(x, dtype, gpu), "1x128")
    assert e.stride() == (1, rows)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), qr)
    assert np.array_equal(e.cpu().numpy(), er)
    w = O.randn((384, k), 6, 1)
    qwr, ewr = O.quant_bs_e8m0_wgt(w)
    qw, ew = qgemm.quant_fp8_e8m0_blockscale(_src(w, torch.float32, gpu), "128x128")
    assert np.array_equal(qw.view(torch.uint8).cpu().numpy(), qwr)
    assert np.array_equal(ew.cpu().numpy(), ewr)


@pytest.mark.parametrize("fp4", [False, True])
@pytest.mark.parametrize("rows,k", [(513, 8192), (3, 96), (64, 2048), (40, 7168)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_quant_mx(qgemm, gpu, fp4, rows, k, dtype):
    x = _data(rows, k, 7 * rows + k)
    ref_x = x if dtype == torch.float32 else _bf16_round(x)
    qr, er = (O.quant_mx4 if fp4 else O.quant_mx8)(ref_x)
    fn = qgemm.quant_mxfp4 if fp4 else qgemm.quant_mxfp8
    q, e = fn(_src(x, dtype, gpu))
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), qr)
    assert np.array_equal(e.cpu().numpy(), er)
    q2, es = fn(_src(x, dtype, gpu), shuffle=True)                  # aiter quant(..., shuffle=True)
    assert np.array_equal(q2.view(torch.uint8).cpu().numpy(), qr)
    assert np.array_equal(es.cpu().numpy(), O.e8m0_shuffle(er))


def _tie_rows(qmax, grid):
    """Rows of 32 whose group amax is exactly qmax (scale 2^0), filled with
    every grid point, every midpoint between neighbours (ties), points just
    off the midpoints, and values past saturation, both signs."""
    g = np.array(grid, np.float64)
    mids = (g[:-1] + g[1:]) / 2
    eps = np.abs(mids) * 2.0 ** -20 + 2.0 ** -30
    vals = np.concatenate([g, mids, mids + eps, mids - eps, [qmax * 1.01, qmax * 1.5, 1e6, qmax]])
    vals = np.concatenate([vals, -vals]).astype(np.float32)
    per = 31
    nrow = -(-vals.size // per)
    out = np.zeros((nrow, 32), np.float32)
    out[:, 0] = qmax
    flat = np.zeros(nrow * per, np.float32)
    flat[:vals.size] = vals
    out[:, 1:] = flat.reshape(nrow, per)
    return out


def _e4m3_grid():
    return sorted({float(O.e4m3_decode(np.array([c], np.uint8))[0]) for c in range(0x7f)})


def test_quant_mx_rounding_ties_and_saturation(qgemm, gpu):
    """Every grid point, midpoint (tie -> even code) and near-midpoint of
    e4m3 and e2m1 in groups whose amax is exactly the top code (scale 2^0);
    then the same rows with values past the top code, which lift the group
    exponent instead."""
    for qmax, grid, fn, ofn in ((448.0, _e4m3_grid(), qgemm.quant_mxfp8, O.quant_mx8),
                                (6.0, [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], qgemm.quant_mxfp4, O.quant_mx4)):
        rows = _tie_rows(qmax, grid)
        for x in (np.clip(rows, -qmax, qmax), rows):
            qr, er = ofn(x)
            q, e = fn(_src(x, torch.float32, gpu))
            assert np.array_equal(q.view(torch.uint8).cpu().numpy(), qr)
            assert np.array_equal(e.cpu().numpy(), er)


def test_quant_mx_random_bits_exponent_zero(qgemm, gpu):
    """Two million random fp32 values (uniform in magnitude and in bit
    pattern below qmax) through groups whose scale is 2^0."""
    rng = np.random.default_rng(77)
    n = 1 << 21
    bits = rng.integers(0, 0x43e00000, n, dtype=np.uint32)          # every float in [0, 448)
    sign = rng.integers(0, 2, n, dtype=np.uint32) << 31
    v = (bits | sign).view(np.float32).reshape(-1, 32)
    v[:, 0] = 448.0
    qr, er = O.quant_mx8(v)
    q, e = qgemm.quant_mxfp8(_src(v, torch.float32, gpu))
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), qr)
    v4 = (rng.integers(0, 0x40c00000, n, dtype=np.uint32) | sign).view(np.float32).reshape(-1, 32)   # [0, 6)
    v4[:, 0] = 6.0
    qr, er = O.quant_mx4(v4)
    q, e = qgemm.quant_mxfp4(_src(v4, torch.float32, gpu))
    assert np.array_equal(q.cpu().numpy(), qr)


def test_quant_extreme_magnitudes(qgemm, gpu):
    """Group amax from subnormal to 1e37: exponent clamps (a subnormal amax
    whose quotient by qmax underflows takes the clamp -127) and subnormal
    scale arithmetic match.  The fp32-scale recipe (x / (amax/448)) is
    checked down to amax ~ 1e-36, where its scale is still a normal float."""
    mags = np.float32([1e-44, 1e-40, 3e-38, 1e-20, 1.0, 1e20, 1e37])
    x = (O.randn((mags.size, 256), 9, 0) * mags[:, None]).astype(np.float32)
    for fn, ofn in ((qgemm.quant_mxfp8, O.quant_mx8), (qgemm.quant_mxfp4, O.quant_mx4)):
        qr, er = ofn(x)
        q, e = fn(_src(x, torch.float32, gpu))
        assert np.array_equal(q.view(torch.uint8).cpu().numpy(), qr)
        assert np.array_equal(e.cpu().numpy(), er)
    x = x[3:]
    qr, sr = O.quant_bs_act(x)
    q, s = qgemm.quant_fp8_blockscale(_src(x, torch.float32, gpu))
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), qr)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), sr.view(np.uint32))


# ----------------------------------------------------------------- layouts
@pytest.mark.parametrize("n,k", [(48, 384), (7168, 512), (37, 256)])
def test_device_layouts_match_host(qgemm, gpu, n, k):
    b = np.random.default_rng(n + k).integers(0, 256, (n, k), dtype=np.uint8)
    B = torch.from_numpy(b).to(gpu)
    assert np.array_equal(qgemm.shuffle_b_kpanel(B).cpu().numpy(), O.shuffle_b_kpanel(b))
    assert qgemm.last_launch() == "relayout<KPANEL>"
    assert np.array_equal(qgemm.ldsbypass_pack_b(B).cpu().numpy(), qgemm.ldsbypass_pack_b(torch.from_numpy(b)).numpy())
    # the GPU B' -> B'' repack and the direct pack agree
    assert torch.equal(qgemm.ldsbypass_pack_b(B), qgemm.ldsbypass_repack(qgemm.shuffle_b_kpanel(B)))
    if n % 16 == 0:
        assert np.array_equal(qgemm.shuffle_weight_16x16(B).cpu().numpy(), O.shuffle_weight_16x16(b))
    # padded source pitch
    wide = torch.zeros((n, k + 64), dtype=torch.uint8, device=gpu)
    wide[:, :k] = B
    assert torch.equal(qgemm.shuffle_b_kpanel(wide[:, :k]), qgemm.shuffle_b_kpanel(B))


# dword-aligned rows take the block kernel (one 32-row block x 16 K-tiles per
# workgroup; partial last chunk, padded groups), odd pitches the byte kernel
@pytest.mark.parametrize("rows,kg", [(64, 24), (100, 13), (32, 8), (1, 256), (300, 1040), (77, 36), (33, 2048)])
def test_device_e8m0_shuffle(qgemm, gpu, rows, kg):
    e = np.random.default_rng(rows * kg).integers(100, 150, (rows, kg), dtype=np.uint8)
    got = qgemm.e8m0_shuffle(torch.from_numpy(e).to(gpu)).cpu().numpy()
    assert qgemm.last_launch() == ("e8m0_shuffle" if kg % 4 else "e8m0_shuffle_blocks<1>")
    assert np.array_equal(got, O.e8m0_shuffle(e))


# ----------------------------------------------------------------- into the GEMM
def test_device_quantized_operands_feed_the_gemms(qgemm, gpu):
    """fp32 -> device quantizers -> GEMM equals the oracle GEMM on the
    oracle's own quantization of the same data (identical bytes)."""
    m, n, k = 96, 512, 2048
    a, b = O.randn((m, k), 3, 0), O.randn((n, k), 3, 1)
    A, B = _src(a, torch.float32, gpu), _src(b, torch.float32, gpu)
    qa, ea = qgemm.quant_mxfp8(A)
    qb, eb = qgemm.quant_mxfp8(B)
    (ra, rea), (rb, reb) = O.quant_mx8(a), O.quant_mx8(b)
    assert_close(O.gemm_mx8(ra, rb, rea, reb),
                 qgemm.gemm_a8w8_mxfp8(qa, qb, ea, eb, dtype=torch.float32).cpu().numpy(), "mxfp8")
    qa4, ea4 = qgemm.quant_mxfp4(A)
    qb4, eb4 = qgemm.quant_mxfp4(B)
    (ra, rea), (rb, reb) = O.quant_mx4(a), O.quant_mx4(b)
    assert_close(O.gemm_mx4(ra, rb, rea, reb),
                 qgemm.gemm_a4w4_mxfp4(qa4, qb4, ea4, eb4, dtype=torch.float32).cpu().numpy(), "mxfp4")
    qa8, sa = qgemm.quant_fp8_blockscale(A, "1x128")
    qb8, sb = qgemm.quant_fp8_blockscale(B, "128x128")
    (ra8, rsa), (rb8, rsb) = O.quant_bs_act(a), O.quant_bs_wgt(b)
    y = qgemm.gemm_a8w8_bpreshuffle(qa8, qgemm.shuffle_b_kpanel(qb8), sa, sb, dtype=torch.float32)
    assert_close(O.gemm_bs_fp32(ra8, rb8, rsa, rsb), y.cpu().numpy(), "bs fp32")
