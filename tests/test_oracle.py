"""CPU checks that pin the oracle (no GPU).

Every oracle function is checked against something it does not compute
itself: torch's fp8 / e8m0 / bf16 casts, closed forms and special values of
the formats, quantizer invariants (range, minimal exponent, rounding error),
brute-force fp64 GEMMs on tiny shapes, and the layout transforms' published
numpy view/permute forms.
"""
import numpy as np
import pytest
import torch

import oracle as O


# ----------------------------------------------------------------- e4m3
def _e4m3_table():
    codes = np.arange(256, dtype=np.uint8)
    return codes, torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()


def test_e4m3_decode_exhaustive_vs_torch():
    codes, ref = _e4m3_table()
    ours = O.e4m3_decode(codes)
    nan = np.isnan(ref)
    assert set(np.nonzero(nan)[0].tolist()) == {0x7F, 0xFF}
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan], ref[~nan])
    # closed forms: bias 7, 3 mantissa bits, max 448, min subnormal 2^-9
    assert ours[0x38] == 1.0 and ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9 and ours[0xB8] == -1.0


def test_e4m3_encode_matches_torch_in_range():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000) * s for s in (1e-3, 0.1, 1.0, 30.0, 150.0)]).astype(np.float32)
    x = x[np.abs(x) <= 448]
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(O.e4m3_encode(x), ref)


def test_e4m3_encode_ties_to_even_and_saturates():
    codes, val = _e4m3_table()
    pos = [c for c in range(0x00, 0x7E)]                  # finite positive codes below max
    mids = np.array([(val[c] + val[c + 1]) / 2 for c in pos], np.float32)
    expect = np.array([c if c % 2 == 0 else c + 1 for c in pos], np.uint8)
    assert np.array_equal(O.e4m3_encode(mids), expect)
    assert np.array_equal(O.e4m3_encode(-mids), expect | 0x80)
    # SATFINITE: beyond 448 clamps to +-448 instead of NaN
    assert O.e4m3_encode(np.float32([449.0, 1e6, -1e6])).tolist() == [0x7E, 0x7E, 0xFE]


# ----------------------------------------------------------------- e8m0 / e2m1
def test_e8m0_decode_vs_torch_and_closed_form():
    e = np.arange(255, dtype=np.uint8)
    ours = O.e8m0_decode(e)
    ref = torch.from_numpy(e).view(torch.float8_e8m0fnu).float().numpy()
    assert np.array_equal(ours, ref)
    assert np.array_equal(ours, np.ldexp(np.float64(1.0), e.astype(np.int64) - 127).astype(np.float32))


E2M1_GRID = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def test_e2m1_decode_table():
    d = O.e2m1_decode(np.arange(16))
    assert d[:8].tolist() == E2M1_GRID
    assert d[8:].tolist() == [-v for v in E2M1_GRID]


def test_e2m1_encode_grid_ties_and_saturation():
    grid = np.float32(E2M1_GRID)
    assert O.e2m1_encode(grid).tolist() == list(range(8))
    assert O.e2m1_encode(-grid[1:]).tolist() == list(range(9, 16))
    # midpoints round to the even code (even mantissa bit)
    mids = np.float32([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
    assert O.e2m1_encode(mids).tolist() == [0, 2, 2, 4, 4, 6, 6]
    off = np.float32([0.26, 0.74, 1.3, 2.6, 4.9, 5.1])
    assert O.e2m1_encode(off).tolist() == [1, 1, 3, 5, 6, 7]
    assert O.e2m1_encode(np.float32([7.0, 100.0, -9.0])).tolist() == [7, 7, 15]


# ----------------------------------------------------------------- bf16
def test_bf16_rne_vs_torch():
    rng = np.random.default_rng(2)
    x = np.concatenate([
        rng.standard_normal(50000).astype(np.float32) * 1e3,
        rng.integers(0, 2 ** 32, 50000, dtype=np.uint64).astype(np.uint32).view(np.float32),
        np.float32([0.0, -0.0, np.inf, -np.inf, 3.4028235e38, 1e-45, -1e-45, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8]),
    ])
    x = x[~np.isnan(x)]
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.bf16_round_bits(x), ref)
    nan = O.bf16_round_bits(np.float32([np.nan]))
    assert np.isnan(O.bf16_bits_to_f32(nan))[0]


# ----------------------------------------------------------------- data
def test_randn_is_counter_based_and_normal():
    a = O.randn((4096,), seed=0, stream=0)
    b = O.randn((64, 128), seed=0, stream=0).reshape(-1)
    assert np.array_equal(a[:1000], b[:1000])                 # element i depends on (seed, stream, i) only
    assert not np.array_equal(a, O.randn((4096,), seed=0, stream=1))
    big = O.randn((1 << 18,), seed=3)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1.0) < 0.01


# ----------------------------------------------------------------- quantizers
def _e4m3_err_ok(x, deq, scale):
    # half an e4m3 ulp (2^-4 relative) plus half the subnormal step
    return np.all(np.abs(deq - x) <= np.abs(x) * 2.0 ** -4 + scale * 2.0 ** -10 + 1e-30)


def test_quant_bs_act_properties():
    x = O.randn((5, 384), seed=4)
    x[2, 128:256] = 0.0
    q, s = O.quant_bs_act(x)
    dq = O.e4m3_decode(q)
    assert s.shape == (5, 3) and s[2, 1] == 1.0
    for i in range(5):
        for g in range(3):
            blk = x[i, g * 128:(g + 1) * 128]
            if not blk.any():
                continue
            assert np.isclose(np.abs(dq[i, g * 128:(g + 1) * 128]).max(), 448.0)   # amax hits the top code
            assert _e4m3_err_ok(blk, dq[i, g * 128:(g + 1) * 128] * s[i, g], s[i, g])


def test_quant_bs_wgt_blocks_are_128x128():
    w = O.randn((200, 256), seed=5)
    w[128:, :128] *= 100.0                                      # second row block, first K block
    q, s = O.quant_bs_wgt(w)
    assert s.shape == (2, 2)
    assert s[1, 0] > 50 * s[0, 0] and s[1, 1] < 2 * s[0, 1]
    deq = O.e4m3_decode(q) * np.repeat(np.repeat(s, 128, 0), 128, 1)[:200]
    assert np.all(np.abs(deq - w) <= np.abs(w) * 2.0 ** -4 + np.repeat(np.repeat(s, 128, 0), 128, 1)[:200] * 2.0 ** -10)


@pytest.mark.parametrize("kind,qmax", [("mx8", 448.0), ("mx4", 6.0)])
def test_mx_exponent_is_minimal_power_of_two(kind, qmax):
    x = O.randn((6, 256), seed=6) * np.float32(np.logspace(-3, 3, 6))[:, None]
    x[3, 32:64] = 0.0
    q, e = O.quant_mx8(x) if kind == "mx8" else O.quant_mx4(x)
    assert e[3, 1] == 127
    amax = np.abs(x.reshape(6, 8, 32)).max(-1)
    p = np.ldexp(1.0, e.astype(np.int64) - 127)
    nz = amax > 0
    assert np.all(amax[nz] / p[nz] <= qmax)                      # fits the element range
    assert np.all(amax[nz] / (p[nz] / 2) > qmax)                 # and one step less would not
    # a subnormal group amax: amax / qmax underflows in fp32, the exponent is the clamp -127
    tiny = np.zeros((1, 64), np.float32)
    tiny[0, 0], tiny[0, 32] = np.float32(1e-44), np.float32(1e-30)
    _, e = O.quant_mx8(tiny) if kind == "mx8" else O.quant_mx4(tiny)
    assert e[0, 0] == 0 and e[0, 1] == 127 + int(np.ceil(np.log2(1e-30 / qmax)))


def test_quant_bs_e8m0_minimal_power_of_two_blocks():
    """E8M0 block scales: 1x128 activation and 128x128 weight blocks, the
    minimal power of two that fits amax into e4m3 (448), top code reached."""
    x = O.randn((4, 384), seed=14) * np.float32(np.logspace(-2, 2, 4))[:, None]
    x[1, 128:256] = 0.0
    q, e = O.quant_bs_e8m0_act(x)
    assert e.shape == (4, 3) and e[1, 1] == 127
    amax = np.abs(x.reshape(4, 3, 128)).max(-1)
    p = np.ldexp(1.0, e.astype(np.int64) - 127)
    nz = amax > 0
    assert np.all(amax[nz] / p[nz] <= 448.0) and np.all(amax[nz] / (p[nz] / 2) > 448.0)
    deq = O.e4m3_decode(q) * np.repeat(p, 128, 1)
    assert _e4m3_err_ok(x, deq, np.repeat(p, 128, 1))
    w = O.randn((200, 256), seed=15)
    w[128:, :128] *= 64.0
    qw, ew = O.quant_bs_e8m0_wgt(w)
    assert ew.shape == (2, 2)
    blk = np.abs(w[:128, :128]).max(), np.abs(w[128:, :128]).max()
    assert ew[1, 0] - ew[0, 0] == int(np.ceil(np.log2(blk[1] / 448))) - int(np.ceil(np.log2(blk[0] / 448)))
    pw = np.repeat(np.repeat(np.ldexp(1.0, ew.astype(np.int64) - 127), 128, 0), 128, 1)[:200]
    assert _e4m3_err_ok(w, O.e4m3_decode(qw) * pw, pw)


def test_mx4_packing_and_rounding():
    x = np.zeros((1, 64), np.float32)
    x[0, :4] = [1.0, 2.0, -0.5, 6.0]
    q, e = O.quant_mx4(x)
    assert e[0, 0] == 127                                         # amax 6 -> 2^0
    assert q[0, 0] == 0x42 and q[0, 1] == 0x79                    # even k in the low nibble
    y = O.randn((4, 256), seed=7)
    q, e = O.quant_mx4(y)
    codes = np.stack([q & 15, q >> 4], -1).reshape(4, 256)
    step = np.repeat(np.ldexp(1.0, e.astype(np.int64) - 127), 32, 1)
    deq = O.e2m1_decode(codes) * step
    # round to nearest on the grid: error <= half the local spacing (0.5 / 1 / 2 below 2 / 4 / 6)
    v = np.abs(y) / step
    half = np.where(v < 2, 0.25, np.where(v < 4, 0.5, 1.0))
    assert np.all(np.abs(deq - y) <= half * step)


# ----------------------------------------------------------------- GEMM oracles vs brute force
def _dec8(q):
    return torch.from_numpy(np.ascontiguousarray(q)).view(torch.float8_e4m3fn).double().numpy()


def _dec4(q):
    codes = np.stack([q & 15, q >> 4], -1).reshape(q.shape[0], -1)
    grid = np.array(E2M1_GRID + [-v for v in E2M1_GRID], np.float64)
    return grid[codes]


def test_gemm_bs_fp32_vs_fp64():
    m, n, k = 3, 130, 384
    a, b = O.randn((m, k), 8, 0), O.randn((n, k), 8, 1)
    qa, sa = O.quant_bs_act(a)
    qb, sb = O.quant_bs_wgt(b)
    A = _dec8(qa) * np.repeat(sa.astype(np.float64), 128, 1)
    B = _dec8(qb) * np.repeat(np.repeat(sb.astype(np.float64), 128, 0), 128, 1)[:n]
    ref = A @ B.T
    got = O.gemm_bs_fp32(qa, qb, sa, sb)
    mag = np.abs(A) @ np.abs(B).T
    assert np.all(np.abs(got - ref) <= 1e-5 * mag + 1e-30)
    assert np.array_equal(got, O.gemm_bs_fp32(qa, qb, np.ascontiguousarray(sa.T), sb, sfa_layout="km"))
    rows, cols = np.array([0, 2, 1]), np.array([129, 0, 64])
    assert np.array_equal(O.gemm_bs_fp32_points(qa, qb, sa, sb, rows, cols), got[rows, cols])


def test_gemm_mx8_vs_fp64_and_unit_scales():
    m, n, k = 4, 48, 256
    qa, ea = O.quant_mx8(O.randn((m, k), 9, 0))
    qb, eb = O.quant_mx8(O.randn((n, k), 9, 1))
    A =_dec8(qa) * np.repeat(np.ldexp(1.0, ea.astype(np.int64) - 127), 32, 1)
    B = _dec8(qb) * np.repeat(np.ldexp(1.0, eb.astype(np.int64) - 127), 32, 1)
    got = O.gemm_mx8(qa, qb, ea, eb)
    mag = np.abs(A) @ np.abs(B).T
    assert np.all(np.abs(got - A @ B.T) <= 1e-5 * mag + 1e-30)
    ones_a, ones_b = np.full_like(ea, 127), np.full_like(eb, 127)
    plain = _dec8(qa) @ _dec8(qb).T
    assert np.all(np.abs(O.gemm_mx8(qa, qb, ones_a, ones_b) - plain) <= 1e-5 * (np.abs(_dec8(qa)) @ np.abs(_dec8(qb)).T))
    rows, cols = np.array([3, 0]), np.array([47, 5])
    assert np.array_equal(O.gemm_mx8_points(qa, qb, ea, eb, rows, cols), got[rows, cols])


def test_gemm_mx4_exact_small_k():
    m, n, k = 3, 40, 64
    qa, ea = O.quant_mx4(O.randn((m, k), 10, 0))
    qb, eb = O.quant_mx4(O.randn((n, k), 10, 1))
    A = _dec4(qa) * np.repeat(np.ldexp(1.0, ea.astype(np.int64) - 127), 32, 1)
    B = _dec4(qb) * np.repeat(np.ldexp(1.0, eb.astype(np.int64) - 127), 32, 1)
    # every product and partial sum is exact in fp32 at this K
    assert np.array_equal(O.gemm_mx4(qa, qb, ea, eb).astype(np.float64), A @ B.T)
    assert np.array_equal(O.gemm_mx4(qa, qb, ea, eb, literal=True).astype(np.float64), A @ B.T)


@pytest.mark.parametrize("data", ["recipe", "random_bytes", "k_pattern", "scale_spread"])
def test_gemm_mx4_grouped_equals_literal(data):
    """The grouped gemm_ref_gpu form (MX4 host.cc:66-94) that the tests use
    for speed is bit-identical to the literal gemm_ref_cpu loop (MX4
    host.cc:96-115): BASELINE-recipe data, the reference's own random fp4
    bytes with scales in [124, 130] (MX4 host.cc:46-54, 178-180), per-K-group
    scale patterns and a wider scale spread; and the sampled-point entry
    equals the full grid."""
    m, n, k = 5, 96, 4096
    rng = np.random.default_rng(21)
    if data == "recipe":
        qa, ea = O.quant_mx4(O.randn((m, k), 21, 0))
        qb, eb = O.quant_mx4(O.randn((n, k), 21, 1))
    else:
        qa = rng.integers(0, 256, (m, k // 2), dtype=np.uint8)
        qb = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
        lo, hi = (124, 131) if data != "scale_spread" else (112, 143)
        ea = rng.integers(lo, hi, (m, k // 32)).astype(np.uint8)
        eb = rng.integers(lo, hi, (n, k // 32)).astype(np.uint8)
        if data == "k_pattern":
            ea = np.broadcast_to((120 + np.arange(k // 32) % 13).astype(np.uint8), ea.shape).copy()
    grouped = O.gemm_mx4(qa, qb, ea, eb)
    literal = O.gemm_mx4(qa, qb, ea, eb, literal=True)
    assert np.array_equal(grouped, literal)
    A = _dec4(qa) * np.repeat(np.ldexp(1.0, ea.astype(np.int64) - 127), 32, 1)
    B = _dec4(qb) * np.repeat(np.ldexp(1.0, eb.astype(np.int64) - 127), 32, 1)
    assert np.all(np.abs(grouped - A @ B.T) <= 2.0 ** -24 * np.abs(A @ B.T) + 1e-30)
    rows, cols = rng.integers(0, m, 200).astype(np.int32), rng.integers(0, n, 200).astype(np.int32)
    assert np.array_equal(O.gemm_mx4_points(qa, qb, ea, eb, rows, cols), grouped[rows, cols])


def test_gemm_mx4_k_group_pattern():
    m, n, k = 2, 16, 512
    qa, ea = O.quant_mx4(O.randn((m, k), 11, 0))
    qb, eb = O.quant_mx4(O.randn((n, k), 11, 1))
    ea = np.broadcast_to((120 + np.arange(k // 32) % 7).astype(np.uint8), ea.shape).copy()
    A = _dec4(qa) * np.repeat(np.ldexp(1.0, ea.astype(np.int64) - 127), 32, 1)
    B = _dec4(qb) * np.repeat(np.ldexp(1.0, eb.astype(np.int64) - 127), 32, 1)
    got = O.gemm_mx4(qa, qb, ea, eb)
    assert np.all(np.abs(got - A @ B.T) <= 1e-6 * (np.abs(A) @ np.abs(B).T))


def test_gemm_bs_e8m0_vs_fp64():
    m, n, k = 256, 256, 256
    rng = np.random.default_rng(12)
    a = O.e4m3_encode(rng.uniform(-1, 1, (m, k)).astype(np.float32))
    b = O.e4m3_encode(rng.uniform(-1, 1, (n, k)).astype(np.float32))
    sfa_km = rng.integers(124, 131, (k // 128, m)).astype(np.uint8)
    sfb = rng.integers(124, 131, (n // 128, k // 128)).astype(np.uint8)
    A = _dec8(a) * np.repeat(np.ldexp(1.0, sfa_km.T.astype(np.int64) - 127), 128, 1)
    B = _dec8(b) * np.repeat(np.repeat(np.ldexp(1.0, sfb.astype(np.int64) - 127), 128, 0), 128, 1)
    got = O.gemm_bs_e8m0(a, b, sfa_km, sfb)
    assert np.all(np.abs(got - A @ B.T) <= 1e-6 * (np.abs(A) @ np.abs(B).T) + 1e-30)
    rows, cols = rng.integers(0, m, 300).astype(np.int32), rng.integers(0, n, 300).astype(np.int32)
    assert np.array_equal(O.gemm_bs_e8m0_points(a, b, sfa_km, sfb, rows, cols), got[rows, cols])


# ----------------------------------------------------------------- tolerance checker
def test_check_tolerance_catches_planted_errors():
    ref = O.randn((64, 64), seed=13)
    assert O.check_tolerance(ref, ref.copy())[0] == 0
    r = O.rms(ref)
    ok = ref + np.sign(ref) * (np.abs(ref) * 2.0 ** -8)           # inside 2^-7 |ref|
    assert O.check_tolerance(ref, ok)[0] == 0
    bad = ref.copy()
    bad[5, 7] += 2.0 ** -6 * abs(ref[5, 7]) + 0.01 * r
    nbad, _, idx = O.check_tolerance(ref, bad)
    assert nbad == 1 and idx == 5 * 64 + 7


# ----------------------------------------------------------------- layouts
def test_kpanel_matches_transpose():
    b = np.random.default_rng(14).integers(0, 256, (48, 512), dtype=np.uint8)
    assert np.array_equal(O.shuffle_b_kpanel(b), b.reshape(48, 4, 128).transpose(1, 0, 2))


def test_shuffle_weight_forms_agree():
    """SNAP [N/16][K/16][16][16] and aiter view(N/16,16,K/32,2,16).permute(0,2,3,1,4)."""
    b = np.random.default_rng(15).integers(0, 256, (64, 256), dtype=np.uint8)
    snap = b.reshape(4, 16, 16, 16).transpose(0, 2, 1, 3).reshape(64, 256)
    aiter = b.reshape(4, 16, 8, 2, 16).transpose(0, 2, 3, 1, 4).reshape(64, 256)
    assert np.array_equal(snap, aiter)
    assert np.array_equal(O.shuffle_weight_16x16(b), snap)


def test_e8m0_shuffle_matches_view_permute():
    """aiter e8m0_shuffle: view(M/32, 2, 16, K/8, 2, 4).permute(0, 3, 5, 2, 4, 1)."""
    rows, kg = 64, 16
    e = np.random.default_rng(16).integers(0, 255, (rows, kg), dtype=np.uint8)
    ref = e.reshape(rows // 32, 2, 16, kg // 8, 2, 4).transpose(0, 3, 5, 2, 4, 1).reshape(-1)
    assert np.array_equal(O.e8m0_shuffle(e), ref)
    # ragged shapes pad with 127 (scale 1.0) and stay a bijection on the real entries
    e2 = np.random.default_rng(17).integers(0, 127, (40, 12), dtype=np.uint8)
    out = O.e8m0_shuffle(e2)
    assert out.size == 64 * 16 and np.sum(out == 127) == out.size - e2.size + np.sum(e2 == 127)
    assert np.array_equal(np.sort(out[out != 127]), np.sort(e2[e2 != 127]))
