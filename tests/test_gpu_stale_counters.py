"""Split-K launches whose workspace counter words hold stale values.

Every kernel with a fused last-slice reduce (burst, skinny, decode, band,
row-streaming, and the 256 x 256 kernel's tail split) tags its arrival
counters with a per-launch epoch, so the counter block needs no clearing: a
never-zeroed workspace, or one left mid-count by an interrupted launch, must
give the same bits as a zeroed one.  Each case fills the counter block with
a pattern -- all ones, every word one arrival short of a finished count, and
random words -- runs the split plan, and compares the output bit for bit with
the zeroed-workspace call and against the oracle.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, make_bs, make_mx4, make_mx8, out_to_f32

pytestmark = pytest.mark.gpu

KID = dict(auto=0, tile256=1, skinny=3, decode=4, burst=5, stream=6, band=7)


def _patterns(splitk_hint):
    rng = np.random.default_rng(7)
    return {
        "ones": np.full(512, 0xFFFFFFFF, dtype=np.uint32),
        "one_short": np.full(512, max(splitk_hint - 1, 1), dtype=np.uint32),
        "random": rng.integers(0, 1 << 32, 512, dtype=np.uint64).astype(np.uint32),
    }


def _run(qgemm, gpu, entry, query, args, kid, m, n, counters):
    L = qgemm.lib()
    need = getattr(L, query)(ctypes.byref(args), kid)
    assert need > 2048, f"{entry} kid {kid}: no split planned (workspace {need})"
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
    if counters is not None:
        ws[:2048] = torch.from_numpy(counters.view(np.uint8)).to(gpu)
    C = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
    args.ptr_c = C.data_ptr()
    st = getattr(L, entry)(ctypes.byref(args), 1, kid, ws.data_ptr(), need,
                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, f"{entry} kid {kid}: error {st}"
    trace = qgemm.last_launch()
    torch.cuda.synchronize()
    return C, trace


def _bs_args(qgemm, gpu, m, n, k, keep):
    qa, qb, sa, sb = make_bs(m, n, k, seed=m + n)
    kg, nbk = k // 128, (n + 127) // 128
    A, SA, SB = (torch.from_numpy(x).to(gpu) for x in (qa, sa, sb))
    Bk = qgemm.shuffle_b_kpanel(torch.from_numpy(qb)).to(gpu)
    keep += [A, SA, SB, Bk]
    args = qgemm.Kargs(A.data_ptr(), Bk.data_ptr(), 0, m, n, k, 1, k, 128, n, m * k, n * k, m * n,
                       SA.data_ptr(), SB.data_ptr(), 1, kg, m * kg, nbk * kg)
    return args, O.gemm_bs_fp32(qa, qb, sa, sb)


def _mx_args(qgemm, gpu, m, n, k, fp4, keep):
    qa, qb, ea, eb = (make_mx4 if fp4 else make_mx8)(m, n, k, seed=m + n)
    A, B, SA, SB = (torch.from_numpy(np.ascontiguousarray(x)).to(gpu) for x in (qa, qb, ea, eb))
    keep += [A, B, SA, SB]
    kb, kg = (k // 2 if fp4 else k), k // 32
    args = qgemm.Kargs(A.data_ptr(), B.data_ptr(), 0, m, n, k, 1, kb, kb, n, m * kb, n * kb, m * n,
                       SA.data_ptr(), SB.data_ptr(), kg, kg, m * kg, n * kg)
    return args, (O.gemm_mx4 if fp4 else O.gemm_mx8)(qa, qb, ea, eb)


# (family, kernel id, M, N, K, expected kernel name)
CASES = [
    ("bs", "auto", 32, 1536, 7168, "burst_gemm"),          # configs[0]: burst, K split 5
    ("bs", "decode", 32, 1536, 7168, "decode_gemm"),
    ("bs", "skinny", 16, 512, 16384, "skinny_gemm"),
    ("bs", "tile256", 300, 520, 1536, "bsf32_gemm"),      # every tile in the tail: tail split
    ("mx8", "skinny", 32, 1024, 8192, "skinny_gemm"),
    ("mx8", "band", 32, 2048, 8192, "band_gemm"),
    ("mx4", "stream", 4, 7168, 32768, "stream_gemm"),
    ("mx4", "burst", 32, 1024, 8192, "burst_gemm"),
]


@pytest.mark.parametrize("fam,kid,m,n,k,kern", CASES)
def test_split_ignores_stale_counters(qgemm, gpu, fam, kid, m, n, k, kern):
    keep = []
    if fam == "bs":
        args, ref = _bs_args(qgemm, gpu, m, n, k, keep)
        entry = "gemm_a8w8_blockscale_bpreshuffle_kid"
    else:
        args, ref = _mx_args(qgemm, gpu, m, n, k, fam == "mx4", keep)
        entry = "gemm_a4w4_mxfp4_kid" if fam == "mx4" else "gemm_a8w8_mxfp8_kid"
    query = entry + "_workspace_bytes"
    C0, trace = _run(qgemm, gpu, entry, query, args, KID[kid], m, n, None)
    assert kern in trace and ("splitk1>" not in trace or ",tail" in trace), trace
    assert_close(ref, out_to_f32(C0), f"{fam} {m}x{n}x{k} ({trace}), zeroed counters")
    split = int(trace.split("splitk")[-1].rstrip(">").split(">")[0]) if "splitk" in trace else 2
    for name, words in _patterns(split).items():
        C1, trace1 = _run(qgemm, gpu, entry, query, args, KID[kid], m, n, words)
        assert trace1 == trace
        assert torch.equal(C0.view(torch.int16), C1.view(torch.int16)), \
            f"{fam} {m}x{n}x{k} ({trace}): counters '{name}' changed the output"
