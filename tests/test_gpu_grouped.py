"""GPU parity of the grouped decode entries: several decode GEMMs with their
own M, N, K, operands, scales and outputs in one launch of the grouped burst
kernel (one grid over every problem's (tile, K slice) items, each split
problem summed in its own counters and partial planes).

* configs[2]'s decode shapes (N, K) = (2112, 7168), (4096, 7168),
  (7168, 2048) together at M = 16 and M = 64, for all four families (fp32
  block scales on K-panel B' and on B'', MXFP8, MXFP4), every output against
  the oracle;
* mixed M (1, 16, 33, 64) with ragged N (1000, 2112, 520) and a long K that
  forces K splits; without a workspace (refused while a problem needs a
  split, every problem unsplit otherwise); bf16 and fp32 output;
* determinism: two calls, a persistent grid (grid_blocks) and a workspace
  whose counter words hold garbage all give the same bits.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, make_bs, make_mx4, make_mx8, out_to_f32

pytestmark = pytest.mark.gpu

C2_DECODE = [(2112, 7168), (4096, 7168), (7168, 2048)]


def _problems(qgemm, gpu, kind, shapes, seed=0):
    """(device problems for gemm_grouped, oracle references)."""
    probs, refs = [], []
    for i, (m, n, k) in enumerate(shapes):
        s = seed + 17 * i + m
        if kind in ("bpreshuffle", "ldsbypass"):
            qa, qb, sa, sb = make_bs(m, n, k, seed=s)
            A = torch.from_numpy(qa).to(gpu).view(torch.float8_e4m3fn)
            Bk = qgemm.shuffle_b_kpanel(torch.from_numpy(qb).to(gpu))
            SA, SB = torch.from_numpy(sa).to(gpu), torch.from_numpy(sb).to(gpu)
            if kind == "bpreshuffle":
                probs.append((A, Bk.view(torch.float8_e4m3fn), SA, SB))
            else:
                probs.append((A, qgemm.ldsbypass_repack(Bk), SA, SB, n))
            refs.append(O.gemm_bs_fp32(qa, qb, sa, sb))
        else:
            fp4 = kind == "mxfp4"
            qa, qb, ea, eb = (make_mx4 if fp4 else make_mx8)(m, n, k, seed=s)
            A, B = torch.from_numpy(qa).to(gpu), torch.from_numpy(qb).to(gpu)
            if not fp4:
                A, B = A.view(torch.float8_e4m3fn), B.view(torch.float8_e4m3fn)
            probs.append((A, B, torch.from_numpy(ea).to(gpu), torch.from_numpy(eb).to(gpu)))
            refs.append((O.gemm_mx4 if fp4 else O.gemm_mx8)(qa, qb, ea, eb))
    return probs, refs


def _bits(ys):
    return [y.view(torch.int16 if y.dtype == torch.bfloat16 else torch.int32).clone() for y in ys]


@pytest.mark.parametrize("kind", ["bpreshuffle", "ldsbypass", "mxfp8", "mxfp4"])
@pytest.mark.parametrize("m", [16, 64])
def test_grouped_configs2_decode(qgemm, gpu, kind, m):
    shapes = [(m, n, k) for n, k in C2_DECODE]
    probs, refs = _problems(qgemm, gpu, kind, shapes)
    ys = qgemm.gemm_grouped(kind, probs)
    trace = qgemm.last_launch()
    torch.cuda.synchronize()
    assert trace.startswith("burst_grouped<") and ",g3," in trace, trace
    for (mm, n, k), ref, y in zip(shapes, refs, ys):
        assert_close(ref, out_to_f32(y), f"{kind} grouped {mm}x{n}x{k} ({trace})")
    first = _bits(ys)
    # the same call again, a persistent grid, and garbage counter words
    ys2 = qgemm.gemm_grouped(kind, probs)
    ys3 = qgemm.gemm_grouped(kind, probs, grid_blocks=97)
    trace3 = qgemm.last_launch()
    L = qgemm.lib()
    name = qgemm._GROUPED[kind][0]
    ktype = qgemm._GROUPED[kind][1]
    arr = (ktype * len(probs))(*[qgemm._group_kargs(kind, pr[0], pr[1], pr[2], pr[3], y, pr[4] if len(pr) > 4 else None)
                                 for pr, y in zip(probs, ys)])
    need = getattr(L, name + "_workspace_bytes")(arr, len(probs))
    junk = torch.full((max(need, 256),), 0xFF, dtype=torch.uint8, device=gpu) if need else None
    ys4 = qgemm.gemm_grouped(kind, probs, workspace=junk) if need else ys
    torch.cuda.synchronize()
    assert ",grid97>" in trace3, trace3
    for other in (ys2, ys3, ys4):
        assert all(torch.equal(a, b) for a, b in zip(first, _bits(other))), f"{kind} M={m}: outputs differ ({trace})"


@pytest.mark.parametrize("kind", ["bpreshuffle", "ldsbypass", "mxfp8", "mxfp4"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_grouped_mixed_m_ragged_n_long_k(qgemm, gpu, kind, dtype):
    shapes = [(1, 1000, 4096), (16, 2112, 16384), (33, 520, 2048), (64, 1536, 7168)]
    probs, refs = _problems(qgemm, gpu, kind, shapes, seed=5)
    ys = qgemm.gemm_grouped(kind, probs, dtype=dtype)
    trace = qgemm.last_launch()
    torch.cuda.synchronize()
    assert trace.startswith("burst_grouped<") and ",g4," in trace and ",mb4," in trace, trace
    for (m, n, k), ref, y in zip(shapes, refs, ys):
        assert y.dtype == dtype
        assert_close(ref, out_to_f32(y), f"{kind} grouped {m}x{n}x{k} ({trace})")
    # no workspace: refused while a problem needs a K split (K = 16384 past
    # one workgroup's reach at M = 64), every problem unsplit without it
    with pytest.raises(RuntimeError, match="HIP error 1"):
        qgemm.gemm_grouped(kind, probs, dtype=dtype, workspace=False)
    keep = [0, 2]
    ys0 = qgemm.gemm_grouped(kind, [probs[i] for i in keep], dtype=dtype, workspace=False)
    trace0 = qgemm.last_launch()
    torch.cuda.synchronize()
    for i, y in zip(keep, ys0):
        m, n, k = shapes[i]
        assert_close(refs[i], out_to_f32(y), f"{kind} grouped unsplit {m}x{n}x{k} ({trace0})")


def test_grouped_sixteen_problems(qgemm, gpu):
    """The largest group: 16 MXFP4 problems of mixed shape in one launch."""
    rng = np.random.default_rng(3)
    shapes = [(int(rng.choice([1, 8, 24, 48])), int(rng.choice([256, 1024, 1800])), int(rng.choice([1024, 4096])))
              for _ in range(16)]
    probs, refs = _problems(qgemm, gpu, "mxfp4", shapes, seed=9)
    ys = qgemm.gemm_grouped("mxfp4", probs)
    trace = qgemm.last_launch()
    torch.cuda.synchronize()
    assert ",g16," in trace, trace
    for (m, n, k), ref, y in zip(shapes, refs, ys):
        assert_close(ref, out_to_f32(y), f"mxfp4 grouped {m}x{n}x{k} ({trace})")
