"""Throughput of the quantized-GEMM hot path on one MI355X.

Default workload (the configuration the headline
metric is quoted on): MXFP8 TN GEMM, M = N = K = 8192, e4m3 operands with one
E8M0 scale per 32 K elements, bf16 output.  A "step" is one GEMM launch.
Other workloads (--workload) cover configs[0] (block-scale FP8 decode, both
B layouts), configs[2] (--sweep), configs[3] (MXFP4 8192^3), configs[4]
(MXFP4 decode, --m) and the device quantizers.

Inputs: N(0,1) fp32 drawn on the GPU from a generator seeded with 0 (A) and
1 (B), quantized on the GPU by this library's quantizers per the BASELINE
recipe, resident in HBM before the timed region.  Launches go straight
through the C ABI with prebuilt argument blocks.

Timing: a clock-settle phase of back-to-back launches (>= --settle-s
seconds; short warm-ups sit in the power controller's downclock window,
MX4 HANDOVER.md:8), then --warmup launches, then exactly --steps launches
between HIP events on the launch stream.  MFMA-bound workloads are timed
launch by launch (an event after every launch gives the spread);
HBM-bound decode workloads run as one HIP graph over rotating weight copies
(more bytes than the 256 MB last-level cache, so B streams from HBM).

After timing, 4096 output points are checked against the CPU oracle on the
same quantized bytes (tolerance |y - y_ref| <= 2^-7|y_ref| + 1e-3 rms);
a failure exits non-zero.  The oracle is used only for that check and for
the cpu_baseline leg (its restatement of the reference CPU GEMM, timed on a
bounded row band on this host).

Prints ONE JSON line with the metric, a roofline block for the dominant
kernel and the cpu_baseline block.
"""
import argparse
import ctypes
import importlib
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "TFLOPS and % of MI355X peak: block-FP8/MXFP8/MXFP4 GEMM at 8192^3 + decode M"
PEAK_TFLOPS = {"fp8": 5000.0, "fp4": 10100.0}
HBM_GBPS = 8000.0
ROTATE_BYTES = 512 << 20
CHECK_POINTS = 4096

WORKLOADS = {
    # name: (family, M, N, K, BASELINE config index)
    "mxfp8_8192": ("mx8", 8192, 8192, 8192, 1),
    "mxfp4_8192": ("mx4", 8192, 8192, 8192, 3),
    # configs[3] with aiter's gemm_a4w4(bpreshuffle=True) operands: the weight
    # pre-shuffled once (shuffle_weight(16,16)), scales in e8m0_shuffle order
    "mxfp4_8192_aiter": ("mx4a", 8192, 8192, 8192, 3),
    "bs_fp32_8192": ("bs", 8192, 8192, 8192, 2),
    "bs_c0": ("bs", 32, 1536, 7168, 0),
    "ldsbypass_c0": ("lbp", 32, 1536, 7168, 0),
    "mxfp4_c4": ("mx4", 32, 7168, 16384, 4),
    # configs[4] in aiter's formats (W16 weight, e8m0_shuffle scales)
    "mxfp4_c4_aiter": ("mx4a", 32, 7168, 16384, 4),
    # the reference's headline block-scale kernel (E8M0 1x128 / 128x128 scales,
    # shuffle_weight(16,16) B: 3.31 PFLOPS at 8192^3)
    "bs_e8m0_8192": ("bs8", 8192, 8192, 8192, None),
    # the same GEMM in aiter's other physical layouts (opus_gemm_mxfp8_{nn,tt,tn}):
    # B [K][N] (NN, TN), A [K][M] (TT, TN), read in place by the tile kernel
    "bs_e8m0_8192_nn": ("bs8nn", 8192, 8192, 8192, None),
    "bs_e8m0_8192_tt": ("bs8tt", 8192, 8192, 8192, None),
    "bs_e8m0_8192_tn": ("bs8tn", 8192, 8192, 8192, None),
}
BS8_FAMS = ("bs8", "bs8nn", "bs8tt", "bs8tn")
LAYOUT_CODE = {"bs8nn": 1, "bs8tt": 2, "bs8tn": 3}   # QGEMM_LAYOUT_*

# the other BASELINE configs the default run measures after the headline:
# (workload, M override)
EXTRA_WORKLOADS = (("mxfp4_8192", None), ("mxfp4_8192_aiter", None), ("bs_c0", None), ("mxfp4_c4", 32),
                   ("mxfp4_c4_aiter", 32))

NAMES = {"mx8": "MXFP8 TN GEMM, e4m3 x e4m3, E8M0 per 32 K",
         "mx4": "MXFP4 A4W4 GEMM, e2m1 x e2m1, E8M0 per 32 K",
         "mx4a": "MXFP4 A4W4 GEMM, e2m1 x e2m1, E8M0 per 32 K, aiter gemm_a4w4 bpreshuffle formats "
                 "(shuffle_weight(16,16) B, e8m0_shuffle scales)",
         "bs": "block-scale FP8 GEMM, fp32 1x128 / 128x128 scales, K-panel B (bpreshuffle)",
         "lbp": "block-scale FP8 GEMM, fp32 1x128 / 128x128 scales, fragment-order B'' (ldsbypass)",
         "bs8": "block-scale FP8 GEMM, E8M0 1x128 / 128x128 scales, shuffle_weight(16,16) B",
         "bs8nn": "block-scale FP8 GEMM, E8M0 1x128 / 128x128 scales, NN layout (B [K][N] N-contiguous)",
         "bs8tt": "block-scale FP8 GEMM, E8M0 1x128 / 128x128 scales, TT layout (A [K][M] M-contiguous, B [N][K])",
         "bs8tn": "block-scale FP8 GEMM, E8M0 1x128 / 128x128 scales, TN layout (A [K][M], B [K][N])"}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--settle-s", type=float, default=1.0,
                   help="seconds of back-to-back launches before the warm-up (clock settle)")
    p.add_argument("--workload", default="mxfp8_8192", choices=sorted(WORKLOADS))
    p.add_argument("--m", type=int, default=None, help="override M (decode sweeps)")
    p.add_argument("--n", type=int, default=None, help="override N")
    p.add_argument("--k", type=int, default=None, help="override K")
    p.add_argument("--grid-blocks", type=int, default=0,
                   help="mxfp4_8192_aiter: persistent grid of this many workgroups (0 = one per tile)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-check", action="store_true", help="skip the output check against the oracle")
    p.add_argument("--no-extra", action="store_true",
                   help="default run only: skip the extra records (configs[3] row-major and in aiter's "
                        "formats, configs[0], configs[4] M = 32 row-major and in aiter's formats)")
    p.add_argument("--sfa-km", action="store_true",
                   help="block-scale fp32 workloads: pass A's scales column-major [K/128][M] (the reference's "
                        "layout) instead of BASELINE's row-major [M][K/128]")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--sweep", nargs="?", const="configs2", default=None, choices=["configs2", "dsv4"],
                   help="time a block-scale shape sweep (bpreshuffle and ldsbypass), one JSON line per shape: "
                        "configs2 = BASELINE configs[2] (default), dsv4 = the 125 traced DeepSeek-V4 a8w8 shapes "
                        "(355_1_trans_amd/configs/dsv4_a8w8_shapes.csv)")
    p.add_argument("--grouped", default=None, choices=["bpreshuffle", "ldsbypass", "mxfp8", "mxfp4"],
                   help="time configs[2]'s decode shapes (N, K) = (2112, 7168), (4096, 7168), (7168, 2048) at M = "
                        "--m (default 16) as ONE grouped launch and as three single launches; one JSON line")
    p.add_argument("--group-grid", type=int, default=0, help="--grouped: persistent grid (0 = one per item)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="run only a plain 256 MiB device copy 5 times (PMC byte-counter calibration)")
    return p.parse_args()


def traffic_from_profiles(kernel_tag):
    """HBM bytes per launch recorded by the committed rocprofv3 PMC summary."""
    f = ROOT / "profiles" / f"{kernel_tag}_pmc.md"
    if not f.exists():
        return None
    m = re.search(r"hbm_bytes_per_launch:\s*([0-9.eE+]+)", f.read_text())
    return float(m.group(1)) if m else None


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ------------------------------------------------------------------ inputs
def randn(shape, seed, dev):
    """N(0,1) fp32 on the GPU from a generator seeded with `seed`."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.randn(shape, generator=g, device=dev, dtype=torch.float32)


def make_operands(q, fam, M, N, K, dev, sfa_km=False):
    """Quantized operands on the GPU (this library's device quantizers, the
    BASELINE recipes).  Returns a dict with the GEMM inputs and the host
    copies the checker and the CPU baseline use."""
    import torch
    a, b = randn((M, K), 0, dev), randn((N, K), 1, dev)
    ops = {}
    if fam == "mx8":
        A, SA = q.quant_mxfp8(a)
        B, SB = q.quant_mxfp8(b)
        ops.update(A=A.view(torch.uint8), SA=SA, B=B.view(torch.uint8), SB=SB)
    elif fam in ("mx4", "mx4a"):
        A, SA = q.quant_mxfp4(a)
        B, SB = q.quant_mxfp4(b)
        ops.update(A=A, SA=SA, B=B, SB=SB)
    elif fam in BS8_FAMS:
        A, SA = q.quant_fp8_e8m0_blockscale(a, "1x128")          # SA: [M, K/128] view of [K/128][M] bytes
        B, SB = q.quant_fp8_e8m0_blockscale(b, "128x128")
        ops.update(A=A.view(torch.uint8), SA=SA, B=B.view(torch.uint8), SB=SB)
    else:
        A, SA = q.quant_fp8_blockscale(a, "1x128", "km" if sfa_km else "mk")
        B, SB = q.quant_fp8_blockscale(b, "128x128")
        ops.update(A=A.view(torch.uint8), SA=SA, B=B.view(torch.uint8), SB=SB)
    del a, b
    ops["B_raw"] = ops["B"]
    if fam == "bs":
        ops["B"] = q.shuffle_b_kpanel(ops["B"]).reshape(-1)
    elif fam == "lbp":
        ops["B"] = q.ldsbypass_pack_b(ops["B"])
    elif fam == "bs8":
        ops["B"] = q.shuffle_weight_16x16(ops["B"])
    elif fam in ("bs8nn", "bs8tn"):
        ops["B"] = ops["B"].t().contiguous()                      # [K][N]
    if fam in ("bs8tt", "bs8tn"):
        ops["A_raw"] = ops["A"]
        ops["A"] = ops["A"].t().contiguous()                      # [K][M]
    elif fam == "mx4a":
        ops["B"] = q.shuffle_weight_16x16(ops["B"])
        ops["SA_raw"], ops["SB_raw"] = ops["SA"], ops["SB"]
        ops["SA"], ops["SB"] = q.e8m0_shuffle(ops["SA"]), q.e8m0_shuffle(ops["SB"])
    torch.cuda.synchronize()
    return ops


def kargs_for(q, fam, M, N, K, A, B, C, SA, SB, sfa_km, grid_blocks=0):
    kg32, kg128 = K // 32, K // 128
    kb = K // 2 if fam in ("mx4", "mx4a") else K
    if fam == "mx4a":
        blk = 32 * ((kg32 + 7) // 8 * 8)       # e8m0_shuffle bytes per 32-row block
        return q.Mxfp4Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, 1, kb, kb, N, M * kb, N * kb, M * N,
                            SA.data_ptr(), SB.data_ptr(), blk, blk, SA.numel(), SB.numel(), grid_blocks)
    if fam in ("mx8", "mx4"):
        return q.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, 1, kb, kb, N, M * kb, N * kb, M * N,
                       SA.data_ptr(), SB.data_ptr(), kg32, kg32, M * kg32, N * kg32)
    if fam in BS8_FAMS:
        return q.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, 1, M if fam in ("bs8tt", "bs8tn") else K,
                       N if fam in ("bs8nn", "bs8tn") else K, N, M * K, N * K, M * N,
                       SA.data_ptr(), SB.data_ptr(), M, kg128, M * kg128, SB.numel())
    sfa_stride = M if sfa_km else (1 if M > 1 else M)
    if fam == "bs":
        return q.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, 1, K, 128, N, M * K, N * K, M * N,
                       SA.data_ptr(), SB.data_ptr(), sfa_stride, kg128, M * kg128, SB.numel())
    return q.LdsBypassKargs(A.data_ptr(), None, B.data_ptr(), C.data_ptr(), M, N, K, 1, K, 128, N, M * K, N * K,
                            M * N, SA.data_ptr(), SB.data_ptr(), sfa_stride, kg128, M * kg128, SB.numel(), B.numel())


def entry_for(L, fam):
    """(launch(kargs_ptr, ws_ptr, ws_bytes, stream), workspace query) of a family."""
    if fam == "bs8":
        return (lambda ka, wp, wb, s: L.launch_blockscale_bpreshuffle(ka, 1, 0, s)), (lambda ka: 0)
    if fam in LAYOUT_CODE:
        code = LAYOUT_CODE[fam]
        return ((lambda ka, wp, wb, s: L.gemm_a8w8_blockscale_layout(ka, code, 1, None, 0, s)),
                (lambda ka: L.gemm_a8w8_blockscale_layout_workspace_bytes(ka, code)))
    if fam == "mx4a":    # the library's choice, with the workspace its decode plans split K in
        return ((lambda ka, wp, wb, s: L.gemm_a4w4_mxfp4_bpreshuffle_kid(ka, 1, 0, wp, wb, s)),
                (lambda ka: L.gemm_a4w4_mxfp4_bpreshuffle_kid_workspace_bytes(ka, 0)))
    name = {"mx8": "gemm_a8w8_mxfp8", "mx4": "gemm_a4w4_mxfp4", "bs": "gemm_a8w8_blockscale_bpreshuffle",
            "lbp": "gemm_a8w8_blockscale_ldsbypass"}[fam]
    fn = getattr(L, name)
    return (lambda ka, wp, wb, s: fn(ka, 1, wp, wb, s)), getattr(L, name + "_workspace_bytes")


# ------------------------------------------------------------------ timing
def run_timed(launch, n_calls, stream, graph_mode, steps, warmup, settle_s):
    """Settle, warm up, then time exactly `steps` launches.  Returns
    (ms per launch, timing dict)."""
    import torch
    with torch.cuda.stream(stream):
        launch(0)
    torch.cuda.synchronize()
    graph = None
    if graph_mode:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                launch(i)

    # clock settle: back-to-back work for >= settle_s seconds; one batch is
    # queued while the previous one runs (the host never runs far ahead)
    t0 = time.perf_counter()
    settle, prev = 0, None
    while True:
        with torch.cuda.stream(stream):
            if graph_mode:
                graph.replay()
                settle += steps
            else:
                for i in range(32):
                    launch(settle + i)
                settle += 32
        ev = torch.cuda.Event()
        ev.record(stream)
        if prev is not None:
            prev.synchronize()
        prev = ev
        if time.perf_counter() - t0 >= settle_s:
            break
    torch.cuda.synchronize()
    settle_wall = time.perf_counter() - t0
    with torch.cuda.stream(stream):
        for i in range(warmup):
            launch(i)
    torch.cuda.synchronize()

    timing = {"settle_s": round(settle_wall, 3), "settle_launches": settle, "warmup": warmup}
    if graph_mode:
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(6)]
        wall0 = time.perf_counter()
        evs[0].record(stream)
        with torch.cuda.stream(stream):
            graph.replay()
        evs[1].record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - wall0
        # spread: four more replays, each timed on its own (not part of the value)
        reps = []
        for r in range(4):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            with torch.cuda.stream(stream):
                graph.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            reps.append(e0.elapsed_time(e1) / steps)
        ms = evs[0].elapsed_time(evs[1]) / steps
        timing.update(mode=f"one HIP graph of {steps} launches over {n_calls} rotating weight copies",
                      replay_us=[round(ms * 1e3, 3)] + [round(x * 1e3, 3) for x in reps], wall_s_timed=round(wall, 4))
        return ms, timing
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    wall0 = time.perf_counter()
    evs[0].record(stream)
    with torch.cuda.stream(stream):
        for i in range(steps):
            launch(i)
            evs[i + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = evs[0].elapsed_time(evs[-1]) / steps
    per = np.array([evs[i].elapsed_time(evs[i + 1]) for i in range(steps)]) * 1e3
    quart = max(1, steps // 4)
    timing.update(mode="back-to-back launches, an event after each",
                  launch_us={"min": round(float(per.min()), 2), "median": round(float(np.median(per)), 2),
                             "max": round(float(per.max()), 2),
                             "first_vs_last_quartile": round(float(per[:quart].mean() / per[-quart:].mean()), 4)},
                  wall_s_timed=round(wall, 4))
    return ms, timing


# ------------------------------------------------------------------ checker
def check_points(O, fam, M, N, K, host, C, sfa_km):
    """4096 sampled outputs against the oracle on the same quantized bytes."""
    rng = np.random.default_rng(12345)
    rows = rng.integers(0, M, CHECK_POINTS).astype(np.int32)
    cols = rng.integers(0, N, CHECK_POINTS).astype(np.int32)
    A, B, SA, SB = host["A"], host["B_raw"], host["SA"], host["SB"]
    if fam == "mx8":
        ref = O.gemm_mx8_points(A, B, SA, SB, rows, cols)
    elif fam in ("mx4", "mx4a"):
        ref = O.gemm_mx4_points(A, B, SA, SB, rows, cols)
    elif fam in BS8_FAMS:
        ref = O.gemm_bs_e8m0_points(A, B, SA, SB, rows, cols)     # SA physical [K/128][M]
    else:
        ref = O.gemm_bs_fp32_points(A, B, SA, SB, rows, cols, sfa_layout="km" if sfa_km else "mk")
    got = C.float().cpu().numpy()[rows, cols]
    bad, ratio, _ = O.check_tolerance(ref, got)
    return {"points": CHECK_POINTS, "violations": bad, "max_err_over_bound": round(ratio, 4), "ok": bad == 0}


def host_copies(fam, ops, sfa_km):
    """Host arrays of the quantized operands in the oracle's layouts."""
    h = {k: ops[k].cpu().numpy() for k in ("B_raw", "SB")}
    h["A"] = ops.get("A_raw", ops["A"]).cpu().numpy()           # [M][K] for the oracle
    sa = ops["SA"]
    if fam == "mx4a":                                           # the row-major scales
        h["SB"] = ops["SB_raw"].cpu().numpy()
        sa = ops["SA_raw"]
    if fam in BS8_FAMS:
        h["SA"] = sa.t().contiguous().cpu().numpy()               # physical [K/128][M]
    elif fam in ("bs", "lbp") and sfa_km:
        h["SA"] = sa.t().contiguous().cpu().numpy()
    else:
        h["SA"] = sa.contiguous().cpu().numpy()
    return h


def cpu_baseline(O, fam, M, N, K, h, sfa_km, seconds):
    """The oracle's restatement of the reference CPU GEMM on a bounded row
    band of the same GEMM, OpenMP over this host's cores, extrapolated per
    FLOP."""
    A, B, SA, SB = h["A"], h["B_raw"], h["SA"], h["SB"]
    if fam == "mx8":
        fn = lambda r: O.gemm_mx8(A[r], B, SA[r], SB)
        which = "MX8 gemm_ref (mxfp8_gemm/gemm_a8w8_mxfp8_host.cc:96-122)"
    elif fam in ("mx4", "mx4a"):
        fn = lambda r: O.gemm_mx4(A[r], B, SA[r], SB)
        which = "MX4 gemm_ref_gpu grouped form (gemm_a4w4_mxfp4_4wave_host.cc:66-94)"
    elif fam in BS8_FAMS:
        fn = lambda r: O.gemm_bs_e8m0(A[r], B, np.ascontiguousarray(SA[:, r]), SB)
        which = "SNAP gemm_ref (gemm_a8w8_blockscale_bpreshuffle_host.cc:219-248)"
    else:
        if sfa_km:
            fn = lambda r: O.gemm_bs_fp32(A[r], B, np.ascontiguousarray(SA[:, r]), SB, sfa_layout="km")
        else:
            fn = lambda r: O.gemm_bs_fp32(A[r], B, SA[r], SB)
        which = "BPS gemm_ref (gemm_a8w8_blockscale_bpreshuffle_host.cc:66-90)"
    rows, elapsed = 1, 0.0
    while True:
        t = time.perf_counter()
        fn(slice(0, rows))
        elapsed = time.perf_counter() - t
        if elapsed * 2 > seconds or rows >= M:
            break
        rows = min(M, max(rows * 2, int(rows * seconds / max(elapsed, 1e-3) * 0.5)))
    tflops = 2.0 * rows * N * K / elapsed / 1e12
    full = rows >= M
    return {"value": round(tflops, 6), "unit": "TFLOPS", "cores": O.num_threads(), "kind": "port",
            "nproc": os.cpu_count(), "cpu_model": cpu_model(),
            "sample": (f"rows 0..{rows - 1} of the same {M}x{N}x{K} GEMM ({elapsed:.2f} s"
                       + (", the whole GEMM)" if full else ", extrapolated per FLOP)")
                       + f"; oracle restatement of the {which}, OpenMP")}


# ------------------------------------------------------------------ sweep
SWEEP_M = (1, 16, 64, 256, 1024, 4096, 16384)
SWEEP_NK = ((24576, 1536), (32768, 512), (7168, 16384), (4096, 7168), (7168, 2048), (2112, 7168))


def sweep_shapes(which):
    """{(N, K): [M, ...]} of a sweep, in file / table order."""
    import csv
    if which == "configs2":
        return {(n, k): list(SWEEP_M) for n, k in SWEEP_NK}
    groups = {}
    with open(ROOT / "355_1_trans_amd" / "configs" / "dsv4_a8w8_shapes.csv", newline="") as fh:
        for r in csv.DictReader(fh):
            groups.setdefault((int(r["N"]), int(r["K"])), []).append(int(r["M"]))
    return groups


def sweep(args):
    """Block-scale shape sweep for both entry points (library plan, bf16
    out): BASELINE configs[2] (M x (N, K)) or the traced dsv4 shapes.
    HBM-bound shapes (M <= 256) replay a graph over rotating weight copies
    (> 512 MB, beyond the last-level cache); the others launch back to back."""
    import torch
    q = importlib.import_module("355_1_trans_amd")
    L = q.lib()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(dev)
    for (n, k), ms in sweep_shapes(args.sweep).items():
        qb, sb = q.quant_fp8_blockscale(randn((n, k), 1, dev), "128x128")
        bk = q.shuffle_b_kpanel(qb.view(torch.uint8))
        bpp = q.ldsbypass_pack_b(qb.view(torch.uint8))
        kg = k // 128
        for m in ms:
            qa, sa = q.quant_fp8_blockscale(randn((m, k), 0, dev), "1x128")
            qa = qa.view(torch.uint8)
            C = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
            hbm = m <= 256
            for variant, B0 in (("bpreshuffle", bk), ("ldsbypass", bpp)):
                b_bytes = B0.numel() + sb.numel() * 4
                copies = max(2, ROTATE_BYTES // b_bytes + 1) if hbm else 1
                Bs = [B0] + [B0.clone() for _ in range(copies - 1)]
                SBs = [sb] + [sb.clone() for _ in range(copies - 1)]
                fam = "bs" if variant == "bpreshuffle" else "lbp"
                launch_fn, wq = entry_for(L, fam)
                calls = [kargs_for(q, fam, m, n, k, qa, B, C, sa, SB, False) for B, SB in zip(Bs, SBs)]
                wsb = max(1, wq(ctypes.byref(calls[0])))
                ws = torch.zeros((wsb + 255) // 256 * 256, dtype=torch.uint8, device=dev)
                sptr = ctypes.c_void_p(stream.cuda_stream)
                torch.cuda.synchronize()    # inputs made on the default stream; launches on `stream`

                def launch(i):
                    st = launch_fn(ctypes.byref(calls[i % len(calls)]), ws.data_ptr(), ws.numel(), sptr)
                    if st:
                        raise RuntimeError(f"{variant} failed: HIP error {st}")

                flops = 2.0 * m * n * k
                steps = max(8, min(50, int(2e13 / flops)))
                ms, timing = run_timed(launch, len(calls), stream, hbm, steps, max(4, steps // 2), 0.2)
                alg = m * k + sa.numel() * 4 + b_bytes + m * n * 2
                tf = flops / (ms * 1e-3) / 1e12
                gbps = alg / (ms * 1e-3) / 1e9
                print(json.dumps({"sweep": args.sweep, "variant": variant, "M": m, "N": n, "K": k,
                                  "us": round(ms * 1e3, 2), "TFLOPS": round(tf, 1), "mfma_frac": round(tf / 5000.0, 4),
                                  "GBps": round(gbps, 1), "hbm_frac": round(gbps / HBM_GBPS, 4),
                                  "bound": "hbm" if hbm else "mfma", "kernel": q.last_launch(),
                                  "spread_us": timing.get("replay_us") or timing.get("launch_us")}), flush=True)
                del Bs, SBs, calls, ws
            del qa, sa, C
        del qb, sb, bk, bpp
        torch.cuda.empty_cache()


# ------------------------------------------------------------------ grouped decode
GROUP_NK = ((2112, 7168), (4096, 7168), (7168, 2048))


def grouped(args):
    """configs[2]'s decode shapes at one M as one grouped launch against
    the same three GEMMs launched one by one (each with the library plan):
    both as HIP graphs over rotating weight copies (> 512 MB, past the last
    level cache), algorithmic bytes = every A, B, scale and C byte once."""
    import torch
    q = importlib.import_module("355_1_trans_amd")
    L = q.lib()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(dev)
    sptr = ctypes.c_void_p(stream.cuda_stream)
    kind = args.grouped
    fam = {"bpreshuffle": "bs", "ldsbypass": "lbp", "mxfp8": "mx8", "mxfp4": "mx4"}[kind]
    m = args.m or 16
    probs, alg = [], 0
    for i, (n, k) in enumerate(GROUP_NK):
        ops = make_operands(q, fam, m, n, k, dev)
        ops["C"] = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        probs.append((n, k, ops))
        alg += (ops["A"].numel() + ops["SA"].numel() * ops["SA"].element_size() + ops["B"].numel()
                + ops["SB"].numel() * ops["SB"].element_size() + m * n * 2)
    b_bytes = sum(o["B"].numel() + o["SB"].numel() * o["SB"].element_size() for _, _, o in probs)
    copies = max(2, ROTATE_BYTES // b_bytes + 1)
    rot = [[(o["B"], o["SB"]) if c == 0 else (o["B"].clone(), o["SB"].clone()) for _, _, o in probs]
           for c in range(copies)]
    name, ktype = q._GROUPED[kind]
    single_fn, single_q = entry_for(L, fam)
    group_calls, single_calls = [], []
    for c in range(copies):
        ks = [kargs_for(q, fam, m, n, k, o["A"], rot[c][j][0], o["C"], o["SA"], rot[c][j][1], False)
              for j, (n, k, o) in enumerate(probs)]
        group_calls.append((ktype * len(ks))(*ks))
        single_calls.append(ks)
    gws_b = max(256, getattr(L, name + "_workspace_bytes")(group_calls[0], len(probs)))
    gws = torch.zeros(gws_b, dtype=torch.uint8, device=dev)
    sws_b = [max(256, single_q(ctypes.byref(k))) for k in single_calls[0]]
    sws = [torch.zeros(b, dtype=torch.uint8, device=dev) for b in sws_b]
    torch.cuda.synchronize()

    def launch_group(i):
        st = getattr(L, name)(group_calls[i % copies], len(probs), 1, args.group_grid, gws.data_ptr(), gws.numel(),
                              sptr)
        if st:
            raise RuntimeError(f"{name} failed: HIP error {st}")

    kern = {}

    def launch_single(i):
        for j, ka in enumerate(single_calls[i % copies]):
            st = single_fn(ctypes.byref(ka), sws[j].data_ptr(), sws[j].numel(), sptr)
            if st:
                raise RuntimeError(f"single launch {j} failed: HIP error {st}")
            kern[j] = q.last_launch()

    with torch.cuda.stream(stream):
        launch_group(0)
    gkern = q.last_launch()
    steps = args.steps
    ms_g, t_g = run_timed(launch_group, copies, stream, True, steps, args.warmup // 4, args.settle_s / 2)
    ms_s, t_s = run_timed(launch_single, copies, stream, True, steps, args.warmup // 4, args.settle_s / 2)
    check = None
    if not args.no_check:
        import oracle as O
        launch_group(0)
        torch.cuda.synchronize()
        bad, worst = 0, 0.0
        for n, k, o in probs:
            h = host_copies(fam, o, False)
            r = check_points(O, fam, m, n, k, h, o["C"], False)
            bad += r["violations"]
            worst = max(worst, r["max_err_over_bound"])
        check = {"points": CHECK_POINTS * len(probs), "violations": bad, "max_err_over_bound": worst, "ok": bad == 0}
    gb_g, gb_s = alg / (ms_g * 1e-3) / 1e9, alg / (ms_s * 1e-3) / 1e9
    print(json.dumps({
        "grouped": kind, "M": m, "shapes_NK": [list(x) for x in GROUP_NK], "algorithmic_bytes": int(alg),
        "grouped_us": round(ms_g * 1e3, 2), "grouped_GBps": round(gb_g, 1), "grouped_hbm_frac": round(gb_g / HBM_GBPS, 4),
        "singles_us": round(ms_s * 1e3, 2), "singles_GBps": round(gb_s, 1), "singles_hbm_frac": round(gb_s / HBM_GBPS, 4),
        "speedup": round(ms_s / ms_g, 3), "grouped_kernel": gkern, "single_kernels": [kern[j] for j in sorted(kern)],
        "spread_us": {"grouped": t_g.get("replay_us"), "singles": t_s.get("replay_us")}, "check": check}), flush=True)
    if check is not None and not check["ok"]:
        sys.exit(1)


def measure(args, workload, m_over, n_over, k_over, with_cpu):
    """Time one workload (settle, warm up, `--steps` launches) and return its
    JSON record: throughput, roofline block of the dominant kernel, the
    4096-point check and, with_cpu, the CPU baseline."""
    import torch
    q = importlib.import_module("355_1_trans_amd")
    L = q.lib()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    fam, M, N, K, cfg = WORKLOADS[workload]
    M, N, K = m_over or M, n_over or N, k_over or K
    hbm_bound = M <= 256
    ops = make_operands(q, fam, M, N, K, dev, args.sfa_km)
    A, SA, B0, SB0 = ops["A"], ops["SA"], ops["B"], ops["SB"]
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    b_bytes = B0.numel() * B0.element_size() + SB0.numel() * SB0.element_size()
    copies = max(2, ROTATE_BYTES // b_bytes + 1) if hbm_bound else 1
    Bs = [B0] + [B0.clone() for _ in range(copies - 1)]
    SBs = [SB0] + [SB0.clone() for _ in range(copies - 1)]

    launch_fn, wq = entry_for(L, fam)
    calls = [kargs_for(q, fam, M, N, K, A, B, C, SA, SB, args.sfa_km, args.grid_blocks) for B, SB in zip(Bs, SBs)]
    ws_bytes = max(1, wq(ctypes.byref(calls[0])))
    ws = torch.zeros((ws_bytes + 255) // 256 * 256, dtype=torch.uint8, device=dev)
    stream = torch.cuda.Stream(dev)
    sptr = ctypes.c_void_p(stream.cuda_stream)

    def launch(i):
        st = launch_fn(ctypes.byref(calls[i % len(calls)]), ws.data_ptr(), ws.numel(), sptr)
        if st:
            raise RuntimeError(f"{workload} launch failed: HIP error {st}")

    with torch.cuda.stream(stream):
        launch(0)
    kernel = q.last_launch()
    ms, timing = run_timed(launch, len(calls), stream, hbm_bound, args.steps, args.warmup, args.settle_s)
    flops = 2.0 * M * N * K
    tflops = flops / (ms * 1e-3) / 1e12

    kind = "fp4" if fam in ("mx4", "mx4a") else "fp8"
    tag = workload + (f"_m{M}" if m_over else "") + (f"_n{N}" if n_over else "") + (f"_k{K}" if k_over else "")
    if hbm_bound:
        # algorithmic bytes: A, B and both scale arrays read once, C written once
        alg = A.numel() * A.element_size() + SA.numel() * SA.element_size() + b_bytes + C.numel() * 2
        gbps = alg / (ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_GBPS, "unit": "GB/s",
                    "frac": round(gbps / HBM_GBPS, 4), "traffic": traffic_from_profiles(tag),
                    "algorithmic_bytes": int(alg)}
    else:
        peak = PEAK_TFLOPS[kind]
        roofline = {"bound": "mfma", "achieved": round(tflops, 2), "peak": peak, "unit": "TFLOP/s",
                    "frac": round(tflops / peak, 4), "traffic": traffic_from_profiles(tag)}

    check, cpu = None, None
    if not (args.no_check and not with_cpu):
        import oracle as O
        h = host_copies(fam, ops, args.sfa_km)
        if not args.no_check:
            torch.cuda.synchronize()
            check = check_points(O, fam, M, N, K, h, C, args.sfa_km)
        if with_cpu:
            cpu = cpu_baseline(O, fam, M, N, K, h, args.sfa_km, args.cpu_seconds)

    line = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": kind,
        "data": "synthetic N(0,1) (torch GPU generator, seeds 0 / 1), quantized on the GPU per the BASELINE recipe",
        "config": {"workload": f"{NAMES[fam]} M={M} N={N} K={K}, bf16 out " +
                               (f"(BASELINE configs[{cfg}])" if cfg is not None
                                else "(the reference's headline block-scale kernel, BASELINE.md)"),
                   "M": M, "N": N, "K": K, "out": "bf16", "kernel": kernel},
        "timing": timing, "roofline": roofline, "cpu_baseline": cpu, "check": check,
    }
    del Bs, SBs, calls, ws, ops
    torch.cuda.empty_cache()
    return line


# ------------------------------------------------------------------ main
def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU sharding plan is described in DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        # known traffic: 256 MiB read + 256 MiB written per copy launch; the
        # FETCH_SIZE / WRITE_SIZE counters of these launches give the factors
        # that turn the counters into bytes
        x = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        y = torch.empty_like(x)
        for _ in range(5):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration": {"bytes_read": 256 << 20, "bytes_written": 256 << 20,
                                               "launches": 5}}), flush=True)
        return

    if args.sweep:
        sweep(args)
        return
    if args.grouped:
        grouped(args)
        return

    line = measure(args, args.workload, args.m, args.n, args.k, with_cpu=not args.no_cpu)
    failed = [line] if line["check"] is not None and not line["check"]["ok"] else []
    if not args.no_extra and args.workload == "mxfp8_8192" and not (args.m or args.n or args.k):
        # the other BASELINE configs from the same run, so that the driver's
        # record carries them too (GPU time, roofline, kernel, 4096-point check)
        line["extra"] = []
        for wl, m in EXTRA_WORKLOADS:
            x = measure(args, wl, m, None, None, with_cpu=False)
            line["extra"].append({k: x[k] for k in ("value", "unit", "ms_per_step", "dtype", "config", "roofline",
                                                   "check", "timing")})
            if x["check"] is not None and not x["check"]["ok"]:
                failed.append(x)
    print(json.dumps(line), flush=True)
    for x in failed:
        print(f"bench.py: output check FAILED for {x['config']['workload']} ({x['check']['violations']} of "
              f"{CHECK_POINTS} points out of tolerance)", file=sys.stderr)
    if failed:
        sys.exit(1)


if __name__ == "__main__":
    main()
