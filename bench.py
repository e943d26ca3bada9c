"""Throughput of the quantized-GEMM hot path on one MI355X.

Default workload (the configuration the headline
metric is quoted on): MXFP8 TN GEMM, M = N = K = 8192, e4m3 operands with one
E8M0 scale per 32 K elements, bf16 output.  A "step" is one GEMM launch on
synthetic N(0,1) data (seed 0) quantized per the BASELINE recipe; inputs are
resident in HBM before the timed region.

Prints ONE JSON line with the metric, a roofline block for the GEMM kernel
(achieved = algorithmic FLOPs / average launch time measured with HIP events
on the launch stream) and a cpu_baseline block (the CPU oracle's restatement
of the reference CPU GEMM, timed on a bounded row band on this host).
"""
import argparse
import importlib
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "TFLOPS and % of MI355X peak: block-FP8/MXFP8/MXFP4 GEMM at 8192^3 + decode M"
PEAK_TFLOPS = {"fp8": 5000.0, "fp4": 10100.0}
HBM_GBPS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--workload", default="mxfp8_8192",
                   choices=["mxfp8_8192", "mxfp4_8192", "bs_fp32_8192", "bs_c0"])
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    return p.parse_args()


def traffic_from_profiles(kernel_tag):
    """HBM bytes per launch recorded by the committed rocprofv3 PMC summary."""
    f = ROOT / "profiles" / f"{kernel_tag}_pmc.md"
    if not f.exists():
        return None
    m = re.search(r"hbm_bytes_per_launch:\s*([0-9.eE+]+)", f.read_text())
    return float(m.group(1)) if m else None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU sharding plan is described in DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import oracle as O

    q = importlib.import_module("355_1_trans_amd")
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    w = args.workload
    if w in ("mxfp8_8192", "mxfp4_8192", "bs_fp32_8192"):
        M = N = K = 8192
    else:
        M, N, K = 32, 1536, 7168
    a = O.randn((M, K), 0, 0)
    b = O.randn((N, K), 0, 1)

    if w == "mxfp8_8192":
        qa, ea = O.quant_mx8(a)
        qb, eb = O.quant_mx8(b)
        A = torch.from_numpy(qa).to(dev).view(torch.float8_e4m3fn)
        B = torch.from_numpy(qb).to(dev).view(torch.float8_e4m3fn)
        SA, SB = torch.from_numpy(ea).to(dev), torch.from_numpy(eb).to(dev)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        step = lambda: q.gemm_a8w8_mxfp8(A, B, SA, SB, out=out)
        dtype, kind, tag = "fp8", "fp8", "mxfp8_8192"
        workload = "MXFP8 TN GEMM M=N=K=8192, e4m3 x e4m3, E8M0 per 32 K, bf16 out (BASELINE configs[1])"
        cpu_fn = lambda rows: O.gemm_mx8(qa[rows], qb, ea[rows], eb)
    elif w == "mxfp4_8192":
        qa, ea = O.quant_mx4(a)
        qb, eb = O.quant_mx4(b)
        A, B = torch.from_numpy(qa).to(dev), torch.from_numpy(qb).to(dev)
        SA, SB = torch.from_numpy(ea).to(dev), torch.from_numpy(eb).to(dev)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        step = lambda: q.gemm_a4w4_mxfp4(A, B, SA, SB, out=out)
        dtype, kind, tag = "fp4", "fp4", "mxfp4_8192"
        workload = "MXFP4 A4W4 GEMM M=N=K=8192, e2m1 x e2m1, E8M0 per 32 K, bf16 out (BASELINE configs[3])"
        cpu_fn = lambda rows: O.gemm_mx4(qa[rows], qb, ea[rows], eb)
    else:
        qa, sa = O.quant_bs_act(a)
        qb, sb = O.quant_bs_wgt(b)
        A = torch.from_numpy(qa).to(dev).view(torch.float8_e4m3fn)
        Bk = q.shuffle_b_kpanel(torch.from_numpy(qb).to(dev)).view(torch.float8_e4m3fn)
        SA, SB = torch.from_numpy(sa).to(dev), torch.from_numpy(sb).to(dev)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        step = lambda: q.gemm_a8w8_bpreshuffle(A, Bk, SA, SB, out=out)
        dtype, kind, tag = "fp8", "fp8", w
        workload = (f"block-scale FP8 GEMM M={M} N={N} K={K}, fp32 1x128/128x128 scales, K-panel B, bf16 out "
                    f"(BASELINE configs[{0 if w == 'bs_c0' else 2}])")
        cpu_fn = lambda rows: O.gemm_bs_fp32(qa[rows], qb, sa[rows], sb)
    torch.cuda.synchronize()

    flops = 2.0 * M * N * K
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    tflops = flops / (ms * 1e-3) / 1e12

    peak = PEAK_TFLOPS[kind]
    roofline = {"bound": "mfma", "achieved": round(tflops, 2), "peak": peak, "unit": "TFLOP/s",
                "frac": round(tflops / peak, 4), "traffic": traffic_from_profiles(tag)}

    cpu = None
    if not args.no_cpu:
        # bounded row band of the same GEMM on this host's cores, extrapolated per FLOP
        rows, elapsed = 1, 0.0
        while True:
            t = time.perf_counter()
            cpu_fn(slice(0, rows))
            elapsed = time.perf_counter() - t
            if elapsed * 2 > args.cpu_seconds or rows >= M:
                break
            rows = min(M, max(rows * 2, int(rows * args.cpu_seconds / max(elapsed, 1e-3) * 0.5)))
        cpu_tflops = 2.0 * rows * N * K / elapsed / 1e12
        cpu = {"value": round(cpu_tflops, 6), "unit": "TFLOPS", "cores": O.num_threads(), "kind": "port",
               "sample": f"rows 0..{rows - 1} of the same {M}x{N}x{K} GEMM ({elapsed:.1f} s, extrapolated "
                         f"per FLOP); oracle restatement of the reference CPU gemm_ref, OpenMP"}

    line = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dtype, "data": "synthetic N(0,1) seed 0, BASELINE quantization recipe",
        "config": {"workload": workload, "M": M, "N": N, "K": K, "out": "bf16"},
        "roofline": roofline, "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 4),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
