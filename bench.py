"""Throughput of the quantized-GEMM hot path on one MI355X.

Default workload (the configuration the headline
metric is quoted on): MXFP8 TN GEMM, M = N = K = 8192, e4m3 operands with one
E8M0 scale per 32 K elements, bf16 output.  A "step" is one GEMM launch on
synthetic N(0,1) data (seed 0) quantized per the BASELINE recipe; inputs are
resident in HBM before the timed region.  Other workloads (--workload) cover
configs[0] (block-scale FP8 decode, both B layouts), configs[3] (MXFP4
8192^3) and configs[4] (MXFP4 decode).

Launches go straight through the C ABI with prebuilt argument blocks.  The
MFMA-bound 8192^3 workloads are timed launch by launch; the HBM-bound decode
workloads are captured in a HIP graph over rotating copies of the weights
(more bytes than the 256 MB last-level cache, so B streams from HBM) and the
replays are timed.  Either way the timing is HIP events on the launch stream.

Prints ONE JSON line with the metric, a roofline block for the GEMM kernel
(algorithmic FLOPs or bytes per launch / average launch time) and a
cpu_baseline block (the CPU oracle's restatement of the reference CPU GEMM,
timed on a bounded row band on this host).
"""
import argparse
import ctypes
import importlib
import json
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

WORKLOADS = {
    # name: (family, M, N, K, BASELINE config index)
    "mxfp8_8192": ("mx8", 8192, 8192, 8192, 1),
    "mxfp4_8192": ("mx4", 8192, 8192, 8192, 3),
    "bs_fp32_8192": ("bs", 8192, 8192, 8192, 2),
    "bs_c0": ("bs", 32, 1536, 7168, 0),
    "ldsbypass_c0": ("lbp", 32, 1536, 7168, 0),
    "mxfp4_c4": ("mx4", 32, 7168, 16384, 4),
    # the reference's headline block-scale kernel (E8M0 1x128 / 128x128 scales,
    # shuffle_weight(16,16) B: 3.31 PFLOPS at 8192^3)
    "bs_e8m0_8192": ("bs8", 8192, 8192, 8192, None),
}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--workload", default="mxfp8_8192", choices=sorted(WORKLOADS))
    p.add_argument("--m", type=int, default=None, help="override M (decode sweeps)")
    p.add_argument("--n", type=int, default=None, help="override N")
    p.add_argument("--k", type=int, default=None, help="override K")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--sfa-km", action="store_true",
                   help="block-scale fp32 workloads: pass A's scales column-major [K/128][M] (the reference's "
                        "layout) instead of BASELINE's row-major [M][K/128]")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--sweep", action="store_true",
                   help="BASELINE configs[2]: time the block-scale shape sweep (bpreshuffle and ldsbypass), "
                        "one JSON line per shape")
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


SWEEP_M = (1, 16, 64, 256, 1024, 4096, 16384)
SWEEP_NK = ((24576, 1536), (32768, 512), (7168, 16384), (4096, 7168), (7168, 2048), (2112, 7168))


def _gpu_quant_bs(rows, k, block_rows, gen, dev):
    """N(0,1) data quantized to e4m3 with one fp32 scale (amax / 448) per
    block_rows x 128 block, on the GPU (the sweep's operands are too large for
    the host quantizer to be quick); returns (uint8 [rows, k], fp32 scales
    [ceil(rows / block_rows), k / 128])."""
    import torch
    rp = -(-rows // block_rows) * block_rows
    x = torch.randn((rp, k), generator=gen, device=dev)
    blk = x.view(rp // block_rows, block_rows, k // 128, 128)
    sc = blk.abs().amax(dim=(1, 3)).clamp_min(1e-12) / 448.0
    qx = (blk / sc[:, None, :, None]).to(torch.float8_e4m3fn).view(rp, k)[:rows]
    return qx.contiguous().view(torch.uint8), sc.contiguous()


def _gpu_quant_e8m0(rows, k, block_rows, gen, dev):
    """N(0,1) data quantized to e4m3 with one E8M0 scale 2^ceil(log2(amax /
    448)) per block_rows x 128 block, on the GPU; returns (uint8 [rows, k],
    uint8 exponent codes [ceil(rows / block_rows), k / 128])."""
    import torch
    rp = -(-rows // block_rows) * block_rows
    x = torch.randn((rp, k), generator=gen, device=dev)
    blk = x.view(rp // block_rows, block_rows, k // 128, 128)
    e = torch.ceil(torch.log2(blk.abs().amax(dim=(1, 3)).clamp_min(1e-30) / 448.0)).clamp(-127, 127)
    qx = (blk / torch.exp2(e)[:, None, :, None]).to(torch.float8_e4m3fn).view(rp, k)[:rows]
    return qx.contiguous().view(torch.uint8), (e + 127).to(torch.uint8).contiguous()


def _time_calls(calls, ws, stream, graph_mode, steps, warmup):
    """Average launch time (ms) of `steps` launches cycling through `calls`:
    back-to-back launches, or (graph_mode) one HIP graph replay of them."""
    import torch
    sptr = ctypes.c_void_p(stream.cuda_stream)

    def launch(i):
        fn, ka = calls[i % len(calls)]
        st = fn(ctypes.byref(ka), 1, ws.data_ptr(), ws.numel(), sptr)
        if st:
            raise RuntimeError(f"{fn.__name__} failed: HIP error {st}")

    with torch.cuda.stream(stream):
        launch(0)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    if graph_mode:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                launch(i)
        with torch.cuda.stream(stream):
            for i in range(warmup):
                launch(i)
            graph.replay()
        torch.cuda.synchronize()
        e0.record(stream)
        with torch.cuda.stream(stream):
            graph.replay()
        e1.record(stream)
    else:
        with torch.cuda.stream(stream):
            for i in range(warmup):
                launch(i)
        torch.cuda.synchronize()
        e0.record(stream)
        with torch.cuda.stream(stream):
            for i in range(steps):
                launch(i)
        e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def sweep(args):
    """M x (N, K) for both block-scale entry points.
    HBM-bound shapes (M <= 256) replay a graph over rotating weight copies
    (> 512 MB, beyond the last-level cache); the others launch back to back."""
    import torch
    q = importlib.import_module("355_1_trans_amd")
    L = q.lib()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    stream = torch.cuda.Stream(dev)
    for n, k in SWEEP_NK:
        qb, sb = _gpu_quant_bs(n, k, 128, gen, dev)
        bk = q.shuffle_b_kpanel(qb)
        bpp = q.ldsbypass_repack(bk)
        kg = k // 128
        for m in SWEEP_M:
            qa, sa = _gpu_quant_bs(m, k, 1, gen, dev)
            C = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
            hbm = m <= 256
            for variant, B0 in (("bpreshuffle", bk), ("ldsbypass", bpp)):
                b_bytes = B0.numel() + sb.numel() * 4
                copies = max(2, ROTATE_BYTES // b_bytes + 1) if hbm else 1
                Bs = [B0] + [B0.clone() for _ in range(copies - 1)]
                SBs = [sb] + [sb.clone() for _ in range(copies - 1)]
                calls = []
                for B, SB in zip(Bs, SBs):
                    if variant == "bpreshuffle":
                        ka = q.Kargs(qa.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, 1, k, 128, n, m * k, n * k,
                                     m * n, sa.data_ptr(), SB.data_ptr(), 1 if m > 1 else m, kg, m * kg, SB.numel())
                        fn, wq = L.gemm_a8w8_blockscale_bpreshuffle, L.gemm_a8w8_blockscale_bpreshuffle_workspace_bytes
                    else:
                        ka = q.LdsBypassKargs(qa.data_ptr(), None, B.data_ptr(), C.data_ptr(), m, n, k, 1, k, 128, n,
                                              m * k, n * k, m * n, sa.data_ptr(), SB.data_ptr(), 1 if m > 1 else m, kg,
                                              m * kg, SB.numel(), B.numel())
                        fn, wq = L.gemm_a8w8_blockscale_ldsbypass, L.gemm_a8w8_blockscale_ldsbypass_workspace_bytes
                    calls.append((fn, ka))
                wsb = max(1, wq(ctypes.byref(calls[0][1])))
                ws = torch.zeros((wsb + 255) // 256 * 256, dtype=torch.uint8, device=dev)
                flops = 2.0 * m * n * k
                steps = max(8, min(50, int(2e13 / flops)))
                ms = _time_calls(calls, ws, stream, hbm, steps, max(4, steps // 2))
                alg = m * k + sa.numel() * 4 + b_bytes + m * n * 2
                tf = flops / (ms * 1e-3) / 1e12
                gbps = alg / (ms * 1e-3) / 1e9
                print(json.dumps({"sweep": "configs[2]", "variant": variant, "M": m, "N": n, "K": k,
                                  "us": round(ms * 1e3, 2), "TFLOPS": round(tf, 1), "mfma_frac": round(tf / 5000.0, 4),
                                  "GBps": round(gbps, 1), "hbm_frac": round(gbps / HBM_GBPS, 4),
                                  "bound": "hbm" if hbm else "mfma"}), flush=True)
                del Bs, SBs, calls, ws
            del qa, sa, C
        del qb, sb, bk, bpp
        torch.cuda.empty_cache()


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

    import oracle as O

    q = importlib.import_module("355_1_trans_amd")
    L = q.lib()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    fam, M, N, K, cfg = WORKLOADS[args.workload]
    if args.m:
        M = args.m
    if args.n:
        N = args.n
    if args.k:
        K = args.k
    hbm_bound = M <= 256
    kg32, kg128 = K // 32, K // 128
    if fam == "bs8":
        # N(0,1) quantized on the GPU with E8M0 block scales 2^ceil(log2(amax / 448))
        gen = torch.Generator(device=dev)
        gen.manual_seed(0)
        qa, sa = _gpu_quant_e8m0(M, K, 1, gen, dev)
        qb, sb = _gpu_quant_e8m0(N, K, 128, gen, dev)
        A = qa
        SA = sa.t().contiguous()                        # physical [K/128][M], stride_sfa = M
        B0 = q.shuffle_weight_16x16(qb)
        SB0 = sb
        a = b = None
    else:
        a = O.randn((M, K), 0, 0)
        b = O.randn((N, K), 0, 1)

    # quantize once on the host (BASELINE recipe); device copies of the operands
    if fam == "bs8":
        pass
    elif fam == "mx8":
        qa, sa = O.quant_mx8(a)
        qb, sb = O.quant_mx8(b)
    elif fam == "mx4":
        qa, sa = O.quant_mx4(a)
        qb, sb = O.quant_mx4(b)
    else:
        qa, sa = O.quant_bs_act(a)
        qb, sb = O.quant_bs_wgt(b)
    if fam != "bs8":
        A = torch.from_numpy(qa).to(dev)
        SA = torch.from_numpy(np.ascontiguousarray(sa.T) if args.sfa_km else sa).to(dev)
        B0 = torch.from_numpy(qb).to(dev)
        SB0 = torch.from_numpy(sb).to(dev)
    if fam == "bs":
        B0 = q.shuffle_b_kpanel(B0)
    elif fam == "lbp":
        B0 = q.ldsbypass_repack(q.shuffle_b_kpanel(B0))
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    b_bytes = B0.numel() * B0.element_size() + SB0.numel() * SB0.element_size()
    copies = max(2, ROTATE_BYTES // b_bytes + 1) if hbm_bound else 1
    Bs = [B0] + [B0.clone() for _ in range(copies - 1)]
    SBs = [SB0] + [SB0.clone() for _ in range(copies - 1)]

    kb = K // 2 if fam == "mx4" else K
    calls = []
    for B, SB in zip(Bs, SBs):
        if fam in ("mx8", "mx4"):
            args_ = q.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, 1, kb, kb, N, M * kb, N * kb, M * N,
                            SA.data_ptr(), SB.data_ptr(), kg32, kg32, M * kg32, N * kg32)
            fn = L.gemm_a8w8_mxfp8 if fam == "mx8" else L.gemm_a4w4_mxfp4
            wq = L.gemm_a8w8_mxfp8_workspace_bytes if fam == "mx8" else L.gemm_a4w4_mxfp4_workspace_bytes
        elif fam == "bs8":
            args_ = q.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, 1, K, K, N, M * K, N * K, M * N,
                            SA.data_ptr(), SB.data_ptr(), M, kg128, M * kg128, SB.numel())

            def fn(ka, out_bf16, ws_ptr, ws_bytes, stream):
                return L.launch_blockscale_bpreshuffle(ka, out_bf16, 0, stream)
            fn.__name__ = "launch_blockscale_bpreshuffle"

            def wq(ka):
                return 0
        elif fam == "bs":
            args_ = q.Kargs(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, 1, K, 128, N, M * K, N * K, M * N,
                            SA.data_ptr(), SB.data_ptr(), M if args.sfa_km else (1 if M > 1 else M), kg128,
                            M * kg128, SB.numel())
            fn, wq = L.gemm_a8w8_blockscale_bpreshuffle, L.gemm_a8w8_blockscale_bpreshuffle_workspace_bytes
        else:
            args_ = q.LdsBypassKargs(A.data_ptr(), None, B.data_ptr(), C.data_ptr(), M, N, K, 1, K, 128, N, M * K,
                                     N * K, M * N, SA.data_ptr(), SB.data_ptr(),
                                     M if args.sfa_km else (1 if M > 1 else M), kg128, M * kg128, SB.numel(),
                                     B.numel())
            fn, wq = L.gemm_a8w8_blockscale_ldsbypass, L.gemm_a8w8_blockscale_ldsbypass_workspace_bytes
        calls.append((fn, args_))
    ws_bytes = max(1, wq(ctypes.byref(calls[0][1])))
    ws = torch.zeros((ws_bytes + 255) // 256 * 256, dtype=torch.uint8, device=dev)

    stream = torch.cuda.Stream(dev)
    sptr = ctypes.c_void_p(stream.cuda_stream)

    def launch(i):
        fn, ka = calls[i % len(calls)]
        st = fn(ctypes.byref(ka), 1, ws.data_ptr(), ws.numel(), sptr)
        if st:
            raise RuntimeError(f"{fn.__name__} failed: HIP error {st}")

    with torch.cuda.stream(stream):
        launch(0)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    if hbm_bound:
        # one graph of exactly `steps` launches over the rotating weight copies;
        # a warm replay, then the timed replay
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(args.steps):
                launch(i)
        with torch.cuda.stream(stream):
            for i in range(args.warmup):
                launch(i)
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        with torch.cuda.stream(stream):
            graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
    else:
        with torch.cuda.stream(stream):
            for i in range(args.warmup):
                launch(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        with torch.cuda.stream(stream):
            for i in range(args.steps):
                launch(i)
        e1.record(stream)
        torch.cuda.synchronize()
    launches = args.steps
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / launches
    flops = 2.0 * M * N * K
    tflops = flops / (ms * 1e-3) / 1e12

    kind = "fp4" if fam == "mx4" else "fp8"
    tag = args.workload + (f"_m{M}" if args.m else "") + (f"_n{N}" if args.n else "") + (f"_k{K}" if args.k else "")
    if hbm_bound:
        # algorithmic bytes: A, B and both scale arrays read once, C written once
        alg = (A.numel() * A.element_size() + SA.numel() * SA.element_size() + b_bytes + C.numel() * 2)
        gbps = alg / (ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_GBPS, "unit": "GB/s",
                    "frac": round(gbps / HBM_GBPS, 4), "traffic": traffic_from_profiles(tag),
                    "algorithmic_bytes": alg}
    else:
        peak = PEAK_TFLOPS[kind]
        roofline = {"bound": "mfma", "achieved": round(tflops, 2), "peak": peak, "unit": "TFLOP/s",
                    "frac": round(tflops / peak, 4), "traffic": traffic_from_profiles(tag)}

    cpu = None
    if not args.no_cpu:
        if fam == "mx8":
            cpu_fn = lambda rows: O.gemm_mx8(qa[rows], qb, sa[rows], sb)
        elif fam == "mx4":
            cpu_fn = lambda rows: O.gemm_mx4(qa[rows], qb, sa[rows], sb)
        elif fam == "bs8":
            qa_h, qb_h = qa.cpu().numpy(), qb.cpu().numpy()
            sa_h, sb_h = SA.cpu().numpy(), sb.cpu().numpy()
            cpu_fn = lambda rows: O.gemm_bs_e8m0(qa_h[rows], qb_h, np.ascontiguousarray(sa_h[:, rows]), sb_h)
        else:
            cpu_fn = lambda rows: O.gemm_bs_fp32(qa[rows], qb, sa[rows], sb)
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

    names = {"mx8": "MXFP8 TN GEMM, e4m3 x e4m3, E8M0 per 32 K",
             "mx4": "MXFP4 A4W4 GEMM, e2m1 x e2m1, E8M0 per 32 K",
             "bs": "block-scale FP8 GEMM, fp32 1x128 / 128x128 scales, K-panel B (bpreshuffle)",
             "lbp": "block-scale FP8 GEMM, fp32 1x128 / 128x128 scales, fragment-order B'' (ldsbypass)",
             "bs8": "block-scale FP8 GEMM, E8M0 1x128 / 128x128 scales, shuffle_weight(16,16) B"}
    line = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOPS", "n_gpus": 1, "steps": launches,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": kind, "data": "synthetic N(0,1) seed 0, BASELINE quantization recipe",
        "config": {"workload": f"{names[fam]} M={M} N={N} K={K}, bf16 out " +
                               (f"(BASELINE configs[{cfg}])" if cfg is not None
                                else "(the reference's headline block-scale kernel, BASELINE.md)"),
                   "M": M, "N": N, "K": K, "out": "bf16",
                   "timing": ("one HIP graph of the timed launches over %d rotating weight copies" % len(calls))
                   if hbm_bound else "back-to-back launches"},
        "roofline": roofline, "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 4),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
