"""Kernel tuner: times every kernel id (QGEMM_KID_*) of an entry point on a
list of (M, N, K) shapes.

    python -m 355_1_trans_amd.tune [--family bs] [--variant bpreshuffle|ldsbypass]
                                   [--shapes CSV | --grid NS:KS:MS] [--out CSV] [--summary MD]
    python -m 355_1_trans_amd.tune --family mx4|mx8 [--shapes CSV | --grid NS:KS:MS] [--summary MD]

fp32 block scales (``--family bs``, the default) write the tuned table that
``opus.gemm_a8w8_bpreshuffle_opus`` reads (the reference's tuning loop:
opus_a8w8_bpreshuffle_integration_and_benchmark.md section 4.2-4.3, same
CSV schema); default shapes: configs/dsv4_a8w8_shapes.csv, the 125 a8w8
shapes traced from DeepSeek-V4 inference
(/root/reference/dsv4_a8w8_all_traced_shapes.csv).  The MX families time
the MXFP4 / MXFP8 entries' ids (the evidence behind the MX planner) and
print the same per-shape lines; ``--grid 24576,32768:1536:32,64`` is the
cross product of comma lists of N, K and M.

Inputs follow the BASELINE recipes on the GPU (N(0,1) data; 1x128
activation and 128x128 weight blocks with scale = amax / 448, or E8M0 per 32
K elements).  Each kernel's output is checked against a float32 torch
reference of the dequantized operands with the BASELINE tolerance
(|y - ref| <= 2^-7 |ref| + 1e-3 rms(ref)); a kernel with any violation is
not eligible.  HBM-bound shapes (M <= 256) are timed as one HIP graph over
rotating weight copies (> 512 MB, beyond the last-level cache), the others
as back-to-back launches, after a short clock-settle phase.  One progress
line per shape goes to stdout.
"""
import argparse
import csv
import ctypes
import importlib
import json
import sys
import time
from pathlib import Path

import torch

PKG = Path(__file__).resolve().parent
CONFIGS = PKG / "configs"
ROTATE_BYTES = 512 << 20
HBM_GBPS, FP8_TFLOPS = 8000.0, 5000.0
SCHEMA = ["gfx", "cu_num", "M", "N", "K", "bias", "dtype", "outdtype", "scaleAB", "bpreshuffle", "libtype",
          "solidx", "splitK", "us", "kernelName", "err_ratio", "tflops", "bw"]


def _pkg():
    if str(PKG.parent) not in sys.path:
        sys.path.insert(0, str(PKG.parent))
    return importlib.import_module(PKG.name)


def _randn(shape, seed, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.randn(shape, generator=g, device=dev, dtype=torch.float32)


def _dequant(q8, scale, rows_per_block):
    """float32 of e4m3 codes times their block scales (128 K per block)."""
    x = q8.view(torch.float8_e4m3fn).float()
    s = scale.repeat_interleave(128, dim=1)[:, : x.shape[1]]
    if rows_per_block > 1:
        s = s.repeat_interleave(rows_per_block, dim=0)[: x.shape[0]]
    return x * s


_E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def _dequant_mx(q8, e, fp4):
    """float32 of MX codes [rows, K or K/2] times their E8M0 scales (32 K per
    group); fp4 element 2i is the low nibble of byte i."""
    if fp4:
        lut = torch.tensor(_E2M1 + tuple(-v for v in _E2M1), device=q8.device)
        lo, hi = (q8 & 15).long(), (q8 >> 4).long()
        x = torch.stack((lut[lo], lut[hi]), dim=-1).reshape(q8.shape[0], -1)
    else:
        x = q8.view(torch.float8_e4m3fn).float()
    return x * torch.exp2(e.float() - 127.0).repeat_interleave(32, dim=1)[:, : x.shape[1]]


def _violations(y, ref):
    rms = ref.pow(2).mean().sqrt()
    bound = ref.abs() * (2.0 ** -7) + 1e-3 * rms
    return int(((y.float() - ref).abs() > bound).sum())


def _time(launch, n_calls, stream, graph_mode, settle_s=0.15):
    """us per launch: settle, warm up, then a timed run."""
    flops_steps = 20
    with torch.cuda.stream(stream):
        launch(0)
    torch.cuda.synchronize()
    if graph_mode:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(flops_steps):
                launch(i)
        run = lambda: graph.replay()
    else:
        def run():
            for i in range(flops_steps):
                launch(i)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < settle_s:
        with torch.cuda.stream(stream):
            run()
        torch.cuda.synchronize()
    best = None
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        with torch.cuda.stream(stream):
            run()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / flops_steps
        best = us if best is None else min(best, us)
    return best


def tune_shape(q, m, n, k, variant, kids, dev, stream):
    """Per kernel id: dict(us, violations, kernel) or None when the id does
    not take the shape."""
    L = q.lib()
    qa, sa = q.quant_fp8_blockscale(_randn((m, k), 0, dev), "1x128")
    qb, sb = q.quant_fp8_blockscale(_randn((n, k), 1, dev), "128x128")
    ref = _dequant(qa.view(torch.uint8), sa, 1) @ _dequant(qb.view(torch.uint8), sb, 128).t()
    qa = qa.view(torch.uint8)
    b0 = q.shuffle_b_kpanel(qb.view(torch.uint8)).reshape(-1) if variant == "bpreshuffle" else \
        q.ldsbypass_pack_b(qb.view(torch.uint8))
    del qb
    hbm = m <= 256
    b_bytes = b0.numel() + sb.numel() * 4
    copies = max(2, ROTATE_BYTES // b_bytes + 1) if hbm else 1
    Bs = [b0] + [b0.clone() for _ in range(copies - 1)]
    SBs = [sb] + [sb.clone() for _ in range(copies - 1)]
    C = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    kg = k // 128
    if variant == "bpreshuffle":
        calls = [q.Kargs(qa.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, 1, k, 128, n, m * k, n * k, m * n,
                         sa.data_ptr(), SB.data_ptr(), 1 if m > 1 else m, kg, m * kg, SB.numel())
                 for B, SB in zip(Bs, SBs)]
        entry, query = L.gemm_a8w8_blockscale_bpreshuffle_kid, L.gemm_a8w8_blockscale_bpreshuffle_kid_workspace_bytes
    else:
        calls = [q.LdsBypassKargs(qa.data_ptr(), None, B.data_ptr(), C.data_ptr(), m, n, k, 1, k, 128, n, m * k,
                                  n * k, m * n, sa.data_ptr(), SB.data_ptr(), 1 if m > 1 else m, kg, m * kg,
                                  SB.numel(), B.numel())
                 for B, SB in zip(Bs, SBs)]
        entry, query = L.gemm_a8w8_blockscale_ldsbypass_kid, L.gemm_a8w8_blockscale_ldsbypass_kid_workspace_bytes
    sptr = ctypes.c_void_p(stream.cuda_stream)
    # the kernels run on `stream`: the inputs, the reference and the
    # temporaries freed on the default stream must be done first (C may
    # reuse a freed temporary's memory)
    torch.cuda.synchronize()
    res = {}
    for kid in kids:
        need = query(ctypes.byref(calls[0]), kid)
        ws = torch.zeros(max(256, (need + 255) // 256 * 256), dtype=torch.uint8, device=dev)
        wp = ws.data_ptr() if need else None
        with torch.cuda.stream(stream):
            st = entry(ctypes.byref(calls[0]), 1, kid, wp, need, sptr)
        if st:
            res[kid] = None
            continue
        torch.cuda.synchronize()
        kernel = q.last_launch()
        bad = _violations(C, ref)

        def launch(i, kid=kid, wp=wp, need=need):
            s = entry(ctypes.byref(calls[i % len(calls)]), 1, kid, wp, need, sptr)
            if s:
                raise RuntimeError(f"kernel id {kid} failed: HIP error {s}")

        us = _time(launch, len(calls), stream, hbm)
        res[kid] = {"us": us, "violations": bad, "kernel": kernel}
        del ws
    alg = m * k + sa.numel() * 4 + b_bytes + m * n * 2
    del Bs, SBs, calls, ref, C, qa, sa
    torch.cuda.empty_cache()
    return res, alg


MX_KIDS = {0: "auto", 1: "tile256", 2: "mid128", 3: "skinny", 4: "decode", 5: "burst", 6: "stream", 7: "band",
           8: "quad", 9: "runs", 10: "slice"}


def tune_shape_mx(q, m, n, k, fp4, kids, dev, stream):
    """tune_shape for the MXFP4 / MXFP8 entries (row-major operands and
    scales)."""
    L = q.lib()
    quant = q.quant_mxfp4 if fp4 else q.quant_mxfp8
    qa, sa = quant(_randn((m, k), 0, dev))
    qb, sb = quant(_randn((n, k), 1, dev))
    qa, qb = qa.view(torch.uint8), qb.view(torch.uint8)
    ref = _dequant_mx(qa, sa, fp4) @ _dequant_mx(qb, sb, fp4).t()
    kb = k // 2 if fp4 else k
    hbm = m <= 256
    b_bytes = qb.numel() + sb.numel()
    copies = max(2, ROTATE_BYTES // b_bytes + 1) if hbm else 1
    Bs = [qb] + [qb.clone() for _ in range(copies - 1)]
    SBs = [sb] + [sb.clone() for _ in range(copies - 1)]
    C = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    kg = k // 32
    calls = [q.Kargs(qa.data_ptr(), B.data_ptr(), C.data_ptr(), m, n, k, 1, kb, kb, n, m * kb, n * kb, m * n,
                     sa.data_ptr(), SB.data_ptr(), kg, kg, m * kg, n * kg)
             for B, SB in zip(Bs, SBs)]
    name = "gemm_a4w4_mxfp4_kid" if fp4 else "gemm_a8w8_mxfp8_kid"
    entry, query = getattr(L, name), getattr(L, name + "_workspace_bytes")
    sptr = ctypes.c_void_p(stream.cuda_stream)
    torch.cuda.synchronize()
    res = {}
    for kid in kids:
        need = query(ctypes.byref(calls[0]), kid)
        ws = torch.zeros(max(256, (need + 255) // 256 * 256), dtype=torch.uint8, device=dev)
        wp = ws.data_ptr() if need else None
        with torch.cuda.stream(stream):
            st = entry(ctypes.byref(calls[0]), 1, kid, wp, need, sptr)
        if st:
            res[kid] = None
            continue
        torch.cuda.synchronize()
        kernel = q.last_launch()
        bad = _violations(C, ref)

        def launch(i, kid=kid, wp=wp, need=need):
            s2 = entry(ctypes.byref(calls[i % len(calls)]), 1, kid, wp, need, sptr)
            if s2:
                raise RuntimeError(f"kernel id {kid} failed: HIP error {s2}")

        us = _time(launch, len(calls), stream, hbm)
        res[kid] = {"us": us, "violations": bad, "kernel": kernel}
        del ws
    alg = qa.numel() + sa.numel() + b_bytes + m * n * 2
    del Bs, SBs, calls, ref, C, qa, sa
    torch.cuda.empty_cache()
    return res, alg


def _grid(spec):
    ns, ks, ms = (tuple(int(x) for x in part.split(",")) for part in spec.split(":"))
    return [(m, n, k) for n in ns for k in ks for m in ms]


def main_mx(args, q, dev, stream):
    fp4 = args.family == "mx4"
    kids = [int(x) for x in args.kids.split(",")] if args.kids else list(MX_KIDS)
    if args.grid:
        shapes = _grid(args.grid)
    else:
        with open(args.shapes, newline="") as fh:
            shapes = [(int(r["M"]), int(r["N"]), int(r["K"])) for r in csv.DictReader(fh)]
    if args.limit:
        shapes = shapes[: args.limit]
    table = []
    for i, (m, n, k) in enumerate(shapes):
        res, alg = tune_shape_mx(q, m, n, k, fp4, kids, dev, stream)
        ok = {kid: r for kid, r in res.items() if r and r["violations"] == 0}
        best = min(ok, key=lambda kk: ok[kk]["us"]) if ok else None
        auto = res.get(0)
        print(json.dumps({"i": i, "M": m, "N": n, "K": k, "family": args.family,
                          "us": {MX_KIDS[kk]: (round(r["us"], 2) if r else None) for kk, r in res.items()},
                          "violations": {MX_KIDS[kk]: r["violations"] for kk, r in res.items() if r},
                          "best": MX_KIDS.get(best), "auto_kernel": auto["kernel"] if auto else None}), flush=True)
        if best is not None:
            table.append((m, n, k, auto, best, ok[best], alg))
    if args.summary:
        with open(args.summary, "w") as fh:
            fh.write("| M | N | K | auto us | auto kernel | best id | best us | best/auto | GB/s | frac of HBM |\n")
            fh.write("|---|---|---|---|---|---|---|---|---|---|\n")
            for m, n, k, auto, best, r, alg in table:
                a_us = auto["us"] if auto else float("nan")
                bw = alg / r["us"] / 1e3
                fh.write(f"| {m} | {n} | {k} | {a_us:.2f} | {auto['kernel'] if auto else '-'} | {MX_KIDS[best]} | "
                         f"{r['us']:.2f} | {r['us'] / a_us:.3f} | {bw:.0f} | {bw / HBM_GBPS:.3f} |\n")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--family", default="bs", choices=["bs", "mx4", "mx8"],
                    help="bs: fp32 block scales (tuned table); mx4 / mx8: the MX entries' kernel ids")
    ap.add_argument("--shapes", default=str(CONFIGS / "dsv4_a8w8_shapes.csv"))
    ap.add_argument("--grid", default=None, help="N,N..:K,K..:M,M.. cross product instead of --shapes")
    ap.add_argument("--variant", default="bpreshuffle", choices=["bpreshuffle", "ldsbypass"])
    ap.add_argument("--kids", default=None, help="comma list of kernel ids (default: all of the family)")
    ap.add_argument("--out", default=None, help="tuned CSV (default configs/qgemm_a8w8_<variant>_tuned.csv)")
    ap.add_argument("--summary", default=None, help="also write a markdown summary here")
    ap.add_argument("--limit", type=int, default=0, help="first N shapes only")
    args = ap.parse_args()
    q = _pkg()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(dev)
    if args.family != "bs":
        main_mx(args, q, dev, stream)
        return
    props = torch.cuda.get_device_properties(dev)
    gfx = getattr(props, "gcnArchName", "gfx950").split(":")[0]
    cu_num = props.multi_processor_count
    kids = [int(x) for x in (args.kids or "0,1,2,3,4,5").split(",")]
    if args.grid:
        shapes = _grid(args.grid)
    else:
        with open(args.shapes, newline="") as fh:
            shapes = [(int(r["M"]), int(r["N"]), int(r["K"])) for r in csv.DictReader(fh)]
    if args.limit:
        shapes = shapes[: args.limit]
    rows, table = [], []
    for i, (m, n, k) in enumerate(shapes):
        res, alg = tune_shape(q, m, n, k, args.variant, kids, dev, stream)
        ok = {kid: r for kid, r in res.items() if r and r["violations"] == 0}
        auto = res.get(0)
        best = min(ok, key=lambda kk: ok[kk]["us"]) if ok else None
        line = {"i": i, "M": m, "N": n, "K": k, "variant": args.variant,
                "us": {q.opus.KID_NAMES[kk]: (round(r["us"], 2) if r else None) for kk, r in res.items()},
                "violations": {q.opus.KID_NAMES[kk]: r["violations"] for kk, r in res.items() if r},
                "best": q.opus.KID_NAMES.get(best), "auto_kernel": auto["kernel"] if auto else None}
        print(json.dumps(line), flush=True)
        if best is None:
            continue
        r = ok[best]
        tf = 2.0 * m * n * k / r["us"] / 1e6
        bw = alg / r["us"] / 1e3
        rows.append({"gfx": gfx, "cu_num": cu_num, "M": m, "N": n, "K": k, "bias": False,
                     "dtype": "torch.float8_e4m3fn", "outdtype": "torch.bfloat16", "scaleAB": True,
                     "bpreshuffle": args.variant == "bpreshuffle", "libtype": "qgemm", "solidx": best,
                     "splitK": 0, "us": round(r["us"], 2), "kernelName": r["kernel"], "err_ratio": 0.0,
                     "tflops": round(tf, 1), "bw": round(bw, 1)})
        table.append((m, n, k, auto, best, r, tf, bw))
    out = Path(args.out) if args.out else CONFIGS / f"qgemm_a8w8_{args.variant}_tuned.csv"
    with open(out, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=SCHEMA)
        w.writeheader()
        w.writerows(rows)
    print(json.dumps({"tuned_rows": len(rows), "out": str(out)}), flush=True)
    if args.summary:
        with open(args.summary, "w") as fh:
            fh.write("| M | N | K | auto us | auto kernel | best id | best us | gain | TFLOPS | GB/s | frac |\n")
            fh.write("|---|---|---|---|---|---|---|---|---|---|---|\n")
            for m, n, k, auto, best, r, tf, bw in table:
                frac = bw / HBM_GBPS if m <= 256 else tf / FP8_TFLOPS
                a_us = auto["us"] if auto else float("nan")
                fh.write(f"| {m} | {n} | {k} | {a_us:.2f} | {auto['kernel'] if auto else '-'} | "
                         f"{q.opus.KID_NAMES[best]} | {r['us']:.2f} | {a_us / r['us']:.3f} | {tf:.0f} | {bw:.0f} | "
                         f"{frac:.3f} ({'hbm' if m <= 256 else 'mfma'}) |\n")


if __name__ == "__main__":
    main()
