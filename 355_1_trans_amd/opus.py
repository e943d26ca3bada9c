"""aiter-facing wrappers: the names and argument conventions the reference's
aiter integration uses, over this library's C ABI.

* ``gemm_a8w8_bpreshuffle_opus`` -- fp32 block-scale FP8 (1x128 / 128x128),
  batched, with the tuned-table kernel lookup
  (opus_a8w8_bpreshuffle_integration_and_benchmark.md sections 2.3, 3, 4.3);
* ``gemm_a8w8_mxfp8_opus`` -- MXFP8 (E8M0 per 32 K), batched, fp32 output
  (opus_mxfp8_gemm_integration_plan.md step 6);
* ``opus_gemm_mxfp8_nt / _nn / _tt / _tn`` -- the E8M0 block-scale GEMM in
  the four physical layouts (opus_mxfp8_layouts_trace_8192_20261027T005846Z/
  capture.py:42-62);
* ``gemm_a4w4`` (package root) -- MXFP4 with aiter's bpreshuffle operands.

Tuned table: CSV files ``configs/*tuned*.csv`` next to this module with the
reference's tuner schema (gfx, cu_num, M, N, K, bias, dtype, outdtype,
scaleAB, bpreshuffle, libtype, solidx, splitK, us, kernelName, err_ratio,
tflops, bw); rows with libtype ``qgemm`` map a shape to a kernel id
(QGEMM_KID_*), the fastest row winning on duplicate keys.  An explicit
``kernelId`` skips the lookup; a shape with no row runs the library's own
plan (kernel id 0).  ``tune.py`` writes the table.
"""
import csv
import ctypes
from functools import lru_cache
from pathlib import Path

import torch

from . import Kargs, _check, _out_code, _record, _require_gpu, _stream, lib, shuffle_b_kpanel

CONFIGS = Path(__file__).resolve().parent / "configs"

KID_AUTO, KID_TILE256, KID_MID, KID_SKINNY, KID_DECODE, KID_BURST = range(6)
KID_NAMES = {KID_AUTO: "auto", KID_TILE256: "tile256", KID_MID: "mid128", KID_SKINNY: "skinny",
             KID_DECODE: "decode", KID_BURST: "burst"}
LAYOUTS = {"nt": 0, "nn": 1, "tt": 2, "tn": 3}

_WS = {}


def _scratch(tag, need, dev, stream):
    """A cached device buffer of at least `need` bytes per (tag, device,
    stream), zero-filled on allocation; the tag separates workspaces of
    different entries.  A query of zero bytes gives no buffer."""
    if need == 0:
        return None, 0
    key = (tag, dev.index, stream.cuda_stream)
    buf = _WS.get(key)
    if buf is None or buf.numel() < need:
        buf = torch.zeros((need + 255) // 256 * 256, dtype=torch.uint8, device=dev)
        _WS[key] = buf
    return buf.data_ptr(), buf.numel()


def _cu_num(dev):
    return torch.cuda.get_device_properties(dev).multi_processor_count


@lru_cache(maxsize=None)
def _tuned_rows():
    rows = {}
    for f in sorted(CONFIGS.glob("*tuned*.csv")):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                if r.get("libtype") != "qgemm":
                    continue
                key = (int(r["cu_num"]), int(r["M"]), int(r["N"]), int(r["K"]), r["bias"], r["dtype"],
                       r["outdtype"], r["scaleAB"], r["bpreshuffle"])
                if key not in rows or float(r["us"]) < float(rows[key]["us"]):
                    rows[key] = r
    return rows


def lookup_tuned(cu_num, m, n, k, out_dtype, bpreshuffle=True):
    """Kernel id of the tuned row for this shape, or None."""
    key = (cu_num, m, n, k, "False", "torch.float8_e4m3fn", str(out_dtype), "True", str(bool(bpreshuffle)))
    r = _tuned_rows().get(key)
    return int(r["solidx"]) if r else None


def _batched(t, name, dims):
    if t.dim() == dims - 1:
        return t.unsqueeze(0), True
    if t.dim() != dims:
        raise ValueError(f"{name} must have {dims - 1} or {dims} dimensions")
    return t, False


def gemm_a8w8_bpreshuffle_opus(A, B, x_scale, w_scale, out_dtype=torch.bfloat16, kernelId=None, preshuffled=False):
    """Block-scale FP8 GEMM, fp32 scales.

    A [M, K] or [batch, M, K] e4m3; B [N, K] / [batch, N, K] e4m3, K-panel
    shuffled here unless ``preshuffled`` (then B holds the K-panel bytes
    [K/128][N][128] per batch, as ``shuffle_b_kpanel`` returns them);
    x_scale fp32 [batch, M, K/128] (or [M, K/128]); w_scale fp32
    [batch, ceil(N/128), K/128].  Returns [M, N] / [batch, M, N] of
    ``out_dtype`` (bf16 or fp32).  ``kernelId``: a QGEMM_KID_* value, or None
    for the tuned-table lookup."""
    dev = _require_gpu(A, B, x_scale, w_scale)
    A3, squeeze = _batched(A, "A", 3)
    batch, m, k = A3.shape
    if preshuffled:
        n = B.numel() // (batch * k)
        if B.numel() != batch * n * k:
            raise ValueError("preshuffled B must hold batch * N * K bytes")
        Bk = B.reshape(batch, n * k)
    else:
        B3, _ = _batched(B, "B", 3)
        if B3.shape[0] != batch or B3.shape[2] != k:
            raise ValueError("B must be [batch, N, K] with A's batch and K")
        n = B3.shape[1]
        Bk = torch.stack([shuffle_b_kpanel(B3[i]).reshape(-1) for i in range(batch)])
    kg, nbk = k // 128, (n + 127) // 128
    if k % 128:
        raise ValueError("K must be a multiple of 128")
    xs = x_scale.reshape(batch, m, kg) if x_scale.numel() == batch * m * kg else None
    ws_ = w_scale.reshape(batch, nbk, kg) if w_scale.numel() == batch * nbk * kg else None
    if xs is None or ws_ is None or x_scale.dtype != torch.float32 or w_scale.dtype != torch.float32:
        raise ValueError("x_scale must be fp32 [batch, M, K/128] and w_scale fp32 [batch, ceil(N/128), K/128]")
    for t in (A3, Bk, xs, ws_):
        if not t.is_contiguous():
            raise ValueError("A, B and the scales must be contiguous")
    out = torch.empty((batch, m, n), dtype=out_dtype, device=dev)
    if kernelId is None:
        kernelId = lookup_tuned(_cu_num(dev), m, n, k, out_dtype) if batch == 1 else None
        kernelId = KID_AUTO if kernelId is None else kernelId
    args = Kargs(A3.data_ptr(), Bk.data_ptr(), out.data_ptr(), m, n, k, batch, k, 128, n, m * k, n * k, m * n,
                 xs.data_ptr(), ws_.data_ptr(), 1 if m > 1 else m, kg, m * kg, nbk * kg)
    L = lib()
    with torch.cuda.device(dev):
        s = _stream(dev)
        need = L.gemm_a8w8_blockscale_bpreshuffle_kid_workspace_bytes(ctypes.byref(args), int(kernelId))
        wp, wb = _scratch("splitk", need, dev, s)
        st = L.gemm_a8w8_blockscale_bpreshuffle_kid(ctypes.byref(args), _out_code(out_dtype), int(kernelId), wp, wb,
                                                    ctypes.c_void_p(s.cuda_stream))
        _record(s, A3, Bk, xs, ws_, out)
    _check(st, f"gemm_a8w8_blockscale_bpreshuffle_kid (kernelId {kernelId})")
    return out[0] if squeeze else out


def gemm_a8w8_mxfp8_opus(A, B, x_scale, w_scale, out=None):
    """MXFP8 GEMM: A [batch, M, K], B [batch, N, K] e4m3 (2-D accepted);
    x_scale [batch, M, K/32], w_scale [batch, N, K/32] E8M0 bytes; fp32
    output Y [batch, M, N] (``out`` reused when given: [batch, M, N], or
    [M, N] when batch is 1).  Shapes are checked before the device."""
    A3, squeeze = _batched(A, "A", 3)
    B3, _ = _batched(B, "B", 3)
    batch, m, k = A3.shape
    if B3.shape[0] != batch or B3.shape[2] != k or k % 128:
        raise ValueError("B must be [batch, N, K] with A's batch and K, K % 128 == 0")
    n, kg = B3.shape[1], k // 32
    xs = x_scale.reshape(batch, m, kg) if x_scale.numel() == batch * m * kg else None
    wsc = w_scale.reshape(batch, n, kg) if w_scale.numel() == batch * n * kg else None
    if xs is None or wsc is None or x_scale.element_size() != 1 or w_scale.element_size() != 1:
        raise ValueError("scales must be E8M0 bytes [batch, M, K/32] and [batch, N, K/32]")
    for t in (A3, B3, xs, wsc):
        if not t.is_contiguous():
            raise ValueError("A, B and the scales must be contiguous")
    if out is not None:
        # a 2-D out holds one batch entry only: the kernel writes batch * M * N values
        shapes = ((batch, m, n), (m, n)) if batch == 1 else ((batch, m, n),)
        if tuple(out.shape) not in shapes or out.dtype != torch.float32 or not out.is_contiguous():
            raise ValueError("out must be a contiguous fp32 [batch, M, N] tensor ([M, N] only when batch is 1)")
    dev = _require_gpu(A, B, x_scale, w_scale) if out is None else _require_gpu(A, B, x_scale, w_scale, out)
    if out is None:
        out = torch.empty((batch, m, n), dtype=torch.float32, device=dev)
    args = Kargs(A3.data_ptr(), B3.data_ptr(), out.data_ptr(), m, n, k, batch, k, k, n, m * k, n * k, m * n,
                 xs.data_ptr(), wsc.data_ptr(), kg, kg, m * kg, n * kg)
    L = lib()
    with torch.cuda.device(dev):
        s = _stream(dev)
        wp, wb = _scratch("splitk", L.gemm_a8w8_mxfp8_workspace_bytes(ctypes.byref(args)), dev, s)
        st = L.gemm_a8w8_mxfp8(ctypes.byref(args), 0, wp, wb, ctypes.c_void_p(s.cuda_stream))
        _record(s, A3, B3, xs, wsc, out)
    _check(st, "gemm_a8w8_mxfp8")
    return out[0] if squeeze and out.dim() == 3 else out


def _layout_gemm(layout, A, B, sfa, sfb, out):
    """E8M0 block-scale GEMM C[M,N] = A[M,K] x B[K,N] in a physical layout:
    A [M,K] (N) or [K,M] (T); B shuffle_weight(16,16) of [N,K] (NT), [N,K]
    (TT) or [K,N] (NN, TN); sfa the [M, K/128] view of [K/128][M] bytes,
    sfb [N/128, K/128]; out [M, N] bf16 or fp32."""
    dev = _require_gpu(A, B, sfa, sfb, out)
    code = LAYOUTS[layout]
    a_t, b_n = layout[0] == "t", layout[1] == "n"
    m, n = out.shape
    k = A.shape[0] if a_t else A.shape[1]
    if A.shape != ((k, m) if a_t else (m, k)):
        raise ValueError(f"{layout.upper()}: A must be {'[K, M]' if a_t else '[M, K]'}")
    if B.numel() != n * k or (b_n and B.shape != (k, n)):
        raise ValueError(f"{layout.upper()}: B must hold N * K bytes{' as [K, N]' if b_n else ''}")
    if sfa.shape != (m, k // 128) or sfa.stride() != (1, m):
        raise ValueError("sfa must be the [M, K/128] view of [K/128, M] E8M0 bytes")
    if sfb.shape != (n // 128, k // 128) or not sfb.is_contiguous():
        raise ValueError("sfb must be contiguous E8M0 bytes [N/128, K/128]")
    if not (A.is_contiguous() and B.is_contiguous() and out.is_contiguous()):
        raise ValueError("A, B and out must be contiguous")
    kg = k // 128
    args = Kargs(A.data_ptr(), B.data_ptr(), out.data_ptr(), m, n, k, 1, m if a_t else k, n if b_n else k, n,
                 m * k, n * k, m * n, sfa.data_ptr(), sfb.data_ptr(), m, kg, m * kg, (n // 128) * kg)
    L = lib()
    with torch.cuda.device(dev):
        s = _stream(dev)
        need = L.gemm_a8w8_blockscale_layout_workspace_bytes(ctypes.byref(args), code)
        wp, wb = _scratch("layout", need, dev, s)
        st = L.gemm_a8w8_blockscale_layout(ctypes.byref(args), code, _out_code(out.dtype), wp, wb,
                                           ctypes.c_void_p(s.cuda_stream))
        _record(s, A, B, sfa, sfb, out)
    _check(st, f"gemm_a8w8_blockscale_layout ({layout.upper()})")
    return out


def opus_gemm_mxfp8_nt(A, B, sfa, sfb, out):
    """NT: A [M, K]; B = shuffle_weight(16,16) of [N, K] (``shuffle_weight_16x16``)."""
    return _layout_gemm("nt", A, B, sfa, sfb, out)


def opus_gemm_mxfp8_nn(A, B, sfa, sfb, out):
    """NN: A [M, K]; B [K, N]."""
    return _layout_gemm("nn", A, B, sfa, sfb, out)


def opus_gemm_mxfp8_tt(A, B, sfa, sfb, out):
    """TT: A [K, M]; B [N, K]."""
    return _layout_gemm("tt", A, B, sfa, sfb, out)


def opus_gemm_mxfp8_tn(A, B, sfa, sfb, out):
    """TN: A [K, M]; B [K, N]."""
    return _layout_gemm("tn", A, B, sfa, sfb, out)


__all__ = ["gemm_a8w8_bpreshuffle_opus", "gemm_a8w8_mxfp8_opus", "opus_gemm_mxfp8_nt", "opus_gemm_mxfp8_nn",
           "opus_gemm_mxfp8_tt", "opus_gemm_mxfp8_tn", "lookup_tuned", "KID_NAMES"]
