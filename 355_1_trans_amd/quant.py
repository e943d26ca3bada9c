"""Device-side quantizers and weight layouts (libqgemm.so ``qgemm_quant_*``
and ``*_device`` entry points), PyTorch-facing.

These produce every operand format the GEMM entry points consume, on the
GPU, from fp32 or bf16 tensors:

* ``quant_fp8_blockscale`` -- e4m3 with fp32 scales amax/448 per 1x128
  (activation) or 128x128 (weight) block: the inputs of
  ``gemm_a8w8_bpreshuffle`` / ``gemm_a8w8_ldsbypass``;
* ``quant_fp8_e8m0_blockscale`` -- the same blocks with E8M0 scales, the
  inputs of the E8M0 adapter ``blockscale_bpreshuffle``;
* ``quant_mxfp8`` / ``quant_mxfp4`` -- MX formats with one E8M0 scale per
  32 K elements, row-major or in aiter's e8m0_shuffle order (the reference's
  MXFP4 inputs come from aiter ``quant(..., shuffle=True)``,
  MX4 candidate_m9/README.md:6-12);
* ``e8m0_shuffle`` and (in the package root) ``shuffle_b_kpanel``,
  ``shuffle_weight_16x16``, ``ldsbypass_pack_b`` -- run on the GPU for GPU
  tensors.

Codes are bit-identical to the host recipes (round to nearest even,
saturating); the tests compare them with the CPU oracle byte for byte.
"""
import ctypes

import torch

from . import _check, _record, _require_gpu, _stream, lib

IN_FP32, IN_BF16 = 0, 1


def _source(x, k_align):
    _require_gpu(x)
    if x.dim() != 2 or x.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("x must be a 2-D float32 or bfloat16 GPU tensor")
    if x.stride(1) != 1 or x.stride(0) % 4 or x.shape[1] % k_align:
        raise ValueError(f"x needs contiguous rows, a row pitch that is a multiple of 4 elements and "
                         f"K % {k_align} == 0")
    return (IN_FP32 if x.dtype == torch.float32 else IN_BF16), x.stride(0)


def _launch(x, fn_name, *args, keep=()):
    with torch.cuda.device(x.device):
        s = _stream(x.device)
        st = getattr(lib(), fn_name)(*args, ctypes.c_void_p(s.cuda_stream))
        _record(s, x, *keep)
    _check(st, fn_name)


def quant_fp8_blockscale(x, block="1x128", scale_layout="mk"):
    """(q, scale): q float8_e4m3fn like x; block "1x128" gives scale [M, K/128]
    (scale_layout "mk": row-major; "km": the BPS column-major [K/128][M],
    returned as the [M, K/128] view with strides (1, M)); block "128x128"
    gives scale [ceil(N/128), K/128]."""
    code, ld = _source(x, 128)
    rows, k = x.shape
    kg = k // 128
    q = torch.empty((rows, k), dtype=torch.uint8, device=x.device)
    if block == "1x128":
        if scale_layout == "mk":
            s = torch.empty((rows, kg), dtype=torch.float32, device=x.device)
            sm, sk, view = kg, 1, s
        elif scale_layout == "km":
            s = torch.empty((kg, rows), dtype=torch.float32, device=x.device)
            sm, sk, view = 1, rows, s.t()
        else:
            raise ValueError("scale_layout must be 'mk' or 'km'")
        _launch(x, "qgemm_quant_fp8_blockscale_act", x.data_ptr(), code, rows, k, ld, q.data_ptr(), k, s.data_ptr(),
                sm, sk, keep=(q, s))
        return q.view(torch.float8_e4m3fn), view
    if block == "128x128":
        s = torch.empty(((rows + 127) // 128, kg), dtype=torch.float32, device=x.device)
        _launch(x, "qgemm_quant_fp8_blockscale_wgt", x.data_ptr(), code, rows, k, ld, q.data_ptr(), k, s.data_ptr(),
                kg, keep=(q, s))
        return q.view(torch.float8_e4m3fn), s
    raise ValueError("block must be '1x128' or '128x128'")


def quant_fp8_e8m0_blockscale(x, block="1x128"):
    """(q, e): E8M0 block scales (codes E+127).  "1x128": e is the [M, K/128]
    view with strides (1, M) of column-major bytes, as
    blockscale_bpreshuffle.gemm_a8w8_blockscale_bpreshuffle takes it;
    "128x128": e [N/128, K/128] (N % 128 == 0 for that kernel)."""
    code, ld = _source(x, 128)
    rows, k = x.shape
    kg = k // 128
    q = torch.empty((rows, k), dtype=torch.uint8, device=x.device)
    if block == "1x128":
        e = torch.empty((kg, rows), dtype=torch.uint8, device=x.device)
        _launch(x, "qgemm_quant_fp8_e8m0_act", x.data_ptr(), code, rows, k, ld, q.data_ptr(), k, e.data_ptr(), 1, rows,
                keep=(q, e))
        return q.view(torch.float8_e4m3fn), e.t()
    if block == "128x128":
        e = torch.empty(((rows + 127) // 128, kg), dtype=torch.uint8, device=x.device)
        _launch(x, "qgemm_quant_fp8_e8m0_wgt", x.data_ptr(), code, rows, k, ld, q.data_ptr(), k, e.data_ptr(), kg,
                keep=(q, e))
        return q.view(torch.float8_e4m3fn), e
    raise ValueError("block must be '1x128' or '128x128'")


def e8m0_shuffle_bytes(rows, groups_k):
    return lib().qgemm_e8m0_shuffle_bytes(rows, groups_k)


def _quant_mx(x, fp4, shuffle):
    code, ld = _source(x, 32)
    rows, k = x.shape
    qcols = k // 2 if fp4 else k
    q = torch.empty((rows, qcols), dtype=torch.uint8, device=x.device)
    if shuffle:
        e = torch.empty(e8m0_shuffle_bytes(rows, k // 32), dtype=torch.uint8, device=x.device)
    else:
        e = torch.empty((rows, k // 32), dtype=torch.uint8, device=x.device)
    _launch(x, "qgemm_quant_mxfp4" if fp4 else "qgemm_quant_mxfp8", x.data_ptr(), code, rows, k, ld, q.data_ptr(),
            qcols, e.data_ptr(), k // 32, int(bool(shuffle)), keep=(q, e))
    return q, e


def quant_mxfp8(x, shuffle=False):
    """(q float8_e4m3fn [rows, K], e uint8 [rows, K/32] or the e8m0_shuffle bytes)."""
    q, e = _quant_mx(x, False, shuffle)
    return q.view(torch.float8_e4m3fn), e


def quant_mxfp4(x, shuffle=False):
    """(q uint8 [rows, K/2] packed e2m1, e uint8 [rows, K/32] or the e8m0_shuffle bytes)."""
    return _quant_mx(x, True, shuffle)


def e8m0_shuffle(e):
    """aiter e8m0_shuffle of row-major E8M0 scales [rows, K/32] (GPU tensor)."""
    _require_gpu(e)
    if e.dim() != 2 or e.element_size() != 1 or e.stride(1) != 1:
        raise ValueError("e must be a 2-D byte tensor with contiguous rows")
    rows, kg = e.shape
    out = torch.empty(e8m0_shuffle_bytes(rows, kg), dtype=torch.uint8, device=e.device)
    _launch(e, "qgemm_e8m0_shuffle_device", e.data_ptr(), out.data_ptr(), rows, kg, e.stride(0), keep=(out,))
    return out


def relayout_device(fn_name, B, out_bytes):
    """Run one of the *_device weight-layout kernels on a 2-D byte tensor."""
    _require_gpu(B)
    if B.dim() != 2 or B.element_size() != 1 or B.stride(1) != 1 or B.stride(0) % 16:
        raise ValueError("B must be a 2-D byte tensor with contiguous rows and a pitch that is a multiple of 16")
    n, kb = B.shape
    out = torch.empty(out_bytes, dtype=torch.uint8, device=B.device)
    _launch(B, fn_name, B.data_ptr(), out.data_ptr(), n, kb, B.stride(0), keep=(out,))
    return out
