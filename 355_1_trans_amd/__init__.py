"""MI355X (gfx950) quantized-GEMM hot path: host-side mirror of the reference.

The compute lives in ``libqgemm.so`` (hand-written HIP for gfx950, C ABI in
``include/qgemm.h``).  This module loads that library with ctypes and exposes
PyTorch-facing wrappers that validate tensors, build the 96-byte kargs block
and launch on the current stream:

* ``blockscale_bpreshuffle.gemm_a8w8_blockscale_bpreshuffle`` -- the
  reference's E8M0 block-scale adapter (SNAP blockscale_bpreshuffle.py:37-97);
* ``gemm_a8w8_bpreshuffle`` -- block-scale FP8 with fp32 1x128 / 128x128
  scales and a K-panel pre-shuffled B (BPS host.cc:66-111, 254-284);
* ``gemm_a8w8_ldsbypass`` -- the same GEMM with B in the fragment order
  B'' that the LDS-bypass kernel streams straight into registers
  (LBP host.cc:283-294), with ``ldsbypass_repack`` (GPU, from the K-panel
  B') and ``ldsbypass_pack_b`` (CPU, from raw B) to build B'';
* ``gemm_a8w8_mxfp8`` -- MXFP8 TN GEMM (MX8 host.cc:96-122, 266-296);
* ``gemm_a4w4_mxfp4`` -- MXFP4 A4W4 GEMM (MX4 host.cc:96-115, 201-216);
* ``opus`` -- the aiter-facing names (``gemm_a8w8_bpreshuffle_opus`` with
  the tuned kernel table, ``gemm_a8w8_mxfp8_opus``,
  ``opus_gemm_mxfp8_{nt,nn,tt,tn}``);
* ``gemm_a4w4`` -- MXFP4 with aiter's ``gemm_a4w4(..., bpreshuffle=True)``
  operands: B in shuffle_weight(16,16) order, both scales in e8m0_shuffle
  order (MX4 candidate_m10/gemm_a4w4_mxfp4_4wave_host.cc:194-250).

There is no CPU fallback: every wrapper raises if the library is missing or
the tensors are not on a GPU.

Skinny-M calls split K across workgroups and reduce the fp32 partials in the
same launch; the workspace's counter words are tagged with a per-launch
epoch, so any initial contents work.  ``workspace=None`` uses one cached
buffer per (device, stream); pass a tensor to supply your own, or
``workspace=False`` to run without split-K.
"""
import ctypes
from functools import lru_cache
from pathlib import Path

import torch

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libqgemm.so"

OUT_FP32 = 0
OUT_BF16 = 1


class Kargs(ctypes.Structure):
    """opus_gemm_scale_kargs: 96 bytes, field order of the reference ABI."""

    _fields_ = (
        [(name, ctypes.c_void_p) for name in ("ptr_a", "ptr_b", "ptr_c")]
        + [(name, ctypes.c_int) for name in (
            "m", "n", "k", "batch", "stride_a", "stride_b", "stride_c",
            "stride_a_batch", "stride_b_batch", "stride_c_batch")]
        + [(name, ctypes.c_void_p) for name in ("ptr_sfa", "ptr_sfb")]
        + [(name, ctypes.c_int) for name in (
            "stride_sfa", "stride_sfb", "stride_sfa_batch", "stride_sfb_batch")]
    )


class LdsBypassKargs(ctypes.Structure):
    """opus_gemm_ldsbypass_kargs: ptr_b_pp after ptr_b, stride_b_pp_batch appended."""

    _fields_ = (
        [(name, ctypes.c_void_p) for name in ("ptr_a", "ptr_b", "ptr_b_pp", "ptr_c")]
        + [(name, ctypes.c_int) for name in (
            "m", "n", "k", "batch", "stride_a", "stride_b", "stride_c",
            "stride_a_batch", "stride_b_batch", "stride_c_batch")]
        + [(name, ctypes.c_void_p) for name in ("ptr_sfa", "ptr_sfb")]
        + [(name, ctypes.c_int) for name in (
            "stride_sfa", "stride_sfb", "stride_sfa_batch", "stride_sfb_batch", "stride_b_pp_batch")]
    )


class Mxfp4Kargs(ctypes.Structure):
    """opus_gemm_mxfp4_scale_kargs: the 96-byte block plus grid_blocks."""

    _fields_ = Kargs._fields_ + [("grid_blocks", ctypes.c_int)]


assert ctypes.sizeof(Kargs) == 96
assert Mxfp4Kargs.grid_blocks.offset == 96


_V, _I = ctypes.c_void_p, ctypes.c_int

EXPORTS = {
    # name: (restype, argtypes)
    "launch_blockscale_bpreshuffle": (ctypes.c_int, [ctypes.POINTER(Kargs), ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "gemm_a8w8_blockscale_bpreshuffle": (ctypes.c_int, [ctypes.POINTER(Kargs), ctypes.c_int, ctypes.c_void_p,
                                                        ctypes.c_size_t, ctypes.c_void_p]),
    "gemm_a8w8_blockscale_bpreshuffle_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Kargs)]),
    "gemm_a8w8_blockscale_layout": (ctypes.c_int, [ctypes.POINTER(Kargs), ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                                   ctypes.c_size_t, ctypes.c_void_p]),
    "gemm_a8w8_blockscale_layout_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Kargs), ctypes.c_int]),
    "gemm_a8w8_blockscale_bpreshuffle_kid": (ctypes.c_int, [ctypes.POINTER(Kargs), ctypes.c_int, ctypes.c_int,
                                                            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "gemm_a8w8_blockscale_bpreshuffle_kid_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Kargs), ctypes.c_int]),
    "gemm_a8w8_blockscale_ldsbypass_kid": (ctypes.c_int, [ctypes.POINTER(LdsBypassKargs), ctypes.c_int, ctypes.c_int,
                                                          ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "gemm_a8w8_blockscale_ldsbypass_kid_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(LdsBypassKargs),
                                                                             ctypes.c_int]),
    "gemm_a8w8_mxfp8_kid": (ctypes.c_int, [ctypes.POINTER(Kargs), ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                           ctypes.c_size_t, ctypes.c_void_p]),
    "gemm_a8w8_mxfp8_kid_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Kargs), ctypes.c_int]),
    "gemm_a4w4_mxfp4_kid": (ctypes.c_int, [ctypes.POINTER(Kargs), ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                           ctypes.c_size_t, ctypes.c_void_p]),
    "gemm_a4w4_mxfp4_kid_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Kargs), ctypes.c_int]),
    "gemm_a4w4_mxfp4_bpreshuffle": (ctypes.c_int, [ctypes.POINTER(Mxfp4Kargs), ctypes.c_int, ctypes.c_void_p]),
    "gemm_a4w4_mxfp4_bpreshuffle_kid": (ctypes.c_int, [ctypes.POINTER(Mxfp4Kargs), ctypes.c_int, ctypes.c_int,
                                                       ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "gemm_a4w4_mxfp4_bpreshuffle_kid_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Mxfp4Kargs), ctypes.c_int]),
    "gemm_a8w8_mxfp8": (ctypes.c_int, [ctypes.POINTER(Kargs), ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
                                       ctypes.c_void_p]),
    "gemm_a8w8_mxfp8_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Kargs)]),
    "gemm_a4w4_mxfp4": (ctypes.c_int, [ctypes.POINTER(Kargs), ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
                                       ctypes.c_void_p]),
    "gemm_a4w4_mxfp4_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Kargs)]),
    "gemm_a4w4_mxfp4_noalloc": (ctypes.c_int, [ctypes.POINTER(Kargs), ctypes.c_int, ctypes.c_void_p]),
    "gemm_a4w4_mxfp4_noalloc_max_workspace_bytes": (ctypes.c_size_t, []),
    "gemm_a8w8_blockscale_ldsbypass": (ctypes.c_int, [ctypes.POINTER(LdsBypassKargs), ctypes.c_int,
                                                      ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "gemm_a8w8_blockscale_ldsbypass_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(LdsBypassKargs)]),
    "gemm_a8w8_blockscale_ldsbypass_repack": (ctypes.c_int, [ctypes.POINTER(LdsBypassKargs), ctypes.c_void_p]),
    "qgemm_ldsbypass_b_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int]),
    "qgemm_pack_b_ldsbypass": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]),
    "qgemm_shuffle_b_kpanel": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]),
    "qgemm_shuffle_weight_16x16": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]),
    "qgemm_e8m0_shuffle_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int]),
    "qgemm_e8m0_shuffle": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]),
    "qgemm_probe_words": (ctypes.c_int, []),
    "qgemm_probe_mfma_layout": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "qgemm_quant_fp8_blockscale_act": (ctypes.c_int, [_V, _I, _I, _I, _I, _V, _I, _V, _I, _I, _V]),
    "qgemm_quant_fp8_blockscale_wgt": (ctypes.c_int, [_V, _I, _I, _I, _I, _V, _I, _V, _I, _V]),
    "qgemm_quant_fp8_e8m0_act": (ctypes.c_int, [_V, _I, _I, _I, _I, _V, _I, _V, _I, _I, _V]),
    "qgemm_quant_fp8_e8m0_wgt": (ctypes.c_int, [_V, _I, _I, _I, _I, _V, _I, _V, _I, _V]),
    "qgemm_quant_mxfp8": (ctypes.c_int, [_V, _I, _I, _I, _I, _V, _I, _V, _I, _I, _V]),
    "qgemm_quant_mxfp4": (ctypes.c_int, [_V, _I, _I, _I, _I, _V, _I, _V, _I, _I, _V]),
    "qgemm_shuffle_b_kpanel_device": (ctypes.c_int, [_V, _V, _I, _I, _I, _V]),
    "qgemm_shuffle_weight_16x16_device": (ctypes.c_int, [_V, _V, _I, _I, _I, _V]),
    "qgemm_pack_b_ldsbypass_device": (ctypes.c_int, [_V, _V, _I, _I, _I, _V]),
    "qgemm_e8m0_shuffle_device": (ctypes.c_int, [_V, _V, _I, _I, _I, _V]),
    "gemm_a8w8_blockscale_bpreshuffle_grouped": (ctypes.c_int, [ctypes.POINTER(Kargs), _I, _I, _I, _V, ctypes.c_size_t,
                                                                _V]),
    "gemm_a8w8_blockscale_bpreshuffle_grouped_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Kargs), _I]),
    "gemm_a8w8_blockscale_ldsbypass_grouped": (ctypes.c_int, [ctypes.POINTER(LdsBypassKargs), _I, _I, _I, _V,
                                                              ctypes.c_size_t, _V]),
    "gemm_a8w8_blockscale_ldsbypass_grouped_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(LdsBypassKargs), _I]),
    "gemm_a8w8_mxfp8_grouped": (ctypes.c_int, [ctypes.POINTER(Kargs), _I, _I, _I, _V, ctypes.c_size_t, _V]),
    "gemm_a8w8_mxfp8_grouped_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Kargs), _I]),
    "gemm_a4w4_mxfp4_grouped": (ctypes.c_int, [ctypes.POINTER(Kargs), _I, _I, _I, _V, ctypes.c_size_t, _V]),
    "gemm_a4w4_mxfp4_grouped_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Kargs), _I]),
    "qgemm_reference_gemm": (ctypes.c_int, [_I, ctypes.POINTER(Kargs), _V]),
    "qgemm_version": (ctypes.c_char_p, []),
    "qgemm_last_launch": (ctypes.c_char_p, []),
}


@lru_cache(None)
def lib():
    """Load libqgemm.so; raises if it has not been built (no fallback)."""
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                           "(the HIP library is the only implementation)")
    L = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in EXPORTS.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def last_launch():
    """Kernel instantiations launched by this thread's most recent library
    call (qgemm_last_launch), e.g. 'wide_gemm<fp8,MX,RAW,bf16,pb16>'."""
    return lib().qgemm_last_launch().decode()


def _check(status, what):
    if status:
        raise RuntimeError(f"{what} failed: HIP error {status}")


def _stream(device):
    return torch.cuda.current_stream(device)


def _record(stream, *tensors):
    for t in tensors:
        if t is not None:
            t.record_stream(stream)


def _require_gpu(*tensors):
    dev = tensors[0].device
    if not tensors[0].is_cuda:
        raise ValueError("inputs must be GPU tensors (there is no CPU implementation)")
    for t in tensors:
        if t.device != dev:
            raise ValueError("all tensors must be on the same GPU")
    return dev


_WORKSPACES = {}


def _workspace(query, args, workspace, dev, stream):
    """(pointer, bytes) of the split-K workspace for this call.

    ``query`` is the entry's *_workspace_bytes function; 0 means the call
    does not split K.  The cached buffer is zero-filled on allocation (on the
    call's stream, so it is ordered before the launch); split launches count
    their slices in epoch-tagged counter words, so no clearing is needed
    between calls."""
    if workspace is False:
        return None, 0
    need = query(ctypes.byref(args))
    if workspace is not None:
        return workspace.data_ptr(), workspace.numel() * workspace.element_size()
    if need == 0:
        return None, 0
    key = (dev.index, stream.cuda_stream)
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < need:
        buf = torch.zeros((need + 255) // 256 * 256, dtype=torch.uint8, device=dev)
        _WORKSPACES[key] = buf
    return buf.data_ptr(), buf.numel()


def _ws_tensor(workspace):
    return workspace if isinstance(workspace, torch.Tensor) else None


def _u8(t):
    return t.view(torch.uint8) if t.dtype != torch.uint8 else t


def _out(out, shape, dtype, device):
    if out is None:
        return torch.empty(shape, dtype=dtype, device=device)
    if tuple(out.shape) != tuple(shape) or out.dtype != dtype or out.device != device or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor of the requested shape/dtype/device")
    return out


def _out_code(dtype):
    if dtype == torch.bfloat16:
        return OUT_BF16
    if dtype == torch.float32:
        return OUT_FP32
    raise ValueError("output dtype must be torch.bfloat16 or torch.float32")


def gemm_a8w8_mxfp8(A, B, A_scale, B_scale, dtype=torch.bfloat16, out=None, workspace=None):
    """MXFP8 TN GEMM: A [M,K] e4m3, B [N,K] e4m3, A_scale [M,K/32], B_scale [N,K/32] E8M0 bytes."""
    dev = _require_gpu(A, B, A_scale, B_scale)
    m, k = A.shape
    n = B.shape[0]
    if B.shape[1] != k or k % 128:
        raise ValueError("requires matching K with K % 128 == 0")
    if A_scale.shape != (m, k // 32) or B_scale.shape != (n, k // 32):
        raise ValueError("requires A_scale [M,K/32] and B_scale [N,K/32]")
    for t in (A, B, A_scale, B_scale):
        if not t.is_contiguous():
            raise ValueError("A, B and scales must be contiguous")
    out = _out(out, (m, n), dtype, dev)
    args = Kargs(A.data_ptr(), B.data_ptr(), out.data_ptr(), m, n, k, 1, k, k, n, m * k, n * k, m * n,
                 A_scale.data_ptr(), B_scale.data_ptr(), k // 32, k // 32, m * (k // 32), n * (k // 32))
    with torch.cuda.device(dev):
        s = _stream(dev)
        ws_ptr, ws_bytes = _workspace(lib().gemm_a8w8_mxfp8_workspace_bytes, args, workspace, dev, s)
        st = lib().gemm_a8w8_mxfp8(ctypes.byref(args), _out_code(dtype), ws_ptr, ws_bytes,
                                   ctypes.c_void_p(s.cuda_stream))
        _record(s, A, B, A_scale, B_scale, out, _ws_tensor(workspace))
    _check(st, "gemm_a8w8_mxfp8")
    return out


def gemm_a4w4_mxfp4(A, B, A_scale, B_scale, dtype=torch.bfloat16, out=None, workspace=None):
    """MXFP4 A4W4 GEMM: A [M,K/2], B [N,K/2] packed e2m1 bytes, scales [rows,K/32] E8M0."""
    dev = _require_gpu(A, B, A_scale, B_scale)
    m, kb = A.shape
    n = B.shape[0]
    k = 2 * kb
    if B.shape[1] != kb or k % 256:
        raise ValueError("requires matching K with K % 256 == 0")
    if A_scale.shape != (m, k // 32) or B_scale.shape != (n, k // 32):
        raise ValueError("requires A_scale [M,K/32] and B_scale [N,K/32]")
    for t in (A, B, A_scale, B_scale):
        if not t.is_contiguous():
            raise ValueError("A, B and scales must be contiguous")
    out = _out(out, (m, n), dtype, dev)
    args = Kargs(A.data_ptr(), B.data_ptr(), out.data_ptr(), m, n, k, 1, kb, kb, n, m * kb, n * kb, m * n,
                 A_scale.data_ptr(), B_scale.data_ptr(), k // 32, k // 32, m * (k // 32), n * (k // 32))
    with torch.cuda.device(dev):
        s = _stream(dev)
        ws_ptr, ws_bytes = _workspace(lib().gemm_a4w4_mxfp4_workspace_bytes, args, workspace, dev, s)
        st = lib().gemm_a4w4_mxfp4(ctypes.byref(args), _out_code(dtype), ws_ptr, ws_bytes,
                                   ctypes.c_void_p(s.cuda_stream))
        _record(s, A, B, A_scale, B_scale, out, _ws_tensor(workspace))
    _check(st, "gemm_a4w4_mxfp4")
    return out


def _shuffled_scale(e, rows, kg, name):
    """Bytes per 32-row block of an e8m0_shuffle'd scale tensor (rows padded
    to 32, groups to 8; any shape with that many contiguous bytes)."""
    kg8 = (kg + 7) // 8 * 8
    need = (rows + 31) // 32 * 32 * kg8
    if e.element_size() != 1 or not e.is_contiguous() or e.numel() < need:
        raise ValueError(f"{name} must be contiguous e8m0_shuffle bytes, at least {need} of them")
    return 32 * kg8


def gemm_a4w4(A, B, A_scale, B_scale, out=None, bias=None, alpha=1.0, beta=0.0, bpreshuffle=True, *,
              dtype=None, grid_blocks=0, kernel_id=0, workspace=None):
    """MXFP4 GEMM with aiter's gemm_a4w4 operand formats.

    A [M, K/2] packed e2m1 (row-major); B [N, K/2] bytes in
    shuffle_weight(16,16) order (``shuffle_weight_16x16``), N % 16 == 0;
    A_scale / B_scale: E8M0 in e8m0_shuffle order (``e8m0_shuffle``, or
    ``quant_mxfp4(x, shuffle=True)``), rows padded to 32; out [M, N], bf16
    unless ``dtype`` (or a given ``out``) says fp32.  ``grid_blocks`` > 0 runs a persistent grid of that
    many workgroups.  ``kernel_id``: 0 = the library's choice (M = 9-64 on
    the slice kernel where its plan fills the CUs in one round, else M <= 64
    on the burst kernel, else the one-by-four wave kernel), 1 = the two-by-two
    wave 256x256 kernel, 5 = the burst kernel (M <= 64), 8 = the one-by-four
    wave kernel (no persistent grid), 10 = the slice kernel (M <= 64).
    ``workspace``: as for the other entries (None: a cached buffer when a
    plan splits K; False: none, so only unsplit plans).  The epilogue has no bias or alpha/beta: anything but
    the defaults raises, and so does bpreshuffle=False (row-major B goes
    through gemm_a4w4_mxfp4)."""
    if bias is not None or alpha != 1.0 or beta != 0.0:
        raise NotImplementedError("gemm_a4w4: bias, alpha and beta are not supported")
    if not bpreshuffle:
        raise NotImplementedError("gemm_a4w4: row-major B goes through gemm_a4w4_mxfp4")
    dev = _require_gpu(A, B, A_scale, B_scale)
    if dtype is None:
        dtype = out.dtype if out is not None else torch.bfloat16
    m, kb = A.shape
    k = 2 * kb
    if B.dim() != 2 or B.shape[1] != kb or k % 256 or B.shape[0] % 16:
        raise ValueError("requires B [N, K/2] with N % 16 == 0 and K % 256 == 0")
    n = B.shape[0]
    if not (A.is_contiguous() and B.is_contiguous()):
        raise ValueError("A and B must be contiguous")
    sfa = _shuffled_scale(A_scale, m, k // 32, "A_scale")
    sfb = _shuffled_scale(B_scale, n, k // 32, "B_scale")
    out = _out(out, (m, n), dtype, dev)
    args = Mxfp4Kargs(A.data_ptr(), B.data_ptr(), out.data_ptr(), m, n, k, 1, kb, kb, n, m * kb, n * kb, m * n,
                      A_scale.data_ptr(), B_scale.data_ptr(), sfa, sfb, A_scale.numel(), B_scale.numel(),
                      int(grid_blocks))
    kid = int(kernel_id)
    with torch.cuda.device(dev):
        s = _stream(dev)
        query = lambda a: lib().gemm_a4w4_mxfp4_bpreshuffle_kid_workspace_bytes(a, kid)
        ws_ptr, ws_bytes = _workspace(query, args, workspace, dev, s)
        st = lib().gemm_a4w4_mxfp4_bpreshuffle_kid(ctypes.byref(args), _out_code(dtype), kid, ws_ptr, ws_bytes,
                                                   ctypes.c_void_p(s.cuda_stream))
        _record(s, A, B, A_scale, B_scale, out, _ws_tensor(workspace))
    _check(st, "gemm_a4w4_mxfp4_bpreshuffle")
    return out


def gemm_a8w8_bpreshuffle(A, B_kpanel, A_scale, B_scale, dtype=torch.bfloat16, out=None, workspace=None):
    """Block-scale FP8 with fp32 scales.

    A [M,K] e4m3; B_kpanel [K/128, N, 128] e4m3 (shuffle_b_kpanel of B [N,K]);
    A_scale fp32 [M,K/128] (row-major, BASELINE) or a [M,K/128] view with
    strides (1, M) (the reference's column-major [K/128][M]); B_scale fp32
    [ceil(N/128), K/128]."""
    dev = _require_gpu(A, B_kpanel, A_scale, B_scale)
    m, k = A.shape
    if B_kpanel.dim() != 3 or B_kpanel.shape[0] * 128 != k or B_kpanel.shape[2] != 128:
        raise ValueError("B_kpanel must be [K/128, N, 128]")
    n = B_kpanel.shape[1]
    kg = k // 128
    if k % 128 or A_scale.shape != (m, kg) or B_scale.shape != ((n + 127) // 128, kg):
        raise ValueError("requires K % 128 == 0, A_scale [M,K/128], B_scale [ceil(N/128),K/128]")
    if A_scale.dtype != torch.float32 or B_scale.dtype != torch.float32:
        raise ValueError("block scales must be fp32")
    if not (A.is_contiguous() and B_kpanel.is_contiguous() and B_scale.is_contiguous()):
        raise ValueError("A, B_kpanel and B_scale must be contiguous")
    stride_sfa = _sfa_stride(A_scale, m)
    out = _out(out, (m, n), dtype, dev)
    args = Kargs(A.data_ptr(), B_kpanel.data_ptr(), out.data_ptr(), m, n, k, 1, k, 128, n, m * k, n * k, m * n,
                 A_scale.data_ptr(), B_scale.data_ptr(), stride_sfa, kg, m * kg, B_scale.shape[0] * kg)
    with torch.cuda.device(dev):
        s = _stream(dev)
        ws_ptr, ws_bytes = _workspace(lib().gemm_a8w8_blockscale_bpreshuffle_workspace_bytes, args, workspace,
                                      dev, s)
        st = lib().gemm_a8w8_blockscale_bpreshuffle(ctypes.byref(args), _out_code(dtype), ws_ptr, ws_bytes,
                                                    ctypes.c_void_p(s.cuda_stream))
        _record(s, A, B_kpanel, A_scale, B_scale, out, _ws_tensor(workspace))
    _check(st, "gemm_a8w8_blockscale_bpreshuffle")
    return out


def _sfa_stride(A_scale, m):
    if A_scale.is_contiguous():
        return 1 if m > 1 else m
    if A_scale.stride() == (1, m):
        return m
    raise ValueError("A_scale must be row-major [M,K/128] or column-major with strides (1,M)")


def ldsbypass_b_bytes(n, k):
    """Bytes of B'' for an [N, K] fp8 weight (N padded to a multiple of 16)."""
    return lib().qgemm_ldsbypass_b_bytes(n, k)


def ldsbypass_pack_b(B):
    """B'' from raw B [N, K] (1-byte elements): on the GPU for a GPU tensor
    (qgemm_pack_b_ldsbypass_device), else the host pack."""
    if B.dim() != 2 or B.element_size() != 1:
        raise ValueError("B must be a 2-D [N, K] tensor of 1-byte elements")
    n, k = B.shape
    nbytes = ldsbypass_b_bytes(n, k)
    if nbytes == 0:
        raise ValueError("requires N >= 1 and K % 128 == 0")
    if B.is_cuda:
        from .quant import relayout_device
        return relayout_device("qgemm_pack_b_ldsbypass_device", _u8(B), nbytes)
    if not B.is_contiguous():
        raise ValueError("a host B must be contiguous")
    out = torch.empty(nbytes, dtype=torch.uint8)
    _check(lib().qgemm_pack_b_ldsbypass(B.data_ptr(), out.data_ptr(), n, k), "qgemm_pack_b_ldsbypass")
    return out


def ldsbypass_repack(B_kpanel, out=None):
    """GPU repack of the K-panel B' [K/128, N, 128] into B'' (LBP host.cc:289-294)."""
    dev = _require_gpu(B_kpanel)
    if B_kpanel.dim() != 3 or B_kpanel.shape[2] != 128 or not B_kpanel.is_contiguous():
        raise ValueError("B_kpanel must be a contiguous [K/128, N, 128] tensor")
    k, n = B_kpanel.shape[0] * 128, B_kpanel.shape[1]
    out = _out(out, (ldsbypass_b_bytes(n, k),), torch.uint8, dev)
    args = LdsBypassKargs(None, B_kpanel.data_ptr(), out.data_ptr(), None, 0, n, k, 1, 0, 128, 0, 0, n * k, 0,
                          None, None, 0, 0, 0, 0, out.numel())
    with torch.cuda.device(dev):
        s = _stream(dev)
        st = lib().gemm_a8w8_blockscale_ldsbypass_repack(ctypes.byref(args), ctypes.c_void_p(s.cuda_stream))
        _record(s, B_kpanel, out)
    _check(st, "gemm_a8w8_blockscale_ldsbypass_repack")
    return out


def gemm_a8w8_ldsbypass(A, B_pp, A_scale, B_scale, n, dtype=torch.bfloat16, out=None, workspace=None):
    """Block-scale FP8 (fp32 scales) with B given as B'' (``ldsbypass_repack``
    or ``ldsbypass_pack_b``); A, A_scale, B_scale as in gemm_a8w8_bpreshuffle."""
    dev = _require_gpu(A, B_pp, A_scale, B_scale)
    m, k = A.shape
    kg = k // 128
    if k % 128 or A_scale.shape != (m, kg) or B_scale.shape != ((n + 127) // 128, kg):
        raise ValueError("requires K % 128 == 0, A_scale [M,K/128], B_scale [ceil(N/128),K/128]")
    if A_scale.dtype != torch.float32 or B_scale.dtype != torch.float32:
        raise ValueError("block scales must be fp32")
    if B_pp.numel() * B_pp.element_size() != ldsbypass_b_bytes(n, k):
        raise ValueError("B_pp must hold ldsbypass_b_bytes(N, K) bytes")
    if not (A.is_contiguous() and B_pp.is_contiguous() and B_scale.is_contiguous()):
        raise ValueError("A, B_pp and B_scale must be contiguous")
    stride_sfa = _sfa_stride(A_scale, m)
    out = _out(out, (m, n), dtype, dev)
    args = LdsBypassKargs(A.data_ptr(), None, B_pp.data_ptr(), out.data_ptr(), m, n, k, 1, k, 128, n, m * k,
                          n * k, m * n, A_scale.data_ptr(), B_scale.data_ptr(), stride_sfa, kg, m * kg,
                          B_scale.shape[0] * kg, B_pp.numel() * B_pp.element_size())
    with torch.cuda.device(dev):
        s = _stream(dev)
        ws_ptr, ws_bytes = _workspace(lib().gemm_a8w8_blockscale_ldsbypass_workspace_bytes, args, workspace,
                                      dev, s)
        st = lib().gemm_a8w8_blockscale_ldsbypass(ctypes.byref(args), _out_code(dtype), ws_ptr, ws_bytes,
                                                  ctypes.c_void_p(s.cuda_stream))
        _record(s, A, B_pp, A_scale, B_scale, out, _ws_tensor(workspace))
    _check(st, "gemm_a8w8_blockscale_ldsbypass")
    return out


def probe_mfma_layout(device=None):
    """Run the layout probes; returns the int32 word tensor (see csrc/probe.hip)."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    words = lib().qgemm_probe_words()
    out = torch.zeros(words, dtype=torch.int32, device=device)
    with torch.cuda.device(device):
        s = _stream(device)
        st = lib().qgemm_probe_mfma_layout(ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(s.cuda_stream))
    _check(st, "qgemm_probe_mfma_layout")
    torch.cuda.synchronize(device)
    return out.cpu()


# ------------------------------------------------------------------ layouts
def shuffle_b_kpanel(B):
    """K-panel pre-shuffle (BPS host.cc:92-111): [N, K] -> [K/128, N, 128].
    A GPU tensor is shuffled by qgemm_shuffle_b_kpanel_device."""
    n, k = B.shape
    if k % 128:
        raise ValueError("K must be a multiple of 128")
    if B.is_cuda:
        from .quant import relayout_device
        return relayout_device("qgemm_shuffle_b_kpanel_device", _u8(B), n * k).view(B.dtype).view(k // 128, n, 128)
    return B.reshape(n, k // 128, 128).permute(1, 0, 2).contiguous()


def shuffle_weight_16x16(B):
    """shuffle_weight(layout=(16,16)) over bytes: [N, Kb] -> [N/16, Kb/16, 16, 16]
    (SNAP host.cc:161-179), returned as [N, Kb].  A GPU tensor is shuffled
    by qgemm_shuffle_weight_16x16_device."""
    n, kb = B.shape
    if n % 16 or kb % 16:
        raise ValueError("N and K bytes must be multiples of 16")
    if B.is_cuda:
        from .quant import relayout_device
        return relayout_device("qgemm_shuffle_weight_16x16_device", _u8(B), n * kb).view(B.dtype).view(n, kb)
    return B.reshape(n // 16, 16, kb // 16, 16).permute(0, 2, 1, 3).contiguous().reshape(n, kb)


from . import blockscale_bpreshuffle  # noqa: E402  (reference adapter mirror)
from .opus import (gemm_a8w8_bpreshuffle_opus, gemm_a8w8_mxfp8_opus, opus_gemm_mxfp8_nn,  # noqa: E402,F401
                   opus_gemm_mxfp8_nt, opus_gemm_mxfp8_tn, opus_gemm_mxfp8_tt)
from .quant import (e8m0_shuffle, quant_fp8_blockscale, quant_fp8_e8m0_blockscale,  # noqa: E402,F401
                    quant_mxfp4, quant_mxfp8)


GROUP_MAX = 16
_GROUPED = {
    "bpreshuffle": ("gemm_a8w8_blockscale_bpreshuffle_grouped", Kargs),
    "ldsbypass": ("gemm_a8w8_blockscale_ldsbypass_grouped", LdsBypassKargs),
    "mxfp8": ("gemm_a8w8_mxfp8_grouped", Kargs),
    "mxfp4": ("gemm_a4w4_mxfp4_grouped", Kargs),
}


def _group_kargs(kind, A, B, A_scale, B_scale, out, n):
    """kargs of one grouped problem (batch 1, M <= 64, contiguous operands)."""
    m = A.shape[0]
    if kind in ("mxfp8", "mxfp4"):
        fp4 = kind == "mxfp4"
        kb = A.shape[1]
        k = 2 * kb if fp4 else kb
        if B.dim() != 2 or B.shape[1] != kb or A_scale.shape != (m, k // 32) or B_scale.shape != (B.shape[0], k // 32):
            raise ValueError(f"{kind}: A [M,{'K/2' if fp4 else 'K'}], B [N,...], scales [rows, K/32]")
        n = B.shape[0]
        return Kargs(A.data_ptr(), B.data_ptr(), out.data_ptr(), m, n, k, 1, kb, kb, n, m * kb, n * kb, m * n,
                     A_scale.data_ptr(), B_scale.data_ptr(), k // 32, k // 32, m * (k // 32), n * (k // 32))
    k = A.shape[1]
    kg = k // 128
    if kind == "bpreshuffle":
        if B.dim() != 3 or B.shape[0] * 128 != k or B.shape[2] != 128:
            raise ValueError("bpreshuffle: B must be the K-panel [K/128, N, 128]")
        n = B.shape[1]
    elif n is None:
        raise ValueError("ldsbypass: give N for each B'' (problems as (A, B'', A_scale, B_scale, N))")
    if A_scale.shape != (m, kg) or B_scale.shape != ((n + 127) // 128, kg) or not B_scale.is_contiguous():
        raise ValueError("block scales: A_scale fp32 [M,K/128], B_scale fp32 [ceil(N/128),K/128]")
    sfa = _sfa_stride(A_scale, m)
    if kind == "bpreshuffle":
        return Kargs(A.data_ptr(), B.data_ptr(), out.data_ptr(), m, n, k, 1, k, 128, n, m * k, n * k, m * n,
                     A_scale.data_ptr(), B_scale.data_ptr(), sfa, kg, m * kg, B_scale.shape[0] * kg)
    return LdsBypassKargs(A.data_ptr(), None, B.data_ptr(), out.data_ptr(), m, n, k, 1, k, 128, n, m * k, 0, m * n,
                          A_scale.data_ptr(), B_scale.data_ptr(), sfa, kg, m * kg, B_scale.shape[0] * kg, B.numel())


def gemm_grouped(kind, problems, dtype=torch.bfloat16, outs=None, grid_blocks=0, workspace=None):
    """Several decode GEMMs (M <= 64 each, up to GROUP_MAX) in one launch.

    ``kind``: "bpreshuffle" (problems (A, B_kpanel, A_scale, B_scale), fp32
    block scales), "ldsbypass" ((A, B'', A_scale, B_scale, N)), "mxfp8" or
    "mxfp4" ((A, B, A_scale, B_scale), row-major, E8M0 per 32).  Each problem
    has its own N, K, M, operands and output; one grid walks all their
    (tile, K slice) items.  ``grid_blocks`` > 0 runs a persistent grid of
    that many workgroups.  Returns the list of outputs [M, N]."""
    if kind not in _GROUPED:
        raise ValueError(f"kind must be one of {sorted(_GROUPED)}")
    if not 1 <= len(problems) <= GROUP_MAX:
        raise ValueError(f"1 to {GROUP_MAX} problems")
    name, ktype = _GROUPED[kind]
    flat = [t for pr in problems for t in pr[:4]]
    dev = _require_gpu(*flat)
    for pr in problems:
        if not all(t.is_contiguous() for t in (pr[0], pr[1], pr[3])):
            raise ValueError("A, B and B_scale must be contiguous")
        if kind in ("mxfp8", "mxfp4") and not pr[2].is_contiguous():
            raise ValueError("E8M0 scales must be contiguous")
    if outs is None:
        outs = []
        for pr in problems:
            n = pr[1].shape[1] if kind == "bpreshuffle" else (pr[4] if kind == "ldsbypass" else pr[1].shape[0])
            outs.append(torch.empty((pr[0].shape[0], n), dtype=dtype, device=dev))
    arr = (ktype * len(problems))(*[_group_kargs(kind, pr[0], pr[1], pr[2], pr[3], o, pr[4] if len(pr) > 4 else None)
                                    for pr, o in zip(problems, outs)])
    L = lib()
    with torch.cuda.device(dev):
        s = _stream(dev)
        if workspace is False:
            wp, wb = None, 0
        elif workspace is not None:
            wp, wb = workspace.data_ptr(), workspace.numel() * workspace.element_size()
        else:
            need = getattr(L, name + "_workspace_bytes")(arr, len(problems))
            buf = _WORKSPACES.get(("grouped", dev.index, s.cuda_stream))
            if need and (buf is None or buf.numel() < need):
                buf = torch.zeros((need + 255) // 256 * 256, dtype=torch.uint8, device=dev)
                _WORKSPACES[("grouped", dev.index, s.cuda_stream)] = buf
            wp, wb = (buf.data_ptr(), buf.numel()) if need else (None, 0)
        st = getattr(L, name)(arr, len(problems), _out_code(dtype), int(grid_blocks), wp, wb,
                              ctypes.c_void_p(s.cuda_stream))
        _record(s, *flat, *outs)
    _check(st, name)
    return outs


_REF_FAMILY = {"bs_fp32": 0, "bs_e8m0": 1, "mxfp8": 2, "mxfp4": 3}


def reference_gemm(kind, A, B, A_scale, B_scale):
    """The whole-output GPU reference GEMM (qgemm_reference_gemm): fp32
    [M, N] from fp64 sums of decoded, scaled products.  Row-major codes A
    [M, K] (fp4: [M, K/2]) and B [N, K]; scales as the family's entry takes
    them -- "bs_fp32": fp32 [M, K/128] (row-major, or the strides-(1, M) view
    of [K/128][M]) and [ceil(N/128), K/128]; "bs_e8m0": the same in E8M0
    bytes; "mxfp8" / "mxfp4": E8M0 [rows, K/32]."""
    if kind not in _REF_FAMILY:
        raise ValueError(f"kind must be one of {sorted(_REF_FAMILY)}")
    dev = _require_gpu(A, B, A_scale, B_scale)
    fp4 = kind == "mxfp4"
    m, kb = A.shape
    n = B.shape[0]
    k = 2 * kb if fp4 else kb
    if B.shape[1] != kb or not (A.is_contiguous() and B.is_contiguous() and B_scale.is_contiguous()):
        raise ValueError("A [M, K] and B [N, K] contiguous codes, B_scale contiguous")
    if kind in ("mxfp8", "mxfp4"):
        if not A_scale.is_contiguous():
            raise ValueError("A_scale must be contiguous")
        sfa, sfb = A_scale.stride(0), B_scale.stride(0)
    else:
        sfa, sfb = _sfa_stride(A_scale, m), B_scale.stride(0)
    out = torch.empty((m, n), dtype=torch.float32, device=dev)
    args = Kargs(A.data_ptr(), B.data_ptr(), out.data_ptr(), m, n, k, 1, kb, kb, n, 0, 0, 0,
                 A_scale.data_ptr(), B_scale.data_ptr(), sfa, sfb, 0, 0)
    with torch.cuda.device(dev):
        s = _stream(dev)
        st = lib().qgemm_reference_gemm(_REF_FAMILY[kind], ctypes.byref(args), ctypes.c_void_p(s.cuda_stream))
        _record(s, A, B, A_scale, B_scale, out)
    _check(st, "qgemm_reference_gemm")
    return out
