"""Block-scale FP8 GEMM with E8M0 scales, behind the reference's Python entry.

The reference's caller-facing function is
``gemm_a8w8_blockscale_bpreshuffle(A, B, A_scale, B_scale, dtype=torch.bfloat16,
out=None, *, tiles=0)`` (SNAP blockscale_bpreshuffle.py:37-97).  This module
keeps that name, signature and error behaviour -- ``ValueError`` for an
argument the launcher would reject, ``RuntimeError`` when the launch itself
fails -- and runs ``launch_blockscale_bpreshuffle`` of libqgemm.so on the
current stream.

Operand formats (the launcher's contract): A e4m3 [M, K]; B e4m3 bytes in
shuffle_weight(16, 16) order; A_scale E8M0 bytes, logical [M, K/128] with
column-major bytes (strides (1, M), or a contiguous tensor whose bytes the
quantizer already transposed); B_scale E8M0 [N/128, K/128].  M and N are
multiples of 256, K of 128.  Nothing is converted, copied or allocated
besides ``out``.

The checks are data: ``_RULES`` lists, in order, the condition each call must
meet and the message raised when it does not, so the contract reads in one
place and the tests can walk it.
"""
import ctypes

import torch

from . import Kargs, lib

_FP8 = torch.float8_e4m3fn
_E8M0 = {torch.uint8} | ({torch.float8_e8m0fnu} if hasattr(torch, "float8_e8m0fnu") else set())
_OUT = {torch.bfloat16: (1, 2), torch.float32: (0, 4)}    # dtype -> (output_bf16 flag, bytes)
_I32_MAX = 2 ** 31 - 1


def _dims(c):
    m, k = c["A"].shape
    n, kb = c["B"].shape
    return m, n, k, kb


# (condition on the call, message) -- evaluated in order, first failure raises.
_RULES = (
    (lambda c: all(t.dim() == 2 for t in c["inputs"]),
     "A, B, A_scale and B_scale must be 2-D tensors"),
    (lambda c: c["A"].is_cuda and all(t.device == c["A"].device for t in c["inputs"]),
     "A, B, A_scale and B_scale must live on one GPU"),
    (lambda c: c["A"].dtype == _FP8 and c["B"].dtype in (_FP8, torch.uint8),
     "A must be float8_e4m3fn and B e4m3 bytes (float8_e4m3fn or uint8)"),
    (lambda c: c["A_scale"].dtype in _E8M0 and c["B_scale"].dtype in _E8M0,
     "A_scale and B_scale must hold E8M0 exponent bytes (uint8 or float8_e8m0fnu), not fp32 scales"),
    (lambda c: (lambda m, n, k, kb: min(m, n, k) > 0 and k == kb and m % 256 == 0 and n % 256 == 0
                and k % 128 == 0)(*_dims(c)),
     "shapes must satisfy K(A) == K(B), M % 256 == 0, N % 256 == 0 and K % 128 == 0"),
    (lambda c: c["dtype"] in _OUT and c["tiles"] in (0, 1),
     "dtype must be torch.bfloat16 or torch.float32 and tiles must be 0 or 1"),
    (lambda c: c["A"].is_contiguous() and c["B"].is_contiguous() and c["B_scale"].is_contiguous(),
     "A, the shuffled B and B_scale must be contiguous"),
    (lambda c: (lambda m, n, k, kb: tuple(c["A_scale"].shape) == (m, k // 128)
                and tuple(c["B_scale"].shape) == (n // 128, k // 128))(*_dims(c)),
     "A_scale must be [M, K/128] and B_scale [N/128, K/128]"),
    (lambda c: c["A_scale"].is_contiguous() or c["A_scale"].stride() == (1, c["A"].shape[0]),
     "A_scale must be column-major bytes: strides (1, M), or contiguous pre-transposed bytes"),
    (lambda c: (lambda m, n, k, kb: max(m * k, n * k, m * n * _OUT[c["dtype"]][1]) <= _I32_MAX)(*_dims(c)),
     "each operand must stay below 2 GiB (the kernels use 32-bit offsets)"),
)


def _extent(t):
    """[first, last) byte addresses a strided tensor can touch."""
    span = 1 + sum((s - 1) * st for s, st in zip(t.shape, t.stride()) if s > 0)
    return t.data_ptr(), t.data_ptr() + span * t.element_size()


def _disjoint(x, y):
    (a0, a1), (b0, b1) = _extent(x), _extent(y)
    return a1 <= b0 or b1 <= a0


def gemm_a8w8_blockscale_bpreshuffle(A, B, A_scale, B_scale, dtype=torch.bfloat16, out=None, *, tiles=0):
    """Y[M, N] = sum over K blocks of (A_blk . B_blk^T) * 2^(ea - 127) * 2^(eb - 127), one launch.

    Raises ValueError for arguments outside the contract above and
    RuntimeError if the launch returns a HIP error."""
    call = {"A": A, "B": B, "A_scale": A_scale, "B_scale": B_scale, "dtype": dtype, "tiles": tiles,
            "inputs": (A, B, A_scale, B_scale)}
    for ok, message in _RULES:
        if not ok(call):
            raise ValueError(message)
    m, n, k, _ = _dims(call)
    flag, _ = _OUT[dtype]

    if out is None:
        out = torch.empty((m, n), dtype=dtype, device=A.device)
    elif not (tuple(out.shape) == (m, n) and out.dtype == dtype and out.device == A.device and out.is_contiguous()):
        raise ValueError("out must be a contiguous [M, N] tensor of the requested dtype on A's device")
    if not all(_disjoint(out, t) for t in call["inputs"]):
        raise ValueError("out must not share memory with an input")

    kb = k // 128
    kargs = Kargs(ptr_a=A.data_ptr(), ptr_b=B.data_ptr(), ptr_c=out.data_ptr(), m=m, n=n, k=k, batch=1,
                  stride_a=k, stride_b=k, stride_c=n, stride_a_batch=m * k, stride_b_batch=n * k,
                  stride_c_batch=m * n, ptr_sfa=A_scale.data_ptr(), ptr_sfb=B_scale.data_ptr(),
                  stride_sfa=m, stride_sfb=kb, stride_sfa_batch=m * kb, stride_sfb_batch=(n // 128) * kb)
    with torch.cuda.device(A.device):
        stream = torch.cuda.current_stream(A.device)
        status = lib().launch_blockscale_bpreshuffle(ctypes.byref(kargs), flag, tiles,
                                                     ctypes.c_void_p(stream.cuda_stream))
        # the kernel reads and writes these tensors on `stream`, outside the
        # caching allocator's view: keep their memory alive until it is done
        for t in (*call["inputs"], out):
            t.record_stream(stream)
    if status != 0:
        raise RuntimeError(f"launch_blockscale_bpreshuffle returned HIP error {status}")
    return out
