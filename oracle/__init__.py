"""CPU oracle for the quantized-GEMM hot path -- TEST INFRASTRUCTURE ONLY.

numpy/ctypes front end of ``qgemm_oracle.c``: value codecs, seeded N(0,1)
data, the BASELINE.json quantizers, the layout transforms and the CPU
reference GEMMs restated from the reference drivers (file:line citations in
qgemm_oracle.h / qgemm_oracle.c).  Only ``tests/``, ``__graft_entry__.smoke``
and the ``cpu_baseline`` leg of ``bench.py`` may import this package, and
only as the checker; the product library never calls it.
"""
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "liboracle.so"
_lib = None

_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i = ctypes.c_int
_sz = ctypes.c_size_t


def build(force=False):
    """Compile liboracle.so with the committed Makefile (gcc, OpenMP)."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", str(_DIR)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        sigs = {
            "ora_e4m3_to_f32": (ctypes.c_float, [ctypes.c_uint8]),
            "ora_f32_to_e4m3": (ctypes.c_uint8, [ctypes.c_float]),
            "ora_e8m0_to_f32": (ctypes.c_float, [ctypes.c_uint8]),
            "ora_e2m1_to_f32": (ctypes.c_float, [ctypes.c_uint]),
            "ora_f32_to_e2m1": (ctypes.c_uint, [ctypes.c_float]),
            "ora_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "ora_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "ora_f32_to_bf16_array": (None, [_f32p, _u16p, _sz]),
            "ora_bf16_to_f32_array": (None, [_u16p, _f32p, _sz]),
            "ora_e4m3_decode_array": (None, [_u8p, _f32p, _sz]),
            "ora_mix_bits": (ctypes.c_uint64, [ctypes.c_uint64]),
            "ora_randn": (None, [_f32p, _sz, ctypes.c_uint64, ctypes.c_uint64]),
            "ora_quant_bs_act": (None, [_f32p, _i, _i, _u8p, _f32p]),
            "ora_quant_bs_wgt": (None, [_f32p, _i, _i, _u8p, _f32p]),
            "ora_quant_mx8": (None, [_f32p, _i, _i, _u8p, _u8p]),
            "ora_quant_mx4": (None, [_f32p, _i, _i, _u8p, _u8p]),
            "ora_quant_bs_e8m0_act": (None, [_f32p, _i, _i, _u8p, _u8p]),
            "ora_quant_bs_e8m0_wgt": (None, [_f32p, _i, _i, _u8p, _u8p]),
            "ora_ceil_log2": (_i, [ctypes.c_float]),
            "ora_shuffle_b_kpanel": (None, [_u8p, _u8p, _i, _i, _i]),
            "ora_shuffle_weight_16x16": (None, [_u8p, _u8p, _i, _i]),
            "ora_e8m0_shuffle_bytes": (_sz, [_i, _i]),
            "ora_e8m0_shuffle": (None, [_u8p, _u8p, _i, _i]),
            "ora_gemm_bs_fp32": (None, [_u8p, _u8p, _f32p, _f32p, _f32p] + [_i] * 10),
            "ora_gemm_mx8": (None, [_u8p, _u8p, _u8p, _u8p, _f32p] + [_i] * 8),
            "ora_gemm_mx4": (None, [_u8p, _u8p, _u8p, _u8p, _f32p] + [_i] * 8),
            "ora_gemm_mx4_grouped": (None, [_u8p, _u8p, _u8p, _u8p, _f32p] + [_i] * 8),
            "ora_gemm_bs_e8m0": (None, [_u8p, _u8p, _u8p, _u8p, _f32p, ctypes.c_void_p] + [_i] * 8),
            "ora_gemm_bs_fp32_points": (None, [_u8p, _u8p, _f32p, _f32p] + [_i] * 7 + [_i32p, _i32p, _sz, _f32p]),
            "ora_gemm_mx8_points": (None, [_u8p, _u8p, _u8p, _u8p] + [_i] * 5 + [_i32p, _i32p, _sz, _f32p]),
            "ora_gemm_bs_e8m0_points": (None, [_u8p, _u8p, _u8p, _u8p] + [_i] * 5 + [_i32p, _i32p, _sz, _f32p]),
            "ora_gemm_mx4_points": (None, [_u8p, _u8p, _u8p, _u8p] + [_i] * 5 + [_i32p, _i32p, _sz, _f32p]),
            "ora_check_tolerance": (_sz, [_f32p, _f32p, _sz, ctypes.c_double,
                                          ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_size_t)]),
            "ora_rms": (ctypes.c_double, [_f32p, _sz]),
            "ora_num_threads": (_i, []),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _c(x, dtype):
    return np.ascontiguousarray(x, dtype=dtype)


# ---------------------------------------------------------------- codecs
def e4m3_decode(q):
    q = _c(q, np.uint8)
    out = np.empty(q.shape, np.float32)
    lib().ora_e4m3_decode_array(q.reshape(-1), out.reshape(-1), q.size)
    return out


def e4m3_encode(x):
    x = np.asarray(x, np.float32)
    return np.array([lib().ora_f32_to_e4m3(float(v)) for v in x.reshape(-1)], np.uint8).reshape(x.shape)


def e2m1_encode(x):
    x = np.asarray(x, np.float32)
    return np.array([lib().ora_f32_to_e2m1(float(v)) for v in x.reshape(-1)], np.uint8).reshape(x.shape)


def e2m1_decode(codes):
    codes = np.asarray(codes)
    return np.array([lib().ora_e2m1_to_f32(int(c)) for c in codes.reshape(-1)], np.float32).reshape(codes.shape)


def e8m0_decode(e):
    e = np.asarray(e, np.uint8)
    return np.array([lib().ora_e8m0_to_f32(int(v)) for v in e.reshape(-1)], np.float32).reshape(e.shape)


def bf16_round_bits(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().ora_f32_to_bf16_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_bits_to_f32(b):
    b = _c(b, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().ora_bf16_to_f32_array(b.reshape(-1), out.reshape(-1), b.size)
    return out


def round_bf16(x):
    return bf16_bits_to_f32(bf16_round_bits(x))


# ---------------------------------------------------------------- data
def randn(shape, seed=0, stream=0):
    out = np.empty(shape, np.float32)
    lib().ora_randn(out.reshape(-1), out.size, int(seed), int(stream))
    return out


def quant_bs_act(x):
    x = _c(x, np.float32)
    m, k = x.shape
    assert k % 128 == 0
    q = np.empty((m, k), np.uint8)
    s = np.empty((m, k // 128), np.float32)
    lib().ora_quant_bs_act(x, m, k, q, s)
    return q, s


def quant_bs_wgt(w):
    w = _c(w, np.float32)
    n, k = w.shape
    assert k % 128 == 0
    q = np.empty((n, k), np.uint8)
    s = np.empty(((n + 127) // 128, k // 128), np.float32)
    lib().ora_quant_bs_wgt(w, n, k, q, s)
    return q, s


def quant_mx8(x):
    x = _c(x, np.float32)
    r, k = x.shape
    assert k % 32 == 0
    q = np.empty((r, k), np.uint8)
    e = np.empty((r, k // 32), np.uint8)
    lib().ora_quant_mx8(x, r, k, q, e)
    return q, e


def quant_mx4(x):
    x = _c(x, np.float32)
    r, k = x.shape
    assert k % 32 == 0
    q = np.empty((r, k // 2), np.uint8)
    e = np.empty((r, k // 32), np.uint8)
    lib().ora_quant_mx4(x, r, k, q, e)
    return q, e


def quant_bs_e8m0_act(x):
    """e4m3 [M,K] and E8M0 codes [M,K/128], one 2^ceil(log2(amax/448)) per 1x128 block."""
    x = _c(x, np.float32)
    m, k = x.shape
    assert k % 128 == 0
    q = np.empty((m, k), np.uint8)
    e = np.empty((m, k // 128), np.uint8)
    lib().ora_quant_bs_e8m0_act(x, m, k, q, e)
    return q, e


def quant_bs_e8m0_wgt(w):
    """e4m3 [N,K] and E8M0 codes [ceil(N/128),K/128], one per 128x128 block."""
    w = _c(w, np.float32)
    n, k = w.shape
    assert k % 128 == 0
    q = np.empty((n, k), np.uint8)
    e = np.empty(((n + 127) // 128, k // 128), np.uint8)
    lib().ora_quant_bs_e8m0_wgt(w, n, k, q, e)
    return q, e


# ---------------------------------------------------------------- layouts
def shuffle_b_kpanel(b, block_k=128):
    b = _c(b, np.uint8)
    n, kb = b.shape
    assert kb % block_k == 0
    out = np.empty(kb * n, np.uint8)
    lib().ora_shuffle_b_kpanel(b, out, n, kb, block_k)
    return out.reshape(kb // block_k, n, block_k)


def shuffle_weight_16x16(b):
    b = _c(b, np.uint8)
    n, kb = b.shape
    assert n % 16 == 0 and kb % 16 == 0
    out = np.empty(n * kb, np.uint8)
    lib().ora_shuffle_weight_16x16(b, out, n, kb)
    return out.reshape(n, kb)


def e8m0_shuffle(e):
    e = _c(e, np.uint8)
    rows, kg = e.shape
    nbytes = lib().ora_e8m0_shuffle_bytes(rows, kg)
    out = np.empty(nbytes, np.uint8)
    lib().ora_e8m0_shuffle(e, out, rows, kg)
    return out


# ---------------------------------------------------------------- GEMMs
def gemm_bs_fp32(a, b, sfa, sfb, sfa_layout="mk"):
    """C[M,N] fp32 of the block-scale FP8 reference (BPS host.cc:66-90).

    a [M,K], b [N,K] e4m3 bytes (raw, K-contiguous); sfb [ceil(N/128),K/128];
    sfa [M,K/128] when sfa_layout == "mk", or [K/128,M] when "km"."""
    a, b = _c(a, np.uint8), _c(b, np.uint8)
    sfa, sfb = _c(sfa, np.float32), _c(sfb, np.float32)
    m, k = a.shape
    n = b.shape[0]
    kg = k // 128
    if sfa_layout == "mk":
        sm, sk = kg, 1
    else:
        sm, sk = 1, m
    c = np.empty((m, n), np.float32)
    lib().ora_gemm_bs_fp32(a, b, sfa, sfb, c, m, n, k, k, k, n, sm, sk, kg, 1)
    return c


def gemm_bs_fp32_points(a, b, sfa, sfb, rows, cols, sfa_layout="mk"):
    a, b = _c(a, np.uint8), _c(b, np.uint8)
    sfa, sfb = _c(sfa, np.float32), _c(sfb, np.float32)
    m, k = a.shape
    kg = k // 128
    sm, sk = (kg, 1) if sfa_layout == "mk" else (1, m)
    rows, cols = _c(rows, np.int32), _c(cols, np.int32)
    out = np.empty(rows.size, np.float32)
    lib().ora_gemm_bs_fp32_points(a, b, sfa, sfb, k, k, k, sm, sk, kg, 1, rows, cols, rows.size, out)
    return out


def gemm_mx8(a, b, sfa, sfb):
    a, b, sfa, sfb = (_c(t, np.uint8) for t in (a, b, sfa, sfb))
    m, k = a.shape
    n = b.shape[0]
    c = np.empty((m, n), np.float32)
    lib().ora_gemm_mx8(a, b, sfa, sfb, c, m, n, k, k, k, n, sfa.shape[1], sfb.shape[1])
    return c


def gemm_mx8_points(a, b, sfa, sfb, rows, cols):
    a, b, sfa, sfb = (_c(t, np.uint8) for t in (a, b, sfa, sfb))
    k = a.shape[1]
    rows, cols = _c(rows, np.int32), _c(cols, np.int32)
    out = np.empty(rows.size, np.float32)
    lib().ora_gemm_mx8_points(a, b, sfa, sfb, k, k, k, sfa.shape[1], sfb.shape[1], rows, cols, rows.size, out)
    return out


def gemm_mx4(a, b, sfa, sfb, literal=False):
    """a [M,K/2], b [N,K/2] packed e2m1 bytes; scales [rows, K/32].

    Default: the grouped form of the reference's gemm_ref_gpu (MX4
    host.cc:66-94); literal=True: the per-element gemm_ref_cpu loop
    (MX4 host.cc:96-115).  Both are exact up to the final fp32 rounding and
    agree bit for bit on every recipe here (tests/test_oracle.py)."""
    a, b, sfa, sfb = (_c(t, np.uint8) for t in (a, b, sfa, sfb))
    m, kb = a.shape
    n = b.shape[0]
    c = np.empty((m, n), np.float32)
    fn = lib().ora_gemm_mx4 if literal else lib().ora_gemm_mx4_grouped
    fn(a, b, sfa, sfb, c, m, n, 2 * kb, kb, kb, n, sfa.shape[1], sfb.shape[1])
    return c


def gemm_mx4_points(a, b, sfa, sfb, rows, cols):
    a, b, sfa, sfb = (_c(t, np.uint8) for t in (a, b, sfa, sfb))
    kb = a.shape[1]
    rows, cols = _c(rows, np.int32), _c(cols, np.int32)
    out = np.empty(rows.size, np.float32)
    lib().ora_gemm_mx4_points(a, b, sfa, sfb, 2 * kb, kb, kb, sfa.shape[1], sfb.shape[1], rows, cols,
                              rows.size, out)
    return out


def gemm_bs_e8m0(a, b, sfa_km, sfb, with_mag=False):
    """SNAP reference: sfa_km physical [K/128, M], sfb [N/128, K/128] e8m0."""
    a, b, sfa_km, sfb = (_c(t, np.uint8) for t in (a, b, sfa_km, sfb))
    m, k = a.shape
    n = b.shape[0]
    c = np.empty((m, n), np.float32)
    mag = np.empty((m, n), np.float64) if with_mag else None
    lib().ora_gemm_bs_e8m0(a, b, sfa_km, sfb, c, mag.ctypes.data if with_mag else None,
                           m, n, k, k, k, n, m, k // 128)
    return (c, mag) if with_mag else c


def gemm_bs_e8m0_points(a, b, sfa_km, sfb, rows, cols):
    """Sampled (rows[t], cols[t]) outputs of gemm_bs_e8m0."""
    a, b, sfa_km, sfb = (_c(t, np.uint8) for t in (a, b, sfa_km, sfb))
    m, k = a.shape
    rows, cols = _c(rows, np.int32), _c(cols, np.int32)
    out = np.empty(rows.size, np.float32)
    lib().ora_gemm_bs_e8m0_points(a, b, sfa_km, sfb, k, k, k, m, k // 128, rows, cols, rows.size, out)
    return out


# ---------------------------------------------------------------- tolerance
def check_tolerance(ref, got, rms=None):
    """(#violations, max ratio, worst index) of |got-ref| <= 2^-7|ref| + 1e-3 rms(ref)."""
    ref, got = _c(ref, np.float32).reshape(-1), _c(got, np.float32).reshape(-1)
    mr = ctypes.c_double()
    wi = ctypes.c_size_t()
    bad = lib().ora_check_tolerance(ref, got, ref.size, float(rms or 0.0), ctypes.byref(mr), ctypes.byref(wi))
    return int(bad), float(mr.value), int(wi.value)


def rms(x):
    x = _c(x, np.float32).reshape(-1)
    return float(lib().ora_rms(x, x.size))


def num_threads():
    return int(lib().ora_num_threads())
