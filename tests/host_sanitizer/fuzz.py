"""Random-argument fuzz of the host side of libqgemm.so (CPU only; meant to
run against the sanitized build of build.py, see run.sh).

* every workspace query and kernel-id query over random and extreme shapes
  (the planners);
* every GEMM entry, quantizer and device layout entry with random, mostly
  invalid arguments: on a host without a GPU each must return an error;
* the host layout helpers on exact-size buffers.

Usage: python fuzz.py <libqgemm.so> [seed] [iterations]
"""
import ctypes
import importlib
import pathlib
import random
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
q = importlib.import_module("355_1_trans_amd")
q.LIB_PATH = pathlib.Path(sys.argv[1])
L = q.lib()
rng = random.Random(int(sys.argv[2]) if len(sys.argv) > 2 else 0)
ITERS = int(sys.argv[3]) if len(sys.argv) > 3 else 3000
INT_MAX = (1 << 31) - 1


def dim():
    r = rng.random()
    if r < 0.3:
        return rng.randint(1, 128)
    if r < 0.6:
        return rng.randint(1, 40000)
    if r < 0.8:
        return rng.choice([256, 2048, 7168, 8192, 24576, 32768, 129280])
    return rng.choice([rng.randint(1, 1 << 20), INT_MAX, INT_MAX - 15])


def v():
    return rng.choice([0, 1, -1, 7, 16, 128, 256, 4096, 1 << 20, INT_MAX, -INT_MAX - 1, rng.randint(-1000, 100000)])


def p():
    return rng.choice([None, 0x1000, 0x1001, 0x100000, 0x7fff00000000])


def lv():
    return rng.choice([0, 1, 16, 1 << 40, 1 << 62, -(1 << 62), rng.randint(0, 1 << 34)])


def queries():
    m, n = dim(), dim()
    k = rng.choice([128, 256]) * rng.choice([1, 2, 4, 12, 56, 64, 128, rng.randint(1, 512)])
    batch = rng.choice([1, 1, 2, 3, 64])
    kg, kg32 = k // 128, k // 32
    a = q.Kargs(1 << 20, 1 << 21, 1 << 22, m, n, k, batch, k, 128, n, m * k, n * k, m * n, 1 << 23, 1 << 24, 1, kg,
                m * kg, ((n + 127) // 128) * kg)
    L.gemm_a8w8_blockscale_bpreshuffle_workspace_bytes(ctypes.byref(a))
    for lay in range(-1, 5):
        L.gemm_a8w8_blockscale_layout_workspace_bytes(ctypes.byref(a), lay)
    mx = q.Kargs(1 << 20, 1 << 21, 1 << 22, m, n, k, batch, k, k, n, m * k, n * k, m * n, 1 << 23, 1 << 24, kg32,
                 kg32, m * kg32, n * kg32)
    nbp = ((n + 15) // 16) * 16 * k
    lb = q.LdsBypassKargs(1 << 20, None, 1 << 21, 1 << 22, m, n, k, batch, k, 128, n, m * k, nbp, m * n, 1 << 23,
                          1 << 24, 1, kg, m * kg, ((n + 127) // 128) * kg, nbp)
    L.gemm_a8w8_blockscale_ldsbypass_workspace_bytes(ctypes.byref(lb))
    for name in ("gemm_a8w8_mxfp8", "gemm_a4w4_mxfp4"):
        getattr(L, name + "_workspace_bytes")(ctypes.byref(mx))
    for kid in range(-1, 9):
        L.gemm_a8w8_blockscale_bpreshuffle_kid_workspace_bytes(ctypes.byref(a), kid)
        L.gemm_a8w8_blockscale_ldsbypass_kid_workspace_bytes(ctypes.byref(lb), kid)
        L.gemm_a8w8_mxfp8_kid_workspace_bytes(ctypes.byref(mx), kid)
        L.gemm_a4w4_mxfp4_kid_workspace_bytes(ctypes.byref(mx), kid)


def entries():
    """Returns how many calls reported success (must stay 0 without a GPU)."""
    ok = 0
    a = q.Kargs(p(), p(), p(), v(), v(), v(), rng.choice([0, 1, 2, -1, 64]), v(), v(), v(), lv(), lv(), lv(), p(),
                p(), v(), v(), lv(), lv())
    lb = q.LdsBypassKargs(p(), p(), p(), p(), v(), v(), v(), rng.choice([0, 1, 64, -3]), v(), v(), v(), lv(), lv(),
                          lv(), p(), p(), v(), v(), lv(), lv(), lv())
    m4 = q.Mxfp4Kargs(*[getattr(a, f) for f, _ in q.Kargs._fields_], rng.choice([0, 1, 37, 256, -5]))
    ws, wsb = rng.choice([None, 0x2000, 0x2001]), rng.choice([0, 255, 2048, 1 << 30])
    calls = [L.gemm_a8w8_mxfp8(ctypes.byref(a), rng.choice([0, 1, 2]), ws, wsb, None),
             L.gemm_a4w4_mxfp4(ctypes.byref(a), 1, ws, wsb, None),
             L.gemm_a8w8_blockscale_bpreshuffle(ctypes.byref(a), 1, ws, wsb, None),
             L.gemm_a8w8_mxfp8_kid(ctypes.byref(a), 1, rng.randint(-2, 9), ws, wsb, None),
             L.gemm_a4w4_mxfp4_kid(ctypes.byref(a), 1, rng.randint(-2, 9), ws, wsb, None),
             L.gemm_a8w8_blockscale_bpreshuffle_kid(ctypes.byref(a), 1, rng.randint(-2, 9), ws, wsb, None),
             L.launch_blockscale_bpreshuffle(ctypes.byref(a), rng.choice([0, 1]), rng.randint(-1, 2), None),
             L.gemm_a8w8_blockscale_layout(ctypes.byref(a), rng.randint(-1, 5), 1, ws, wsb, None),
             L.gemm_a4w4_mxfp4_noalloc(ctypes.byref(a), 1, None),
             L.gemm_a4w4_mxfp4_bpreshuffle(ctypes.byref(m4), 1, None),
             L.gemm_a8w8_blockscale_ldsbypass(ctypes.byref(lb), 1, ws, wsb, None),
             L.gemm_a8w8_blockscale_ldsbypass_kid(ctypes.byref(lb), 1, rng.randint(-2, 9), ws, wsb, None),
             L.gemm_a8w8_blockscale_ldsbypass_repack(ctypes.byref(lb), None)]
    for f in ("qgemm_quant_fp8_blockscale_act", "qgemm_quant_fp8_e8m0_act", "qgemm_quant_mxfp8", "qgemm_quant_mxfp4"):
        calls.append(getattr(L, f)(p(), rng.randint(-1, 3), v(), v(), v(), p(), v(), p(), v(), rng.randint(-1, 2),
                                   None))
    for f in ("qgemm_quant_fp8_blockscale_wgt", "qgemm_quant_fp8_e8m0_wgt"):
        calls.append(getattr(L, f)(p(), rng.randint(-1, 3), v(), v(), v(), p(), v(), p(), v(), None))
    for f in ("qgemm_shuffle_b_kpanel_device", "qgemm_shuffle_weight_16x16_device", "qgemm_pack_b_ldsbypass_device",
              "qgemm_e8m0_shuffle_device"):
        calls.append(getattr(L, f)(p(), p(), v(), v(), v(), None))
    return sum(1 for st in calls if st == 0)


def host_layouts():
    P = lambda x: x.ctypes.data_as(ctypes.c_void_p)
    n = rng.choice([1, 15, 16, 17, 300, rng.randint(1, 700)])
    kb = rng.choice([0, 64, 127, 128, 384, rng.randint(0, 1200)])
    src = np.random.randint(0, 256, size=max(1, n * kb), dtype=np.uint8)
    dst = np.zeros(max(1, n * kb), dtype=np.uint8)
    L.qgemm_shuffle_b_kpanel(P(src), P(dst), n, kb)
    L.qgemm_shuffle_weight_16x16(P(src), P(dst), n, kb)
    k = rng.choice([0, 128, 384, 7168, rng.randint(0, 2000)])
    need = L.qgemm_ldsbypass_b_bytes(n, k)
    if 0 < need < (1 << 28):
        b = np.random.randint(0, 256, size=max(1, n * k), dtype=np.uint8)
        L.qgemm_pack_b_ldsbypass(P(b), P(np.zeros(need, dtype=np.uint8)), n, k)
    rows, gk = rng.randint(0, 300), rng.randint(0, 300)
    need = L.qgemm_e8m0_shuffle_bytes(rows, gk)
    if 0 < need < (1 << 28):
        s = np.random.randint(0, 256, size=max(1, rows * gk), dtype=np.uint8)
        L.qgemm_e8m0_shuffle(P(s), P(np.zeros(need, dtype=np.uint8)), rows, gk)


succeeded = 0
for i in range(ITERS):
    queries()
    succeeded += entries()
    if i % 10 == 0:
        host_layouts()
assert succeeded == 0, f"{succeeded} calls reported success without a GPU"
print(f"fuzz ok: {ITERS} iterations")
