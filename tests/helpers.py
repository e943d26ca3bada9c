"""Shared test helpers: seeded problem generation through the CPU oracle and
the BASELINE tolerance check."""
import numpy as np
import torch

import oracle as O


def to_dev(x, dtype, device):
    t = torch.from_numpy(np.ascontiguousarray(x))
    if dtype in (torch.float8_e4m3fn,):
        return t.view(torch.uint8).to(device).view(dtype)
    return t.to(device)


def out_to_f32(y):
    y = y.detach().cpu()
    if y.dtype == torch.bfloat16:
        return y.float().numpy()
    return y.numpy().astype(np.float32)


def assert_close(ref, got, what=""):
    bad, ratio, idx = O.check_tolerance(ref, got)
    assert bad == 0, f"{what}: {bad} elements out of tolerance, worst ratio {ratio:.3f} at {idx} " \
                     f"(ref={ref.reshape(-1)[idx]}, got={got.reshape(-1)[idx]})"
    return ratio


def make_mx8(m, n, k, seed=0):
    a = O.randn((m, k), seed, 0)
    b = O.randn((n, k), seed, 1)
    qa, ea = O.quant_mx8(a)
    qb, eb = O.quant_mx8(b)
    return qa, qb, ea, eb


def make_mx4(m, n, k, seed=0):
    a = O.randn((m, k), seed, 0)
    b = O.randn((n, k), seed, 1)
    qa, ea = O.quant_mx4(a)
    qb, eb = O.quant_mx4(b)
    return qa, qb, ea, eb


def make_bs(m, n, k, seed=0):
    a = O.randn((m, k), seed, 0)
    b = O.randn((n, k), seed, 1)
    qa, sa = O.quant_bs_act(a)
    qb, sb = O.quant_bs_wgt(b)
    return qa, qb, sa, sb


def assert_close_all(ref, got, what=""):
    """Every element of two GPU tensors against the BASELINE tolerance,
    |got - ref| <= 2^-7 |ref| + 1e-3 rms(ref) (rms over all of ref), computed
    on the GPU; NaN or Inf in either counts as a violation."""
    ref, got = ref.float(), got.float()
    rms = float(torch.sqrt(torch.mean(ref.double() ** 2)))
    bound = ref.abs() * 2.0 ** -7 + 1e-3 * rms
    err = (got - ref).abs()
    ok = err <= bound
    bad = int((~ok).sum())
    ratio = float(torch.nan_to_num(err / bound, nan=float("inf")).max())
    if bad:
        idx = int(torch.nonzero(~ok.reshape(-1))[0])
        raise AssertionError(f"{what}: {bad} of {ref.numel()} elements out of tolerance, worst ratio {ratio:.3f}; "
                             f"first at flat index {idx} (ref={float(ref.reshape(-1)[idx])}, "
                             f"got={float(got.reshape(-1)[idx])})")
    return ratio
