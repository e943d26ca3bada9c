"""The committed tuned kernel tables (355_1_trans_amd/configs/*tuned*.csv):
schema of the reference's tuner, one winner per traced dsv4 shape, and the
lookup that gemm_a8w8_bpreshuffle_opus runs when no kernelId is given."""
import csv
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent.parent
CONFIGS = ROOT / "355_1_trans_amd" / "configs"
SCHEMA = ["gfx", "cu_num", "M", "N", "K", "bias", "dtype", "outdtype", "scaleAB", "bpreshuffle", "libtype",
          "solidx", "splitK", "us", "kernelName", "err_ratio", "tflops", "bw"]


def _rows(name):
    with open(CONFIGS / name, newline="") as fh:
        r = csv.DictReader(fh)
        assert r.fieldnames == SCHEMA
        return list(r)


def test_tables_cover_the_traced_shapes():
    with open(CONFIGS / "dsv4_a8w8_shapes.csv", newline="") as fh:
        shapes = {(int(r["M"]), int(r["N"]), int(r["K"])) for r in csv.DictReader(fh)}
    assert len(shapes) == 125
    for name, pre in (("qgemm_a8w8_bpreshuffle_tuned.csv", "True"), ("qgemm_a8w8_ldsbypass_tuned.csv", "False")):
        rows = _rows(name)
        assert {(int(r["M"]), int(r["N"]), int(r["K"])) for r in rows} == shapes
        for r in rows:
            assert r["libtype"] == "qgemm" and r["bpreshuffle"] == pre and float(r["err_ratio"]) == 0.0
            assert 0 <= int(r["solidx"]) <= 5 and float(r["us"]) > 0


def test_lookup_returns_the_table_winner(qgemm):
    rows = _rows("qgemm_a8w8_bpreshuffle_tuned.csv")
    for r in rows[:: max(1, len(rows) // 10)]:
        kid = qgemm.opus.lookup_tuned(int(r["cu_num"]), int(r["M"]), int(r["N"]), int(r["K"]), torch.bfloat16)
        assert kid == int(r["solidx"])
    assert qgemm.opus.lookup_tuned(int(rows[0]["cu_num"]), 7, 7, 128, torch.bfloat16) is None
    assert qgemm.opus.lookup_tuned(1, int(rows[0]["M"]), int(rows[0]["N"]), int(rows[0]["K"]), torch.bfloat16) is None


def test_tuner_mx_reference_dequant():
    """The MX tuner's float32 reference decodes codes and E8M0 scales as the
    oracle does (fp4: element 2i in the low nibble of byte i)."""
    import importlib

    import numpy as np

    import oracle as O
    tune = importlib.import_module("355_1_trans_amd.tune")
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 256, (3, 64), dtype=np.uint8)
    e = rng.integers(120, 135, (3, 4), dtype=np.uint8)
    got = tune._dequant_mx(torch.from_numpy(codes), torch.from_numpy(e), True).numpy()
    elems = np.stack((codes & 15, codes >> 4), axis=-1).reshape(3, 128)
    want = O.e2m1_decode(elems) * np.repeat(O.e8m0_decode(e), 32, axis=1)
    assert np.array_equal(got, want)
    fp8 = rng.integers(0, 256, (2, 64), dtype=np.uint8)
    fp8[(fp8 & 0x7F) == 0x7F] = 0    # no NaN codes
    e2 = rng.integers(120, 135, (2, 2), dtype=np.uint8)
    got8 = tune._dequant_mx(torch.from_numpy(fp8), torch.from_numpy(e2), False).numpy()
    assert np.array_equal(got8, O.e4m3_decode(fp8) * np.repeat(O.e8m0_decode(e2), 32, axis=1))
    assert tune._grid("24576,32768:1536:32,64") == [(32, 24576, 1536), (64, 24576, 1536), (32, 32768, 1536),
                                                  (64, 32768, 1536)]
