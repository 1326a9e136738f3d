"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py): the oracle
must still reproduce them (CPU), and the HIP kernels must reproduce them bit for bit (GPU; the stem
within its 1-LSB tolerance)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import checks, lib

GOLDEN = Path(__file__).resolve().parent / "golden"


def fx(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_oracle_reproduces_fixtures():
    f = fx("prologue")
    assert np.array_equal(lib.prologue_lut(f["abh"]), f["lut"])
    f = fx("conv1")
    acc, byt = lib.conv1(f["in0"], f["seg"], int(f["G0"]), int(f["G"]), int(f["N"]), int(f["HW"]),
                         f["abh"], f["w1"], f["gd"], np.arange(len(f["acc"])))
    assert np.array_equal(acc, f["acc"]) and np.array_equal(byt, f["bott"])
    f = fx("conv2")
    acc, q = lib.conv2(f["bott"], int(f["N"]), int(f["H"]), int(f["W"]), f["w2k"], f["sc"],
                       np.arange(len(f["q"])))
    assert np.array_equal(acc, f["acc"]) and np.array_equal(q, f["q"])
    f = fx("trans")
    S, q = lib.trans(f["in0"], f["seg"], int(f["G0"]), int(f["G"]), int(f["N"]), int(f["HW"]),
                     int(f["W"]), f["abh"], f["w"], f["gdf"], int(f["cout"]), np.arange(len(f["q"])))
    assert np.array_equal(S, f["S"]) and np.array_equal(q, f["q"])
    f = fx("final")
    assert np.array_equal(lib.final(f["in0"], int(f["G0"]), f["seg"], int(f["N"]), int(f["HW"]),
                                    f["ab"], int(f["ctot"])), f["out"])
    f = fx("stem")
    sel = np.arange(len(f["out"]))
    w16 = f["w16"].view(np.float16)
    assert np.array_equal(lib.stem(f["x"], 1, f["lut"], False, w16, f["bias"], f["inv"], sel), f["out"])
    assert np.array_equal(lib.stem(f["x"], 1, f["lut"], True, w16, f["bias"], f["inv"], sel),
                          f["out_flip"])


@pytest.mark.gpu
def test_kernels_reproduce_fixtures(dev):
    from oracle import cases
    f = fx("conv1")
    c = cases.GemmCase(S=int(f["W"]), N=int(f["N"]), G0=int(f["G0"]), G=int(f["G"]), in0=f["in0"],
                       seg=f["seg"], q=None, abh=f["abh"], ab=None, w=None, w1=f["w1"], gd=f["gd"])
    acc, byt = checks.run_conv1(c, dev)
    assert np.array_equal(acc, f["acc"]) and np.array_equal(byt, f["bott"])
    f = fx("conv2")
    n, h, w = int(f["N"]), int(f["H"]), int(f["W"])
    v = f["bott"].reshape(4, n, h * w, 32).transpose(1, 0, 3, 2).reshape(n, 128, h, w)
    c2 = cases.Conv2Case(S=h, N=n, v=v, bott=f["bott"], w2=None, w2k=f["w2k"], sc=f["sc"])
    got, _ = checks.run_conv2(c2, dev)
    assert np.array_equal(got, f["q"])
    f = fx("trans")
    t = {"S": int(f["W"]), "N": int(f["N"]), "cout": int(f["cout"]), "in0": f["in0"], "seg": f["seg"],
         "w": f["w"], "abh": f["abh"], "gdf": f["gdf"], "G0": int(f["G0"]), "G": int(f["G"])}
    assert np.array_equal(checks.run_trans(t, dev), f["q"])
    f = fx("final")
    got = checks.run_final(f["in0"], int(f["G0"]), f["seg"], int(f["N"]), int(f["HW"]), f["ab"],
                           int(f["ctot"]), dev)
    assert np.array_equal(got, f["out"])
    f = fx("stem")
    w16 = f["w16"].view(np.float16)
    for flip, key in ((False, "out"), (True, "out_flip")):
        got = checks.run_stem(f["x"], 1, f["lut"], flip, w16, f["bias"], f["inv"], dev)
        got = got.transpose(0, 2, 3, 1).reshape(-1, 64)
        cmp_ = checks.bytes_cmp(got, f[key])
        assert cmp_["max_diff"] <= 1 and cmp_["mismatch_frac"] < 1e-2, cmp_
