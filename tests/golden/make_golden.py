"""Writes the golden fixtures of tests/golden/ (run from the repository root):

    python tests/golden/make_golden.py

The reference ships no golden vectors for this path (its checks recompute formulas on CUDA-seeded
random data, kaggle/int8_pack/pack_dense8s.py:216-447), so these are the oracle's outputs on small
seeded inputs, pinned by tests/test_oracle.py and frozen here: tests/test_golden.py checks that the
oracle still reproduces them (CPU) and that the HIP kernels reproduce them bit for bit (GPU).
Every file is a plain .npz of numeric arrays (no pickles).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()
from oracle import cases, lib  # noqa: E402
from rsna_knee_efficiency_amd import dense8s  # noqa: E402


def conv1_fixture() -> dict:
    c = cases.gemm_case(4, 96, N=2, seed=101)
    in0, seg = cases.store_from_q(c.q, 1)
    acc, byt = lib.conv1(in0, seg, 1, 3, 2, 16, c.abh, c.w1, c.gd, np.arange(32))
    return {"in0": in0, "seg": seg, "abh": c.abh, "w1": c.w1, "gd": c.gd, "G0": 1, "G": 3, "N": 2,
            "HW": 16, "W": 4, "acc": acc, "bott": byt}


def conv2_fixture() -> dict:
    c = cases.conv2_case(6, N=2, seed=102, W=5)
    acc, q = lib.conv2(c.bott, 2, 6, 5, c.w2k, c.sc, np.arange(60))
    return {"bott": c.bott, "w2k": c.w2k, "sc": c.sc, "N": 2, "H": 6, "W": 5, "acc": acc, "q": q}


def trans_fixture() -> dict:
    t = cases.trans_case(8, 128, N=2, c0=64, seed=103)
    S, q = lib.trans(t["in0"], t["seg"], t["G0"], t["G"], 2, 64, 8, t["abh"], t["w"], t["gdf"],
                     t["cout"], np.arange(32))
    return {"in0": t["in0"], "seg": t["seg"], "abh": t["abh"], "w": t["w"], "gdf": t["gdf"],
            "G0": t["G0"], "G": t["G"], "N": 2, "HW": 64, "W": 8, "cout": t["cout"], "S": S, "q": q}


def final_fixture() -> dict:
    rng = np.random.default_rng(104)
    q = rng.integers(-127, 128, (2, 96, 9)).astype(np.int8)
    in0, seg = cases.store_from_q(q, 1)
    ab = np.stack([rng.uniform(0.001, 0.05, 96), rng.normal(0, 0.3, 96)], 1).astype(np.float32)
    return {"in0": in0, "seg": seg, "ab": ab, "G0": 1, "N": 2, "HW": 9, "ctot": 96,
            "out": lib.final(in0, 1, seg, 2, 9, ab, 96)}


def stem_fixture() -> dict:
    rng = np.random.default_rng(105)
    w = rng.normal(0, np.sqrt(2 / 147), (64, 3, 7, 7)).astype(np.float32)
    w16 = dense8s.stem_weights16(w)
    bias = rng.normal(0, 0.1, 64).astype(np.float32)
    inv = (1.0 / rng.uniform(0.02, 0.05, 64)).astype(np.float32)
    lut = dense8s.input_lut([0.5] * 3, [0.25] * 3)
    x = rng.integers(0, 256, (2, 3, 20, 24)).astype(np.uint8)
    sel = np.arange(2 * 5 * 6)
    return {"x": x, "w16": w16.view(np.int16), "bias": bias, "inv": inv, "lut": lut,
            "out": lib.stem(x, 1, lut, False, w16, bias, inv, sel),
            "out_flip": lib.stem(x, 1, lut, True, w16, bias, inv, sel)}


def prologue_fixture() -> dict:
    rng = np.random.default_rng(106)
    ab = np.stack([rng.normal(0, 0.01, 64), rng.normal(0.2, 0.4, 64)], 1).astype(np.float32)
    abh = cases.abh_table(ab)
    return {"abh": abh, "lut": lib.prologue_lut(abh)}


FIXTURES = {"prologue": prologue_fixture, "conv1": conv1_fixture, "conv2": conv2_fixture,
            "trans": trans_fixture, "final": final_fixture, "stem": stem_fixture}


def main() -> None:
    for name, fn in FIXTURES.items():
        arrays = {k: np.asarray(v) for k, v in fn().items()}
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print(name, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main()
