"""The host-side calibration, plan and tables against frozen fixtures and closed forms (CPU only).

- `tests/golden/tables_small.npz` / `tables_169.json` (written by tests/golden/make_tables.py): every
  table of `kernel_params` is bit-identical to the frozen one (full arrays for the float / fp16 tables
  of a small seeded DenseNet, SHA-256 of its int8 weights and of every table of DenseNet169), and
  `calibrate` gives the frozen maxima;
- closed form of `calibrate`: each maximum equals max|t| (per channel or per tensor) of the matching
  intermediate of the independent functional forward `oracle/fp32.py`: a maximum taken without the
  absolute value, or on the wrong tensor (before a ReLU, after a pooling), fails it;
- the plan's sign fold, weight and activation scales against their definitions.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import fp32
from rsna_knee_efficiency_amd import dense8s, densenet

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import make_tables as mt  # noqa: E402


@pytest.fixture(scope="module")
def small():
    with np.load(GOLDEN / "tables_small.npz", allow_pickle=False) as z:
        data = {k: np.array(z[k]) for k in z.files}
    return {"cal": json.loads(bytes(data.pop("cal")).decode()),
            "ints": json.loads(bytes(data.pop("int8_digests")).decode()),
            "par": {k[4:]: v for k, v in data.items()}}


def test_small_tables_are_the_frozen_ones(small):
    par = dense8s.kernel_params(dense8s.make_plan(mt.small_model(), small["cal"], 64))
    assert set(par) == set(small["par"]) | set(small["ints"])
    for k, v in par.items():
        if k in small["ints"]:
            assert mt.digest(v) == small["ints"][k], k
        else:
            want = small["par"][k]
            assert v.dtype == want.dtype and v.shape == want.shape, k
            assert np.array_equal(v.view(np.uint8), want.view(np.uint8)), k


def test_calibrate_gives_the_frozen_maxima(small):
    cal = dense8s.calibrate(mt.small_model(), [mt.small_inputs()])
    assert cal.keys() == small["cal"].keys()
    for k, v in small["cal"].items():
        assert cal[k] == v, k


def test_densenet169_table_digests():
    want = json.loads((GOLDEN / "tables_169.json").read_text())
    par = dense8s.kernel_params(dense8s.make_plan(densenet.seeded_densenet169(0), mt.fake_cal(), 512))
    assert set(par) == set(want)
    bad = [k for k, v in par.items() if mt.digest(v) != want[k]]
    assert not bad, bad[:8]


def test_calibrate_is_the_maxima_of_the_intermediates():
    """Two batches; every maximum against max|t| of the functional forward's intermediates."""
    model = mt.small_model()
    rng = np.random.default_rng(9)
    batches = [torch.from_numpy(rng.normal(0, 1, (2, 3, 64, 64)).astype(np.float32)) for _ in range(2)]
    cal = dense8s.calibrate(model, batches)
    chan: dict = {}
    tens: dict = {}

    def tap(name, t):
        kind, rest = name.split(".", 1) if "." in name else (name, "")
        per_ch = t.abs().amax(dim=(0, 2, 3)).double().numpy()
        per_t = float(t.abs().max())
        key = {"pool0": lambda: ("c", "seg0.0"), "conv2": lambda: ("c", f"conv2.{rest}"),
               "tpool": lambda: ("c", f"seg0.{int(rest) + 1}"),
               "relu1": lambda: ("t", f"in1.{rest}"), "relu2": lambda: ("t", f"in2.{rest}"),
               "trelu": lambda: ("t", f"tin.{rest}")}[kind]()
        if key[0] == "c":
            chan[key[1]] = np.maximum(chan.get(key[1], per_ch), per_ch)
        else:
            tens[key[1]] = max(tens.get(key[1], 0.0), per_t)

    sd = model.state_dict()
    for x in batches:
        fp32.forward(sd, x, tap=tap)
    assert set(cal) == set(chan) | set(tens)
    for k, v in chan.items():
        np.testing.assert_allclose(np.asarray(cal[k]), v, rtol=1e-6, atol=0, err_msg=k)
    for k, v in tens.items():
        assert cal[k] == pytest.approx(v, rel=1e-6), k
    # the closed form tells the right tensors apart: conv2 outputs and transition-pool outputs have
    # negative values, so a maximum without the absolute value would differ
    assert any(np.any(np.asarray(cal[k]) > 0) for k in chan)


def test_plan_definitions():
    """Sign fold, scales and the dead-channel rule, from the definitions: w1 rows carry sign(a2),
    w1s = (max|w| / 127) |a2| per output channel (the weight scale alone where |a2| < 1e-30, whose
    rows are zero), s1 = max(in1, 1e-12) / 255, s2 = max(in2, 1e-12) / 127, sigma = max(amax, 1e-6)
    / 127."""
    model = mt.small_model()
    layer = model.features.denseblock2.denselayer2
    with torch.no_grad():
        layer.norm2.weight[5] = -layer.norm2.weight[5]          # a negative gamma: sign folded
        layer.norm2.weight[9] = 0.0                             # a dead channel
    cal = mt.fake_cal(mt.SMALL_BLOCKS, seed=3)
    cal["conv2.1.1"][4] = 1e-9                                  # floored scale
    plan = dense8s.make_plan(model, cal, 64)
    L = plan.blocks[1].layers[1]
    bn2 = layer.norm2
    a2 = (bn2.weight.detach().double() / torch.sqrt(bn2.running_var.double() + bn2.eps)).numpy()
    w = layer.conv1.weight.detach().float().reshape(128, -1)
    ws = (w.abs().amax(1).clamp_min(1e-12) / 127).numpy()
    q = torch.round(w * (1.0 / torch.from_numpy(ws)).view(-1, 1)).clamp(-128, 127).numpy()
    assert L.c_in == plan.blocks[1].c0 + 32
    assert np.array_equal(L.w1[5], -q[5]) and np.array_equal(L.w1[6], q[6])
    assert not L.w1[9].any() and L.w1s[9] == pytest.approx(float(ws[9]), rel=1e-7)
    np.testing.assert_allclose(L.w1s[[5, 6]], ws[[5, 6]] * np.abs(a2[[5, 6]]), rtol=1e-7)
    assert L.s1 == max(cal["in1.1.1"], 1e-12) / 255 and L.s2 == max(cal["in2.1.1"], 1e-12) / 127
    assert L.sig[4] == 1e-6 / 127 and L.sig[0] == cal["conv2.1.1"][0] / 127
    b2 = bn2.bias.detach().double() - bn2.running_mean.double() * torch.from_numpy(a2)
    assert np.array_equal(L.bias1, b2.numpy())
