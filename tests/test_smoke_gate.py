"""The smoke gate on the CPU: a whole pass computed by the C oracle alone (`checks.oracle_trace`) passes
`checks.check_trace` with no mismatch in any family, and a single byte planted in one layer's output,
or no checked layer at all, makes `checks.smoke_gate` fail.  The smoke network (2 layers per block at
64 x 64) runs every block as one whole-block launch (family "block"), with no conv1 / conv2 launch,
so the fused families are the ones that must be gated."""
from __future__ import annotations

import types

import numpy as np
import pytest
import torch

from oracle import checks
from rsna_knee_efficiency_amd import dense8s, densenet


@pytest.fixture(scope="module")
def small_pass():
    torch.manual_seed(0)
    model = densenet.seeded_densenet169(0, blocks=(2, 2, 2, 2))
    rng = np.random.default_rng(5)
    mean, std = 0.5, 0.25
    cal_u8 = rng.integers(0, 256, (4, 3, 64, 64), dtype=np.uint8)
    cal = dense8s.calibrate(model, [(torch.from_numpy(cal_u8).float() / 255 - mean) / std])
    plan = dense8s.make_plan(model, cal, 64)
    pack = dense8s.make_pack(plan, 2, input_kind="u8", mean=(mean,) * 3, std=(std,) * 3)
    par = dense8s.kernel_params(plan)
    x = rng.integers(0, 256, (2, 3, 64, 64), dtype=np.uint8)
    lut = dense8s.input_lut([mean] * 3, [std] * 3)
    stem_q = checks.stem_reference(x, 1, lut, False, par["S_w16"], par["S_bias"], par["S_inv"])
    trace, feats = checks.oracle_trace(pack["meta"], par, stem_q, 2)
    enc = types.SimpleNamespace(meta=pack["meta"], nb=2, fused=dense8s.fused_blocks(pack["meta"]))
    return {"enc": enc, "trace": trace, "feats": feats, "par": par}


def _res(p, trace) -> dict:
    res = checks.summarize(checks.check_trace(p["enc"], trace, p["feats"], p["par"], max_rows=None))
    res["stem"] = {"n": 1, "mismatch": 0, "mismatch_frac": 0.0, "max_diff": 0}
    res["call_vs_trace"] = True
    res["vs_emulate"] = {"max_abs": 0.0, "rel_l2": 0.0, "cos_min": 1.0}
    return res


def test_oracle_pass_is_clean(small_pass):
    res = _res(small_pass, small_pass["trace"])
    assert res["block"]["launches"] == 8 and res["block"]["mismatch"] == 0, res
    assert res["dense"]["launches"] == 0, res
    assert res["trans"]["launches"] == 3 and res["trans"]["mismatch"] == 0, res
    assert res["conv1"]["launches"] == 0 and res["final"]["equal"], res
    assert checks.smoke_gate(res)["ok"]


@pytest.mark.parametrize("key", [(0, 1), (1, 2), (3, 2)])
def test_planted_byte_fails_the_gate(small_pass, key):
    trace = dict(small_pass["trace"])
    t = trace[key].clone()
    t[1, 7, 1, 0] += 1                        # one byte of one fused layer's output, image 1
    trace[key] = t
    res = _res(small_pass, trace)
    assert res["block"]["mismatch"] >= 1, res
    with pytest.raises(AssertionError):
        checks.smoke_gate(res)


def test_planted_byte_in_a_fused_layer_fails_the_gate(small_pass):
    """The same pass read as per-layer fused launches ("dense" family)."""
    enc = types.SimpleNamespace(meta=small_pass["enc"].meta, nb=2, fused={})
    trace = dict(small_pass["trace"])
    t = trace[(2, 1)].clone()
    t[0, 31, 3, 3] -= 1
    trace[(2, 1)] = t
    p = dict(small_pass, enc=enc)
    res = _res(p, trace)
    assert res["dense"]["launches"] == 8 and res["dense"]["mismatch"] >= 1, res
    with pytest.raises(AssertionError):
        checks.smoke_gate(res)


def test_gate_needs_checked_launches(small_pass):
    res = _res(small_pass, small_pass["trace"])
    res["block"] = {"launches": 0, "mismatch": 0, "max_diff": 0}
    with pytest.raises(AssertionError):
        checks.smoke_gate(res)


def test_expired_band_wait_fails_the_gate(small_pass):
    res = _res(small_pass, small_pass["trace"])
    res["wait_errors"] = 2
    with pytest.raises(AssertionError):
        checks.smoke_gate(res)
