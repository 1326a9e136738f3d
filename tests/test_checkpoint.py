"""Packages from trained weights (CPU): a KneeBaseline-layout checkpoint on disk -> weights-only load ->
the DenseNet of its `encoder.features.*` -> calibrate -> plan -> package, with the same tables as the
direct path from the module; the loader refuses files holding objects; the committed reference-layout
package (`tests/golden/refpack_small.npz`, written by make_refpack.py) loads with every table the
runner needs and holds the tables this build's checkpoint path computes."""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from rsna_knee_efficiency_amd import checkpoint, dense8s, densenet

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import make_refpack as mr  # noqa: E402


class NotAWeight:
    """An object a weights-only load must refuse."""


def _direct_tables(model, cal_u8, img, mean=(0.0,) * 3, std=(1.0,) * 3) -> dict:
    cal = dense8s.calibrate(model, [checkpoint.normalised(torch.from_numpy(cal_u8), mean, std)])
    return dense8s.pack_params(dense8s.make_plan(model, cal, img))


def _same_tables(a: dict, b: dict) -> None:
    assert set(a) == set(b)
    for k in a:
        assert a[k].dtype == b[k].dtype and np.array_equal(a[k].view(np.uint8), b[k].view(np.uint8)), k


def test_pack_from_checkpoint_file(tmp_path):
    ck = mr.knee_state()
    torch.save(ck, tmp_path / "fold0.pt")
    res = checkpoint.build_pack(tmp_path / "fold0.pt", [torch.from_numpy(mr.cal_windows())], 2,
                                out=tmp_path / "pack.npz")
    assert res["plan"].img == mr.IMG                               # from cfg["cache"]["img"]
    model = densenet.seeded_densenet169(3, blocks=mr.BLOCKS)
    _same_tables(res["pack"]["par"], _direct_tables(model, mr.cal_windows(), mr.IMG))
    pk = dense8s.load_pack(tmp_path / "pack.npz")
    dense8s.validate_meta(pk["meta"])
    assert pk["meta"]["input"] == {"kind": "u8", "mean": [0.0] * 3, "std": [1.0] * 3}
    _same_tables(pk["par"], res["pack"]["par"])


def test_loader_forms_and_errors(tmp_path):
    ck = mr.knee_state()
    model = densenet.seeded_densenet169(3, blocks=mr.BLOCKS)
    # a compiled model's prefix, a bare state dict of the DenseNet itself
    wrapped = {"cfg": ck["cfg"], "model": {f"_orig_mod.{k}": v for k, v in ck["model"].items()}}
    torch.save(wrapped, tmp_path / "a.pt")
    torch.save(model.state_dict(), tmp_path / "b.pt")
    for name in ("a.pt", "b.pt"):
        m = checkpoint.encoder_from_state(checkpoint.load_checkpoint(tmp_path / name)["model"])
        for k, v in model.state_dict().items():
            assert torch.equal(m.state_dict()[k], v), (name, k)
    # objects in the file: refused by the weights-only loader, nothing executed
    torch.save({"cfg": {"x": NotAWeight()}, "model": ck["model"]}, tmp_path / "c.pt")
    with pytest.raises(Exception, match="[Ww]eights.only"):
        checkpoint.load_checkpoint(tmp_path / "c.pt")
    # a missing encoder weight, no encoder at all
    sd = dict(ck["model"])
    del sd["encoder.features.denseblock2.denselayer1.conv2.weight"]
    with pytest.raises(RuntimeError):
        checkpoint.encoder_from_state(sd)
    with pytest.raises(ValueError):
        checkpoint.encoder_from_state({"slot_emb": torch.zeros(8, 4)})
    assert mr.BLOCKS == checkpoint.block_config(checkpoint.encoder_state(ck["model"]))


def test_input_norm_from_cfg():
    assert checkpoint.input_norm({}) == ((0.0,) * 3, (1.0,) * 3)
    mean, std = checkpoint.input_norm({"model": {"input_norm": "imagenet"}})
    assert mean == checkpoint.IMAGENET_MEAN and std == checkpoint.IMAGENET_STD
    ck = mr.knee_state()
    ck["cfg"]["model"]["input_norm"] = "imagenet"
    res = checkpoint.build_pack(ck, [torch.from_numpy(mr.cal_windows())], 2)
    assert res["pack"]["meta"]["input"]["mean"] == list(mean)
    model = densenet.seeded_densenet169(3, blocks=mr.BLOCKS)
    _same_tables(res["pack"]["par"], _direct_tables(model, mr.cal_windows(), mr.IMG, mean, std))
    with pytest.raises(ValueError):
        checkpoint.input_norm({"model": {"input_norm": "other"}})


def test_cli_writes_a_package(tmp_path, capsys):
    torch.save(mr.knee_state(), tmp_path / "fold0.pt")
    np.save(tmp_path / "cal.npy", mr.cal_windows())
    if torch.cuda.is_available():
        pytest.skip("the CPU path of the command")
    checkpoint.main([str(tmp_path / "fold0.pt"), "--cal", str(tmp_path / "cal.npy"), "--n", "2",
                     "--out", str(tmp_path / "p.npz"), "--batch", "2"])
    rep = json.loads(capsys.readouterr().out.strip().splitlines()[-1])
    assert rep["img"] == mr.IMG and rep["n"] == 2
    dense8s.validate_meta(dense8s.load_pack(tmp_path / "p.npz")["meta"])


def test_reference_layout_fixture_loads():
    pk = dense8s.load_pack(GOLDEN / "refpack_small.npz")
    meta = pk["meta"]
    dense8s.validate_meta(meta)
    for key in ("format", "kind", "n", "img", "in_ch", "kernels_sha", "n_features", "stem_c",
                "conv2_int8", "stem_int8", "conv2", "stem", "blocks", "engines"):
        assert key in meta, key
    assert "input" not in meta                                    # fp16 windows, as the reference
    assert set(pk["engines"]) == {"stem"} and pk["cubin"] is not None
    assert all({"bm", "c2", "tbm", "fused"} <= set(b) for b in meta["blocks"])
    missing = [k for k in dense8s.needed_tables(meta) if k not in pk["par"]]
    assert not missing
    extra = set(pk["par"]) - set(dense8s.needed_tables(meta))
    assert {"T0_wh", "S_w8", "S_w8f", "S_kc", "S_w0", "S_b0"} <= extra
    # the fixture's tables are what this build's checkpoint path computes
    res = checkpoint.build_pack(mr.knee_state(), [torch.from_numpy(mr.cal_windows())], mr.NB, mr.IMG)
    par = dense8s.kernel_params(res["plan"])
    for k, v in par.items():
        assert np.array_equal(pk["par"][k].view(np.uint8), v.view(np.uint8)), k
