"""Packages on the GPU.

- The committed reference-layout package (`tests/golden/refpack_small.npz`: the reference's meta keys,
  `eng_stem`, `cubin`, its full table set, fp16 input) runs through `load_pack` -> `Dense8SEncoder`
  unchanged: every launch exact against the C oracle on its own inputs, the final features exact, the
  stem within 1 LSB, and the same tables with uint8 input give the same bytes (graphs too).
- A DenseNet169 checkpoint in the `KneeBaseline` layout goes through the weights-only loader,
  calibration, plan, save and reload, and the reloaded package passes the reference's gate against
  the float32 forward (kaggle/int8_pack/pack_dense8s.py:1242-1257) and equals the in-memory package.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import checks
from rsna_knee_efficiency_amd import checkpoint, dense8s, densenet, synthetic

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_reference_layout_package_runs(dev):
    pk = dense8s.load_pack(GOLDEN / "refpack_small.npz")
    enc = dense8s.Dense8SEncoder(pk, dev.index or 0, 2)
    assert enc.in_dtype == torch.float16 and enc.nb == 2
    x = np.random.default_rng(23).integers(0, 256, (2, 3, 32, 32), dtype=np.uint8)
    lut = torch.from_numpy(dense8s.input_lut([0.0] * 3, [1.0] * 3).view(np.float16).copy()).to(dev)
    xd = torch.from_numpy(x).to(dev)
    x16 = lut[torch.arange(3, device=dev).view(1, 3, 1, 1), xd.long()].contiguous()   # u / 255 fp16
    trace, f = enc.trace(x16)
    feats = f.cpu().numpy()
    res = checks.summarize(checks.check_trace(enc, trace, feats, pk["par"], max_rows=None))
    print(res)
    for fam in ("conv1", "conv2", "dense", "block", "trans"):
        assert res[fam]["mismatch"] == 0, (fam, res[fam])
    assert sum(res[f]["launches"] for f in ("conv1", "dense", "block")) == 4 and res["trans"]["launches"] == 1
    assert res["final"]["equal"], res["final"]
    got0 = trace[(0, 0)].cpu().numpy().astype(np.int8)
    want0 = checks.stem_reference(x16.cpu().numpy(), 0, None, False, pk["par"]["S_w16"],
                                  pk["par"]["S_bias"], pk["par"]["S_inv"])
    st = checks.bytes_cmp(got0, want0)
    assert st["max_diff"] <= 1 and st["mismatch_frac"] < 1e-3, st
    plain = enc(x16).clone()
    assert np.array_equal(plain.cpu().numpy(), feats)
    pk8 = dict(pk, meta=dict(pk["meta"], input={"kind": "u8", "mean": [0.0] * 3, "std": [1.0] * 3}))
    enc8 = dense8s.Dense8SEncoder(pk8, dev.index or 0, 2)
    assert torch.equal(enc8(xd), plain)
    enc.capture(2)
    for _ in range(2):
        got = enc(x16).clone()
        torch.cuda.synchronize(dev)
        assert torch.equal(got, plain)


def test_checkpoint_to_gated_package(dev, tmp_path):
    model = densenet.seeded_densenet169(5)
    sd = {f"encoder.{k}": v for k, v in model.state_dict().items()}
    sd["slot_emb"] = torch.zeros(8, 1664)
    torch.save({"cfg": {"cache": {"img": 512}, "model": {"arch": "densenet169"}}, "model": sd},
               tmp_path / "fold5.pt")
    cal = synthetic.study_u8(16, 512, seed=[7, 5])
    print("checkpoint -> package (DenseNet169, 512 px)", flush=True)
    res = checkpoint.build_pack(tmp_path / "fold5.pt", [torch.from_numpy(c) for c in np.split(cal, 2)],
                                8, device=dev, out=tmp_path / "pack.npz")
    pk = dense8s.load_pack(tmp_path / "pack.npz")
    x = torch.from_numpy(synthetic.study_u8(8, 512, seed=[1234, 9])).to(dev)
    g = checkpoint.gate(pk, res["model"], x, res["mean"], res["std"])
    print(g)
    assert g["ok"], g
    a = dense8s.Dense8SEncoder(pk, dev.index or 0, 8)(x).clone()
    b = dense8s.Dense8SEncoder(res["pack"], dev.index or 0, 8)(x).clone()
    assert torch.equal(a, b)
