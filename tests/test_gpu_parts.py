"""Whole dense blocks split into row bands across workgroups (`d8s_dense_block_parts`, block kind
"parts") on the GPU: every band count of the 32 x 32 and 16 x 16 blocks of the configuration-4 encoder
gives the bytes of the default encoder (two launches per layer / one workgroup per image), exact
against the C oracle on sampled pixels of its own inputs, under graph replay too (the kernel clears its
own synchronisation words for the next launch), with no bounded wait running out.  Two such runners on
two streams at once stay exact.  The 64- and 128-wide blocks split into bands give the same bytes too,
and an error word planted from the host makes the pass's features NaN and the next call raise."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import checks
from rsna_knee_efficiency_amd import dense8s, densenet, synthetic

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def c4(dev):
    model = densenet.seeded_densenet169(0).to(dev)
    cal = dense8s.calibrate(model, [synthetic.normalise(torch.from_numpy(c).to(dev))
                                    for c in np.split(synthetic.study_u8(64, 512, seed=7), 8)])
    plan = dense8s.make_plan(model.cpu(), cal, 512)
    pack = dense8s.make_pack(plan, 24, input_kind="u8")
    x = torch.from_numpy(synthetic.c5_study(0)[:24]).to(dev)
    base = dense8s.Dense8SEncoder(pack, dev.index or 0, 24, fused={0: "tile"})
    return {"plan": plan, "pack": pack, "x": x, "want": base(x).clone()}


def test_parts_options():
    meta = dense8s.pack_meta(dense8s.make_plan(densenet.seeded_densenet169(0), _fake_cal(), 512), 24)
    b = meta["blocks"]
    assert dense8s.parts_options(b[3]) == [1, 2, 4, 8]
    assert dense8s.parts_options(b[2]) == [4, 8, 16, 32]
    assert dense8s.parts_for(b[3], 24) == 8 and dense8s.parts_for(b[3], 96) == 2
    assert dense8s.parts_for(b[2], 24) == 8 and dense8s.parts_for(b[2], 96) is None


def _fake_cal():
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
    import make_tables
    return make_tables.fake_cal()


@pytest.mark.parametrize("kinds", [{2: "parts:8", 3: "parts:8"}, {2: "parts:4", 3: "parts:4"},
                                   {2: "parts:16", 3: "parts:2"}, {2: "parts:32", 3: "parts:1"}])
def test_parts_same_bytes(dev, c4, kinds):
    print(f"parts {kinds}", flush=True)
    enc = dense8s.Dense8SEncoder(c4["pack"], dev.index or 0, 24, fused={0: "tile", **kinds})
    got = enc(c4["x"]).clone()
    assert enc.sync_errors() == 0
    assert torch.equal(got, c4["want"])
    enc.capture(24)
    for _ in range(3):
        g = enc(c4["x"]).clone()
        _ = (c4["x"].float() * 2).sum()
        torch.cuda.synchronize(dev)
        assert torch.equal(g, c4["want"])
    assert enc.sync_errors() == 0


def test_parts_layers_exact(dev, c4):
    """The default band counts at 24 images traced: every layer of the banded blocks exact."""
    enc = dense8s.Dense8SEncoder(c4["pack"], dev.index or 0, 24, fused={0: "tile", 2: "parts", 3: "parts"})
    assert enc.fused[2] == "parts:8" and enc.fused[3] == "parts:8"
    trace, f = enc.trace(c4["x"])
    assert enc.sync_errors() == 0
    par = dense8s.kernel_params(c4["plan"])
    res = checks.summarize(checks.check_trace(enc, trace, f.cpu().numpy(), par, max_rows=1024))
    print(res)
    assert res["block"]["launches"] == 64 and res["block"]["mismatch"] == 0, res["block"]
    assert res["conv1"]["mismatch"] == 0 and res["trans"]["mismatch"] == 0
    assert res["final"]["equal"]


def test_parts_two_runners_at_once(dev, c4):
    encs = [dense8s.Dense8SEncoder(c4["pack"], dev.index or 0, 24, fused={0: "tile", 2: "parts", 3: "parts"})
            for _ in range(2)]
    xs = [c4["x"], torch.flip(c4["x"], dims=[0]).contiguous()]
    want = [c4["want"], None]
    base = dense8s.Dense8SEncoder(c4["pack"], dev.index or 0, 24, fused={0: "tile"})
    want[1] = base(xs[1]).clone()
    for e in encs:
        e.capture(24)
    for k in range(3):
        outs = dense8s.encode_concurrent([(encs[0], xs[0], False), (encs[1], xs[1], False)])
        got = [o.clone() for o in outs]
        torch.cuda.synchronize(dev)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1]), k
    assert sum(e.sync_errors() for e in encs) == 0


@pytest.fixture(scope="module")
def small_first(dev):
    """A seeded DenseNet with 4 layers in its first block at 128 px: that block is 32 x 32 with 2
    groups in (below every prologue chunk of the banded kernel)."""
    model = densenet.seeded_densenet169(5, blocks=(4, 1, 2, 2)).to(dev)
    x_u8 = synthetic.study_u8(8, 128, seed=3)
    cal = dense8s.calibrate(model, [synthetic.normalise(torch.from_numpy(x_u8).to(dev))])
    pack = dense8s.make_pack(dense8s.make_plan(model.cpu(), cal, 128), 8, input_kind="u8")
    assert pack["meta"]["blocks"][0]["c0"] // 32 == 2 and pack["meta"]["blocks"][0]["L"] == 4
    x = torch.from_numpy(x_u8).to(dev)
    kinds = dense8s.fused_blocks(pack["meta"], None)
    kinds[0] = "conv"
    want = dense8s.Dense8SEncoder(pack, dev.index or 0, 8, fused=kinds)(x).clone()
    return {"pack": pack, "x": x, "kinds": kinds, "want": want}


@pytest.mark.parametrize("parts", [4, 8, 16, 32])
def test_parts_groups_below_first_chunk(dev, small_first, parts):
    """Layers whose second-newest group falls in the first prologue chunk (it is stored by the conv2
    that runs after the chunk was requested, and comes from conv2's copy in LDS): every band size
    (256, 128, 64 and 32 pixels) gives the bytes of two launches per layer."""
    print(f"small first block, parts:{parts}", flush=True)
    kinds = dict(small_first["kinds"])
    kinds[0] = f"parts:{parts}"
    enc = dense8s.Dense8SEncoder(small_first["pack"], dev.index or 0, 8, fused=kinds)
    got = enc(small_first["x"]).clone()
    assert enc.sync_errors() == 0
    assert torch.equal(got, small_first["want"])


@pytest.mark.parametrize("kinds", [{1: "parts:16"}, {1: "parts:32"}, {1: "parts:64"}, {0: "parts:128"}])
def test_parts_wide_maps(dev, c4, kinds):
    """The 64 x 64 block (12 layers) in 256-, 128- and 64-pixel bands and the 128 x 128 block (6 layers)
    in one-row bands: more bands than compute units (384 to 3072 workgroups), so images start as
    earlier ones finish; the bytes of the default encoder."""
    print(f"wide parts {kinds}", flush=True)
    enc = dense8s.Dense8SEncoder(c4["pack"], dev.index or 0, 24, fused={0: "tile", **kinds})
    got = enc(c4["x"]).clone()
    assert enc.sync_errors() == 0
    assert torch.equal(got, c4["want"])


def test_parts_wait_error_surfaces(dev, c4):
    """A non-zero error word (planted by the host, as an expired wait would leave it) makes the pass's
    features NaN, reaches the host-mapped report, and makes the next call raise PartsWaitError, which
    clears it: the call after that is exact again.  The same under graph replay."""
    enc = dense8s.Dense8SEncoder(c4["pack"], dev.index or 0, 24, fused={0: "tile", 2: "parts", 3: "parts"})
    assert enc._checked and enc._report is not None
    for graphs in (False, True):
        if graphs:
            enc.capture(24)
        assert torch.equal(enc(c4["x"]).clone(), c4["want"])
        torch.cuda.synchronize(dev)
        enc._sync[2].fill_(3)
        bad = enc(c4["x"]).clone()
        torch.cuda.synchronize(dev)
        assert torch.isnan(bad).all(), graphs
        assert int(enc._report[0]) == 3, graphs
        with pytest.raises(dense8s.PartsWaitError):
            enc(c4["x"])
        assert int(enc._report[0]) == 0 and enc.sync_errors(clear=False) == 0
        assert torch.equal(enc(c4["x"]).clone(), c4["want"]), graphs
    assert enc.calls["graph"] >= 2
