"""Host logic of the encoder (CPU only): plan and table formats, the package round trip, validation
errors (the reference's ValueError paths, src/knee/dense8s.py:954-956,1121-1124,1259-1260,1279-1280)."""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from rsna_knee_efficiency_amd import dense8s, densenet, hip


def fake_cal(blocks=(6, 12, 32, 32), seed=0) -> dict:
    """Calibration maxima of the right keys and sizes (no forward pass needed)."""
    rng = np.random.default_rng(seed)
    cal: dict = {}
    c = 64
    for b, nl in enumerate(blocks):
        cal[f"seg0.{b}"] = list(rng.uniform(0.5, 3, c))
        for li in range(nl):
            cal[f"conv2.{b}.{li}"] = list(rng.uniform(0.5, 3, 32))
            cal[f"in1.{b}.{li}"] = float(rng.uniform(1, 5))
            cal[f"in2.{b}.{li}"] = float(rng.uniform(1, 5))
        c += 32 * nl
        if b < len(blocks) - 1:
            cal[f"tin.{b}"] = float(rng.uniform(1, 5))
            c //= 2
    return cal


@pytest.fixture(scope="module")
def plan169():
    m = densenet.seeded_densenet169(0)
    return m, dense8s.make_plan(m, fake_cal(), 512)


def test_plan_shapes(plan169):
    _, plan = plan169
    assert [len(b.layers) for b in plan.blocks] == [6, 12, 32, 32]
    assert [b.c0 for b in plan.blocks] == [64, 128, 256, 640]
    assert [(b.h, b.w) for b in plan.blocks] == [(128, 128), (64, 64), (32, 32), (16, 16)]
    assert plan.n_features == 1664
    par = dense8s.kernel_params(plan)
    assert par["L0_0_w1"].shape == (2, 128, 32) and par["L0_0_w1"].dtype == np.int8
    assert par["L3_31_w1"].shape == (51, 128, 32)
    assert par["L2_5_abh"].shape == ((256 + 160) // 2, 4) and par["L2_5_abh"].dtype == np.int16
    assert par["L1_0_w2k"].shape == (4, 9, 32, 32)
    assert par["T0_w"].shape == (8, 128, 32) and par["T2_w"].shape == (40, 640, 32)
    assert par["T1_gdf"].shape == (256, 2) and par["F_ab"].shape == (1664, 2)
    assert par["S_w16"].shape == (64, 168) and par["S_w16"].dtype == np.float16
    # the transition tables: T*_gd = T*_gdf / 4 (the mean of four vs the sum)
    assert np.array_equal(par["T0_gd"][:, 0] * 4, par["T0_gdf"][:, 0])


def test_table_layouts(plan169):
    _, plan = plan169
    par = dense8s.kernel_params(plan)
    L = plan.blocks[1].layers[3]
    w1 = par["L1_3_w1"]                                  # chunked [G][128][32]
    for g, o, i in [(0, 0, 0), (3, 77, 31), (6, 127, 5)]:
        assert w1[g, o, i] == L.w1[o, 32 * g + i]
    w2k = par["L1_3_w2k"]                                # [block][tap][o][i]
    for b, tap, o, i in [(0, 0, 0, 0), (3, 8, 31, 31), (2, 4, 7, 19)]:
        assert w2k[b, tap, o, i] == L.w2[o, 32 * b + i, tap // 3, tap % 3]
    a, b = dense8s.abh_values(par["L1_3_abh"])
    assert np.array_equal(a, par["L1_3_ab"][:, 0].astype(np.float16).astype(np.float64))
    assert np.array_equal(b, par["L1_3_ab"][:, 1].astype(np.float16).astype(np.float64))


def test_sign_fold_and_scales(plan169):
    """conv1 rows carry the sign of norm2 (dense8s.py:401-407); |q| <= 127 from the max scaling."""
    m, plan = plan169
    layer = m.features.denseblock1.denselayer1
    a2, _ = dense8s.bn_affine(layer.norm2)
    L = plan.blocks[0].layers[0]
    q, _ = dense8s.quant_weight(layer.conv1.weight)
    sign = np.where(a2 < 0, -1, 1)
    assert np.array_equal(L.w1, (q.reshape(128, -1) * sign[:, None]).astype(np.int8))
    assert np.abs(L.w2).max() <= 127 and np.all(L.w1s > 0)


def test_derived_tables(plan169):
    _, plan = plan169
    pack = dense8s.make_pack(plan, 24)
    d = dense8s.derived_params(pack["meta"], pack["par"])
    w1 = pack["par"]["L2_7_w1"].astype(np.int64)
    assert np.array_equal(d["L2_7_w1sum"], w1.sum(axis=(0, 2)))
    assert np.array_equal(d["L0_1_w2sum"], pack["par"]["L0_1_w2k"].astype(np.int64).sum(axis=(0, 1, 3)))
    assert np.array_equal(d["T1_wsum"], pack["par"]["T1_w"].astype(np.int64).sum(axis=(0, 2)))
    assert d["L0_0_w1sum"].dtype == np.int32


def test_input_lut():
    ref = dense8s.input_lut([0.0] * 3, [1.0] * 3).view(np.float16)
    assert np.array_equal(ref[0], (np.arange(256) / 255.0).astype(np.float16))
    lut = dense8s.input_lut([0.5] * 3, [0.25] * 3).view(np.float16)
    assert lut[1, 0] == -2.0 and lut[2, 255] == 2.0 and lut.shape == (3, 256)


def test_stem_weight_layout():
    w = np.random.default_rng(0).normal(size=(64, 3, 7, 7)).astype(np.float32)
    w16 = dense8s.stem_weights16(w).reshape(64, 3, 7, 8)
    assert np.all(w16[..., 0] == 0) and np.array_equal(w16[..., 1:], w.astype(np.float16))


def test_pack_roundtrip(tmp_path, plan169):
    _, plan = plan169
    p = tmp_path / "enc.npz"
    dense8s.save_pack(p, plan, 24, input_kind="u8")
    pk = dense8s.load_pack(p)
    mem = dense8s.make_pack(plan, 24, input_kind="u8")
    assert pk["meta"] == mem["meta"]
    assert pk["meta"]["kernels_sha"] == hip.source_sha()
    assert set(pk["par"]) == set(mem["par"])
    for k in pk["par"]:
        assert np.array_equal(pk["par"][k], mem["par"][k]) and pk["par"][k].dtype == mem["par"][k].dtype
    assert dense8s.is_pack(pk)
    dense8s.validate_meta(pk["meta"])


@pytest.mark.parametrize("change,msg", [
    ({"kind": "dense8"}, "expected dense8s"), ({"format": 2}, "format"),
    ({"conv2": "trt"}, "TensorRT"), ({"img": 510}, "multiple of 4"), ({"n": 0}, "batch"),
    ({"stem_c": 32}, "stem"),
])
def test_meta_validation(plan169, change, msg):
    _, plan = plan169
    meta = dense8s.pack_meta(plan, 24) | change
    with pytest.raises(ValueError, match=msg):
        dense8s.validate_meta(meta)


def test_encoder_rejects_bad_package(plan169):
    _, plan = plan169
    pack = dense8s.make_pack(plan, 24)
    pack["meta"] = pack["meta"] | {"format": 7}
    with pytest.raises(ValueError):
        dense8s.Dense8SEncoder(pack, 0, 24)
    pack = dense8s.make_pack(plan, 24)
    del pack["par"]["L1_4_w2k"]
    with pytest.raises(ValueError, match="missing"):
        dense8s.Dense8SEncoder(pack, 0, 24)


def test_calibrate_keys():
    m = densenet.seeded_densenet169(1, blocks=(2, 3, 2, 2))
    cal = dense8s.calibrate(m, [torch.randn(2, 3, 32, 32)])
    want = {"seg0.0", "seg0.1", "seg0.2", "seg0.3", "tin.0", "tin.1", "tin.2"}
    want |= {f"{k}.{b}.{l}" for b, n in enumerate((2, 3, 2, 2)) for l in range(n)
             for k in ("conv2", "in1", "in2")}
    assert set(cal) == want
    assert len(cal["seg0.0"]) == 64 and len(cal["conv2.1.2"]) == 32 and len(cal["seg0.1"]) == 64
    assert all(v >= 0 for v in cal["seg0.0"]) and cal["in1.0.0"] > 0


def test_written_bumps_versions():
    """A buffer a kernel writes through a raw pointer gets a new version (base and views share it),
    so the encoder's graph-input key sees new contents in a reused output buffer."""
    buf = torch.zeros((4, 3, 8, 8), dtype=torch.uint8)
    view = buf[1:3]
    key0 = dense8s.contents_id(view)
    v0 = buf._version
    hip.written(view)
    assert buf._version == v0 + 1 and view._version == buf._version
    key1 = dense8s.contents_id(view)
    assert key1 != key0
    with torch.inference_mode():
        t = torch.zeros(3)
        hip.written(t, None)                     # inference tensors and None are accepted
    assert dense8s.contents_id(t) != dense8s.contents_id(t)     # no version counter: always new


def test_concurrent_order_keeps_banded_runners_within_the_cus():
    """encode_concurrent: runners with banded whole blocks overlap while their bands per image sum to at
    most the CU count; one that does not fit waits for every banded runner before it (the group), the
    others run free."""
    import types
    rs = [types.SimpleNamespace(max_bands=k) for k in (8, 0, 8, 200, 100, 0, 8)]
    assert dense8s.concurrent_order(rs, 256) == [[], [], [], [], [0, 2, 3], [], []]
    assert dense8s.concurrent_order(rs, 16) == [[], [], [], [0, 2], [3], [], [4]]
    assert dense8s.concurrent_order([types.SimpleNamespace(max_bands=8)] * 3, 256) == [[], [], []]
    assert dense8s.concurrent_order([]) == []


def test_pass_share_checks_before_any_launch():
    """`Dense8SEncoder.pass_share` refuses a family the pass does not launch, and a runner beside it
    whose banded blocks do not fit the CUs together with its own (their bounded waits could run out),
    before it launches anything."""
    import types
    me = types.SimpleNamespace(program=[dense8s.Step("block", 2, -1, (), "d8s_dense_block_parts")],
                               max_bands=200, dev=0)
    with pytest.raises(ValueError, match="no 'chain' launch"):
        dense8s.Dense8SEncoder.pass_share(me, None, "chain")
    with pytest.raises(ValueError, match="do not fit the CUs"):
        dense8s.Dense8SEncoder.pass_share(me, None, "block", beside=types.SimpleNamespace(max_bands=100))


def test_graph_book_finds_the_smallest_covering_capture():
    """A batch replays the graphs captured for its size, else the first passes of the smallest capture
    that covers it (per flip mode), else none."""
    book = dense8s.GraphBook()
    book.add(48, 0, ["a0", "a1"], "s48")
    book.add(96, 0, ["b0", "b1", "b2", "b3"], "s96")
    book.add(24, 2, ["t0", "t1"], "st")
    assert book.find(48, 0, 24) == (["a0", "a1"], "s48")
    assert book.find(20, 0, 24) == (["a0"], "s48")
    assert book.find(60, 0, 24) == (["b0", "b1", "b2"], "s96")
    assert book.find(97, 0, 24) is None
    assert book.find(12, 2, 12) == (["t0"], "st") and book.find(24, 1, 24) is None
    assert len(book) == 3 and bool(book)
    book.clear()
    assert not book


def test_regions_are_aligned_and_disjoint():
    r = dense8s.Regions()
    r.reserve("a", 1000)
    r.reserve("b", 10)
    r.reserve("c", 300)
    spans = sorted(r.spans.values())
    assert all(start % dense8s.Regions.ALIGN == 0 for start, _ in spans)
    assert all(s0 + n0 <= s1 for (s0, n0), (s1, _) in zip(spans, spans[1:]))
    assert r.size == spans[-1][0] + spans[-1][1] and "b" in r and "z" not in r


def test_step_names_follow_the_family():
    s = dense8s.Step("chain", 2, 5, ((2, 6), ("bott", 2, 6)), "d8s_conv2_conv1")
    assert s.tag() == "chain_2" and s.label() == "cc b2l5"
    assert dense8s.Step("trans", 1, -1, ((2, 0),), "d8s_transition").label() == "t1"
    assert dense8s.Step("block", 3, -1, (), "d8s_dense_block").label() == "blk b3"
    assert dense8s.Step("stem", 0, -1, ((0, 0),), "d8s_stem").tag() == "stem"


def test_inflight_gate_without_a_limit_records_nothing():
    g = dense8s.InflightGate(None)
    g.admit()
    g.done(None)
    assert len(g.events) == 0


def test_recorded_kernel_variants(plan169):
    """Kernel variants recorded per block (`pack_meta(bm=, c2=, tbm=)`: "bm" a list per layer, "c2" per
    side, "tbm" per transition, as the reference's packages record their kernels) map back to variant
    ids; the reference's own kernel names (CUDA kernels) name none and leave the library's choice;
    names that are no variant are refused."""
    _, plan = plan169
    meta = dense8s.pack_meta(plan, 24, bm={"b1l0": "p64", "b2l3": "k2"}, c2={64: "32x4", "32": "16x4"},
                             tbm={"t2": "d4w4"})
    blocks = meta["blocks"]
    assert blocks[1]["bm"][0] == "p64" and blocks[2]["bm"][3] == "k2" and blocks[0]["bm"] == [None] * 6
    assert blocks[1]["c2"] == "32x4" and blocks[2]["c2"] == "16x4" and blocks[0]["c2"] is None
    assert blocks[2]["tbm"] == "d4w4" and blocks[3]["tbm"] is None
    assert dense8s.recorded_variants(meta) == {("conv1", 1, 0): 2, ("conv1", 2, 3): 4, ("conv2", 1): 2,
                                               ("conv2", 2): 4, ("trans", 2): 2}
    dense8s.validate_meta(meta)
    ref = json.loads(json.dumps(meta))
    for b in ref["blocks"]:
        b["bm"], b["c2"], b["tbm"] = ["w64_pl"] * b["L"], [16, 8, "p4u_pl"], "q128"
    assert dense8s.recorded_variants(ref) == {}
    for kw in ({"bm": {"b1l0": "u128h"}}, {"c2": {64: "8x32"}}, {"tbm": {"t0": "q128"}}):
        with pytest.raises(ValueError, match="variant"):
            dense8s.pack_meta(plan, 24, **kw)
    names = [set(t.values()) for t in (dense8s.C1_VARIANTS, dense8s.C2_VARIANTS, dense8s.TRANS_VARIANTS)]
    assert all(len(n) == len(t) for n, t in zip(names, (dense8s.C1_VARIANTS, dense8s.C2_VARIANTS,
                                                        dense8s.TRANS_VARIANTS)))
