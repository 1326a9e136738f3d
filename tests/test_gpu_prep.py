"""Parity of the preprocessing kernels (`d8s_prep`, `d8s_prep_resize`) on the GPU, bit for bit: the
resize against the C oracle and against the reference's own torch operations on the same device, the
uint8 values and percentiles against `cache._to_uint8` (numpy), whole study payloads against the
oracle's chain."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import prep as P
from rsna_knee_efficiency_amd import prep as hp
from rsna_knee_efficiency_amd import synthetic

pytestmark = pytest.mark.gpu


def _region(K, h, w, seed, hi=4096, zero_frac=0.0):
    rng = np.random.default_rng(seed)
    r = rng.integers(0, hi, (K, h, w)).astype(np.uint16)
    if zero_frac:
        r[rng.random(r.shape) < zero_frac] = 0
    return r


# (K, hr, wr, box, img, rescale, slice range)
RESIZE = [
    (3, 480, 480, (64, 416, 64, 416), 512, None, None),          # 110 mm box, bilinear up
    (2, 480, 480, (0, 480, 0, 480), 512, (1.2265625, -5.0), None),
    (2, 750, 750, (100, 650, 100, 650), 512, None, None),        # area 550 -> 512
    (2, 750, 750, (0, 750, 0, 750), 512, (0.75, 13.25), (1, 2)),  # area 750 -> 512
    (2, 1024, 1024, (0, 1024, 0, 1024), 512, None, None),        # area, factor 2
    (2, 700, 520, (0, 700, 4, 516), 512, None, None),            # area rows, columns at img
    (2, 429, 386, (57, 371, 36, 350), 512, None, None),
    (2, 429, 386, (0, 429, 0, 386), 512, None, None),            # non-square bilinear
    (2, 300, 300, (10, 298, 6, 294), 288, None, None),           # identity at 288
    (2, 40, 50, (0, 40, 0, 50), 64, None, None),
    (1, 17, 9, (0, 17, 0, 9), 64, (2.0, 0.5), None),             # strong upscale, odd sizes
    (2, 600, 300, (0, 600, 0, 300), 256, None, None),            # area both axes
]


@pytest.mark.parametrize("case", RESIZE, ids=[f"resize{i}" for i in range(len(RESIZE))])
def test_resize_bit_exact(dev, case):
    K, hr, wr, box, img, resc, kr = case
    print(f"resize {case}", flush=True)
    reg = _region(K, hr, wr, hr * 7 + wr)
    rs = None if resc is None else np.tile(np.asarray(resc, np.float32), (K, 1))
    want = P.resize_stack(reg, rs, box, img, k_range=kr)
    r = torch.from_numpy(reg.view(np.int16)).to(dev)
    got = hp.resize(r, None if rs is None else torch.from_numpy(rs).to(dev), box, img, k_range=kr)
    got = got.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"{int((got != want).sum())} values differ, max {float(np.abs(got - want).max())}"


@pytest.mark.parametrize("h,w,img", [(352, 352, 512), (480, 480, 512), (244, 333, 512), (40, 50, 64)])
def test_bilinear_is_torch_interpolate_on_the_gpu(dev, h, w, img):
    """The reference's own operation (raw_crop.py:431-432) on the same device gives the same bits."""
    reg = _region(2, h, w, h + w)
    x = torch.from_numpy(reg.astype(np.float32)).to(dev)
    ref = F.interpolate(x.unsqueeze(1), size=(img, img), mode="bilinear", align_corners=False,
                        antialias=False).squeeze(1)
    got = hp.resize(torch.from_numpy(reg.view(np.int16)).to(dev), None, (0, h, 0, w), img)
    diff = int((got != ref).sum())
    assert diff == 0, f"{diff} values differ, max {float((got - ref).abs().max())}"


def test_area_is_the_reference_torch_ops_on_the_gpu(dev):
    """`area_resize_torch` (raw_crop.py:396-416) as torch operations on the GPU against the kernel."""
    reg = _region(2, 700, 650, 9)
    sub = torch.from_numpy(reg.astype(np.float32)).to(dev)
    out = sub
    for axis, size in ((2, 650), (1, 700)):
        idx, wt = P.area_taps(size, 512)
        idx_t, wt_t = torch.from_numpy(idx.astype(np.int64)).to(dev), torch.from_numpy(wt).to(dev)
        shape = list(out.shape)
        shape[axis] = 512
        acc = torch.zeros(shape, dtype=torch.float32, device=dev)
        for j in range(idx.shape[1]):
            w = wt_t[:, j] if axis == 2 else wt_t[:, j].unsqueeze(1)
            acc.add_(out.index_select(axis, idx_t[:, j]).mul_(w))
        out = acc
    got = hp.resize(torch.from_numpy(reg.view(np.int16)).to(dev), None, (0, 700, 0, 650), 512)
    assert torch.equal(got, out)


def _stack_cases(K, img):
    rng = np.random.default_rng(5)
    n = K * img * img
    cases = {"normal": rng.normal(0, 100, n), "uniform_pos": rng.uniform(0, 3000, n)}
    z = rng.uniform(1, 2000, n)
    z[rng.random(n) < 0.6] = 0.0
    cases["zero_background"] = z
    cases["integers_ties"] = rng.integers(0, 50, n).astype(np.float64)
    cases["signs_and_zeros"] = np.where(rng.random(n) < 0.5, -0.0, 0.0) + rng.choice([-1, 0, 1], n) * \
        rng.uniform(1e-30, 1e30, n)
    cases["denormals"] = rng.uniform(0, 1e-39, n)
    c = np.full(n, 7.25)
    cases["constant"] = c
    t = rng.uniform(0, 1, n)
    t[:5] = np.nan
    cases["nan"] = t
    t = rng.uniform(0, 1, n)
    t[rng.random(n) < 0.005] = np.inf
    cases["few_inf"] = t
    t = rng.uniform(0, 1, n)
    t[rng.random(n) < 0.05] = np.inf
    cases["many_inf"] = t
    two = np.zeros(n)
    two[: n // 2] = 1.0
    cases["two_values"] = two
    return {k: v.astype(np.float32).reshape(K, img, img) for k, v in cases.items()}


def test_to_uint8_float_stacks(dev):
    K, img = 3, 64
    cases = _stack_cases(K, img)
    names = list(cases)
    x = np.stack([cases[k] for k in names])
    xt = torch.from_numpy(x).to(dev)
    got = hp.to_uint8_hist_batch(xt).cpu().numpy()
    st = hp.stats(hp._WS[str(dev)], len(names))
    for i, k in enumerate(names):
        print(f"stack {k}", flush=True)
        want = P.to_uint8(x[i])
        assert np.array_equal(got[i], want), f"{k}: {int((got[i] != want).sum())} bytes differ"
        ref = P.stats(x[i])
        assert st[i]["bad"] == ref["bad"], k
        if not ref["bad"]:
            assert (st[i]["lo"], st[i]["hi"], st[i]["scale"]) == (ref["lo"], ref["hi"], ref["scale"]), k


@pytest.mark.parametrize("R,K,img", [(20, 2, 64), (1, 1, 8), (2, 5, 96)])
def test_to_uint8_batches(dev, R, K, img):
    """More stacks than one launch holds (16), the smallest side, a side that is not a power of two."""
    rng = np.random.default_rng(R * 100 + img)
    x = rng.gamma(2.0, 300.0, (R, K, img, img)).astype(np.float32)
    got = hp.to_uint8_hist_batch(torch.from_numpy(x).to(dev)).cpu().numpy()
    for i in range(R):
        assert np.array_equal(got[i], P.to_uint8(x[i])), i


def _series(small: bool):
    if small:
        return ((1.25, 1.0, 0, None), (0.8, 1.0, 1, (1.5, -3.0)), (2.0, 0.9, 2, None), (1.0, 1.0, 0, None))
    return synthetic.PAYLOAD_SERIES


@pytest.mark.parametrize("read_slices", [None, (1, 7)])
def test_payload_small_study(dev, read_slices):
    img, K = 128, 8
    pays = [synthetic.study_payload(img, K, 20 + b, cpu_series=b == 1, series=_series(True))
            for b in range(2)]
    spec = hp.PrepSpec(img=img, slices=K, n_seq=4, n_scales=2)
    got = hp.payloads_to_uint8(pays, spec, dev, read_slices=read_slices).cpu().numpy()
    for b, pay in enumerate(pays):
        want = P.payload_to_uint8(pay, img, 4, 2, K, read_slices=read_slices)
        for s in range(8):
            assert np.array_equal(got[b, s], want[s]), (b, s, int((got[b, s] != want[s]).sum()))


def test_payload_full_study(dev):
    """One study at the final configuration: 512 px, 24 slices, 110 + 150 mm, slices 0:23 read."""
    img, K = 512, 24
    pay = synthetic.study_payload(img, K, 3)
    spec = hp.PrepSpec(img=img, slices=K, n_seq=4, n_scales=2)
    got = hp.payloads_to_uint8([pay], spec, dev, read_slices=(0, 23)).cpu().numpy()[0]
    want = P.payload_to_uint8(pay, img, 4, 2, K, read_slices=(0, 23))
    for s in range(8):
        assert np.array_equal(got[s], want[s]), (s, int((got[s] != want[s]).sum()))


def test_payload_missing_series_slots_are_zero(dev):
    """A study without one of its series: that series' slots (both crop scales) are all zeros even
    when the volume's memory held other bytes before, the others equal the oracle's chain."""
    img, K = 64, 6
    pay = synthetic.study_payload(img, K, 31, series=_series(True))
    pay = dict(pay)
    pay["meta"] = np.delete(np.asarray(pay["meta"]), 2, axis=0)        # drop series 2
    spec = hp.PrepSpec(img=img, slices=K, n_seq=4, n_scales=2)
    junk = torch.full((1, *spec.shape), 77, dtype=torch.uint8, device=dev)
    del junk                                                            # its block is reused next
    got = hp.payloads_to_uint8([pay], spec, dev).cpu().numpy()[0]
    want = P.payload_to_uint8(pay, img, 4, 2, K)
    slots = {int(r[0]) for r in pay["meta"]}
    assert 2 not in slots
    for s in range(8):
        assert np.array_equal(got[s], want[s]), (s, int((got[s] != want[s]).sum()))
    assert not got[2].any() and not got[6].any()
