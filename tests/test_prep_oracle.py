"""Pins of the preprocessing oracle (`oracle/prep.py`, `oracle/prep_oracle.c`) on the CPU: closed forms,
library routines and invariants that a dropped term, a wrong index or a transposed axis would break."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import prep as P
from rsna_knee_efficiency_amd import prep as hp
from rsna_knee_efficiency_amd import synthetic


@pytest.mark.parametrize("n", [4, 5, 100, 101, 1000, 4097, 24 * 512 * 512, 23 * 288 * 288])
def test_ranks_reproduce_np_percentile(n):
    """On 0, 1, ..., n-1 the linear percentile is k + gamma exactly: pins the ranks and gammas."""
    k1, k2, g1, g2 = P.ranks(n)
    x = np.arange(n, dtype=np.float64)
    lo, hi = np.percentile(x, P.CLIP_PCT)
    assert lo == k1 + g1 and hi == k2 + g2
    assert 0 <= k1 < k1 + 1 < n and 0 <= k2 < k2 + 1 < n and 0 <= g1 < 1 and 0 <= g2 < 1
    assert hp.ranks(n) == (k1, k2, g1, g2)


def test_ranks_reject_tiny_stacks():
    with pytest.raises(ValueError):
        hp.ranks(3)


def test_to_uint8_closed_forms():
    # constant, NaN, infinite percentiles: all zero (cache.py:331-336)
    assert not P.to_uint8(np.full((2, 8, 8), 3.5, np.float32)).any()
    x = np.random.default_rng(0).normal(size=(2, 8, 8)).astype(np.float32)
    x[1, 3, 3] = np.nan
    assert not P.to_uint8(x).any()
    x = np.arange(2 * 8 * 8, dtype=np.float32).reshape(2, 8, 8)
    x[0, :2] = -np.inf
    assert not P.to_uint8(x).any()                 # lo = -inf
    # a ramp: below the 1st percentile 0, above the 99th 255, monotone in between
    n = 10001
    x = np.arange(n, dtype=np.float32)
    u = P.to_uint8(x)
    k1, k2, g1, g2 = P.ranks(n)
    lo, hi = k1 + g1, k2 + g2
    assert (u[x <= lo] == 0).all() and (u[x >= hi] == 255).all()
    assert (np.diff(u.astype(int)) >= 0).all() and u[n // 2] == int((n // 2 - lo) * 255 / (hi - lo))


def test_to_uint8_matches_sorted_definition():
    """np.percentile against the order statistics themselves (sorted array), ties included."""
    rng = np.random.default_rng(1)
    for trial in range(6):
        n = int(rng.integers(50, 5000))
        x = rng.integers(-3, 40, n).astype(np.float32) * np.float32(0.37)
        if trial % 2:
            x[rng.random(n) < 0.4] = 0.0             # a background of zeros
        s = np.sort(x)
        k1, k2, g1, g2 = P.ranks(n)
        lo, hi = np.percentile(x, P.CLIP_PCT)
        for k, g, v in ((k1, g1, lo), (k2, g2, hi)):
            a, b = s[k], s[k + 1]
            assert min(a, b) <= v <= max(a, b)
            if a == b:
                assert v == a
        st = P.stats(x)
        assert st["lo"] == lo and st["hi"] == hi and st["bad"] == (not hi > lo)


@pytest.mark.parametrize("ssize,dsize", [(1024, 512), (1536, 512), (750, 512), (550, 512),
                                         (513, 512), (4096, 512), (600, 288)])
def test_area_taps_properties(ssize, dsize):
    idx, w = P.area_taps(ssize, dsize)
    scale = ssize / dsize
    assert ((idx >= 0) & (idx < ssize)).all()
    sums = w.astype(np.float64).sum(1)
    assert np.allclose(sums, 1.0, atol=2e-6)
    for d in range(dsize):
        nz = idx[d][w[d] > 0]
        # the taps of output d cover exactly the source pixels its interval [d s, (d + 1) s) touches
        lo, hi = int(np.floor(d * scale + 1e-9)), int(np.ceil((d + 1) * scale - 1e-9)) - 1
        assert list(nz) == list(range(lo, min(hi, ssize - 1) + 1)), d
    if ssize % dsize == 0:
        f = ssize // dsize
        assert idx.shape[1] == f and (w == np.float32(1.0 / f)).all()
        assert (idx == np.arange(dsize)[:, None] * f + np.arange(f)).all()


def _area_np(sub: np.ndarray, img: int) -> np.ndarray:
    """`area_resize_torch` (raw_crop.py:396-416) in numpy float32: columns, then rows, in table order."""
    k, h, w = sub.shape
    out = sub
    if w != img:
        idx, wt = P.area_taps(w, img)
        acc = np.zeros((k, h, img), np.float32)
        for j in range(idx.shape[1]):
            acc = acc + out[:, :, idx[:, j]] * wt[:, j]
        out = acc
    if h != img:
        idx, wt = P.area_taps(h, img)
        acc = np.zeros((k, img, out.shape[2]), np.float32)
        for j in range(idx.shape[1]):
            acc = acc + out[:, idx[:, j], :] * wt[:, j][:, None]
        out = acc
    return out


def _region(K, h, w, seed, hi=4096):
    return np.random.default_rng(seed).integers(0, hi, (K, h, w)).astype(np.uint16)


@pytest.mark.parametrize("h,w,img", [(80, 80, 64), (96, 72, 64), (128, 64, 64), (200, 150, 64)])
def test_area_resize_matches_numpy_restatement(h, w, img):
    reg = _region(2, h + 6, w + 4, 3)
    box = (3, 3 + h, 1, 1 + w)
    got = P.resize_stack(reg, None, box, img)
    want = _area_np(reg[:, 3:3 + h, 1:1 + w].astype(np.float32), img)
    assert np.array_equal(got, want)


def test_area_resize_factor_two_is_block_mean():
    reg = _region(1, 128, 128, 4, hi=1000)
    got = P.resize_stack(reg, None, (0, 128, 0, 128), 64)[0]
    blocks = reg[0].astype(np.float64).reshape(64, 2, 64, 2).mean(axis=(1, 3))
    assert np.array_equal(got, blocks.astype(np.float32))


@pytest.mark.parametrize("h,w", [(48, 48), (40, 56), (63, 17), (64, 40)])
def test_bilinear_matches_torch_interpolate(h, w):
    """The C restatement against torch's own CPU interpolate (same weights, another rounding order)."""
    img = 64
    reg = _region(2, h, w, 5)
    got = P.resize_stack(reg, None, (0, h, 0, w), img)
    ref = F.interpolate(torch.from_numpy(reg.astype(np.float32)).unsqueeze(1), size=(img, img),
                        mode="bilinear", align_corners=False, antialias=False).squeeze(1).numpy()
    assert np.allclose(got, ref, rtol=2e-6, atol=2e-3)
    # half-pixel centres: a linear ramp in x is reproduced at the interior output columns
    ramp = np.tile(np.arange(w, dtype=np.uint16) * 8, (1, h, 1))
    r = P.resize_stack(ramp, None, (0, h, 0, w), img)[0]
    sx = (np.arange(img) + 0.5) * (w / img) - 0.5
    inner = (sx >= 0) & (sx <= w - 1)
    assert np.allclose(r[:, inner], 8 * sx[inner][None, :], atol=1e-3)


def test_identity_and_rescale():
    reg = _region(3, 70, 70, 6)
    resc = np.array([[1.5, -2.0], [0.25, 10.0], [1.0, 0.0]], np.float32)
    got = P.resize_stack(reg, resc, (3, 67, 2, 66), 64)
    want = reg[:, 3:67, 2:66].astype(np.float32) * resc[:, 0, None, None] + resc[:, 1, None, None]
    assert np.array_equal(got, want.astype(np.float32))


def test_slice_range_leaves_other_slices():
    reg = _region(4, 50, 50, 7)
    full = P.resize_stack(reg, None, (0, 50, 0, 50), 64)
    part = P.resize_stack(reg, None, (0, 50, 0, 50), 64, k_range=(1, 3))
    assert np.array_equal(part[1:3], full[1:3]) and not part[0].any() and not part[3].any()


def test_payload_chain_flips_and_ranges():
    """The chain on a small synthetic study: the flips are the reference's views (raw_crop.py:541-545),
    a slice range normalises only its slices, CPU series are copied as they are."""
    img, K = 64, 6
    pay = synthetic.study_payload(img, K, 11, crops=(110.0, 150.0), cpu_series=True,
                                  series=((1.25, 1.0, 0, None), (0.8, 1.0, 1, (1.5, -3.0)),
                                          (2.0, 0.9, 2, None), (1.0, 1.0, 0, None)))
    vol = P.payload_to_uint8(pay, img, 4, 2, K)
    assert vol.shape == (8, K, img, img)
    meta = pay["meta"]
    raw = pay["raw"].view(np.uint16)
    # series 1 (FLIP_X), scale 0: recompute unflipped and compare mirrored
    row = meta[1]
    reg = raw[row[5]: row[5] + K * row[3] * row[4]].reshape(K, row[3], row[4])
    st = P.resize_stack(reg, pay["resc"][:K].astype(np.float32), row[8:12], img)
    assert np.array_equal(vol[1], P.to_uint8(st)[:, :, ::-1])
    # series 2 (FLIP_SLICES) with a range: positions read are reversed
    rng = (1, 5)
    vr = P.payload_to_uint8(pay, img, 4, 2, K, read_slices=rng)
    row = meta[2]
    reg = raw[row[5]: row[5] + K * row[3] * row[4]].reshape(K, row[3], row[4])
    a, z = P.read_range(K, 2, rng)
    assert (a, z) == (K - 5, K - 1)
    st = P.resize_stack(reg, None, row[8:12], img, k_range=(a, z))
    u = np.zeros((K, img, img), np.uint8)
    u[a:z] = P.to_uint8(st[a:z])
    assert np.array_equal(vr[2], u[::-1])
    assert not vr[2][:1].any() and not vr[2][5:].any()
    # the CPU series is the payload's own uint8
    n = K * img * img
    assert np.array_equal(vol[3], pay["u8"][:n].reshape(K, img, img))
    assert np.array_equal(vol[7], pay["u8"][n:2 * n].reshape(K, img, img))
