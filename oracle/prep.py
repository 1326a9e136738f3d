"""CPU oracle of the upstream preprocessing: raw uint16 crop -> resize to img -> exact 1/99 percentiles
-> uint8 -> side flip.  TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Sources followed (all in the reference's `src/knee/data/`):
- `to_uint8`      `cache._to_uint8` (cache.py:319-340) with NumPy 2 promotion: `np.percentile` (linear)
                  at `CLIP_PCT` (cache.py:46), then `(stack - lo) * (255 / (hi - lo))` in float64,
                  clip to [0, 255], truncation; a stack with non-finite percentiles or hi <= lo is 0.
                  This is the reference's own CPU path and the definition the GPU path is bit-identical
                  to (torch_uint8.py:1-16).
- `ranks`         `torch_uint8._ranks` (torch_uint8.py:31-42): the order statistics k1, k2 and gamma of
                  numpy's linear method, virtual index (n - 1) q.
- `stats`         the per-stack values the GPU path derives on the way (percentiles, scale, bad).
- `resize_stack`  the crop + rescale + resize of `payloads_to_uint8_torch` (raw_crop.py:515-531),
                  restated in C (`prep_oracle.c`, which cites the reference lines it follows).
- `payload_to_uint8` the whole chain for one study payload (raw_crop.py:492-549), including the
                  slice range of `read_range`/`_uint8_ranges` (raw_crop.py:79-110) and the flips.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import lib as _lib

CLIP_PCT = (1.0, 99.0)
# columns of the payload's `meta` (src/knee/data/raw_crop.py:44-52)
M_SLOT, M_MODE, M_K, M_HR, M_WR, M_RAW_OFF, M_FLIP, M_U8_OFF = range(8)
M_BOX = 8
MAX_SCALES = 2
M_RESC = M_BOX + 4 * MAX_SCALES
N_META = M_RESC + 1
MODE_GPU, MODE_CPU = 1, 2
FLIP_NONE, FLIP_X, FLIP_SLICES = 0, 1, 2

vp, i32 = ctypes.c_void_p, ctypes.c_int


def _L():
    L = _lib.lib()
    if not getattr(L, "_prep_ready", False):
        L.orc_area_taps.argtypes = [i32, i32, i32, vp, vp]
        L.orc_area_taps.restype = i32
        L.orc_resize_stack.argtypes = [vp, i32, i32, i32, vp, i32, i32, i32, i32, i32, i32, i32, vp]
        L.orc_resize_stack.restype = i32
        L._prep_ready = True
    return L


def ranks(n: int) -> tuple[int, int, float, float]:
    """(k1, k2, gamma1, gamma2): linear `np.percentile` at CLIP_PCT over n values is
    lerp(sorted[k], sorted[k + 1], gamma) for (k1, gamma1) and (k2, gamma2)."""
    q = np.true_divide(np.asarray(CLIP_PCT), 100)
    virtual = (n - 1) * q
    prev = np.floor(virtual)
    g = virtual - prev
    return int(prev[0]), int(prev[1]), float(g[0]), float(g[1])


def to_uint8(stack: np.ndarray) -> np.ndarray:
    """`cache._to_uint8` of one stack (any shape, float32) -> uint8 of the same shape."""
    lo, hi = np.percentile(stack, CLIP_PCT)
    if not np.isfinite([lo, hi]).all() or hi <= lo:
        return np.zeros(stack.shape, np.uint8)
    y = np.subtract(stack, lo)
    np.multiply(y, 255.0 / (hi - lo), out=y)
    np.clip(y, 0, 255, out=y)
    return y.astype(np.uint8)


def stats(stack: np.ndarray) -> dict:
    """The values the GPU records per stack: the two percentiles, the scale and the bad flag."""
    lo, hi = (float(v) for v in np.percentile(stack, CLIP_PCT))
    bad = bool(not np.isfinite([lo, hi]).all() or hi <= lo)
    with np.errstate(all="ignore"):
        scale = float(255.0 / (np.float64(hi) - np.float64(lo)))
    return {"lo": lo, "hi": hi, "scale": scale, "bad": bad}


def area_taps(ssize: int, dsize: int, max_taps: int = 16) -> tuple[np.ndarray, np.ndarray]:
    """cv2 INTER_AREA table (dsize, T): source indices (int32) and float32 weights, zero-padded."""
    idx = np.zeros(dsize * max_taps, np.int32)
    w = np.zeros(dsize * max_taps, np.float32)
    T = _L().orc_area_taps(ssize, dsize, max_taps, idx.ctypes.data, w.ctypes.data)
    if T < 0:
        raise ValueError(f"area table {ssize}->{dsize} longer than {max_taps} taps")
    return idx[:dsize * T].reshape(dsize, T), w[:dsize * T].reshape(dsize, T)


def resize_stack(region: np.ndarray, resc: np.ndarray | None, box, img: int,
                 k_range: tuple[int, int] | None = None, out: np.ndarray | None = None) -> np.ndarray:
    """region (K, hr, wr) uint16, resc (K, 2) float32 slope/intercept or None, box (y0, y1, x0, x1)
    -> (K, img, img) float32; with k_range only those slices are computed (the others stay 0)."""
    region = np.ascontiguousarray(region, dtype=np.uint16)
    K, hr, wr = region.shape
    y0, y1, x0, x1 = (int(v) for v in box)
    if not (0 <= y0 < y1 <= hr and 0 <= x0 < x1 <= wr):
        raise ValueError(f"box {box} outside the region {hr}x{wr}")
    a, z = k_range if k_range is not None else (0, K)
    if out is None:
        out = np.zeros((K, img, img), np.float32)
    rs = None if resc is None else np.ascontiguousarray(resc, dtype=np.float32)
    rc = _L().orc_resize_stack(region.ctypes.data, K, hr, wr, None if rs is None else rs.ctypes.data,
                               y0, y1, x0, x1, img, a, z, out.ctypes.data)
    if rc != 0:
        raise ValueError("resize_stack: area table too long")
    return out


def flip(u: np.ndarray, code: int) -> np.ndarray:
    """`normalise_laterality` as applied by the GPU path (raw_crop.py:541-545): FLIP_X reverses the
    columns, FLIP_SLICES the slices."""
    if code == FLIP_X:
        return u[:, :, ::-1]
    if code == FLIP_SLICES:
        return u[::-1]
    return u


def read_range(k_sl: int, code: int, slices: tuple[int, int] | None) -> tuple[int, int] | None:
    """`raw_crop.read_range` (raw_crop.py:79-90) with the `KNEE_READ_SLICES` range passed in."""
    if slices is None:
        return None
    a, z = slices
    if not 0 <= a < z <= k_sl:
        raise ValueError(f"slice range {a}:{z} outside 0..{k_sl}")
    return (k_sl - z, k_sl - a) if code == FLIP_SLICES else (a, z)


def payload_to_uint8(payload: dict, img: int, n_seq: int, n_scales: int, slices: int,
                     read_slices: tuple[int, int] | None = None) -> np.ndarray:
    """One study payload (`raw` int16 1-D, `u8` uint8 1-D, `resc` float64 (m, 2), `meta` int64
    (n, N_META)) -> the volume (n_seq * n_scales, slices, img, img) uint8."""
    vol = np.zeros((n_seq * n_scales, slices, img, img), np.uint8)
    raw = np.asarray(payload["raw"]).view(np.uint16)
    u8 = np.asarray(payload["u8"])
    resc_all = np.asarray(payload["resc"])
    for row in np.asarray(payload["meta"]):
        j, k_sl = int(row[M_SLOT]), int(row[M_K])
        if row[M_MODE] == MODE_GPU:
            hr, wr, off = int(row[M_HR]), int(row[M_WR]), int(row[M_RAW_OFF])
            region = raw[off: off + k_sl * hr * wr].reshape(k_sl, hr, wr)
            resc = None
            if row[M_RESC] >= 0:
                resc = resc_all[int(row[M_RESC]): int(row[M_RESC]) + k_sl].astype(np.float32)
            code = int(row[M_FLIP])
            rr = read_range(k_sl, code, read_slices)
            for k in range(n_scales):
                box = [int(v) for v in row[M_BOX + 4 * k: M_BOX + 4 * k + 4]]
                st = resize_stack(region, resc, box, img, rr)
                if rr is None:
                    u = to_uint8(st)
                else:
                    u = np.zeros(st.shape, np.uint8)
                    u[rr[0]:rr[1]] = to_uint8(st[rr[0]:rr[1]])
                vol[j + k * n_seq] = flip(u, code)
        else:
            off, n = int(row[M_U8_OFF]), k_sl * img * img
            for k in range(n_scales):
                vol[j + k * n_seq] = u8[off + k * n: off + (k + 1) * n].reshape(k_sl, img, img)
    return vol
