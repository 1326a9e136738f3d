"""Seeded synthetic inputs of the benchmark configurations (there is no dataset offline).

- `study_u8(n, img, seed)`: n slice stacks of 3 x img x img uint8 from one synthetic volume of n + 2
  slices (stack i = slices i, i+1, i+2, the reference's 3-slice windows, `src/knee/models/baseline.py:
  154-164`): a smooth low-frequency field of Gaussian blobs drifting from slice to slice, plus uniform
  noise.
- `c5_study(s)`: study s of configuration 5 (two crops of 24 stacks, seeded 1234 + s).
- `normalise(u8)`: x = (u / 255 - mean) / std as float32 (mean 0.5, std 0.25): the float model's input;
  the INT8 encoder applies the same map in its stem through an fp16 table.
- `linear_head(c_in, c_out, seed)`: the 1664 -> 8 head of configuration 4 (float64 weights, bias).
- `study_payload(...)`: one study as the raw-crop payload the GPU preparation reads
  (src/knee/data/raw_crop.py:28-41): four series of uint16 slices (an MRI-like field with a zero
  background), cropped to the 150 mm box, with the 110 and 150 mm boxes per series; pixel spacings
  chosen so that both resize branches run (bilinear upscaling and INTER_AREA downscaling), one series
  with a non-trivial Rescale, flips of both kinds, and optionally one series already in uint8 (a CPU
  series).
"""
from __future__ import annotations

import numpy as np
import torch

MEAN, STD = 0.5, 0.25


def study_u8(n: int, img: int, seed, blobs: int = 12) -> np.ndarray:
    rng = np.random.default_rng(seed)
    t = np.arange(img) / img
    cy, cx = rng.uniform(0, 1, blobs), rng.uniform(0, 1, blobs)
    sig = rng.uniform(0.05, 0.25, blobs)
    amp = rng.uniform(-1, 1, blobs)
    drift = rng.uniform(-0.01, 0.01, (blobs, 2))
    vol = np.empty((n + 2, img, img), np.uint8)
    for z in range(n + 2):
        # each blob is separable: amp exp(-dy^2 / 2 s^2) exp(-dx^2 / 2 s^2), one outer product
        gy = amp[:, None] * np.exp(-(t[None, :] - (cy + z * drift[:, 0])[:, None]) ** 2
                                   / (2 * sig[:, None] ** 2))
        gx = np.exp(-(t[None, :] - (cx + z * drift[:, 1])[:, None]) ** 2 / (2 * sig[:, None] ** 2))
        field = gy.T @ gx
        field /= max(np.abs(field).max(), 1e-9)
        s = 128 + 90 * field + rng.uniform(-40, 40, (img, img))
        vol[z] = np.clip(np.rint(s), 0, 255).astype(np.uint8)
    return np.ascontiguousarray(np.stack([vol[i:i + 3] for i in range(n)]))


C5_SEED0 = 1234                 # configuration 5's studies are seeded 1234, 1235, ...


def c5_study(s: int, img: int = 512, slices: int = 24) -> np.ndarray:
    """Study `s` of configuration 5: its two crops (110 mm, 150 mm, both at img) of `slices` stacks
    each, (2 slices, 3, img, img) uint8, crop c seeded (C5_SEED0 + s, c)."""
    return np.concatenate([study_u8(slices, img, seed=[C5_SEED0 + s, c]) for c in range(2)])


def normalise(u8: torch.Tensor, mean: float = MEAN, std: float = STD) -> torch.Tensor:
    return (u8.float() / 255.0 - mean) / std


def linear_head(c_in: int, c_out: int, seed: int) -> tuple[np.ndarray, np.ndarray]:
    rng = np.random.default_rng(seed)
    return rng.normal(0, np.sqrt(1.0 / c_in), (c_out, c_in)), rng.normal(0, 0.1, c_out)


# (pixel spacing mm, rows / columns aspect, flip code, Rescale) of the four synthetic series
PAYLOAD_SERIES = ((0.3125, 1.0, 0, None), (0.2, 1.0, 1, (1.2265625, -5.0)),
                  (0.45, 1.0, 2, (0.75, 13.25)), (0.35, 0.9, 0, None))


def _crop_box(rows: int, cols: int, ps: float, mm: float) -> tuple[int, int, int, int]:
    side = int(round(mm / ps))
    h, w = min(side, rows), min(side, cols)
    y0, x0 = (rows - h) // 2, (cols - w) // 2
    return y0, y0 + h, x0, x0 + w


def study_payload(img: int, slices: int, seed: int, crops=(110.0, 150.0), cpu_series: bool = False,
                  series=PAYLOAD_SERIES) -> dict:
    """One study payload: `raw` int16 (uint16 values), `u8` uint8, `resc` float64 (m, 2), `meta` int64
    (n, 17) with the columns of src/knee/data/raw_crop.py:44-52 (boxes relative to the region)."""
    rng = np.random.default_rng(seed)
    raws, u8s, rescs, meta = [], [], [], []
    raw_off = u8_off = resc_off = 0
    for j, (ps, aspect, flip, resc) in enumerate(series):
        side = int(round(max(crops) / ps))
        rows, cols = side, int(round(side * aspect))
        boxes = [_crop_box(rows, cols, ps, mm) for mm in crops]
        row = np.zeros(17, np.int64)
        row[0], row[2] = j, slices
        if cpu_series and j == len(series) - 1:
            row[1], row[7], row[16] = 2, u8_off, -1
            n = len(crops) * slices * img * img
            u8s.append(rng.integers(0, 256, n, dtype=np.uint8))
            u8_off += n
            meta.append(row)
            continue
        yy, xx = np.meshgrid(np.linspace(-1, 1, rows), np.linspace(-1, 1, cols), indexing="ij")
        body = (yy ** 2 + (xx / 0.85) ** 2) < 0.8
        vol = np.zeros((slices, rows, cols), np.uint16)
        for z in range(slices):
            field = 600 + 400 * np.sin(3 * yy + 0.2 * z) * np.cos(2 * xx - 0.1 * z)
            sl = field + rng.normal(0, 60, (rows, cols))
            vol[z] = np.where(body, np.clip(np.rint(sl), 0, 4095), 0).astype(np.uint16)
        row[1], row[3], row[4], row[5], row[6] = 1, rows, cols, raw_off, flip
        for k, b in enumerate(boxes):
            row[8 + 4 * k: 12 + 4 * k] = b
        if resc is not None:
            row[16] = resc_off
            rescs.append(np.tile(np.asarray(resc, np.float64), (slices, 1)))
            resc_off += slices
        else:
            row[16] = -1
        raws.append(vol.reshape(-1).view(np.int16))
        raw_off += vol.size
        meta.append(row)
    return {"raw": np.concatenate(raws) if raws else np.zeros(0, np.int16),
            "u8": np.concatenate(u8s) if u8s else np.zeros(0, np.uint8),
            "resc": np.concatenate(rescs) if rescs else np.zeros((0, 2), np.float64),
            "meta": np.stack(meta)}
