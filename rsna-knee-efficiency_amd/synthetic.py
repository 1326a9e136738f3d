"""Seeded synthetic inputs of the benchmark configurations (there is no dataset offline).

- `study_u8(n, img, seed)`: n slice stacks of 3 x img x img uint8 from one synthetic volume of n + 2
  slices (stack i = slices i, i+1, i+2, the reference's 3-slice windows, `src/knee/models/baseline.py:
  154-164`): a smooth low-frequency field of Gaussian blobs drifting from slice to slice, plus uniform
  noise.
- `normalise(u8)`: x = (u / 255 - mean) / std as float32 (mean 0.5, std 0.25): the float model's input;
  the INT8 encoder applies the same map in its stem through an fp16 table.
- `linear_head(c_in, c_out, seed)`: the 1664 -> 8 head of configuration 4 (float64 weights, bias).
"""
from __future__ import annotations

import numpy as np
import torch

MEAN, STD = 0.5, 0.25


def study_u8(n: int, img: int, seed: int, blobs: int = 12) -> np.ndarray:
    rng = np.random.default_rng(seed)
    yy, xx = np.meshgrid(np.arange(img) / img, np.arange(img) / img, indexing="ij")
    cy, cx = rng.uniform(0, 1, blobs), rng.uniform(0, 1, blobs)
    sig = rng.uniform(0.05, 0.25, blobs)
    amp = rng.uniform(-1, 1, blobs)
    drift = rng.uniform(-0.01, 0.01, (blobs, 2))
    vol = np.empty((n + 2, img, img), np.uint8)
    for z in range(n + 2):
        field = np.zeros((img, img))
        for k in range(blobs):
            d2 = (yy - cy[k] - z * drift[k, 0]) ** 2 + (xx - cx[k] - z * drift[k, 1]) ** 2
            field += amp[k] * np.exp(-d2 / (2 * sig[k] ** 2))
        field /= max(np.abs(field).max(), 1e-9)
        s = 128 + 90 * field + rng.uniform(-40, 40, (img, img))
        vol[z] = np.clip(np.rint(s), 0, 255).astype(np.uint8)
    return np.ascontiguousarray(np.stack([vol[i:i + 3] for i in range(n)]))


def normalise(u8: torch.Tensor, mean: float = MEAN, std: float = STD) -> torch.Tensor:
    return (u8.float() / 255.0 - mean) / std


def linear_head(c_in: int, c_out: int, seed: int) -> tuple[np.ndarray, np.ndarray]:
    rng = np.random.default_rng(seed)
    return rng.normal(0, np.sqrt(1.0 / c_in), (c_out, c_in)), rng.normal(0, 0.1, c_out)
