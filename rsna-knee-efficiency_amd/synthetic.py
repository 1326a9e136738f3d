"""Seeded synthetic inputs of the benchmark configurations (there is no dataset offline).

- `study_u8(n, img, seed)`: n slice stacks of 3 x img x img uint8 from one synthetic volume of n + 2
  slices (stack i = slices i, i+1, i+2, the reference's 3-slice windows, `src/knee/models/baseline.py:
  154-164`): a smooth low-frequency field of Gaussian blobs drifting from slice to slice, plus uniform
  noise.
- `c5_study(s)`: study s of configuration 5 (two crops of 24 stacks, seeded 1234 + s).
- `normalise(u8)`: x = (u / 255 - mean) / std as float32 (mean 0.5, std 0.25): the float model's input;
  the INT8 encoder applies the same map in its stem through an fp16 table.
- `linear_head(c_in, c_out, seed)`: the 1664 -> 8 head of configuration 4 (float64 weights, bias).
- `c2_case(S, c_in)` / `c3_case(S)`: the isolated kernels of configurations 2 and 3 at batch 24 with
  the distributions and seeds of the benchmark's definition: int8 activations from N(0, 1) quantised
  per tensor (seed 11 for the 1 x 1 GEMM, 21 for the 3 x 3 conv), int8 weights per output channel
  from N(0, 2 / K) (seeds 12 and 22), BatchNorms with the configuration-1 distributions, and scales
  calibrated on the data as the encoder's plan calibrates them; arrays in the kernels' layouts.
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


# --- isolated kernels (configurations 2 and 3) ------------------------------------------------
# (side, C_in) of configuration 2 and the block input width at each side (DenseNet169 at 512 px)
C2_CASES = ((128, 64), (128, 160), (128, 224), (64, 128), (64, 320), (64, 480),
            (32, 256), (32, 768), (32, 1248), (16, 640), (16, 1152), (16, 1632))
C0_AT = {128: 64, 64: 128, 32: 256, 16: 640}
C3_SIDES = (128, 64, 32, 16)
SAMPLE_PX = 4096                 # pixels the synthetic scales are calibrated on


def int8_activations(shape: tuple, seed) -> tuple[np.ndarray, float]:
    """x ~ N(0, 1) quantised per tensor: q = RNE(clamp(x / s, +-127)), s = max|x| / 127."""
    x = np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)
    s = float(np.abs(x).max()) / 127
    return np.clip(np.rint(x / s), -127, 127).astype(np.int8), s


def int8_weights(cout: int, k: int, seed) -> tuple[np.ndarray, np.ndarray]:
    """w ~ N(0, 2 / k) [cout][k], int8 per output channel in float32 arithmetic (scale = max|w| / 127,
    q = RNE(w / scale)): the encoder's weight quantisation."""
    w = np.random.default_rng(seed).normal(0, np.sqrt(2.0 / k), (cout, k)).astype(np.float32)
    scale = np.maximum(np.abs(w).max(1), np.float32(1e-12)) / np.float32(127)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    return np.clip(np.rint(w * inv[:, None]), -128, 127).astype(np.int8), scale.astype(np.float32)


def batchnorm_affine(c: int, rng) -> tuple[np.ndarray, np.ndarray]:
    """An eval BatchNorm of the configuration-1 distributions (gamma U(0.8, 1.2), beta N(0, 0.1), mean
    N(0, 0.1), var U(0.5, 1.5)) as y = a x + b."""
    gamma, beta = rng.uniform(0.8, 1.2, c), rng.normal(0, 0.1, c)
    mean, var = rng.normal(0, 0.1, c), rng.uniform(0.5, 1.5, c)
    a = gamma / np.sqrt(var + 1e-5)
    return a, beta - mean * a


def _u8_input(q: np.ndarray, s: float, a: np.ndarray, b: np.ndarray, axis: int) -> tuple[np.ndarray, float]:
    """The u8 conv input of int8 activations q (scale s) through BN (a, b) and ReLU, on the scale
    s1 = max(relu(bn(x))) / 255 (the encoder's per-tensor input scale): (u, s1), u = RNE(y / s1)."""
    shp = [1] * q.ndim
    shp[axis] = -1
    y = np.maximum(a.reshape(shp) * (q.astype(np.float64) * s) + b.reshape(shp), 0.0)
    s1 = max(float(y.max()), 1e-12) / 255
    return np.clip(np.rint(y / s1), 0, 255).astype(np.uint8), s1


def c2_case(S: int, c_in: int, n: int = 24, seeds=(11, 12, 13)) -> dict:
    """Configuration 2's case (S, c_in): n images of S x S pixels, c_in store channels (the block input
    width `C0_AT[S]` in `in0`, the rest in layer slots of `seg`), 128 outputs.  Activations seed
    seeds[0], weights seeds[1], the two BatchNorms (norm1 before the GEMM, norm2 after it) seeds[2];
    the prologue table maps the store's bytes through norm1 + ReLU to u8 on the data's scale, the
    epilogue table through norm2 + ReLU to the u8 bottleneck on the scale of its maximum over
    `SAMPLE_PX` pixels.  Arrays: in0 [n][G0][HW][32], seg [G - G0][n][HW][32] int8 (at least one
    slot), abh [c_in / 2][4] fp16 bits, w1 [G][128][32] int8, gdu [128][2] float32, w1sum [128]
    int32; q [n][c_in][HW] (channel-major, for checks) and the float tables."""
    hw = S * S
    q, s = int8_activations((n, c_in, hw), [seeds[0], S, c_in])
    w, wscale = int8_weights(128, c_in, [seeds[1], S, c_in])
    rng = np.random.default_rng([seeds[2], S, c_in])
    a1, b1 = batchnorm_affine(c_in, rng)
    g2, t2 = batchnorm_affine(128, rng)
    pick = np.random.default_rng([seeds[2], S, c_in, 1]).choice(n * hw, min(SAMPLE_PX, n * hw), replace=False)
    qs = q.transpose(0, 2, 1).reshape(n * hw, c_in)[pick]                     # [P][c_in]
    u, s1 = _u8_input(qs, s, a1, b1, axis=1)
    ab = np.stack([a1 * s / (255 * s1), b1 / (255 * s1)], 1).astype(np.float32)
    w = np.where((g2 < 0)[:, None], -w.astype(np.int16), w.astype(np.int16)).astype(np.int8)
    w1s = wscale.astype(np.float64) * np.abs(g2)
    y = np.maximum(u.astype(np.float64) @ w.astype(np.float64).T * (w1s * s1) + t2, 0.0)
    s2u = max(float(y.max()), 1e-12) / 255
    gdu = np.stack([w1s * s1 / (255 * s2u), t2 / (255 * s2u)], 1).astype(np.float32)
    g = c_in // 32
    g0 = min(C0_AT.get(S, c_in), c_in) // 32
    groups = q.reshape(n, g, 32, hw).transpose(0, 1, 3, 2)                   # [n][G][HW][32]
    in0 = np.ascontiguousarray(groups[:, :g0])
    seg = (np.ascontiguousarray(groups[:, g0:].transpose(1, 0, 2, 3)) if g > g0
           else np.zeros((1, n, hw, 32), np.int8))
    h = ab.astype(np.float16).reshape(-1, 2, 2)
    abh = np.ascontiguousarray(np.swapaxes(h, 1, 2).reshape(-1, 4)).view(np.int16)
    w1 = np.ascontiguousarray(np.swapaxes(w.reshape(128, g, 32), 0, 1))
    return {"S": S, "N": n, "G0": g0, "G": g, "in0": in0, "seg": seg, "q": q, "ab": ab, "abh": abh,
            "w": w, "w1": w1, "gdu": gdu, "w1sum": w1.astype(np.int64).sum(axis=(0, 2)).astype(np.int32)}


def c3_case(S: int, n: int = 24, seeds=(21, 22, 23)) -> dict:
    """Configuration 3's case at side S: n images of S x S, 128 -> 32 channels.  The 128 input channels
    are int8 activations (seed seeds[0]) through a BatchNorm (seeds[2]) and ReLU to the u8 bottleneck
    (`_u8_input`), the weights int8 per output channel from N(0, 2 / 1152) (seeds[1]), and the
    requantisation scale per output channel maps the maximum |acc| over `SAMPLE_PX` pixels to 127 (the
    store's per-channel scale).  Arrays: v [n][128][S][S] uint8, bott [4][n * S * S][32] uint8 (planar),
    w2 [32][128][3][3] int8, w2k [4][9][32][32] int8, c2u [32] float32, w2sum [32] int32."""
    hw = S * S
    q, s = int8_activations((n, 128, S, S), [seeds[0], S])
    rng = np.random.default_rng([seeds[2], S])
    a, b = batchnorm_affine(128, rng)
    v, _ = _u8_input(q, s, a, b, axis=1)
    w2, _ = int8_weights(32, 1152, [seeds[1], S])
    w2 = w2.reshape(32, 128, 3, 3)
    bott = np.ascontiguousarray(v.reshape(n, 4, 32, hw).transpose(1, 0, 3, 2)).reshape(4, n * hw, 32)
    w2k = np.ascontiguousarray(w2.reshape(32, 4, 32, 9).transpose(1, 3, 0, 2))
    # |acc| over sampled output pixels (3 x 3 windows, zero padding)
    pr = np.random.default_rng([seeds[2], S, 1])
    P = min(SAMPLE_PX, n * hw)
    img, pix = pr.integers(0, n, P), pr.integers(0, hw, P)
    y, x = pix // S, pix % S
    vp = np.pad(v, ((0, 0), (0, 0), (1, 1), (1, 1)))
    win = np.stack([vp[img, :, y + dy, x + dx] for dy in range(3) for dx in range(3)], 2)   # [P][128][9]
    acc = win.reshape(P, -1).astype(np.float64) @ w2.reshape(32, -1).astype(np.float64).T
    c2u = (127.0 / np.maximum(np.abs(acc).max(0), 1.0)).astype(np.float32)
    return {"S": S, "N": n, "v": v, "bott": bott, "w2": w2, "w2k": w2k, "c2u": c2u,
            "w2sum": w2k.astype(np.int64).sum(axis=(0, 1, 3)).astype(np.int32)}
