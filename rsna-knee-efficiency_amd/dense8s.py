"""The INT8 DenseNet encoder on gfx950: plan, tables, package format and the runner.

Host side of the reference's `src/knee/dense8s.py` (interface `Dense8SEncoder`, `:944-1651`), with the
arithmetic on the HIP kernels of `libd8s_hip.so` (`hip.py`, C ABI `include/d8s_hip.h`):

- `calibrate(encoder, batches)`: per-channel maxima of every store segment and per-tensor maxima of
  every conv input, by walking the float network (`observe`) with the maxima kept on the device
  (the role of `dense8s.py:272-318`);
- `make_plan(encoder, cal, img)`: BatchNorm as affines, int8 weights per output channel with the sign
  of norm2 folded into conv1 (`fold_norm2`), scales; one helper per layer and per transition (the
  role of `dense8s.py:374-433`, with the arithmetic of `dense8.py:176-188`);
- `kernel_params(plan)`: the kernel tables, float64 expressions cast once to float32 / fp16
  (`dense8s.py:436-519`); `derived_params` adds the tables only this build's kernels use;
- `pack_meta` / `save_pack` / `load_pack`: the `.npz` package (format 1, kind "dense8s",
  `dense8s.py:810-863`, `dense8.py:597-603`);
- `Dense8SEncoder(pack, dev, n_total, max_inflight)`: the runner, same constructor, attributes and
  methods as the reference's (`__call__`, `capture`, `graph_in_buf`, `store`, `trace`, `profile`,
  `time_layers`).

Quantisation (as the reference's final path: fp16 prologues everywhere, u8 bottleneck, our conv2):
  store      q = RNE(x / sigma_c), sigma_c = max|x_c| / 127 per channel (calibration);
  conv input u = RNE(255 sat(fp16(A q + B))), A = a sigma / (255 s), B = b / (255 s), s = amax / 255;
  bottleneck v = RNE(255 sat(g acc + d)) (u8, scale s2u = amax / 255);
  conv2      q = RNE(clamp(acc c2u, +-127)), c2u = s2u w2s / sigma;
  transition q' = RNE(clamp(k' acc_mean, +-127)), k' = ts tws / sigma' (mean of the 2x2 square first);
  final      f = mean relu(a5 sigma q + b5).
"""
from __future__ import annotations

import collections
import ctypes
import itertools
import json
import time
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

from . import hip

QU = 255                        # u8 inputs of the kernels
QS = 127                        # the store
GROUP = 32                      # channels per store group = growth rate
GROWTH = 32
BOTTLENECK = 128
PACK_FORMAT = 1
KIND = "dense8s"
STEM_C = 64


# --- calibration ----------------------------------------------------------------------------
class RunningMax:
    """Maxima of |x| over the calibration batches, kept on the tensors' device until `result()` (one
    host transfer in all, not one per layer and batch): per channel for what goes into the store (a
    block input, a layer's 32 new channels: their int8 scales sigma_c), per tensor for what a conv
    reads (its u8 scale).  The maximum is exact in any order, so the values do not depend on the
    batching."""

    def __init__(self) -> None:
        self.channel: dict[str, torch.Tensor] = {}
        self.tensor: dict[str, torch.Tensor] = {}

    @staticmethod
    def _merge(table: dict, key: str, m: torch.Tensor) -> None:
        old = table.get(key)
        table[key] = m if old is None else torch.maximum(old, m)

    def per_channel(self, key: str, y: torch.Tensor) -> None:
        self._merge(self.channel, key, y.detach().float().abs().amax(dim=(0, 2, 3)))

    def per_tensor(self, key: str, y: torch.Tensor) -> None:
        self._merge(self.tensor, key, y.detach().float().abs().amax())

    def result(self) -> dict:
        out: dict = {k: v.cpu().double().numpy().tolist() for k, v in self.channel.items()}
        out.update({k: float(v.cpu()) for k, v in self.tensor.items()})
        return out


def dense_stages(features) -> list[tuple]:
    """(dense block, the transition after it or None) in network order, from the timm / torchvision
    child names `denseblock{k}` / `transition{k}` of `features`."""
    kids = dict(features.named_children())
    stages = []
    while f"denseblock{len(stages) + 1}" in kids:
        k = len(stages) + 1
        stages.append((kids[f"denseblock{k}"], kids.get(f"transition{k}")))
    return stages


def observe(features, x: torch.Tensor, rec: RunningMax) -> None:
    """The float forward of `features` on x, recording at the points where the INT8 path quantises:
    `seg0.{b}` block b's input (pool0 / the transition's pooled output, per channel), `conv2.{b}.{l}`
    layer l's new channels (per channel), and per tensor the conv inputs `in1.{b}.{l}` (after norm1 +
    ReLU), `in2.{b}.{l}` (after norm2 + ReLU) and `tin.{b}` (the transition's after its norm + ReLU).
    It calls the modules a `densenet.DenseNet` forward calls, in the same order, so the recorded
    values are the float model's own; the ReLU is applied as a function, which also suits norms that
    already include their activation (applying it twice changes nothing)."""
    y = features.pool0(F.relu(features.norm0(features.conv0(x))))
    rec.per_channel("seg0.0", y)
    for b, (block, trans) in enumerate(dense_stages(features)):
        feats = [y]
        for l, layer in enumerate(block.values()):
            z = F.relu(layer.norm1(torch.cat(feats, 1)))
            rec.per_tensor(f"in1.{b}.{l}", z)
            z = F.relu(layer.norm2(layer.conv1(z)))
            rec.per_tensor(f"in2.{b}.{l}", z)
            feats.append(layer.conv2(z))
            rec.per_channel(f"conv2.{b}.{l}", feats[-1])
        y = torch.cat(feats, 1)
        if trans is not None:
            z = F.relu(trans.norm(y))
            rec.per_tensor(f"tin.{b}", z)
            y = trans.pool(trans.conv(z))
            rec.per_channel(f"seg0.{b + 1}", y)


@torch.inference_mode()
def calibrate(encoder, batches) -> dict:
    """The maxima the INT8 plan is scaled by, over `batches` (tensors (N, in, H, W) on the device of
    the float encoder, a `densenet.DenseNet`): keys `seg0.{b}` and `conv2.{b}.{l}` (lists, one value
    per channel), `in1.{b}.{l}`, `in2.{b}.{l}` and `tin.{b}` (numbers) -- the calibration dictionary
    of the reference (`src/knee/dense8s.py:272-318`), computed by walking the network (`observe`)."""
    rec = RunningMax()
    for x in batches:
        observe(encoder.features, x, rec)
    return rec.result()


# --- plan -----------------------------------------------------------------------------------
@dataclass
class SLayer:
    c_in: int
    a1: np.ndarray              # norm1 as an affine [c_in] (float64)
    b1: np.ndarray
    s1: float                   # u8 scale of the conv1 input
    w1: np.ndarray              # int8 [128, c_in], sign of norm2 inside
    w1s: np.ndarray             # [128] > 0: weight scale times |a2|
    bias1: np.ndarray           # [128] = b2 of norm2
    s2: float                   # int8 scale of the conv2 input (amax / 127)
    w2: np.ndarray              # int8 [32, 128, 3, 3]
    w2s: np.ndarray             # [32]
    sig: np.ndarray             # [32] per-channel scale of the output in the store


@dataclass
class SBlock:
    c0: int
    h: int
    w: int
    sig0: np.ndarray            # [c0] per-channel scale of the block input
    layers: list[SLayer]
    ta: np.ndarray | None = None        # transition: norm as an affine [c_tot]
    tb: np.ndarray | None = None
    ts: float | None = None             # u8 scale of the transition conv input
    tw: np.ndarray | None = None        # int8 [c_tot // 2, c_tot]
    tws: np.ndarray | None = None       # [c_tot // 2]

    @property
    def c_tot(self) -> int:
        return self.c0 + GROWTH * len(self.layers)

    @property
    def sig_all(self) -> np.ndarray:
        return np.concatenate([self.sig0] + [L.sig for L in self.layers])


@dataclass
class SPlan:
    img: int
    in_ch: int
    w0: np.ndarray              # stem with norm0 folded in, float32 [64, in_ch, 7, 7]
    b0: np.ndarray
    blocks: list[SBlock] = field(default_factory=list)
    a5: np.ndarray | None = None
    b5: np.ndarray | None = None

    @property
    def n_features(self) -> int:
        return self.blocks[-1].c_tot


def bn_affine(bn) -> tuple[np.ndarray, np.ndarray]:
    """An eval-mode BatchNorm as y = s x + t per channel, in float64: s = gamma / sqrt(var + eps),
    t = beta - mean s (`src/knee/dense8.py:176-179`)."""
    as64 = lambda t: t.detach().to("cpu", torch.float64).numpy()  # noqa: E731
    s = as64(bn.weight) / np.sqrt(as64(bn.running_var) + bn.eps)
    return s, as64(bn.bias) - as64(bn.running_mean) * s


def quant_weight(w: torch.Tensor) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric int8 per output channel in float32 arithmetic: scale = max(max|w|, 1e-12) / 127 per
    row, q = RNE(w * (1 / scale)) clamped to int8 (`src/knee/dense8.py:182-188`).  Returns q (the
    weight's shape) and the scales."""
    w32 = w.detach().to("cpu", torch.float32).numpy()
    rows = w32.reshape(w32.shape[0], -1)
    scale = np.maximum(np.abs(rows).max(axis=1), np.float32(1e-12)) / np.float32(QS)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    q = np.clip(np.rint(rows * inv[:, None]), -128, 127).astype(np.int8)
    return q.reshape(w32.shape), scale.astype(np.float32)


def store_scale(v, floor: float = 1e-6) -> np.ndarray:
    """sigma = max(amax, floor) / 127 per channel: the store's int8 scale (`src/knee/dense8s.py:374-375`)."""
    return np.maximum(np.asarray(v, dtype=np.float64), floor) / QS


def _input_scale(amax, levels: int) -> float:
    """Scale of a conv input quantised to `levels` steps: max(amax, 1e-12) / levels."""
    return max(float(amax), 1e-12) / levels


def fold_norm2(q: np.ndarray, wscale: np.ndarray, g: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """conv1's output goes through norm2, y = g acc + t, before its ReLU.  The epilogue wants a
    positive factor, so each output row's sign of g moves into the row's weights (q_o -> -q_o where
    g_o < 0) and |g_o| into the row scale (wscale_o |g_o|).  A channel with |g_o| < 1e-30 is dead: its
    row is zeroed and keeps the bare weight scale.  q [cout, ...] int8, wscale [cout], g [cout]."""
    dead = np.abs(g) < 1e-30
    neg = g < 0
    rows = q.reshape(q.shape[0], -1).astype(np.int16)
    rows = np.where(neg[:, None], -rows, rows)
    rows[dead] = 0
    folded = rows.astype(np.int8)            # wraps like int8 arithmetic (|q| <= 127 in practice)
    wscale64 = wscale.astype(np.float64)
    return folded, np.where(dead, wscale64, wscale64 * np.abs(g))


def layer_plan(layer, c_in: int, cal: dict, tag: str) -> SLayer:
    """The plan of one dense layer (`tag` = "{block}.{layer}" in the calibration keys)."""
    if not hasattr(layer.norm2, "running_var"):
        raise ValueError(f"dense layer {tag}: norm2 has no running statistics (folded?): the "
                         f"unfolded model is needed")
    a1, b1 = bn_affine(layer.norm1)
    g2, t2 = bn_affine(layer.norm2)
    q1, ws1 = quant_weight(layer.conv1.weight)
    w1, w1s = fold_norm2(q1, ws1, g2)
    q2, ws2 = quant_weight(layer.conv2.weight)
    return SLayer(c_in=c_in, a1=a1, b1=b1, s1=_input_scale(cal[f"in1.{tag}"], QU), w1=w1, w1s=w1s,
                  bias1=t2, s2=_input_scale(cal[f"in2.{tag}"], QS), w2=q2,
                  w2s=ws2.astype(np.float64), sig=store_scale(cal[f"conv2.{tag}"]))


def transition_plan(blk: SBlock, trans, cal: dict, b: int) -> None:
    """Fills the transition fields of `blk` from the transition module after block b."""
    blk.ta, blk.tb = bn_affine(trans.norm)
    q, ws = quant_weight(trans.conv.weight)
    blk.tw, blk.tws = q.reshape(q.shape[0], -1), ws.astype(np.float64)
    blk.ts = _input_scale(cal[f"tin.{b}"], QU)


def make_plan(encoder, cal: dict, img: int) -> SPlan:
    """The plan of `encoder` (a `densenet.DenseNet` in eval, BatchNorms not folded) at img x img with
    the maxima `cal` of `calibrate`: the stem with norm0 folded into its weights, then per block its
    layers (`layer_plan`) and transition (`transition_plan`); the block sides halve at each transition
    (the role of `src/knee/dense8s.py:378-433`)."""
    f = encoder.features
    s0, t0 = bn_affine(f.norm0)
    conv0 = f.conv0.weight.detach().to("cpu", torch.float64).numpy()
    plan = SPlan(img=img, in_ch=conv0.shape[1], w0=(conv0 * s0[:, None, None, None]).astype(np.float32),
                 b0=t0.astype(np.float32))
    width, side = conv0.shape[0], img // 4
    sig_in = store_scale(cal["seg0.0"])
    for b, (block, trans) in enumerate(dense_stages(f)):
        layers = [layer_plan(layer, width + GROWTH * l, cal, f"{b}.{l}")
                  for l, layer in enumerate(block.values())]
        blk = SBlock(c0=width, h=side, w=side, sig0=sig_in, layers=layers)
        width = blk.c_tot
        if trans is not None:
            transition_plan(blk, trans, cal, b)
            sig_in = store_scale(cal[f"seg0.{b + 1}"])
            width, side = width // 2, side // 2
        plan.blocks.append(blk)
    plan.a5, plan.b5 = bn_affine(f.norm5)
    return plan


def chunked(w: np.ndarray) -> np.ndarray:
    """[cout, cin] -> [cin / 32, cout, 32]: each store group's 32 input channels contiguous per output."""
    cout, cin = w.shape
    return np.ascontiguousarray(np.swapaxes(w.reshape(cout, cin // GROUP, GROUP), 0, 1))


def abh_table(ab: np.ndarray) -> np.ndarray:
    """The prologue [c, 2] (A, B) as fp16 [c / 2, 4] (bits as int16): per channel pair p the row
    (A_2p, A_2p+1, B_2p, B_2p+1), one 8-byte load per two channels."""
    h = ab.astype(np.float16).reshape(-1, 2, 2)              # [pair][channel of the pair][A or B]
    return np.ascontiguousarray(np.swapaxes(h, 1, 2).reshape(-1, 4)).view(np.int16)


def abh_values(abh: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(A, B) per channel as float64 from an `abh_table`."""
    h = np.ascontiguousarray(abh).view(np.float16).astype(np.float64)
    return h[:, :2].reshape(-1), h[:, 2:].reshape(-1)


def stem_weights16(w: np.ndarray) -> np.ndarray:
    """Stem weights [64, 3, 7, 7] -> [64, 168] fp16, k = (channel * 7 + ky) * 8 + kx + 1, k % 8 = 0 zero
    (`src/knee/dense8s.py:522-530`)."""
    cout, cin, kh, kw = w.shape
    out = np.zeros((cout, cin, kh, kw + 1), np.float32)
    out[..., 1:] = w
    return np.ascontiguousarray(out.reshape(cout, -1).astype(np.float16))


def kernel_params(plan: SPlan) -> dict[str, np.ndarray]:
    """The tables of the final path (`src/knee/dense8s.py:457-519`), same names and expressions:
    - `L{b}_{l}_ab` [c_in, 2], `L{b}_{l}_abh` [c_in/2, 4]: conv1 prologue a sigma / (255 s1), b / (255 s1);
    - `L{b}_{l}_gdu` [128, 2]: conv1 epilogue into the u8 bottleneck (scale s2u = s2 127 / 255);
    - `L{b}_{l}_w1` [G, 128, 32] int8; `L{b}_{l}_w2k` [4, 9, 32, 32] int8 (input block, tap, output,
      input); `L{b}_{l}_c2u` [32] = s2u w2s / sigma;
    - `T{b}_ab`, `T{b}_abh`, `T{b}_w` [G, cout, 32] int8, `T{b}_gdf` [cout, 2] = (ts tws / sigma', 0);
    - `F_ab` [n_features, 2] = (a5 sigma, b5);
    - `S_w16` [64, 168] fp16, `S_bias` [64] = b0, `S_inv` [64] = 1 / sigma0.
    """
    out: dict[str, np.ndarray] = {}
    for bi, blk in enumerate(plan.blocks):
        sig = blk.sig_all
        for li, L in enumerate(blk.layers):
            s = sig[:L.c_in]
            out[f"L{bi}_{li}_ab"] = np.stack([L.a1 * s / (QU * L.s1),
                                              L.b1 / (QU * L.s1)], 1).astype(np.float32)
            out[f"L{bi}_{li}_abh"] = abh_table(out[f"L{bi}_{li}_ab"])
            out[f"L{bi}_{li}_w1"] = chunked(L.w1)
            s2u = L.s2 * QS / QU
            out[f"L{bi}_{li}_gdu"] = np.stack([L.w1s * L.s1 / (QU * s2u),
                                               L.bias1 / (QU * s2u)], 1).astype(np.float32)
            w2 = L.w2.reshape(GROWTH, 4, GROUP, 9)                 # [o, block, i, tap]
            out[f"L{bi}_{li}_w2k"] = np.ascontiguousarray(w2.transpose(1, 3, 0, 2))
            out[f"L{bi}_{li}_c2u"] = (s2u * L.w2s / L.sig).astype(np.float32)
        if blk.ta is not None:
            nxt = plan.blocks[bi + 1].sig0
            out[f"T{bi}_ab"] = np.stack([blk.ta * sig / (QU * blk.ts),
                                         blk.tb / (QU * blk.ts)], 1).astype(np.float32)
            out[f"T{bi}_abh"] = abh_table(out[f"T{bi}_ab"])
            out[f"T{bi}_w"] = chunked(blk.tw)
            out[f"T{bi}_gd"] = np.stack([0.25 * blk.ts * blk.tws / nxt,
                                         np.zeros_like(nxt)], 1).astype(np.float32)
            out[f"T{bi}_gdf"] = np.stack([blk.ts * blk.tws / nxt, np.zeros_like(nxt)],
                                         1).astype(np.float32)
    last = plan.blocks[-1]
    out["F_ab"] = np.stack([plan.a5 * last.sig_all, plan.b5], 1).astype(np.float32)
    s0 = plan.blocks[0].sig0
    out["S_w0"] = (plan.w0.astype(np.float64) / s0[:, None, None, None]).astype(np.float32)
    out["S_b0"] = (plan.b0.astype(np.float64) / s0).astype(np.float32)
    out["S_w16"] = stem_weights16(plan.w0)
    out["S_bias"] = plan.b0.astype(np.float32)
    out["S_inv"] = (1.0 / s0).astype(np.float32)
    return out


def input_lut(mean, std) -> np.ndarray:
    """[3, 256] fp16 bits of x = (u / 255 - mean_c) / std_c: the fused uint8 normalisation of the stem
    (with mean 0, std 1 it is the reference's u / 255 table, `src/knee/data/fused_uint8.py:735`)."""
    u = np.arange(256, dtype=np.float64) / 255.0
    m = np.asarray(mean, dtype=np.float64).reshape(-1, 1)
    s = np.asarray(std, dtype=np.float64).reshape(-1, 1)
    return np.ascontiguousarray(((u[None, :] - m) / s).astype(np.float16)).view(np.int16)


def needed_tables(meta: dict) -> list[str]:
    """The package tables the runner's kernels read (`par_<name>` of a package): per layer the conv1
    prologue, weights and epilogue and the conv2 weights and scale, per transition its prologue,
    weights and epilogue, the final norm and the fp16 stem's tables."""
    names = ["F_ab", "S_w16", "S_bias", "S_inv"]
    for bi, b in enumerate(meta["blocks"]):
        for li in range(b["L"]):
            names += [f"L{bi}_{li}_{k}" for k in ("abh", "w1", "gdu", "w2k", "c2u")]
        if b["trans"]:
            names += [f"T{bi}_{k}" for k in ("abh", "w", "gdf")]
    return names


def derived_params(meta: dict, par: dict, names_only: bool = False):
    """Tables this build's kernels need beyond the reference's, derived from the package tables (so a
    package with only the reference's tables loads too): per-output weight sums for the offset of the
    unsigned activations (`L*_w1sum`, `L*_w2sum`, `T*_wsum`, int32) and the input table `S_lut`.
    `names_only`: just their names.
    """
    if names_only:
        names = ["S_lut"]
        for bi, b in enumerate(meta["blocks"]):
            names += [f"L{bi}_{li}_{k}" for li in range(b["L"]) for k in ("w1sum", "w2sum")]
            if b["trans"]:
                names.append(f"T{bi}_wsum")
        return names
    out: dict[str, np.ndarray] = {}
    for bi, b in enumerate(meta["blocks"]):
        for li in range(b["L"]):
            w1 = par[f"L{bi}_{li}_w1"].astype(np.int64)           # [G, 128, 32]
            out[f"L{bi}_{li}_w1sum"] = w1.sum(axis=(0, 2)).astype(np.int32)
            w2 = par[f"L{bi}_{li}_w2k"].astype(np.int64)          # [4, 9, 32, 32]
            out[f"L{bi}_{li}_w2sum"] = w2.sum(axis=(0, 1, 3)).astype(np.int32)
        if b["trans"]:
            tw = par[f"T{bi}_w"].astype(np.int64)                 # [G, cout, 32]
            out[f"T{bi}_wsum"] = tw.sum(axis=(0, 2)).astype(np.int32)
    inp = meta.get("input", {})
    out["S_lut"] = input_lut(inp.get("mean", [0.0] * 3), inp.get("std", [1.0] * 3))
    return out


# --- package -------------------------------------------------------------------------------
RUNTIME_TABLES = ("_abh", "_w1", "_gdu", "_w2k", "_c2u", "_w", "_gdf")


def pack_meta(plan: SPlan, n: int, input_kind: str = "u8", mean=(0.5, 0.5, 0.5),
              std=(0.25, 0.25, 0.25)) -> dict:
    """Package metadata: format 1, kind "dense8s" (`src/knee/dense8s.py:810-830`).  `n` = images per
    pass (graph block); `input`: "u8" (raw slices, normalised in the stem with mean / std) or "f16"
    (already normalised fp16, the reference's input)."""
    if input_kind not in ("u8", "f16"):
        raise ValueError(f"input kind {input_kind!r}: expected 'u8' or 'f16'")
    blocks = [{"c0": b.c0, "h": b.h, "w": b.w, "L": len(b.layers), "trans": b.ta is not None}
              for b in plan.blocks]
    return {"format": PACK_FORMAT, "kind": KIND, "n": int(n), "img": plan.img,
            "in_ch": plan.in_ch, "kernels_sha": hip.source_sha(), "n_features": plan.n_features,
            "stem_c": int(plan.w0.shape[0]), "conv2": "ours", "stem": "hip", "conv2_int8": True,
            "stem_int8": False, "engines": [],
            "input": {"kind": input_kind, "mean": [float(v) for v in mean],
                      "std": [float(v) for v in std]},
            "blocks": blocks}


def pack_params(plan: SPlan) -> dict[str, np.ndarray]:
    par = kernel_params(plan)
    keep = ("F_ab", "S_w16", "S_bias", "S_inv")
    return {k: v for k, v in par.items() if k in keep or k.endswith(RUNTIME_TABLES)}


def make_pack(plan: SPlan, n: int, **kw) -> dict:
    """The package in memory, as `load_pack` returns it."""
    return {"meta": pack_meta(plan, n, **kw), "engines": {}, "par": pack_params(plan), "cubin": None}


def save_pack(path: Path, plan: SPlan, n: int, **kw) -> None:
    meta = pack_meta(plan, n, **kw)
    arrays = {"meta": np.frombuffer(json.dumps(meta).encode(), np.uint8)}
    arrays |= {f"par_{k}": v for k, v in pack_params(plan).items()}
    with open(path, "wb") as fh:
        np.savez(fh, **arrays)


def load_pack(path: Path) -> dict:
    """{"meta", "engines", "par", "cubin"} as `src/knee/dense8.py:597-603` (no pickles: numpy arrays
    and a JSON byte vector)."""
    with np.load(path, allow_pickle=False) as z:
        meta = json.loads(bytes(z["meta"]).decode())
        engines = {k[4:]: z[k].tobytes() for k in z.files if k.startswith("eng_")}
        par = {k[4:]: np.array(z[k]) for k in z.files if k.startswith("par_")}
        cubin = z["cubin"].tobytes() if "cubin" in z.files else None
    return {"meta": meta, "engines": engines, "par": par, "cubin": cubin}


def is_pack(pack: dict) -> bool:
    return isinstance(pack, dict) and pack.get("meta", {}).get("kind") == KIND


def validate_meta(meta: dict) -> None:
    """ValueError for a package this runner cannot run (`src/knee/dense8s.py:954-956,1121-1124`)."""
    if meta.get("kind") != KIND or meta.get("format") != PACK_FORMAT:
        raise ValueError(f"package {meta.get('kind')} format {meta.get('format')}, "
                         f"expected {KIND} {PACK_FORMAT}")
    if meta.get("conv2", "trt") != "ours":
        raise ValueError("package with TensorRT conv2 engines: only conv2 'ours' runs here")
    if int(meta.get("stem_c", STEM_C)) != STEM_C or int(meta.get("in_ch", 3)) != 3:
        raise ValueError(f"stem {meta.get('stem_c')} x {meta.get('in_ch')}: 64 channels of 3 "
                         f"inputs expected")
    img = int(meta["img"])
    if img % 4 or img < 8:
        raise ValueError(f"image side {img}: a multiple of 4 (>= 8) expected")
    if int(meta["n"]) < 1:
        raise ValueError(f"package batch {meta['n']} < 1")
    blocks = meta["blocks"]
    if not blocks or blocks[-1]["trans"] or any(not b["trans"] for b in blocks[:-1]):
        raise ValueError("blocks: every block but the last needs a transition")
    for bi, b in enumerate(blocks):
        if b["c0"] % GROUP:
            raise ValueError(f"block {bi}: c0 {b['c0']} not a multiple of {GROUP}")
        if b["trans"] and (b["h"] % 2 or b["w"] % 2):
            raise ValueError(f"block {bi}: odd side {b['h']} x {b['w']} before a transition")
    inp = meta.get("input", {"kind": "f16"})
    if inp.get("kind", "f16") not in ("u8", "f16"):
        raise ValueError(f"input kind {inp.get('kind')!r}")


# --- runner ----------------------------------------------------------------------------------
@dataclass
class GraphInput:
    """The static input buffer of captured graphs, shared by the runners of one GPU that take inputs
    of the same shape and type: the seeds of an ensemble encode the same images, so what one runner
    copied in is reused by the next (the role of the reference's shared graph inputs,
    `src/knee/dense8s.py:911-941`).  `source` is the tensor last copied in, kept alive so that its
    address and version still name those contents, `ident` its identity (`contents_id`), `copied` an
    event after that copy and `readers` the event after each runner's last replay that read the
    buffer.  Runners on different streams are ordered through them: a new copy waits for every
    reader, a reuse waits for the copy."""
    buf: torch.Tensor
    source: torch.Tensor | None = None
    ident: tuple | None = None
    copied: torch.cuda.Event | None = None
    readers: dict = field(default_factory=dict)

    def forget(self) -> None:
        """The buffer's contents no longer come from `source` (a capture, or a caller writing it)."""
        self.source = self.ident = None

    def load(self, x: torch.Tensor, n: int, stream) -> bool:
        """Makes buf[:n] hold x, ordered on `stream`: skips the copy when x is the last source, unchanged.
        Returns whether it copied."""
        ident = contents_id(x) + (n,)
        if ident == self.ident:
            if self.copied is not None:
                stream.wait_event(self.copied)
            return False
        for ev in self.readers.values():
            stream.wait_event(ev)
        self.readers.clear()
        self.buf[:n].copy_(x)
        self.source, self.ident = x, ident
        self.copied = _record_sync(stream)
        return True

    def read_by(self, runner, stream) -> None:
        self.readers[id(runner)] = _record_sync(stream)


_GRAPH_INPUTS: dict[tuple, GraphInput] = {}
_FRESH = itertools.count()


def graph_input(dev: int, shape: tuple, dtype) -> GraphInput:
    """The shared graph input of (GPU, shape, dtype), allocated on first use."""
    key = (dev, tuple(shape), dtype)
    gi = _GRAPH_INPUTS.get(key)
    if gi is None:
        gi = _GRAPH_INPUTS[key] = GraphInput(torch.zeros(shape, dtype=dtype, device=f"cuda:{dev}"))
    return gi


def contents_id(x: torch.Tensor) -> tuple:
    """What names the contents of x from one call to the next: its storage and place in it (storage
    address, data address, shape, strides) and the version counter shared by the tensors of that
    storage, which every in-place write bumps (`hip.written` too).  Tensors made in inference mode have
    no version counter: they get a fresh token, so their contents are always copied."""
    try:
        ver = x._version
    except RuntimeError:
        ver = ("fresh", next(_FRESH))
    return (x.untyped_storage().data_ptr(), x.data_ptr(), tuple(x.shape), tuple(x.stride()), ver)


class Layer(collections.namedtuple("Layer", "c1 c2 dense")):
    """The launches of one dense layer: conv1 and conv2 argument structs, and the fused layer's
    (`hip.DenseArgs`, None when the block runs the two launches)."""


# How a block's layers run: "conv" conv1 + conv2 per layer (d8s_conv1, d8s_conv2); "chain" conv1 of
# layer 0, then conv2 of each layer with conv1 of the next in one launch (d8s_conv2_conv1), conv2 of the
# last layer (L + 1 launches; the bottleneck alternates between two buffers); "tile" one fused launch per
# layer (d8s_dense, the reference's fused kind "tile"); "img" the whole block in one launch, a workgroup
# per image (d8s_dense_block, the reference's "img*" kinds); "parts" the whole block in one launch with
# every image split into row bands, a workgroup per band (d8s_dense_block_parts; "parts:K" for K bands,
# plain "parts" for as many as fill the chip).  The bytes are the same.
BLOCK_KINDS = ("conv", "chain", "tile", "img", "parts")
IMG_MAX_PX = 256                # d8s_dense_block: pixels per image
IMG_MAX_GROUPS = 64             # and groups read by the last layer
LDS_BYTES = 160 * 1024
PARTS_TABLES = 1792             # d8s_dense_block_parts: per-layer tables besides the prologue's


def parts_static_lds(pt: int) -> int:
    """Fixed LDS bytes of d8s_dense_block_parts with pt pixel tiles per band: conv2 weights, two
    prologue chunks, partial sums."""
    cg = 4 if pt == 8 else 8
    s2 = 1 if pt == 8 else 2 if pt == 4 else 4
    nred = 4 * 1024 if pt == 1 else max(1, (s2 - 1) * pt * 1024)
    return 36864 + 2 * cg * pt * 1024 + 4 * nred + 16


def img_fits(b: dict) -> bool:
    """Whether block `b` (meta) fits d8s_dense_block."""
    return b["h"] * b["w"] <= IMG_MAX_PX and b["c0"] // GROUP + b["L"] - 1 <= IMG_MAX_GROUPS


def parts_options(b: dict) -> list[int]:
    """Band counts d8s_dense_block_parts can split block `b`'s images into (increasing)."""
    groups = b["c0"] // GROUP + b["L"] - 1
    if groups > IMG_MAX_GROUPS:
        return []
    out = []
    for k in range(1, b["h"] + 1):
        r = b["h"] // k
        if b["h"] % k or r * b["w"] not in hip.PARTS_PIXELS:
            continue
        lds = (r + 2) * (b["w"] + 2) * 128 + PARTS_TABLES + groups * 128 + parts_static_lds(r * b["w"] // 32)
        if lds > LDS_BYTES:
            continue
        out.append(k)
    return out


def parts_for(b: dict, n: int, cus: int = 256) -> int | None:
    """The band count of block `b` at n images per pass: the most bands with n x bands <= cus
    workgroups (one workgroup per CU: its LDS), or None if no split fits."""
    fit = [k for k in parts_options(b) if n * k <= cus]
    return fit[-1] if fit else None


def _kind_name(kind) -> str:
    return str(kind).split(":", 1)[0]


def chain_fits(b: dict) -> bool:
    """Whether block `b` (meta) runs d8s_conv2_conv1: a map width it takes, whole 128-pixel tiles, at
    least two layers and the last layer's conv1 within its group limit."""
    return (b["w"] in hip.C21_WIDTHS and (b["h"] * b["w"]) % 128 == 0 and b["L"] >= 2
            and b["c0"] // GROUP + b["L"] - 1 <= hip.C21_MAX_GROUPS)


BAND_W = 128                    # d8s_dense runs its band form, faster than two launches, at this width
BAND_MAX_GROUPS = 16            # (the conv1 weights of the layer in LDS)


def band_fits(b: dict) -> bool:
    """Whether every layer of block `b` (meta) runs d8s_dense's band form at its best width."""
    return b["w"] == BAND_W and b["c0"] // GROUP + b["L"] - 1 <= BAND_MAX_GROUPS


def default_kind(b: dict, n: int, cus: int = 256) -> str:
    """The block kind of block `b` at n images per pass: "parts" (the whole block in one launch, images
    split into as many bands as fill the chip) where that takes 4 bands or more and the block either
    fits a workgroup per image (the 16 x 16 maps of a 24-image study: 0.31 ms against 0.49 ms on 24
    CUs) or splits into 8 bands (the 32 x 32 block of a 24-image study: one launch instead of 64
    latency-bound ones); "img" where a workgroup per image fits (at 96 images: its 96 workgroups leave
    room for a second encoder's pass on another stream, which 2-band launches of 192 did not); "tile"
    for 128-wide blocks (the fused layer's band form); "chain" where the block's 128-pixel tiles fill
    one round of three workgroups per CU to at least two thirds (the 32 x 32 block at 96 images: 0.82
    against 0.89 ms per pass; the 64 x 64 block at 24 images: 0.24 against 0.26 ms; at 96 images that
    block's four tiles per workgroup run slower chained than as two launches); else "conv"."""
    k = parts_for(b, n, cus)
    if k is not None and k >= 4 and (img_fits(b) or k >= 8):
        return f"parts:{k}"
    if img_fits(b):
        return "img"
    if band_fits(b):
        return "tile"
    tiles = n * b["h"] * b["w"] // 128
    if chain_fits(b) and 2 * cus < tiles <= 3 * cus:
        return "chain"
    return "conv"


def fused_blocks(meta: dict, fused=None, cus: int = 256) -> dict:
    """{block: kind} for every block.  `fused` None -> the default (`default_kind`); a dict {block:
    kind} (other blocks "conv"); an iterable of blocks -> "tile" for those."""
    nb = len(meta["blocks"])
    if fused is None:
        return {bi: default_kind(b, int(meta["n"]), cus) for bi, b in enumerate(meta["blocks"])}
    req = dict(fused) if isinstance(fused, dict) else {int(b): "tile" for b in fused}
    out = {bi: "conv" for bi in range(nb)}
    for bi, kind in req.items():
        bi = int(bi)
        if not 0 <= bi < nb:
            raise ValueError(f"fused block {bi}: the encoder has blocks 0..{nb - 1}")
        if _kind_name(kind) not in BLOCK_KINDS:
            raise ValueError(f"block kind {kind!r}: expected one of {BLOCK_KINDS}")
        if kind == "img" and not img_fits(meta["blocks"][bi]):
            raise ValueError(f"block {bi} does not fit the whole-block kernel")
        if kind == "chain" and not chain_fits(meta["blocks"][bi]):
            b = meta["blocks"][bi]
            raise ValueError(f"block {bi} ({b['h']} x {b['w']}, {b['L']} layers) does not run chained "
                             f"conv2 + conv1 launches (widths {hip.C21_WIDTHS}, H * W a multiple of 128)")
        if _kind_name(kind) == "parts":
            b = meta["blocks"][bi]
            k = int(kind.split(":", 1)[1]) if ":" in str(kind) else parts_for(b, int(meta["n"]), cus)
            if k is None or k not in parts_options(b):
                raise ValueError(f"block {bi} ({b['h']} x {b['w']}, {b['L']} layers) does not split into "
                                 f"{k} bands (options {parts_options(b)})")
            kind = f"parts:{k}"
        out[bi] = kind
    return out


def _cu_count(dev: int) -> int:
    """Compute units of GPU `dev` (256 on an MI355X; that figure when no GPU is visible, where the
    runner fails later anyway)."""
    if not torch.cuda.is_available():
        return 256
    return int(torch.cuda.get_device_properties(dev).multi_processor_count)


def _ptr(t: torch.Tensor | None) -> int:
    return 0 if t is None else int(t.data_ptr())


class Dense8SEncoder:
    """The INT8 encoder on GPU `dev`: `enc(x)` with x (N, 3, img, img) on that GPU, uint8 (package input
    "u8") or fp16 ("f16"); returns (N, n_features) float32 in its own buffer (valid until the next
    call).  Blocks of `nb` images per pass; N is padded up to a multiple of `nb`.  Interface of the
    reference's runner (`src/knee/dense8s.py:944-1488`): own stream, `max_inflight`, `capture(n)`,
    `graph_in_buf(n)`, `nb`, `graphs`, `calls`, `load_s`, `in_dtype`, `in_shape`, `stream`, `out`.
    `__call__(x, flip=True)` encodes the horizontally mirrored images; `flip="tta"` returns (2N, C): the N
    images, then the same images mirrored (flip TTA fused in the stem: no mirrored copy in memory).
    """

    def __init__(self, pack: dict, dev: int, n_total: int, max_inflight: int | None = None,
                 fused=None) -> None:
        t0 = time.perf_counter()
        meta = pack["meta"]
        validate_meta(meta)
        self.meta, self.dev = meta, int(dev)
        self.fused = fused_blocks(meta, fused, _cu_count(int(dev)))
        self.nb = int(meta["n"])
        self.n_out = -(-int(n_total) // self.nb) * self.nb
        self.max_inflight = max_inflight
        self.inflight: collections.deque = collections.deque()
        self.graphs: dict = {}
        self.calls = {"graph": 0, "plain": 0}
        self._pad: torch.Tensor | None = None
        self.lib = hip.library()
        self.library_version = hip.version()
        self.pack_sha = meta.get("kernels_sha")
        inp = meta.get("input", {"kind": "f16"})
        self.in_kind = hip.IN_U8 if inp.get("kind", "f16") == "u8" else hip.IN_F16
        self.in_dtype = torch.uint8 if self.in_kind == hip.IN_U8 else torch.float16
        self.in_shape = (self.nb, int(meta["in_ch"]), int(meta["img"]), int(meta["img"]))
        missing = [k for k in self._needed_tables() if k not in pack["par"]]
        if missing:
            raise ValueError(f"package tables missing: {missing[:4]}{'...' if len(missing) > 4 else ''}")
        d = f"cuda:{self.dev}"
        with torch.cuda.device(self.dev):
            self.stream = torch.cuda.Stream(self.dev)
            self._buffers(pack, d)
            self.out = torch.empty((self.n_out, meta["n_features"]), dtype=torch.float32, device=d)
        self.load_s = time.perf_counter() - t0

    # -- initialisation --
    def _buffers(self, pack: dict, d: str) -> None:
        meta, n = self.meta, self.nb
        blocks = meta["blocks"]
        par = dict(pack["par"])
        par.update(derived_params(meta, par))
        # two alternating arenas: block b reads arena b % 2, its transition writes the other one
        sizes, lay = [0, 0], []
        for bi, b in enumerate(blocks):
            hw = b["h"] * b["w"]
            in0 = n * (b["c0"] // GROUP) * hw * GROUP
            seg = b["L"] * n * hw * GROUP
            lay.append((bi % 2, in0))
            sizes[bi % 2] = max(sizes[bi % 2], in0 + seg)
        self.arenas = [torch.empty(max(s, 16), dtype=torch.int8, device=d) for s in sizes]
        self.arena_mb = round(sum(sizes) / 2**20, 1)
        self.in0 = [self.arenas[a].data_ptr() for a, _ in lay]
        self.seg = [self.arenas[a].data_ptr() + in0 for a, in0 in lay]
        hw_max = max(b["h"] * b["w"] for b in blocks)
        self.bott = torch.empty(n * BOTTLENECK * hw_max, dtype=torch.uint8, device=d)
        # "chain" blocks: conv2 of a layer reads one bottleneck while conv1 of the next writes the other
        hw_chain = [b["h"] * b["w"] for bi, b in enumerate(blocks) if self.fused[bi] == "chain"]
        self.bott2 = (torch.empty(n * BOTTLENECK * max(hw_chain), dtype=torch.uint8, device=d)
                      if hw_chain else None)
        dev = torch.device(d)
        # only the tables the kernels read go to the device (a reference package also carries the
        # tables of its TensorRT and int8-stem paths)
        used = set(needed_tables(meta)) | set(derived_params(meta, {}, names_only=True))
        self.par = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
                    for k, v in par.items() if k in used}
        self.out_dev = dev
        self._build_launches()

    def _needed_tables(self) -> list[str]:
        return needed_tables(self.meta)

    def _build_launches(self) -> None:
        """Argument structs of every launch of a pass (`src/knee/dense8s.py:1103-1152`)."""
        n, P = self.nb, lambda k: _ptr(self.par[k])  # noqa: E731
        meta = self.meta
        self.plan_l: list = []
        self.block_args: dict = {}                   # "img" / "parts" blocks: their launch
        self._tables: dict = {}                      # and their device layer tables
        self._sync: dict = {}                        # "parts" blocks: sync words and exchange rows
        for bi, b in enumerate(meta["blocks"]):
            hw, g0 = b["h"] * b["w"], b["c0"] // GROUP
            layers = []
            for li in range(b["L"]):
                bott = _ptr(self._bott_of(bi, li))
                c1 = hip.GemmArgs(self.in0[bi], self.seg[bi], P(f"L{bi}_{li}_w1"),
                                  P(f"L{bi}_{li}_abh"), P(f"L{bi}_{li}_gdu"), P(f"L{bi}_{li}_w1sum"),
                                  bott, g0, g0 + li, n, hw, b["w"], n * hw, BOTTLENECK, 0)
                c2 = hip.Conv2Args(bott, P(f"L{bi}_{li}_w2k"), P(f"L{bi}_{li}_c2u"),
                                   P(f"L{bi}_{li}_w2sum"), self.seg[bi] + li * n * hw * GROUP,
                                   n, b["h"], b["w"], 0)
                dn = None
                if self.fused[bi] == "tile":
                    dn = hip.DenseArgs(self.in0[bi], self.seg[bi], P(f"L{bi}_{li}_w1"),
                                       P(f"L{bi}_{li}_abh"), P(f"L{bi}_{li}_gdu"), P(f"L{bi}_{li}_w1sum"),
                                       P(f"L{bi}_{li}_w2k"), P(f"L{bi}_{li}_c2u"), P(f"L{bi}_{li}_w2sum"),
                                       self.seg[bi] + li * n * hw * GROUP, g0, g0 + li, n, b["h"],
                                       b["w"], 0)
                layers.append(Layer(c1, c2, dn))
            kind = _kind_name(self.fused[bi])
            if kind in ("img", "parts"):
                lps = (hip.LayerP * b["L"])()
                for li in range(b["L"]):
                    lps[li] = hip.LayerP(P(f"L{bi}_{li}_w1"), P(f"L{bi}_{li}_abh"), P(f"L{bi}_{li}_gdu"),
                                         P(f"L{bi}_{li}_w1sum"), P(f"L{bi}_{li}_w2k"), P(f"L{bi}_{li}_c2u"),
                                         P(f"L{bi}_{li}_w2sum"))
                table = torch.frombuffer(bytearray(bytes(lps)), dtype=torch.uint8).to(self.out_dev)
                self._tables[bi] = table
                if kind == "img":
                    self.block_args[bi] = hip.BlockArgs(self.in0[bi], self.seg[bi], _ptr(table), n,
                                                        b["h"], b["w"], g0, b["L"], 0)
                else:
                    k = int(self.fused[bi].split(":", 1)[1])
                    sync = torch.zeros(hip.parts_sync_words(n * k), dtype=torch.int32, device=self.out_dev)
                    xchg = torch.zeros(hip.parts_xchg_bytes(n * k, b["w"]), dtype=torch.uint8,
                                       device=self.out_dev)
                    self._sync[bi] = (sync, xchg)
                    self.block_args[bi] = hip.PartsArgs(self.in0[bi], self.seg[bi], _ptr(table),
                                                        _ptr(sync), _ptr(xchg), n, b["h"], b["w"], g0,
                                                        b["L"], k)
            trans = None
            if b["trans"]:
                cout = (b["c0"] + GROWTH * b["L"]) // 2
                trans = hip.GemmArgs(self.in0[bi], self.seg[bi], P(f"T{bi}_w"), P(f"T{bi}_abh"),
                                     P(f"T{bi}_gdf"), P(f"T{bi}_wsum"), self.in0[bi + 1], g0,
                                     g0 + b["L"], n, hw, b["w"], n * hw, cout, cout // GROUP)
            self.plan_l.append((layers, trans))
        img = int(meta["img"])
        self.stem_args = hip.StemArgs(0, P("S_lut"), P("S_w16"), P("S_bias"), P("S_inv"),
                                      self.in0[0], n, img, img, self.in_kind, 0, 0)

    def _bott_of(self, bi: int, li: int) -> torch.Tensor:
        """The bottleneck buffer of layer li of block bi (in "chain" blocks odd layers use the second)."""
        return self.bott2 if self.fused[bi] == "chain" and li % 2 else self.bott

    # -- one pass --
    @staticmethod
    def _mode(flip) -> int:
        """flip -> stem mode: False 0 (as is), True 1 (every image mirrored), "tta" 2 (flip-TTA pairs: a
        pass encodes nb/2 input images, then the same images mirrored)."""
        if isinstance(flip, str):
            if flip != "tta":
                raise ValueError(f"flip {flip!r}: expected False, True or 'tta'")
            return 2
        return 1 if flip else 0

    def _per_pass(self, mode: int) -> int:
        """Input images one pass of `nb` encoded images consumes."""
        return self.nb // 2 if mode == 2 else self.nb

    def _stem(self, x_ptr: int, mode: int, st: int) -> None:
        self.stem_args.x = x_ptr
        self.stem_args.flip = mode
        hip.check(self.lib.d8s_stem(ctypes.byref(self.stem_args), st), "d8s_stem")

    def _final(self, bi: int, f_ptr: int, st: int, n: int | None = None) -> None:
        b = self.meta["blocks"][bi]
        n = self.nb if n is None else n
        hip.check(self.lib.d8s_final(self.in0[bi], b["c0"] // GROUP, self.seg[bi], n,
                                     b["h"] * b["w"], _ptr(self.par["F_ab"]), f_ptr,
                                     self.meta["n_features"], st), "d8s_final")

    def _conv1(self, c1, st: int) -> None:
        hip.check(self.lib.d8s_conv1(ctypes.byref(c1), st), "d8s_conv1")

    def _conv2(self, c2, st: int) -> None:
        hip.check(self.lib.d8s_conv2(ctypes.byref(c2), st), "d8s_conv2")

    def _chain(self, c2, c1, st: int) -> None:
        hip.check(self.lib.d8s_conv2_conv1(ctypes.byref(c2), ctypes.byref(c1), st), "d8s_conv2_conv1")

    def _block(self, bi: int, st: int) -> None:
        args = self.block_args[bi]
        if isinstance(args, hip.PartsArgs):
            hip.check(self.lib.d8s_dense_block_parts(ctypes.byref(args), st), "d8s_dense_block_parts")
        else:
            hip.check(self.lib.d8s_dense_block(ctypes.byref(args), st), "d8s_dense_block")

    def sync_errors(self, clear: bool = True) -> int:
        """Waits that ran out in the "parts" blocks' launches so far (0: every result valid); reads the
        sync words on the runner's stream (a synchronisation) and clears the count when `clear`."""
        total = 0
        with torch.cuda.device(self.dev):
            self.stream.synchronize()
            for sync, _ in self._sync.values():
                total += int(sync[2].item())
                if clear:
                    sync[2].zero_()
            self.stream.synchronize()
        return total

    def _dense(self, d, st: int) -> None:
        hip.check(self.lib.d8s_dense(ctypes.byref(d), st), "d8s_dense")

    def _trans(self, t, st: int) -> None:
        hip.check(self.lib.d8s_transition(ctypes.byref(t), st), "d8s_transition")

    def _pass(self, x_ptr: int, f_ptr: int, mode: int = 0, events: list | None = None) -> None:
        """The launch sequence of one pass (`src/knee/dense8s.py:1354-1385`): stem, then per block
        conv1 / conv2 of every layer, the transition or the final features."""
        st = self.stream.cuda_stream
        mark = ((lambda tag: events.append((tag, _record(self.stream)))) if events is not None
                else (lambda tag: None))
        mark("start")
        self._stem(x_ptr, mode, st)
        mark("stem")
        for bi, (layers, trans) in enumerate(self.plan_l):
            if bi in self.block_args:
                self._block(bi, st)
                mark(f"block_{bi}")
                layers = ()
            if self.fused[bi] == "chain":
                self._conv1(layers[0].c1, st)
                mark(f"conv1_{bi}")
                for La, Lb in zip(layers, layers[1:]):
                    self._chain(La.c2, Lb.c1, st)
                    mark(f"chain_{bi}")
                self._conv2(layers[-1].c2, st)
                mark(f"conv2_{bi}")
                layers = ()
            for L in layers:
                if L.dense is not None:
                    self._dense(L.dense, st)
                    mark(f"dense_{bi}")
                    continue
                self._conv1(L.c1, st)
                mark(f"conv1_{bi}")
                self._conv2(L.c2, st)
                mark(f"conv2_{bi}")
            if trans is not None:
                self._trans(trans, st)
                mark(f"trans{bi}")
            else:
                self._final(bi, f_ptr, st)
                mark("final")

    def _padded(self, chunk: torch.Tensor, mode: int) -> torch.Tensor:
        """One pass worth of input images: `chunk` itself if full (copied if its data is not 16-byte
        aligned: the stem reads uint8 rows as dwords), else copied to the head of a buffer (the rest
        holds old images, whose outputs are computed and discarded)."""
        if chunk.shape[0] == self._per_pass(mode):
            return chunk if chunk.data_ptr() % 16 == 0 else chunk.clone()
        if self._pad is None:
            self._pad = torch.zeros((self.nb, *chunk.shape[1:]), dtype=self.in_dtype,
                                    device=f"cuda:{self.dev}")
        self._pad[:chunk.shape[0]].copy_(chunk)
        return self._pad

    def _enqueue(self, xf: torch.Tensor, mode: int) -> None:
        for i, chunk in enumerate(xf.split(self._per_pass(mode))):
            if self.max_inflight:
                while len(self.inflight) >= self.max_inflight:
                    self.inflight.popleft().synchronize()
            self._pass(self._padded(chunk, mode).data_ptr(), self.out[i * self.nb].data_ptr(), mode)
            if self.max_inflight:
                ev = torch.cuda.Event(blocking=True)
                ev.record(self.stream)
                self.inflight.append(ev)

    def _check_input(self, x: torch.Tensor, mode: int = 0) -> None:
        if x.dtype != self.in_dtype:
            raise ValueError(f"input {x.dtype}: this package takes {self.in_dtype}")
        if tuple(x.shape[1:]) != self.in_shape[1:]:
            raise ValueError(f"input {tuple(x.shape)}: expected (N, "
                             f"{', '.join(map(str, self.in_shape[1:]))})")
        if x.device != torch.device(f"cuda:{self.dev}"):
            raise ValueError(f"input on {x.device}, encoder on cuda:{self.dev}")
        if mode == 2 and self.nb % 2:
            raise ValueError(f"flip-TTA pairs need an even images-per-pass, the package has {self.nb}")
        k = self._per_pass(mode)
        if -(-x.shape[0] // k) * self.nb > self.n_out:
            raise ValueError(f"{x.shape[0]} images: the output holds {self.n_out} encoded images")

    def _result(self, n: int, mode: int) -> torch.Tensor:
        """The features of `n` input images: (n, C) views of `out`, or for flip-TTA (2n, C) with the n
        plain images first, then the n mirrored ones."""
        if mode != 2:
            return self.out[:n]
        k = self.nb // 2
        if n == k:
            return self.out[:self.nb]
        idx = torch.arange(n, device=self.out.device)
        rows = (idx // k) * self.nb + idx % k
        return self.out.index_select(0, torch.cat([rows, rows + k]))

    def capture(self, n: int, flip=False) -> float:
        """One HIP graph per pass over a batch of `n` input images (`src/knee/dense8s.py:1410-1433`);
        returns the seconds spent."""
        mode = self._mode(flip)
        k = self._per_pass(mode)
        n = -(-n // k) * k
        if n // k * self.nb > self.out.shape[0]:
            raise ValueError(f"graph for {n} images: the encoder does {self.nb} per pass, "
                             f"the output holds {self.out.shape[0]}")
        t = time.perf_counter()
        with torch.cuda.device(self.dev):
            shared = graph_input(self.dev, (n, *self.in_shape[1:]), self.in_dtype)
            static_in = shared.buf
            shared.forget()
            with torch.cuda.stream(self.stream):
                self.stream.wait_stream(torch.cuda.current_stream(self.dev))
                self._enqueue(static_in[:k], mode)
            self.stream.synchronize()
            self.inflight.clear()
            graphs = []
            for i, chunk in enumerate(static_in.split(k)):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=self.stream, capture_error_mode="thread_local"):
                    self._pass(chunk.data_ptr(), self.out[i * self.nb].data_ptr(), mode)
                graphs.append(g)
            self.stream.synchronize()
        self.graphs[(n, mode)] = (graphs, shared)
        return time.perf_counter() - t

    def _graphs_for(self, n: int, mode: int):
        gs = self.graphs.get((n, mode))
        if gs is None:
            k = -(-n // self._per_pass(mode))
            for (m_, md), (g_, s_) in sorted(self.graphs.items()):
                if md == mode and m_ >= k * self._per_pass(mode):
                    return g_[:k], s_
        return gs

    def graph_in_buf(self, n: int, flip=False) -> torch.Tensor | None:
        """The static input buffer `[:n]` of the graphs captured for `n` images, or None."""
        gs = self._graphs_for(n, self._mode(flip))
        return None if gs is None else gs[1].buf[:n]

    def __call__(self, x: torch.Tensor, flip=False) -> torch.Tensor:
        mode = self._mode(flip)
        self._check_input(x, mode)
        cur = torch.cuda.current_stream(self.dev)
        self.stream.wait_stream(cur)
        n = x.shape[0]
        with torch.cuda.device(self.dev), torch.cuda.stream(self.stream):
            gs = self._graphs_for(n, mode)
            if gs is not None:
                graphs, shared = gs
                buf = shared.buf[:n]
                if (x.data_ptr() == buf.data_ptr() and x.shape == buf.shape
                        and x.stride() == buf.stride()):
                    shared.forget()                  # the caller wrote the graph input itself
                elif shared.load(x, n, self.stream):
                    self.calls["copy"] = self.calls.get("copy", 0) + 1
                for g in graphs:
                    if self.max_inflight:
                        while len(self.inflight) >= self.max_inflight:
                            self.inflight.popleft().synchronize()
                    g.replay()
                    if self.max_inflight:
                        ev = torch.cuda.Event(blocking=True)
                        ev.record(self.stream)
                        self.inflight.append(ev)
                shared.read_by(self, self.stream)
                self.calls["graph"] += 1
            else:
                self._enqueue(x.contiguous(), mode)
                self.calls["plain"] += 1
            res = self._result(n, mode)
        hip.written(self.out)
        cur.wait_stream(self.stream)
        return res

    # -- diagnostics --
    def store(self, bi: int, j: int) -> torch.Tensor:
        """Store segment (bi, j) as a float tensor (nb, c, h, w) of integers (j = 0 block input, j >= 1
        output of layer j - 1), `src/knee/dense8s.py:1491-1508`."""
        b = self.meta["blocks"][bi]
        n, h, w = self.nb, b["h"], b["w"]
        hw, g0 = h * w, b["c0"] // GROUP
        a = self.arenas[bi % 2]
        if j == 0:
            off = self.in0[bi] - a.data_ptr()
            t = a[off:off + n * g0 * hw * GROUP].view(n, g0, hw, GROUP)
            return t.permute(0, 1, 3, 2).reshape(n, g0 * GROUP, h, w).float()
        off = self.seg[bi] - a.data_ptr() + (j - 1) * n * hw * GROUP
        t = a[off:off + n * hw * GROUP].view(n, hw, GROUP)
        return t.permute(0, 2, 1).reshape(n, GROUP, h, w).float()

    def bottleneck(self, bi: int, li: int = 0) -> torch.Tensor:
        """The planar bottleneck of the last conv1 run in block bi as uint8 (nb, 128, h, w)."""
        b = self.meta["blocks"][bi]
        n, h, w = self.nb, b["h"], b["w"]
        hw = h * w
        t = self._bott_of(bi, li)[:4 * n * hw * GROUP].view(4, n, hw, GROUP)
        return t.permute(1, 0, 3, 2).reshape(n, 4 * GROUP, h, w)

    @torch.no_grad()
    def trace(self, x: torch.Tensor, flip=False) -> tuple[dict, torch.Tensor]:
        """One pass over the first images stopping after every launch: the store {(block, j): tensor},
        the bottleneck {("bott", block, layer): tensor} and the features (`src/knee/dense8s.py:1510-1546`)."""
        mode = self._mode(flip)
        self._check_input(x, mode)
        xf = self._padded(x[:self._per_pass(mode)].contiguous(), mode)
        out: dict = {}
        st = self.stream.cuda_stream
        with torch.cuda.device(self.dev), torch.cuda.stream(self.stream):
            self.stream.wait_stream(torch.cuda.current_stream(self.dev))
            f = torch.zeros((self.nb, self.meta["n_features"]), dtype=torch.float32,
                            device=f"cuda:{self.dev}")
            self._stem(xf.data_ptr(), mode, st)
            for bi, (layers, trans) in enumerate(self.plan_l):
                self.stream.synchronize()
                out[(bi, 0)] = self.store(bi, 0).clone()
                if bi in self.block_args:                    # every layer in one launch
                    self._block(bi, st)
                    self.stream.synchronize()
                    for li in range(len(layers)):
                        out[(bi, li + 1)] = self.store(bi, li + 1).clone()
                    layers = ()
                if self.fused[bi] == "chain":                # conv2 of li and conv1 of li + 1 together
                    self._conv1(layers[0].c1, st)
                    for li, L in enumerate(layers):
                        self.stream.synchronize()
                        out[("bott", bi, li)] = self.bottleneck(bi, li).clone()
                        if li + 1 < len(layers):
                            self._chain(L.c2, layers[li + 1].c1, st)
                        else:
                            self._conv2(L.c2, st)
                        self.stream.synchronize()
                        out[(bi, li + 1)] = self.store(bi, li + 1).clone()
                    layers = ()
                for li, L in enumerate(layers):
                    if L.dense is not None:                  # no bottleneck in memory
                        self._dense(L.dense, st)
                    else:
                        self._conv1(L.c1, st)
                        self.stream.synchronize()
                        out[("bott", bi, li)] = self.bottleneck(bi, li).clone()
                        self._conv2(L.c2, st)
                    self.stream.synchronize()
                    out[(bi, li + 1)] = self.store(bi, li + 1).clone()
                if trans is not None:
                    self._trans(trans, st)
                else:
                    self._final(bi, f.data_ptr(), st)
            self.stream.synchronize()
        return out, f

    def profile(self, x: torch.Tensor, reps: int = 3, flip=False) -> dict:
        """GPU milliseconds per item (stem, conv1 / conv2 per block, transitions, final) of a pass of
        `nb` images, from HIP events between launches (`src/knee/dense8s.py:1548-1563`)."""
        mode = self._mode(flip)
        self._check_input(x, mode)
        xf = self._padded(x[:self._per_pass(mode)].contiguous(), mode)
        tot: dict[str, float] = collections.defaultdict(float)
        with torch.cuda.device(self.dev), torch.cuda.stream(self.stream):
            self.stream.wait_stream(torch.cuda.current_stream(self.dev))
            for r in range(reps + 1):
                ev: list = []
                self._pass(xf.data_ptr(), self.out.data_ptr(), mode, ev)
                self.stream.synchronize()
                if r == 0:
                    continue
                for (_, a), (tag, b) in zip(ev, ev[1:]):
                    tot[tag] += a.elapsed_time(b)
        return {k: round(v / reps, 4) for k, v in sorted(tot.items())}

    def time_families(self, x: torch.Tensor, reps: int = 5, flip=False) -> dict:
        """GPU milliseconds per pass of each kernel family (stem, conv1, conv2, trans, final): the
        family's launches of one pass, in pass order, recorded in a HIP graph `reps` times and replayed
        between events on the runner's stream.  Unlike `profile` no host gap between launches is
        counted, so the figure is the kernels' own time.  One eager pass first fills the arenas."""
        mode = self._mode(flip)
        self._check_input(x, mode)
        xf = self._padded(x[:self._per_pass(mode)].contiguous(), mode)
        st = self.stream.cuda_stream
        fams: dict[str, list] = {"stem": [lambda: self._stem(xf.data_ptr(), mode, st)],
                                 "conv1": [], "conv2": [], "chain": [], "dense": [], "block": [],
                                 "trans": [], "final": []}
        for bi, (layers, trans) in enumerate(self.plan_l):
            if bi in self.block_args:
                fams["block"].append(lambda b=bi: self._block(b, st))
                layers = ()
            if self.fused[bi] == "chain":
                fams["conv1"].append(lambda c=layers[0].c1: self._conv1(c, st))
                for La, Lb in zip(layers, layers[1:]):
                    fams["chain"].append(lambda a=La.c2, b=Lb.c1: self._chain(a, b, st))
                fams["conv2"].append(lambda c=layers[-1].c2: self._conv2(c, st))
                layers = ()
            for L in layers:
                if L.dense is not None:
                    fams["dense"].append(lambda d=L.dense: self._dense(d, st))
                    continue
                fams["conv1"].append(lambda c=L.c1: self._conv1(c, st))
                fams["conv2"].append(lambda c=L.c2: self._conv2(c, st))
            if trans is not None:
                fams["trans"].append(lambda t=trans: self._trans(t, st))
            else:
                fams["final"].append(lambda b=bi: self._final(b, self.out.data_ptr(), st))
        with torch.cuda.device(self.dev), torch.cuda.stream(self.stream):
            self.stream.wait_stream(torch.cuda.current_stream(self.dev))
            self._pass(xf.data_ptr(), self.out.data_ptr(), mode)
            out = {k: self._time(lambda fs=fs: [f() for f in fs], reps) for k, fs in fams.items() if fs}
        return {k: round(v, 4) for k, v in out.items()}

    def _time(self, fn, reps: int = 20) -> float:
        """ms per call of `fn` (launching on the runner's stream): a HIP graph of `reps` calls replayed
        once as warm-up and once under events (`src/knee/dense8s.py:1565-1581`)."""
        with torch.cuda.device(self.dev), torch.cuda.stream(self.stream):
            fn()
            self.stream.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=self.stream, capture_error_mode="thread_local"):
                for _ in range(reps):
                    fn()
            g.replay()
            e0 = _record(self.stream)
            g.replay()
            e1 = _record(self.stream)
            self.stream.synchronize()
        return e0.elapsed_time(e1) / reps

    def time_layers(self, reps: int = 20) -> dict:
        """ms of every conv1, conv2 and transition on the current store."""
        st = self.stream.cuda_stream
        out: dict = {}
        for bi, (layers, trans) in enumerate(self.plan_l):
            if bi in self.block_args:
                out[f"blk b{bi}"] = round(self._time(lambda b=bi: self._block(b, st), reps), 4)
                layers = ()
            if self.fused[bi] == "chain":
                out[f"c1 b{bi}l0"] = round(self._time(lambda c=layers[0].c1: self._conv1(c, st), reps), 4)
                for li, (La, Lb) in enumerate(zip(layers, layers[1:])):
                    out[f"cc b{bi}l{li}"] = round(self._time(lambda a=La.c2, b=Lb.c1: self._chain(a, b, st),
                                                             reps), 4)
                out[f"c2 b{bi}l{len(layers) - 1}"] = round(
                    self._time(lambda c=layers[-1].c2: self._conv2(c, st), reps), 4)
                layers = ()
            for li, L in enumerate(layers):
                if L.dense is not None:
                    out[f"dn b{bi}l{li}"] = round(self._time(lambda d=L.dense: self._dense(d, st), reps), 4)
                    continue
                out[f"c1 b{bi}l{li}"] = round(self._time(lambda c=L.c1: self._conv1(c, st), reps), 4)
                out[f"c2 b{bi}l{li}"] = round(self._time(lambda c=L.c2: self._conv2(c, st), reps), 4)
            if trans is not None:
                out[f"t{bi}"] = round(self._time(lambda t=trans: self._trans(t, st), reps), 4)
        return out


def encode_concurrent(calls) -> list[torch.Tensor]:
    """Several runners at once: `calls` = [(runner, x, flip), ...], every runner on its own stream, the
    caller's current stream joined after all of them.  The seeds of an ensemble read the same input and
    are independent, so one runner's small late-block layers overlap another's work.

    Each call is made with the runner's own stream current: an extra stream per call would share one
    of the device's few hardware queues with another runner, and an event recorded there would make
    that runner wait for everything queued before it.  Returns the runners' outputs (views, as
    `Dense8SEncoder.__call__`)."""
    if not calls:
        return []
    dev = calls[0][0].dev
    cur = torch.cuda.current_stream(dev)
    for enc, _, _ in calls:
        if enc.dev != dev:
            raise ValueError("encode_concurrent: runners on different GPUs")
        enc.stream.wait_stream(cur)
    outs = []
    for enc, x, flip in calls:
        with torch.cuda.stream(enc.stream):
            outs.append(enc(x, flip=flip))
    for enc, _, _ in calls:
        cur.wait_stream(enc.stream)
    return outs


class EncoderPair:
    """Two encoders of one geometry over the same input images -- the final model's two weight seeds
    on one study -- as ONE launch sequence: every step of a pass is a paired launch (`d8s_*_pair`)
    carrying both encoders' arguments, so the two passes' small late layers fill the chip together
    (the 16 x 16 whole block: 192 workgroups in about the time of 96) instead of overlapping by chance
    on two streams (`encode_concurrent`).  Each encoder's outputs are exactly what it gives alone.  The
    pair runs on the first encoder's stream and orders the second's around it.  Steps without a pair
    launch ("parts" blocks, the chained conv2 + conv1 launches of "chain" blocks, the final features)
    run as two launches in the same sequence."""

    def __init__(self, a: Dense8SEncoder, b: Dense8SEncoder):
        if a is b:
            raise ValueError("EncoderPair: the same encoder twice")
        if a.dev != b.dev:
            raise ValueError(f"EncoderPair: encoders on cuda:{a.dev} and cuda:{b.dev}")
        same = (a.nb == b.nb and a.n_out == b.n_out and a.in_dtype == b.in_dtype and a.in_shape == b.in_shape
                and a.fused == b.fused and len(a.meta["blocks"]) == len(b.meta["blocks"])
                and all(all(x[k] == y[k] for k in ("h", "w", "c0", "L"))
                        for x, y in zip(a.meta["blocks"], b.meta["blocks"])))
        if not same:
            raise ValueError("EncoderPair: the encoders differ in geometry, batch, input or block kinds")
        self.a, self.b = a, b
        self.lib = a.lib
        self.graphs: dict = {}
        self.calls = {"graph": 0, "plain": 0, "copy": 0}

    def _pass(self, x_ptr: int, fa: int, fb: int, mode: int) -> None:
        A, B, lib = self.a, self.b, self.lib
        st = A.stream.cuda_stream
        for e in (A, B):
            e.stem_args.x = x_ptr
            e.stem_args.flip = mode
        hip.check(lib.d8s_stem_pair(ctypes.byref(A.stem_args), ctypes.byref(B.stem_args), st), "d8s_stem_pair")
        for bi, ((la, ta), (lb, tb)) in enumerate(zip(A.plan_l, B.plan_l)):
            if bi in A.block_args:
                pa, pb = A.block_args[bi], B.block_args[bi]
                if isinstance(pa, hip.PartsArgs):
                    A._block(bi, st)
                    B._block(bi, st)
                else:
                    hip.check(lib.d8s_dense_block_pair(ctypes.byref(pa), ctypes.byref(pb), st),
                              "d8s_dense_block_pair")
                la = lb = ()
            if A.fused[bi] == "chain":                       # no pair launch of the chained kernel
                hip.check(lib.d8s_conv1_pair(ctypes.byref(la[0].c1), ctypes.byref(lb[0].c1), st),
                          "d8s_conv1_pair")
                for i in range(len(la) - 1):
                    A._chain(la[i].c2, la[i + 1].c1, st)
                    B._chain(lb[i].c2, lb[i + 1].c1, st)
                hip.check(lib.d8s_conv2_pair(ctypes.byref(la[-1].c2), ctypes.byref(lb[-1].c2), st),
                          "d8s_conv2_pair")
                la = lb = ()
            for La, Lb in zip(la, lb):
                if La.dense is not None:
                    hip.check(lib.d8s_dense_pair(ctypes.byref(La.dense), ctypes.byref(Lb.dense), st),
                              "d8s_dense_pair")
                    continue
                hip.check(lib.d8s_conv1_pair(ctypes.byref(La.c1), ctypes.byref(Lb.c1), st), "d8s_conv1_pair")
                hip.check(lib.d8s_conv2_pair(ctypes.byref(La.c2), ctypes.byref(Lb.c2), st), "d8s_conv2_pair")
            if ta is not None:
                hip.check(lib.d8s_transition_pair(ctypes.byref(ta), ctypes.byref(tb), st), "d8s_transition_pair")
            else:
                A._final(bi, fa, st)
                B._final(bi, fb, st)

    def _passes(self, xf: torch.Tensor, mode: int) -> None:
        A, B = self.a, self.b
        for i, chunk in enumerate(xf.split(A._per_pass(mode))):
            xc = A._padded(chunk, mode)
            self._pass(xc.data_ptr(), A.out[i * A.nb].data_ptr(), B.out[i * B.nb].data_ptr(), mode)

    def capture(self, n: int, flip=False) -> float:
        """One HIP graph per pair of passes over a batch of `n` input images; returns the seconds spent."""
        A, B = self.a, self.b
        mode = A._mode(flip)
        k = A._per_pass(mode)
        n = -(-n // k) * k
        if n // k * A.nb > A.out.shape[0]:
            raise ValueError(f"graph for {n} images: the encoders do {A.nb} per pass, "
                             f"the output holds {A.out.shape[0]}")
        t = time.perf_counter()
        with torch.cuda.device(A.dev):
            shared = graph_input(A.dev, (n, *A.in_shape[1:]), A.in_dtype)
            static_in = shared.buf
            shared.forget()
            with torch.cuda.stream(A.stream):
                A.stream.wait_stream(torch.cuda.current_stream(A.dev))
                A.stream.wait_stream(B.stream)
                self._passes(static_in[:k], mode)
            A.stream.synchronize()
            graphs = []
            for i, chunk in enumerate(static_in.split(k)):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=A.stream, capture_error_mode="thread_local"):
                    self._pass(chunk.data_ptr(), A.out[i * A.nb].data_ptr(), B.out[i * B.nb].data_ptr(), mode)
                graphs.append(g)
            A.stream.synchronize()
        self.graphs[(n, mode)] = (graphs, shared)
        return time.perf_counter() - t

    def _graphs_for(self, n: int, mode: int):
        gs = self.graphs.get((n, mode))
        if gs is None:
            k = -(-n // self.a._per_pass(mode))
            for (m_, md), (g_, s_) in sorted(self.graphs.items()):
                if md == mode and m_ >= k * self.a._per_pass(mode):
                    return g_[:k], s_
        return gs

    def __call__(self, x: torch.Tensor, flip=False) -> tuple[torch.Tensor, torch.Tensor]:
        """Both encoders' features of x: (outputs of the first, outputs of the second), as each
        encoder's `__call__` returns them."""
        A, B = self.a, self.b
        mode = A._mode(flip)
        A._check_input(x, mode)
        B._check_input(x, mode)
        cur = torch.cuda.current_stream(A.dev)
        A.stream.wait_stream(cur)
        A.stream.wait_stream(B.stream)
        n = x.shape[0]
        with torch.cuda.device(A.dev), torch.cuda.stream(A.stream):
            gs = self._graphs_for(n, mode)
            if gs is not None:
                graphs, shared = gs
                buf = shared.buf[:n]
                if x.data_ptr() == buf.data_ptr() and x.shape == buf.shape and x.stride() == buf.stride():
                    shared.forget()
                elif shared.load(x, n, A.stream):
                    self.calls["copy"] += 1
                for g in graphs:
                    g.replay()
                shared.read_by(self, A.stream)
                self.calls["graph"] += 1
            else:
                self._passes(x.contiguous(), mode)
                self.calls["plain"] += 1
            ra, rb = A._result(n, mode), B._result(n, mode)
        hip.written(A.out, B.out)
        B.stream.wait_stream(A.stream)
        cur.wait_stream(A.stream)
        return ra, rb


def _record_sync(stream) -> torch.cuda.Event:
    """An event without timing on `stream`: orders the shared graph input between runners' streams."""
    e = torch.cuda.Event()
    e.record(stream)
    return e


def _record(stream) -> torch.cuda.Event:
    e = torch.cuda.Event(enable_timing=True)
    e.record(stream)
    return e
