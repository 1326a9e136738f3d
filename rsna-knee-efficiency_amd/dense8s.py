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
import contextlib
import ctypes
import itertools
import json
import time
from dataclasses import dataclass, field, replace
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
    """What the INT8 path needs of one dense layer reading `c_in` store channels.

    conv1 side: norm1 as the float64 affine (a1, b1) over the c_in inputs and the u8 input scale s1;
    the int8 weights w1 [128, c_in] with norm2's sign folded into their rows (`fold_norm2`), w1s the
    positive per-row factor (weight scale times |norm2 gain|) and bias1 norm2's shift.  conv2 side:
    the int8 input scale s2, the int8 weights w2 [32, 128, 3, 3] with their per-row scales w2s, and
    sig, the store scale of the 32 channels the layer appends."""
    c_in: int
    a1: np.ndarray
    b1: np.ndarray
    s1: float
    w1: np.ndarray
    w1s: np.ndarray
    bias1: np.ndarray
    s2: float
    w2: np.ndarray
    w2s: np.ndarray
    sig: np.ndarray


@dataclass
class SBlock:
    """A dense block of `layers` on h x w maps whose input has c0 channels stored at scales sig0, and,
    for every block but the last, its transition: the norm affine (ta, tb) over all c_tot channels,
    the u8 input scale ts, the int8 1 x 1 weights tw [c_tot / 2, c_tot] and their row scales tws."""
    c0: int
    h: int
    w: int
    sig0: np.ndarray
    layers: list[SLayer]
    ta: np.ndarray | None = None
    tb: np.ndarray | None = None
    ts: float | None = None
    tw: np.ndarray | None = None
    tws: np.ndarray | None = None

    @property
    def c_tot(self) -> int:
        """Channels of the store after the last layer."""
        return self.c0 + GROWTH * len(self.layers)

    @property
    def sig_all(self) -> np.ndarray:
        """Store scale of every channel after the last layer, in store order."""
        return np.concatenate([self.sig0, *(layer.sig for layer in self.layers)])


@dataclass
class SPlan:
    """The whole encoder at img x img: the stem (w0 [64, in_ch, 7, 7] float32 with norm0's gain folded
    in, b0 its shift), the blocks, and the final norm as the affine (a5, b5)."""
    img: int
    in_ch: int
    w0: np.ndarray
    b0: np.ndarray
    blocks: list[SBlock] = field(default_factory=list)
    a5: np.ndarray | None = None
    b5: np.ndarray | None = None

    @property
    def n_features(self) -> int:
        """Length of the pooled feature vector (the last block's channels)."""
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
              std=(0.25, 0.25, 0.25), fused: dict | None = None, bm: dict | None = None,
              c2: dict | None = None, tbm: dict | None = None) -> dict:
    """Package metadata: format 1, kind "dense8s" (`src/knee/dense8s.py:810-830`).  `n` = images per
    pass (graph block); `input`: "u8" (raw slices, normalised in the stem with mean / std) or "f16"
    (already normalised fp16, the reference's input); `fused` {block: kind} (keys ints or "b{block}"):
    the block kinds to record, e.g. `Dense8SEncoder.tune_kinds`'s choice, which runners of the package
    then use (the reference's per-block "fused" field).  `bm` {"b{block}l{layer}": conv1 variant},
    `c2` {side: conv2 variant}, `tbm` {"t{block}": transition variant}: kernel variants to record
    (`C1_VARIANTS`, `C2_VARIANTS`, `TRANS_VARIANTS`; e.g. the fastest of `tune_bm`, `tune_c2`,
    `tune_trans`), kept per block as the reference's packages keep theirs ("bm" a list per layer, "c2",
    "tbm"; `src/knee/dense8s.py:818-826`)."""
    if input_kind not in ("u8", "f16"):
        raise ValueError(f"input kind {input_kind!r}: expected 'u8' or 'f16'")
    fused, bm, c2, tbm = fused or {}, bm or {}, c2 or {}, tbm or {}
    for table, names in ((bm, C1_VARIANTS), (c2, C2_VARIANTS), (tbm, TRANS_VARIANTS)):
        for key, name in table.items():
            if name not in names.values():
                raise ValueError(f"variant {name!r} for {key!r}: expected one of {sorted(names.values())}")
    blocks = [{"c0": b.c0, "h": b.h, "w": b.w, "L": len(b.layers), "trans": b.ta is not None,
               "fused": fused.get(bi) or fused.get(f"b{bi}"),
               "bm": [bm.get(f"b{bi}l{li}") for li in range(len(b.layers))],
               "c2": c2.get(b.h, c2.get(str(b.h))),
               "tbm": tbm.get(f"t{bi}") if b.ta is not None else None}
              for bi, b in enumerate(plan.blocks)]
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
        self.buf[:n].copy_(x)
        self.source, self.ident = x, ident
        if self.copied is None:
            self.copied = torch.cuda.Event()
        self.copied.record(stream)
        return True

    def read_by(self, runner, stream) -> None:
        """Marks the end of `runner`'s last replay reading the buffer (one event per runner, recorded
        again each time: a wait enqueued earlier keeps the record it saw)."""
        ev = self.readers.get(id(runner))
        if ev is None:
            ev = self.readers[id(runner)] = torch.cuda.Event()
        ev.record(stream)


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
# the reference's fused kinds (`src/knee/dense8s.py:174-176`) as this runner's: its whole-block kinds
# ("img3", "band2", "slide", "slide2": one image per thread block) are "img"; "tile" is "tile"
REFERENCE_KINDS = {"img3": "img", "band2": "img", "slide": "img", "slide2": "img", "tile": "tile"}


def block_groups(b: dict) -> int:
    """Store groups the last layer of block `b` (meta) reads."""
    return b["c0"] // GROUP + b["L"] - 1


def img_fits(b: dict) -> bool:
    """Whether block `b` (meta) fits d8s_dense_block."""
    return b["h"] * b["w"] <= IMG_MAX_PX and block_groups(b) <= IMG_MAX_GROUPS


def parts_options(b: dict) -> list[int]:
    """Band counts d8s_dense_block_parts can split block `b`'s images into (increasing): the library's
    own shape and LDS check (`d8s_parts_supported`)."""
    lib = hip.library()
    g = block_groups(b)
    return [k for k in range(1, b["h"] + 1) if lib.d8s_parts_supported(b["h"], b["w"], g, k)]


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
            and block_groups(b) <= hip.C21_MAX_GROUPS)


BAND_W = 128                    # d8s_dense runs its band form, faster than two launches, at this width
BAND_MAX_GROUPS = 16            # (the conv1 weights of the layer in LDS)


def band_fits(b: dict) -> bool:
    """Whether every layer of block `b` (meta) runs d8s_dense's band form at its best width."""
    return b["w"] == BAND_W and block_groups(b) <= BAND_MAX_GROUPS


# Kernel variants of the per-layer launches (include/d8s_hip.h, d8s_conv1_as / d8s_conv2_as /
# d8s_transition_as): id -> name.  Every variant writes the same bytes; 0 is the library's own choice.
C1_VARIANTS = {1: "p32", 2: "p64", 3: "k1", 4: "k2", 5: "k4"}
C2_VARIANTS = {1: "32x8", 2: "32x4", 3: "32x2", 4: "16x4", 5: "8x8", 6: "4x16", 7: "2x32", 8: "1x64"}
TRANS_VARIANTS = {1: "d4w2", 2: "d4w4", 3: "d2w2", 4: "d1w1"}
VARIANTS = {"conv1": C1_VARIANTS, "conv2": C2_VARIANTS, "trans": TRANS_VARIANTS}


def _variant_id(table: dict, name) -> int:
    for v, n in table.items():
        if n == name:
            return v
    return 0


def recorded_variants(meta: dict) -> dict:
    """The kernel variants a package records (per block "bm" per layer, "c2", "tbm", as the reference's
    packages record theirs, `kaggle/int8_pack/pack_dense8s.py:141-147`): {("conv1", block, layer) |
    ("conv2", block) | ("trans", block): variant id}.  Names of this library's variants only: the
    reference's kernel names (CUDA kernels, `src/knee/dense8s.py:818-826`) name nothing here and leave
    the library's choice."""
    out = {}
    for bi, b in enumerate(meta["blocks"]):
        bm = b.get("bm")
        if isinstance(bm, (list, tuple)):
            for li, name in enumerate(bm):
                if isinstance(name, str) and _variant_id(C1_VARIANTS, name):
                    out[("conv1", bi, li)] = _variant_id(C1_VARIANTS, name)
        for fam, key in (("conv2", "c2"), ("trans", "tbm")):
            name = b.get(key)
            if isinstance(name, str) and _variant_id(VARIANTS[fam], name):
                out[(fam, bi)] = _variant_id(VARIANTS[fam], name)
    return out


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


def valid_kind(b: dict, bi: int, kind, n: int, cus: int = 256) -> str:
    """`kind` for block `b` (meta, index bi) at n images per pass, checked and normalised ("parts" ->
    "parts:K"); ValueError if the block cannot run it."""
    name = _kind_name(kind)
    if name not in BLOCK_KINDS:
        raise ValueError(f"block kind {kind!r}: expected one of {BLOCK_KINDS}")
    if name == "img" and not img_fits(b):
        raise ValueError(f"block {bi} does not fit the whole-block kernel")
    if name == "chain" and not chain_fits(b):
        raise ValueError(f"block {bi} ({b['h']} x {b['w']}, {b['L']} layers) does not run chained "
                         f"conv2 + conv1 launches (widths {hip.C21_WIDTHS}, H * W a multiple of 128)")
    if name == "parts":
        k = int(str(kind).split(":", 1)[1]) if ":" in str(kind) else parts_for(b, n, cus)
        if k is None or k not in parts_options(b):
            raise ValueError(f"block {bi} ({b['h']} x {b['w']}, {b['L']} layers) does not split into "
                             f"{k} bands (options {parts_options(b)})")
        return f"parts:{k}"
    return name


def recorded_kind(b: dict, bi: int, n: int, cus: int = 256) -> str | None:
    """The kind a package records for block `b` (meta field "fused", as the reference's packages carry
    their tuned choice, `kaggle/int8_pack/pack_dense8s.py:141-147`), or None if it records none.  This
    runner's own kinds are checked (ValueError if the block cannot run them); the reference's kinds
    map onto this runner's (`REFERENCE_KINDS`), and a whole-block kind whose block does not fit one
    workgroup per image falls back to the default."""
    rec = b.get("fused")
    if not rec:
        return None
    if rec in REFERENCE_KINDS:
        mapped = REFERENCE_KINDS[rec]
        return mapped if mapped != "img" or img_fits(b) else None
    return valid_kind(b, bi, rec, n, cus)


def fused_blocks(meta: dict, fused=None, cus: int = 256) -> dict:
    """{block: kind} for every block.  `fused` None -> what the package records per block
    (`recorded_kind`), else the default (`default_kind`); a dict {block: kind} (other blocks "conv");
    an iterable of blocks -> "tile" for those."""
    nb, n = len(meta["blocks"]), int(meta["n"])
    if fused is None:
        out = {}
        for bi, b in enumerate(meta["blocks"]):
            rec = recorded_kind(b, bi, n, cus)
            out[bi] = rec if rec is not None else default_kind(b, n, cus)
        return out
    req = dict(fused) if isinstance(fused, dict) else {int(b): "tile" for b in fused}
    out = {bi: "conv" for bi in range(nb)}
    for bi, kind in req.items():
        bi = int(bi)
        if not 0 <= bi < nb:
            raise ValueError(f"fused block {bi}: the encoder has blocks 0..{nb - 1}")
        out[bi] = valid_kind(meta["blocks"][bi], bi, kind, n, cus)
    return out


def kind_options(b: dict, n: int) -> list[str]:
    """Every kind block `b` (meta) can run at n images per pass (what `Dense8SEncoder.tune_kinds` times)."""
    out = ["conv"]
    if chain_fits(b):
        out.append("chain")
    out.append("tile")              # d8s_dense takes any map (its band form at 64 and 128 wide)
    if img_fits(b):
        out.append("img")
    out += [f"parts:{k}" for k in parts_options(b)]
    return out


def _cu_count(dev: int) -> int:
    """Compute units of GPU `dev` (256 on an MI355X; that figure when no GPU is visible, where the
    runner fails later anyway)."""
    if not torch.cuda.is_available():
        return 256
    return int(torch.cuda.get_device_properties(dev).multi_processor_count)


def _ptr(t: torch.Tensor | None) -> int:
    return 0 if t is None else int(t.data_ptr())


class PartsWaitError(hip.D8sError):
    """A banded whole-block launch (d8s_dense_block_parts) had bounded waits that ran out: the features
    of the passes since the last check were written as NaN.  The runner has cleared the error words."""


class Regions:
    """One device allocation carved into aligned named regions: sizes are reserved first (byte offsets
    known before anything is allocated), then one tensor holds them all."""

    ALIGN = 256

    def __init__(self) -> None:
        self.spans: dict[str, tuple[int, int]] = {}
        self.size = 0
        self.mem: torch.Tensor | None = None

    def reserve(self, name: str, nbytes: int) -> None:
        start = -(-self.size // self.ALIGN) * self.ALIGN
        self.spans[name] = (start, int(nbytes))
        self.size = start + int(nbytes)

    def allocate(self, device) -> None:
        self.mem = torch.empty(max(self.size, self.ALIGN), dtype=torch.uint8, device=device)

    def __contains__(self, name: str) -> bool:
        return name in self.spans

    def addr(self, name: str, offset: int = 0) -> int:
        return self.mem.data_ptr() + self.spans[name][0] + offset

    def view(self, name: str, offset: int = 0, nbytes: int | None = None) -> torch.Tensor:
        start, size = self.spans[name]
        nbytes = size - offset if nbytes is None else nbytes
        return self.mem[start + offset:start + offset + nbytes]


@dataclass
class Step:
    """One launch of a pass.  `family` names the kernel family (stem, conv1, conv2, chain, dense,
    block, trans, final), `block` / `layer` where it sits (layer -1: the whole block or none), `makes`
    the trace keys whose contents it completes ((b, j): store segment j of block b, ("bott", b, l):
    layer l's bottleneck), `entry` the C entry point and `args` its argument struct (None for the
    stem's and the final's, whose pointers change per pass), `variant` the kernel variant of a conv1,
    conv2 or transition launch (0: the library's choice)."""
    family: str
    block: int
    layer: int
    makes: tuple
    entry: str
    args: object = None
    variant: int = 0

    def tag(self) -> str:
        return self.family if self.family in ("stem", "final") else f"{self.family}_{self.block}"

    def label(self) -> str:
        short = {"conv1": "c1", "conv2": "c2", "chain": "cc", "dense": "dn"}
        if self.family in short:
            return f"{short[self.family]} b{self.block}l{self.layer}"
        return {"block": f"blk b{self.block}", "trans": f"t{self.block}"}.get(self.family, self.family)


class InflightGate:
    """At most `limit` passes in flight on a stream (None: no limit): `admit()` blocks the host on the
    oldest pass's event while the limit is reached, `done(stream)` marks the end of a pass (the role of
    the reference's `max_inflight`, `src/knee/dense8s.py:1400-1408`)."""

    def __init__(self, limit: int | None) -> None:
        self.limit = limit
        self.events: collections.deque = collections.deque()

    def admit(self) -> None:
        while self.limit and len(self.events) >= self.limit:
            self.events.popleft().synchronize()

    def done(self, stream) -> None:
        if self.limit:
            ev = torch.cuda.Event(blocking=True)
            ev.record(stream)
            self.events.append(ev)

    def clear(self) -> None:
        self.events.clear()


class GraphBook:
    """Captured graphs by flip mode: for each mode, batch size -> (graphs, shared input).  A batch of n
    images replays the graphs captured for n, else the first ceil(n / per-pass) graphs of the smallest
    capture that covers them (a short batch: the rows past n hold old images, whose outputs are
    computed and discarded)."""

    def __init__(self) -> None:
        self.by_mode: dict[int, dict[int, tuple]] = {}

    def add(self, n: int, mode: int, graphs: list, shared: GraphInput) -> None:
        self.by_mode.setdefault(mode, {})[n] = (graphs, shared)

    def find(self, n: int, mode: int, per_pass: int):
        book = self.by_mode.get(mode, {})
        if n in book:
            return book[n]
        passes = -(-n // per_pass)
        covering = [m for m in book if m >= passes * per_pass]
        if not covering:
            return None
        graphs, shared = book[min(covering)]
        return graphs[:passes], shared

    def items(self):
        return [((n, mode), v) for mode, book in self.by_mode.items() for n, v in book.items()]

    def __len__(self) -> int:
        return sum(len(b) for b in self.by_mode.values())

    def __bool__(self) -> bool:
        return len(self) > 0

    def clear(self) -> None:
        self.by_mode.clear()


class _PassRunner:
    """What the runner and the pair share: a batch as passes of `nb` encoded images on one launch
    stream, eagerly or by replaying captured graphs, with the input shared between the runners of a GPU
    (`GraphInput`).  Subclasses give `_launch_pass(x_ptr, index, mode)` (the launches of pass `index`
    reading x_ptr), `_accept(x, mode)` (input checks), `_outputs(n, mode)` and `_mark_written()`."""

    def _mode(self, flip) -> int:
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

    def _staged(self, chunk: torch.Tensor, mode: int) -> int:
        """Address of one pass worth of input: the chunk itself when it is whole and 16-byte aligned (the
        stem reads uint8 rows as dwords), else a copy at the head of the staging buffer (whose other rows
        hold old images: their outputs are computed and discarded)."""
        if chunk.shape[0] == self._per_pass(mode) and chunk.data_ptr() % 16 == 0:
            return chunk.data_ptr()
        if self._staging is None:
            self._staging = torch.zeros(self.in_shape, dtype=self.in_dtype, device=f"cuda:{self.dev}")
        self._staging[:chunk.shape[0]].copy_(chunk)
        return self._staging.data_ptr()

    def _run_eager(self, x: torch.Tensor, mode: int) -> None:
        per = self._per_pass(mode)
        for index in range(-(-x.shape[0] // per)):
            self._gate.admit()
            self._launch_pass(self._staged(x[index * per:(index + 1) * per], mode), index, mode)
            self._gate.done(self.stream)

    def _run_graphs(self, x: torch.Tensor, graphs: list, shared: GraphInput, launch) -> None:
        n = x.shape[0]
        own = shared.buf[:n]
        if x.data_ptr() == own.data_ptr() and x.shape == own.shape and x.stride() == own.stride():
            shared.forget()                   # the caller wrote the graph input in place
        elif shared.load(x, n, launch):
            self.calls["copy"] = self.calls.get("copy", 0) + 1
        for g in graphs:
            self._gate.admit()
            g.replay()
            self._gate.done(launch)
        shared.read_by(self, launch)

    def capture(self, n: int, flip=False) -> float:
        """One HIP graph per pass over a batch of `n` input images (the reference's `capture`,
        `src/knee/dense8s.py:1410-1433`), recorded on the runner's stream after one eager pass (which does
        any lazy set-up outside the capture); returns the seconds spent."""
        mode = self._mode(flip)
        per = self._per_pass(mode)
        passes = -(-n // per)
        if passes * self.nb > self.n_out:
            raise ValueError(f"graph for {n} images: the encoder does {self.nb} per pass, "
                             f"the output holds {self.n_out}")
        t0 = time.perf_counter()
        shared = graph_input(self.dev, (passes * per, *self.in_shape[1:]), self.in_dtype)
        shared.forget()
        with self._launching():
            self._launch_pass(shared.buf.data_ptr(), 0, mode)
            self.stream.synchronize()
            self._gate.clear()
            graphs = []
            for index in range(passes):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=self.stream, capture_error_mode="thread_local"):
                    self._launch_pass(shared.buf[index * per].data_ptr(), index, mode)
                graphs.append(g)
        self.stream.synchronize()
        self.graphs.add(passes * per, mode, graphs, shared)
        return time.perf_counter() - t0

    def graph_in_buf(self, n: int, flip=False) -> torch.Tensor | None:
        """The static input buffer `[:n]` of the graphs that a batch of `n` images replays, or None."""
        mode = self._mode(flip)
        hit = self.graphs.find(n, mode, self._per_pass(mode))
        return None if hit is None else hit[1].buf[:n]

    def _event(self, name: str) -> torch.cuda.Event:
        """A synchronisation event of this runner, made once and recorded again at every use (a wait
        enqueued on it keeps the record it saw): no event is created per call."""
        ev = self.__dict__.get(name)
        if ev is None:
            ev = self.__dict__[name] = torch.cuda.Event()
        return ev

    # Ordering.  Every launch of a runner (calls, captures, diagnostics) is made inside `_launching`:
    # on the launch stream, after the caller's current stream's work so far and after the runner's own
    # previous launches (on whichever stream they ran: its buffers are reused), and before what the
    # caller enqueues next.  Each cross-stream dependency is one event wait, which the host pays for
    # (about 16 us on this stack for a pending event): a graph replay of a call is therefore made on
    # the caller's own stream when the runner allows it (`_adopt`), where stream order gives all of
    # that with no wait at all as long as the calls come from one stream.
    _adopt = False
    _tail = None                          # the stream of the runner's last launches (None: none yet)

    def _owners(self) -> tuple:
        """The runners whose buffers this one's launches use (itself; both encoders for a pair)."""
        return (self,)

    @contextlib.contextmanager
    def _launching(self, adopt: bool = False):
        switch = torch.cuda.current_device() != self.dev
        with torch.cuda.device(self.dev) if switch else contextlib.nullcontext():
            caller = torch.cuda.current_stream()
            launch = caller if adopt else self.stream
            if launch != caller:
                ev = self._event("_ev_in")
                ev.record(caller)
                launch.wait_event(ev)
            for r in self._owners():
                if r._tail is not None and r._tail != launch:
                    launch.wait_event(r._event("_ev_tail"))
            try:
                with torch.cuda.stream(launch) if launch != caller else contextlib.nullcontext():
                    yield launch
            finally:                      # also after a failed launch: what was enqueued stays ordered
                for r in self._owners():
                    r._event("_ev_tail").record(launch)
                    r._tail = launch
                if launch != caller:
                    caller.wait_event(self._owners()[0]._event("_ev_tail"))

    def _settle(self) -> None:
        """Waits on the host for the runner's launches so far."""
        for r in self._owners():
            (r._tail or r.stream).synchronize()

    def _encode(self, x: torch.Tensor, flip):
        """Encodes x, ordered after the caller's current stream and before what the caller enqueues next;
        returns `_outputs`."""
        mode = self._mode(flip)
        self._accept(x, mode)
        hit = self.graphs.find(x.shape[0], mode, self._per_pass(mode))
        with self._launching(adopt=self._adopt and hit is not None) as launch:
            if hit is None:
                self._run_eager(x.contiguous(), mode)
                self.calls["plain"] += 1
            else:
                self._run_graphs(x, *hit, launch)
                self.calls["graph"] += 1
            res = self._outputs(x.shape[0], mode)
        self._mark_written()
        return res


class Dense8SEncoder(_PassRunner):
    """The INT8 encoder on GPU `dev`: `enc(x)` with x (N, 3, img, img) on that GPU, uint8 (package input
    "u8") or fp16 ("f16"); returns (N, n_features) float32 in its own buffer (valid until the next
    call).  Blocks of `nb` images per pass; N is padded up to a multiple of `nb`.  Interface of the
    reference's runner (`src/knee/dense8s.py:944-1488`): own stream, `max_inflight`, `capture(n)`,
    `graph_in_buf(n)`, `nb`, `graphs`, `calls`, `load_s`, `in_dtype`, `in_shape`, `stream`, `out`.
    `__call__(x, flip=True)` encodes the horizontally mirrored images; `flip="tta"` returns (2N, C): the N
    images, then the same images mirrored (flip TTA fused in the stem: no mirrored copy in memory).

    A pass is a program of `Step`s compiled once from the package and the block kinds (`fused`,
    `fused_blocks`); running, tracing, profiling and timing a pass all walk that one program.
    """

    def __init__(self, pack: dict, dev: int, n_total: int, max_inflight: int | None = None,
                 fused=None) -> None:
        t0 = time.perf_counter()
        meta = pack["meta"]
        validate_meta(meta)
        missing = [k for k in needed_tables(meta) if k not in pack["par"]]
        if missing:
            raise ValueError(f"package tables missing: {missing[:4]}{'...' if len(missing) > 4 else ''}")
        self.meta, self.dev = meta, int(dev)
        self.device = torch.device(f"cuda:{self.dev}")
        self.lib = hip.library()
        self.library_version = hip.version()
        self.pack_sha = meta.get("kernels_sha")
        self.nb = int(meta["n"])
        self.fused = fused_blocks(meta, fused, _cu_count(self.dev))
        self.variants = recorded_variants(meta)  # {(family, block[, layer]): kernel variant}
        self.n_out = -(-int(n_total) // self.nb) * self.nb
        self.max_inflight = max_inflight
        self._gate = InflightGate(max_inflight)
        self.graphs = GraphBook()
        self.calls = {"graph": 0, "plain": 0}
        inp = meta.get("input", {"kind": "f16"})
        self.in_kind = hip.IN_U8 if inp.get("kind", "f16") == "u8" else hip.IN_F16
        self.in_dtype = torch.uint8 if self.in_kind == hip.IN_U8 else torch.float16
        self.in_shape = (self.nb, int(meta["in_ch"]), int(meta["img"]), int(meta["img"]))
        self._staging: torch.Tensor | None = None
        self._extra: dict = {}                   # per (block, kind): buffers a kind needs beyond the store
        with torch.cuda.device(self.dev):
            self.stream = torch.cuda.Stream(self.dev)
            self._upload(pack)
            self._lay_out()
            self.out = torch.empty((self.n_out, meta["n_features"]), dtype=torch.float32,
                                   device=f"cuda:{self.dev}")
            self._compile()
        self.load_s = time.perf_counter() - t0

    # -- set-up --
    def _upload(self, pack: dict) -> None:
        """The tables the kernels read, on the device (a reference package also carries the tables of
        its TensorRT and int8-stem paths, which stay behind), with this build's derived ones."""
        tables = dict(pack["par"])
        tables.update(derived_params(self.meta, tables))
        wanted = set(needed_tables(self.meta)) | set(derived_params(self.meta, {}, names_only=True))
        dev = torch.device(f"cuda:{self.dev}")
        self.par = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
                    for k, v in tables.items() if k in wanted}

    def _lay_out(self) -> None:
        """Device memory of a pass: the block stores in two regions used in turn (block b in region
        b % 2: its transition writes the next block's input into the other one), the planar bottleneck
        [4][nb * HW][32] of the largest map, the banded blocks' synchronisation words."""
        n = self.nb
        self.mem = Regions()
        need = [0, 0]
        for bi, b in enumerate(self.meta["blocks"]):
            need[bi % 2] = max(need[bi % 2], self._in0_bytes(bi) + b["L"] * self._slot_bytes(bi))
        self.mem.reserve("store0", need[0])
        self.mem.reserve("store1", need[1])
        self.mem.reserve("bott", n * BOTTLENECK * max(b["h"] * b["w"] for b in self.meta["blocks"]))
        self.mem.reserve("sync", 4 * hip.parts_sync_words(0))
        self.mem.allocate(f"cuda:{self.dev}")
        self.mem.view("sync").zero_()
        self.arena_mb = round(sum(need) / 2**20, 1)
        self.in0 = [self.mem.addr(f"store{bi % 2}") for bi in range(len(self.meta["blocks"]))]
        self.seg = [self.mem.addr(f"store{bi % 2}", self._in0_bytes(bi))
                    for bi in range(len(self.meta["blocks"]))]
        self._sync = self.mem.view("sync").view(torch.int32)
        self._report: torch.Tensor | None = None
        self._report_dev = 0

    def _in0_bytes(self, bi: int) -> int:
        b = self.meta["blocks"][bi]
        return self.nb * b["c0"] * b["h"] * b["w"]

    def _slot_bytes(self, bi: int) -> int:
        b = self.meta["blocks"][bi]
        return self.nb * b["h"] * b["w"] * GROUP

    def _slot(self, bi: int, li: int) -> int:
        return self.seg[bi] + li * self._slot_bytes(bi)

    def _buffer(self, key: tuple, make) -> torch.Tensor:
        """A buffer a block kind needs (made on first use and kept)."""
        t = self._extra.get(key)
        if t is None:
            t = self._extra[key] = make()
        return t

    def _bottleneck_buf(self, bi: int, li: int, kind: str) -> torch.Tensor:
        """Layer li's bottleneck buffer: the shared one, or for a "chain" block the second buffer on odd
        layers (conv2 of a layer reads one while conv1 of the next writes the other)."""
        if kind == "chain" and li % 2:
            b = self.meta["blocks"][bi]
            size = self.nb * BOTTLENECK * b["h"] * b["w"]
            return self._buffer(("bott2", size), lambda: torch.empty(size, dtype=torch.uint8,
                                                                     device=f"cuda:{self.dev}"))
        return self.mem.view("bott")

    def _bottleneck(self, bi: int, li: int, kind: str) -> int:
        return _ptr(self._bottleneck_buf(bi, li, kind))

    def _layer_table(self, bi: int) -> int:
        """Device array of block bi's `D8sLayerP` descriptors (for the whole-block kinds)."""
        def make():
            L = self.meta["blocks"][bi]["L"]
            arr = (hip.LayerP * L)(*[hip.LayerP(*(self._tab(bi, li, k) for k in
                                                  ("w1", "abh", "gdu", "w1sum", "w2k", "c2u", "w2sum")))
                                     for li in range(L)])
            return torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8).to(f"cuda:{self.dev}")
        return _ptr(self._buffer(("layers", bi), make))

    def _tab(self, bi: int, li: int, name: str) -> int:
        return _ptr(self.par[f"L{bi}_{li}_{name}"])

    def _conv1_args(self, bi: int, li: int, kind: str) -> hip.GemmArgs:
        b = self.meta["blocks"][bi]
        hw, g0 = b["h"] * b["w"], b["c0"] // GROUP
        return hip.GemmArgs(self.in0[bi], self.seg[bi], self._tab(bi, li, "w1"), self._tab(bi, li, "abh"),
                            self._tab(bi, li, "gdu"), self._tab(bi, li, "w1sum"),
                            self._bottleneck(bi, li, kind), g0, g0 + li, self.nb, hw, b["w"], self.nb * hw,
                            BOTTLENECK, 0)

    def _conv2_args(self, bi: int, li: int, kind: str) -> hip.Conv2Args:
        b = self.meta["blocks"][bi]
        return hip.Conv2Args(self._bottleneck(bi, li, kind), self._tab(bi, li, "w2k"), self._tab(bi, li, "c2u"),
                             self._tab(bi, li, "w2sum"), self._slot(bi, li), self.nb, b["h"], b["w"], 0)

    def block_steps(self, bi: int, kind: str) -> list[Step]:
        """The launches of block bi's layers run as `kind`."""
        b = self.meta["blocks"][bi]
        L, name = b["L"], _kind_name(kind)
        if name in ("img", "parts"):
            g0 = b["c0"] // GROUP
            makes = tuple((bi, j) for j in range(1, L + 1))
            if name == "img":
                args = hip.BlockArgs(self.in0[bi], self.seg[bi], self._layer_table(bi), self.nb,
                                     b["h"], b["w"], g0, L, 0)
                return [Step("block", bi, -1, makes, "d8s_dense_block", args)]
            k = int(kind.split(":", 1)[1])
            size = hip.parts_xchg_bytes(self.nb * k, b["w"])
            xchg = self._buffer(("xchg", bi, k), lambda: torch.zeros(size, dtype=torch.uint8,
                                                                      device=f"cuda:{self.dev}"))
            args = hip.PartsArgs(self.in0[bi], self.seg[bi], self._layer_table(bi), _ptr(self._sync),
                                 _ptr(xchg), self.nb, b["h"], b["w"], g0, L, k)
            return [Step("block", bi, -1, makes, "d8s_dense_block_parts", args)]
        if name == "tile":
            steps = []
            for li in range(L):
                g0 = b["c0"] // GROUP
                args = hip.DenseArgs(self.in0[bi], self.seg[bi], *(self._tab(bi, li, k) for k in
                                     ("w1", "abh", "gdu", "w1sum", "w2k", "c2u", "w2sum")),
                                     self._slot(bi, li), g0, g0 + li, self.nb, b["h"], b["w"], 0)
                steps.append(Step("dense", bi, li, ((bi, li + 1),), "d8s_dense", args))
            return steps
        if name == "chain":
            steps = [Step("conv1", bi, 0, (("bott", bi, 0),), "d8s_conv1", self._conv1_args(bi, 0, kind))]
            for li in range(L - 1):
                pair = (self._conv2_args(bi, li, kind), self._conv1_args(bi, li + 1, kind))
                steps.append(Step("chain", bi, li, ((bi, li + 1), ("bott", bi, li + 1)), "d8s_conv2_conv1",
                                  pair))
            steps.append(Step("conv2", bi, L - 1, ((bi, L),), "d8s_conv2", self._conv2_args(bi, L - 1, kind)))
            return steps
        steps = []
        for li in range(L):
            steps.append(Step("conv1", bi, li, (("bott", bi, li),), "d8s_conv1", self._conv1_args(bi, li, kind)))
            steps.append(Step("conv2", bi, li, ((bi, li + 1),), "d8s_conv2", self._conv2_args(bi, li, kind)))
        return steps

    def _compile(self) -> None:
        """The program of one pass: the stem, each block's layers as its kind, its transition, and the
        final features (the launch sequence of the reference's `_pass`, `src/knee/dense8s.py:1354-1385`)."""
        img = int(self.meta["img"])
        self.stem_args = hip.StemArgs(0, _ptr(self.par["S_lut"]), _ptr(self.par["S_w16"]),
                                      _ptr(self.par["S_bias"]), _ptr(self.par["S_inv"]), self.in0[0],
                                      self.nb, img, img, self.in_kind, 0, 0)
        prog = [Step("stem", 0, -1, ((0, 0),), "d8s_stem", self.stem_args)]
        for bi, b in enumerate(self.meta["blocks"]):
            prog += self.block_steps(bi, self.fused[bi])
            if b["trans"]:
                g0, hw = b["c0"] // GROUP, b["h"] * b["w"]
                cout = (b["c0"] + GROWTH * b["L"]) // 2
                args = hip.GemmArgs(self.in0[bi], self.seg[bi], _ptr(self.par[f"T{bi}_w"]),
                                    _ptr(self.par[f"T{bi}_abh"]), _ptr(self.par[f"T{bi}_gdf"]),
                                    _ptr(self.par[f"T{bi}_wsum"]), self.in0[bi + 1], g0, g0 + b["L"], self.nb,
                                    hw, b["w"], self.nb * hw, cout, cout // GROUP)
                prog.append(Step("trans", bi, -1, ((bi + 1, 0),), "d8s_transition", args))
            else:
                prog.append(Step("final", bi, -1, (), "d8s_final"))
        for step in prog:
            v = self._variant_of(step)
            if v:
                got = getattr(self.lib, step.entry + "_variant")(ctypes.byref(step.args), v)
                if got != v:
                    raise ValueError(f"{step.label()}: kernel variant {VARIANTS[step.family][v]!r} is not "
                                     f"taken for this shape")
                step.variant = v
        self.program = prog
        self._checked = any(s.entry == "d8s_dense_block_parts" for s in prog)
        # bands per image of the widest banded launch: its share of the CUs a wait needs resident
        self.max_bands = max((s.args.parts for s in prog if s.entry == "d8s_dense_block_parts"), default=0)
        if self._checked and self._report is None:
            # a host-mapped word the final kernel copies the banded blocks' error count into
            self._report = torch.zeros(2, dtype=torch.int32).pin_memory()
            self._report_np = self._report.numpy()
            dptr = ctypes.c_void_p()
            hip.check(self.lib.d8s_host_mapped(self._report.data_ptr(), ctypes.byref(dptr)), "d8s_host_mapped")
            self._report_dev = int(dptr.value or 0)

    def _variant_of(self, step: Step) -> int:
        """The kernel variant `variants` gives a conv1, conv2 or transition launch (0: none)."""
        if step.family == "conv1":
            return self.variants.get(("conv1", step.block, step.layer), 0)
        if step.family in ("conv2", "trans"):
            return self.variants.get((step.family, step.block), 0)
        return 0

    # -- launches --
    def _launch(self, step: Step, st: int, x_ptr: int = 0, f_ptr: int = 0, mode: int = 0) -> None:
        lib = self.lib
        if step.family == "stem":
            step.args.x = x_ptr
            step.args.flip = mode
            rc = lib.d8s_stem(ctypes.byref(step.args), st)
        elif step.family == "final":
            b = self.meta["blocks"][step.block]
            common = (self.in0[step.block], b["c0"] // GROUP, self.seg[step.block], self.nb,
                      b["h"] * b["w"], _ptr(self.par["F_ab"]), f_ptr, self.meta["n_features"])
            if self._checked:
                rc = lib.d8s_final_checked(*common, _ptr(self._sync) + 8, self._report_dev, st)
            else:
                rc = lib.d8s_final(*common, st)
        elif step.family == "chain":
            rc = lib.d8s_conv2_conv1(ctypes.byref(step.args[0]), ctypes.byref(step.args[1]), st)
        elif step.variant:
            rc = getattr(lib, step.entry + "_as")(ctypes.byref(step.args), step.variant, st)
        else:
            rc = getattr(lib, step.entry)(ctypes.byref(step.args), st)
        hip.check(rc, step.entry)

    def _launch_pass(self, x_ptr: int, index: int, mode: int, after=None) -> None:
        """The program on the runner's stream, reading x_ptr and writing the features of pass `index`;
        `after(step)` (optional) runs after every launch."""
        st = self.stream.cuda_stream
        f_ptr = self.out[index * self.nb].data_ptr()
        for step in self.program:
            self._launch(step, st, x_ptr, f_ptr, mode)
            if after is not None:
                after(step)

    # -- calls --
    def _accept(self, x: torch.Tensor, mode: int) -> None:
        if x.dtype != self.in_dtype:
            raise ValueError(f"input {x.dtype}: this package takes {self.in_dtype}")
        if tuple(x.shape[1:]) != self.in_shape[1:]:
            raise ValueError(f"input {tuple(x.shape)}: expected (N, "
                             f"{', '.join(map(str, self.in_shape[1:]))})")
        if x.device != self.device:
            raise ValueError(f"input on {x.device}, encoder on cuda:{self.dev}")
        if mode == 2 and self.nb % 2:
            raise ValueError(f"flip-TTA pairs need an even images-per-pass, the package has {self.nb}")
        if -(-x.shape[0] // self._per_pass(mode)) * self.nb > self.n_out:
            raise ValueError(f"{x.shape[0]} images: the output holds {self.n_out} encoded images")
        self._raise_wait_errors()

    def _outputs(self, n: int, mode: int) -> torch.Tensor:
        """The features of `n` input images: (n, C) views of `out`, or for flip-TTA (2n, C) with the n
        plain images first, then the n mirrored ones (pass p holds its images' plain features in rows
        p nb .. p nb + nb/2 - 1, the mirrored ones in the next nb/2 rows)."""
        if mode != 2:
            return self.out[:n]
        half = self.nb // 2
        if n == half:
            return self.out[:self.nb]
        i = torch.arange(n, device=self.out.device)
        plain = i + (i // half) * half
        return self.out.index_select(0, torch.cat([plain, plain + half]))

    def _mark_written(self) -> None:
        hip.written(self.out)

    _adopt = True                         # a call's graph replay runs on the caller's stream

    def __call__(self, x: torch.Tensor, flip=False) -> torch.Tensor:
        return self._encode(x, flip)

    # -- the banded blocks' bounded waits --
    def _raise_wait_errors(self) -> None:
        """Raises PartsWaitError if a pass since the last check reported expired waits (the host-mapped
        word the final kernel writes: read without a synchronisation; a pass still running is seen at
        a later call or by `sync_errors`)."""
        if self._report is None or self._report_np[0] == 0:
            return
        count = self._clear_wait_errors()
        raise PartsWaitError("d8s_dense_block_parts", 1,
                             f"{count} bounded waits ran out: features written as NaN since the last "
                             f"check; the error words are cleared")

    def _clear_wait_errors(self) -> int:
        """Waits for the runner's stream, then zeroes the banded blocks' ticket, end and error words
        (the launch count stays: it names the exchange rows) and the host report; returns the count."""
        with torch.cuda.device(self.dev):
            self._settle()
            count = int(self._sync[2].item())
            self._sync[:3].zero_()
            torch.cuda.synchronize(self.dev)
        if self._report is not None:
            self._report.zero_()
        return count

    def sync_errors(self, clear: bool = True) -> int:
        """Bounded waits that ran out in the banded blocks' launches so far (0: every result valid),
        read after the runner's stream (a synchronisation); `clear` zeroes the words."""
        if clear:
            return self._clear_wait_errors()
        with torch.cuda.device(self.dev):
            self._settle()
            return int(self._sync[2].item())

    # -- diagnostics --
    def store(self, bi: int, j: int) -> torch.Tensor:
        """Store segment j of block bi as a float tensor (nb, c, h, w) of its integers: j = 0 the block
        input (c = c0), j >= 1 the output of layer j - 1 (c = 32)."""
        b = self.meta["blocks"][bi]
        h, w = b["h"], b["w"]
        region = f"store{bi % 2}"
        if j == 0:
            raw = self.mem.view(region, 0, self._in0_bytes(bi)).view(torch.int8)
            groups = raw.view(self.nb, b["c0"] // GROUP, h * w, GROUP).transpose(2, 3)
            return groups.reshape(self.nb, b["c0"], h, w).float()
        off = self._in0_bytes(bi) + (j - 1) * self._slot_bytes(bi)
        raw = self.mem.view(region, off, self._slot_bytes(bi)).view(torch.int8)
        return raw.view(self.nb, h * w, GROUP).transpose(1, 2).reshape(self.nb, GROUP, h, w).float()

    def bottleneck(self, bi: int, li: int = 0) -> torch.Tensor:
        """Layer li's planar bottleneck in block bi as uint8 (nb, 128, h, w) (the last one written there)."""
        b = self.meta["blocks"][bi]
        hw = b["h"] * b["w"]
        raw = self._bottleneck_buf(bi, li, self.fused[bi])[:4 * self.nb * hw * GROUP]
        return raw.view(4, self.nb, hw, GROUP).permute(1, 0, 3, 2).reshape(self.nb, 4 * GROUP, b["h"], b["w"])

    def launch(self, x: torch.Tensor, flip=False, after=None) -> None:
        """Enqueues one eager pass over the first images of x on the runner's stream (after the caller's
        current stream), writing `out[:nb]`, without waiting for it; `after(step)` is called after each
        launch is enqueued (e.g. to record events at chosen steps)."""
        mode = self._mode(flip)
        x_ptr = self._pass_input(x, mode)
        with self._launching():
            self._launch_pass(x_ptr, 0, mode, after)

    def _pass_input(self, x: torch.Tensor, mode: int) -> int:
        self._accept(x, mode)
        return self._staged(x[:self._per_pass(mode)].contiguous(), mode)

    @torch.no_grad()
    def trace(self, x: torch.Tensor, flip=False) -> tuple[dict, torch.Tensor]:
        """One pass over the first images with a synchronisation after every launch: what each launch
        completed -- store segments {(block, j): tensor} and bottlenecks {("bott", block, layer): tensor}
        -- and the features (the reference's `trace`, `src/knee/dense8s.py:1510-1546`)."""
        mode = self._mode(flip)
        x_ptr = self._pass_input(x, mode)
        snaps: dict = {}
        f = torch.zeros((self.nb, self.meta["n_features"]), dtype=torch.float32, device=f"cuda:{self.dev}")

        def snapshot(step: Step) -> None:
            self.stream.synchronize()
            for key in step.makes:
                snaps[key] = (self.bottleneck(key[1], key[2]) if key[0] == "bott" else self.store(*key)).clone()

        st = self.stream.cuda_stream
        with self._launching():
            for step in self.program:
                self._launch(step, st, x_ptr, f.data_ptr(), mode)
                snapshot(step)
        return snaps, f

    def profile(self, x: torch.Tensor, reps: int = 3, flip=False) -> dict:
        """GPU milliseconds per `Step.tag` (stem, conv1 / conv2 / chain / dense / block per block,
        transitions, final) of one pass, mean of `reps` passes after a warm one, from HIP events
        recorded between the launches."""
        mode = self._mode(flip)
        x_ptr = self._pass_input(x, mode)
        sums: dict[str, float] = collections.defaultdict(float)
        with self._launching():
            for r in range(reps + 1):
                marks = [(None, _record(self.stream))]
                self._launch_pass(x_ptr, 0, mode, after=lambda s: marks.append((s.tag(), _record(self.stream))))
                self.stream.synchronize()
                if r:
                    for (_, e0), (tag, e1) in zip(marks, marks[1:]):
                        sums[tag] += e0.elapsed_time(e1)
        return {tag: round(ms / reps, 4) for tag, ms in sorted(sums.items())}

    def _graph_ms(self, steps: list[Step], reps: int, x_ptr: int = 0, mode: int = 0) -> float:
        """ms per run of `steps`: a HIP graph holding `reps` runs of them back to back, replayed three
        times between events after one warm replay; the median replay."""
        st = self.stream.cuda_stream
        f_ptr = self.out.data_ptr()
        with self._launching():
            for s in steps:
                self._launch(s, st, x_ptr, f_ptr, mode)
            self.stream.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=self.stream, capture_error_mode="thread_local"):
                for _ in range(reps):
                    for s in steps:
                        self._launch(s, st, x_ptr, f_ptr, mode)
            g.replay()
            marks = [_record(self.stream)]
            for _ in range(3):
                g.replay()
                marks.append(_record(self.stream))
            self.stream.synchronize()
        self._mark_written()
        times = sorted(a.elapsed_time(b) for a, b in zip(marks, marks[1:]))
        return times[1] / reps

    def _warm(self, x: torch.Tensor, flip) -> tuple[int, int]:
        """One eager pass over x (fills the store every later timing reads); returns (x_ptr, mode)."""
        mode = self._mode(flip)
        x_ptr = self._pass_input(x, mode)
        with self._launching():
            self._launch_pass(x_ptr, 0, mode)
        self._mark_written()
        return x_ptr, mode

    def time_families(self, x: torch.Tensor, reps: int = 5, flip=False) -> dict:
        """GPU milliseconds per pass of each kernel family (stem, conv1, conv2, chain, dense, block,
        trans, final): the family's launches of one pass, in pass order, `reps` times in one HIP graph
        (`_graph_ms`).  Unlike `profile` no host gap between launches is counted: the kernels' own time."""
        x_ptr, mode = self._warm(x, flip)
        by_family: dict[str, list] = {}
        for step in self.program:
            by_family.setdefault(step.family, []).append(step)
        return {fam: round(self._graph_ms(steps, reps, x_ptr, mode), 4) for fam, steps in by_family.items()}

    def pass_share(self, x: torch.Tensor, family: str, reps: int = 5, flip=False, beside=None) -> dict:
        """GPU milliseconds a kernel family adds to a whole pass as the graphs run it: the pass in one HIP
        graph against the same pass without the family's launches in another, each replayed `reps`
        times between events after a warm replay, medians ("share_ms" = "pass_ms" - "without_ms").  The
        pass without them computes nothing useful (it overwrites the outputs of earlier calls, as a call
        does); every later pass rewrites what it read.  `beside`:
        another runner whose own pass (`beside(x, flip)`) starts with each replay on its stream, so the
        two share the GPU as in `encode_concurrent`; the times are then the pair's, from the caller's
        stream."""
        if not any(s.family == family for s in self.program):
            raise ValueError(f"pass_share: no {family!r} launch in this runner's pass")
        if beside is not None and concurrent_order([self, beside], _cu_count(self.dev))[1]:
            raise ValueError("pass_share: the two runners' banded blocks do not fit the CUs together")
        x_ptr, mode = self._warm(x, flip)
        st = self.stream.cuda_stream
        f_ptr = self.out.data_ptr()
        graphs = {}
        with self._launching():
            for key, steps in (("pass_ms", self.program),
                               ("without_ms", [s for s in self.program if s.family != family])):
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr, stream=self.stream, capture_error_mode="thread_local"):
                    for step in steps:
                        self._launch(step, st, x_ptr, f_ptr, mode)
                graphs[key] = gr
        self.stream.synchronize()
        caller = torch.cuda.current_stream(self.dev)
        times: dict[str, list] = {k: [] for k in graphs}
        for r in range(reps + 1):
            for key, gr in graphs.items():
                if beside is None:
                    a = _record(self.stream)
                    with torch.cuda.stream(self.stream):
                        gr.replay()
                    b = _record(self.stream)
                else:
                    a = _record(caller)
                    self.stream.wait_stream(caller)
                    beside.stream.wait_stream(caller)
                    with torch.cuda.stream(beside.stream):
                        beside(x, flip=flip)
                    with torch.cuda.stream(self.stream):
                        gr.replay()
                    caller.wait_stream(self.stream)
                    caller.wait_stream(beside.stream)
                    b = _record(caller)
                torch.cuda.synchronize(self.dev)
                if r:
                    times[key].append(a.elapsed_time(b))
        self._mark_written()
        out = {k: sorted(v)[len(v) // 2] for k, v in times.items()}
        out["share_ms"] = out["pass_ms"] - out["without_ms"]
        out["launches"] = sum(s.family == family for s in self.program)
        return out

    def time_layers(self, reps: int = 20, families=None) -> dict:
        """ms of every launch of the pass but the stem and the final features (or only those of the
        kernel families named in `families`), on the current store (`Step.label`: "c1 b{b}l{l}",
        "c2 ...", "cc ..." chained, "dn ..." fused layer, "blk b{b}", "t{b}")."""
        return {s.label(): round(self._graph_ms([s], reps), 4) for s in self.program
                if s.family not in ("stem", "final") and (families is None or s.family in families)}

    def tune_kinds(self, x: torch.Tensor, reps: int = 10, flip=False, apply: bool = False) -> dict:
        """For every block the ms of its layers run as each kind it can take (`kind_options`), on the
        store a pass over x leaves: {"b{block}": {kind: ms}} (the role of the reference's on-device
        tuners `tune_bm` / `tune_trans` / `tune_c2`, `src/knee/dense8s.py:1598-1651`, for this build's
        choice, the block kind).  Every kind writes the same bytes.  `apply`: the runner then uses the
        fastest kind per block (its graphs are dropped: capture again); `pack_meta(fused=...)` records
        such a choice in a package."""
        self._warm(x, flip)
        out: dict = {}
        for bi, b in enumerate(self.meta["blocks"]):
            times = {}
            for kind in kind_options(b, self.nb):
                times[kind] = round(self._graph_ms(self.block_steps(bi, kind), reps), 4)
            out[f"b{bi}"] = times
        if apply:
            self.fused = {bi: min(out[f"b{bi}"].items(), key=lambda kv: kv[1])[0]
                          for bi in range(len(self.meta["blocks"]))}
            self.graphs.clear()
            self._compile()
        return out

    def _tune_variants(self, steps: list, reps: int) -> dict:
        """{variant name: ms} of the first of `steps` (one family) run as every kernel variant its shape
        takes (`d8s_*_variant`), on the current store."""
        step = steps[0]
        names = VARIANTS[step.family]
        query = getattr(self.lib, step.entry + "_variant")
        return {name: round(self._graph_ms([replace(step, variant=v)], reps), 4)
                for v, name in names.items() if query(ctypes.byref(step.args), v) == v}

    def _apply_variants(self, choices: dict) -> None:
        """Runs the launches with the variants chosen ({(family, block[, layer]): id}); graphs dropped."""
        self.variants.update(choices)
        self.graphs.clear()
        self._compile()

    def tune_bm(self, reps: int = 20, apply: bool = False) -> dict:
        """For every conv1 launch of the pass the ms of every conv1 kernel variant its shape takes
        (`C1_VARIANTS`): {"b{block}l{layer}": {variant: ms}}, on the current store (the reference's
        `tune_bm`, `src/knee/dense8s.py:1598-1617`; here the layers of blocks run as "conv", and the first
        layer of a "chain" block, have conv1 launches of their own).  Every variant writes the same bytes.
        `apply`: the runner then uses the fastest per layer; `pack_meta(bm=...)` records such a choice."""
        out, pick = {}, {}
        for s in self.program:
            if s.family == "conv1":
                res = out[f"b{s.block}l{s.layer}"] = self._tune_variants([s], reps)
                pick[("conv1", s.block, s.layer)] = _variant_id(C1_VARIANTS, min(res, key=res.get))
        if apply:
            self._apply_variants(pick)
        return out

    def tune_c2(self, reps: int = 20, apply: bool = False) -> dict:
        """For every block with conv2 launches of its own the ms of its first one as every conv2 tile the
        map takes (`C2_VARIANTS`): {side: {variant: ms}}, on the current store (the reference's `tune_c2`,
        `src/knee/dense8s.py:1636-1651`, layer 0's conv2 per side).  `apply`: the block's conv2 launches
        then use the fastest; `pack_meta(c2=...)` records such a choice."""
        out, pick = {}, {}
        for bi, b in enumerate(self.meta["blocks"]):
            steps = [s for s in self.program if s.family == "conv2" and s.block == bi]
            if steps:
                res = out[b["h"]] = self._tune_variants(steps, reps)
                pick[("conv2", bi)] = _variant_id(C2_VARIANTS, min(res, key=res.get))
        if apply:
            self._apply_variants(pick)
        return out

    def tune_trans(self, reps: int = 20, apply: bool = False) -> dict:
        """For every transition the ms of every transition variant its shape takes (`TRANS_VARIANTS`):
        {"t{block}": {variant: ms}}, on the current store (the reference's `tune_trans`,
        `src/knee/dense8s.py:1619-1634`).  `apply`: the runner then uses the fastest;
        `pack_meta(tbm=...)` records such a choice."""
        out, pick = {}, {}
        for s in self.program:
            if s.family == "trans":
                res = out[f"t{s.block}"] = self._tune_variants([s], reps)
                pick[("trans", s.block)] = _variant_id(TRANS_VARIANTS, min(res, key=res.get))
        if apply:
            self._apply_variants(pick)
        return out


def encode_concurrent(calls) -> list[torch.Tensor]:
    """Several runners at once: `calls` = [(runner, x, flip), ...], every runner on its own stream, the
    caller's current stream joined after all of them.  The seeds of an ensemble read the same input and
    are independent, so one runner's small late-block layers overlap another's work.  Runners with
    banded whole blocks ("parts" kinds) overlap only while their bands per image fit the CUs together
    (`concurrent_order`): a banded workgroup waits for its neighbour bands, which must be resident at
    the same time.

    Each call is made with the runner's own stream current: an extra stream per call would share one
    of the device's few hardware queues with another runner, and an event recorded there would make
    that runner wait for everything queued before it.  Returns the runners' outputs (views, as
    `Dense8SEncoder.__call__`)."""
    if not calls:
        return []
    dev = calls[0][0].dev
    if any(enc.dev != dev for enc, _, _ in calls):
        raise ValueError("encode_concurrent: runners on different GPUs")
    caller = torch.cuda.current_stream(dev)
    for enc, _, _ in calls:
        enc.stream.wait_stream(caller)
    outs = []
    runners = [enc for enc, _, _ in calls]
    for (enc, x, flip), after in zip(calls, concurrent_order(runners, _cu_count(dev))):
        for j in after:
            enc.stream.wait_stream(runners[j].stream)
        with torch.cuda.stream(enc.stream):
            outs.append(enc(x, flip=flip))
    for enc, _, _ in calls:
        caller.wait_stream(enc.stream)
    return outs


def concurrent_order(runners, cus: int = 256) -> list[list[int]]:
    """For each runner of `encode_concurrent`, the runners whose streams it waits for first.  A banded
    launch progresses while the banded launches in flight together have at most `cus` bands per image
    in all (each then has a whole image resident), so runners with banded blocks (`max_bands` > 0:
    their launches follow each other on their own stream) are grouped in order while their bands per
    image fit `cus`; a runner that does not fit waits for every runner of the group before it and
    starts the next group.  Runners without banded blocks run free."""
    order, group, load = [], [], 0
    for i, enc in enumerate(runners):
        k = int(getattr(enc, "max_bands", 0) or 0)
        if not k:
            order.append([])
            continue
        if group and load + k > cus:
            order.append(list(group))
            group, load = [], 0
        else:
            order.append([])
        group.append(i)
        load += k
    return order


PAIR_ENTRIES = {"d8s_stem": "d8s_stem_pair", "d8s_conv1": "d8s_conv1_pair", "d8s_conv2": "d8s_conv2_pair",
                "d8s_dense": "d8s_dense_pair", "d8s_dense_block": "d8s_dense_block_pair",
                "d8s_transition": "d8s_transition_pair"}


class EncoderPair(_PassRunner):
    """Two encoders of one geometry over the same input images -- the final model's two weight seeds
    on one study -- as ONE launch sequence: the two programs side by side, each step that has a paired
    entry point (`PAIR_ENTRIES`, `d8s_*_pair`) one launch carrying both encoders' arguments, so the two
    passes' small late layers fill the chip together (the 16 x 16 whole block: 192 workgroups in about
    the time of 96) instead of overlapping by chance on two streams (`encode_concurrent`); the other
    steps (banded blocks, chained launches, final features) as two launches in the same sequence.  Each
    encoder's outputs are exactly what it gives alone.  The pair launches on the first encoder's stream
    and orders the second's around it."""

    def __init__(self, a: Dense8SEncoder, b: Dense8SEncoder):
        if a is b:
            raise ValueError("EncoderPair: the same encoder twice")
        if a.dev != b.dev:
            raise ValueError(f"EncoderPair: encoders on cuda:{a.dev} and cuda:{b.dev}")
        geometry = lambda e: (e.nb, e.n_out, e.in_dtype, e.in_shape, e.fused,  # noqa: E731
                              [(x["h"], x["w"], x["c0"], x["L"]) for x in e.meta["blocks"]])
        if geometry(a) != geometry(b):
            raise ValueError("EncoderPair: the encoders differ in geometry, batch, input or block kinds")
        self.a, self.b = a, b
        self.dev, self.nb, self.n_out = a.dev, a.nb, a.n_out
        self.in_shape, self.in_dtype = a.in_shape, a.in_dtype
        self.stream = a.stream
        self.lib = a.lib
        self.device = a.device
        self.graphs = GraphBook()
        self.calls = {"graph": 0, "plain": 0, "copy": 0}
        self._gate = InflightGate(None)
        self._staging: torch.Tensor | None = None

    def _owners(self) -> tuple:
        return (self.a, self.b)

    def _accept(self, x: torch.Tensor, mode: int) -> None:
        self.a._accept(x, mode)
        self.b._accept(x, mode)

    def _launch_pass(self, x_ptr: int, index: int, mode: int) -> None:
        A, B, st = self.a, self.b, self.stream.cuda_stream
        fa, fb = A.out[index * A.nb].data_ptr(), B.out[index * B.nb].data_ptr()
        for sa, sb in zip(A.program, B.program):
            paired = None if sa.variant or sb.variant else PAIR_ENTRIES.get(sa.entry)
            if paired is None:
                A._launch(sa, st, x_ptr, fa, mode)
                B._launch(sb, st, x_ptr, fb, mode)
                continue
            if sa.family == "stem":
                for s in (sa, sb):
                    s.args.x, s.args.flip = x_ptr, mode
            hip.check(getattr(self.lib, paired)(ctypes.byref(sa.args), ctypes.byref(sb.args), st), paired)

    def _outputs(self, n: int, mode: int):
        return self.a._outputs(n, mode), self.b._outputs(n, mode)

    def _mark_written(self) -> None:
        hip.written(self.a.out, self.b.out)

    def __call__(self, x: torch.Tensor, flip=False) -> tuple[torch.Tensor, torch.Tensor]:
        """Both encoders' features of x: (outputs of the first, outputs of the second), as each
        encoder's `__call__` returns them."""
        return self._encode(x, flip)


def _record(stream) -> torch.cuda.Event:
    e = torch.cuda.Event(enable_timing=True)
    e.record(stream)
    return e
