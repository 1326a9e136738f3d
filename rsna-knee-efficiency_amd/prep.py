"""Upstream preprocessing on the GPU: raw uint16 crops -> resize to img -> exact 1/99 percentiles ->
uint8 -> side flip, over the HIP library (`d8s_prep`, `d8s_prep_resize`, include/d8s_hip.h).

The host side of the reference's GPU preparation, same names and meaning:
- `to_uint8_hist_batch(x, out)`   `knee.data.torch_uint8.to_uint8_torch_hist_batch`
  (src/knee/data/torch_uint8.py:332-357): (R, K, H, W) float32 -> uint8, `cache._to_uint8` per stack
  bit for bit (exact mode; the reference's `KNEE_PCT_STRIDE` subsampling is not bit-identical and is
  not offered);
- `resize(region, resc, box, img)` `_resize_torch` after the Rescale (src/knee/data/raw_crop.py:419-432,
  520-522);
- `payloads_to_uint8(payloads, spec, device)` `raw_crop.payloads_to_uint8_torch`
  (src/knee/data/raw_crop.py:492-549): the study payloads (`raw`, `u8`, `resc`, `meta`) -> the volumes
  (B, S, K, img, img) uint8, including `KNEE_READ_SLICES` ranges (`read_range`, raw_crop.py:79-90)
  and the flips;
- `ranks(n)`                       `torch_uint8._ranks` (torch_uint8.py:31-42).
Every stack of a call runs through one `d8s_prep` launch sequence (up to 16 stacks per call): the
resize runs once per stack, into a float32 scratch buffer together with the first histogram pass,
and the later passes (the other two radix levels and the uint8 write) read the stored values.
There is no CPU path: without the library the calls raise.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from functools import lru_cache

import numpy as np
import torch

from . import hip

CLIP_PCT = (1.0, 99.0)
# columns of a payload's `meta` (src/knee/data/raw_crop.py:44-52)
M_SLOT, M_MODE, M_K, M_HR, M_WR, M_RAW_OFF, M_FLIP, M_U8_OFF = range(8)
M_BOX = 8
MAX_SCALES = 2
M_RESC = M_BOX + 4 * MAX_SCALES
N_META = M_RESC + 1
MODE_GPU, MODE_CPU = 1, 2
FLIP_NONE, FLIP_X, FLIP_SLICES = 0, 1, 2


@dataclass(frozen=True)
class PrepSpec:
    """The fields of the reference's `CacheSpec` (src/knee/data/cache.py:50-140) the preparation reads:
    output side, slices per stack, sequences (slots per scale) and crop scales."""
    img: int = 512
    slices: int = 24
    n_seq: int = 4
    n_scales: int = 2

    @property
    def shape(self) -> tuple[int, int, int, int]:
        return (self.n_seq * self.n_scales, self.slices, self.img, self.img)


@lru_cache(maxsize=64)
def ranks(n: int) -> tuple[int, int, float, float]:
    """(k1, k2, gamma1, gamma2) of linear `np.percentile(..., CLIP_PCT)` over n values."""
    q = np.true_divide(np.asarray(CLIP_PCT), 100)
    virtual = (n - 1) * q
    prev = np.floor(virtual).astype(np.intp)
    if n < 4 or not (0 < q[0] < 0.5 < q[1] < 1) or prev[1] + 1 >= n:
        raise ValueError(f"percentiles {CLIP_PCT} over {n} values: unsupported case")
    gamma = virtual - prev.astype(virtual.dtype)
    return int(prev[0]), int(prev[1]), float(gamma[0]), float(gamma[1])


def read_range(k_sl: int, flip: int, read_slices: tuple[int, int] | None) -> tuple[int, int] | None:
    """Payload positions [a, z) read and normalised (`raw_crop.read_range`, raw_crop.py:79-90), with the
    `KNEE_READ_SLICES` range passed in; None = all."""
    if read_slices is None:
        return None
    a, z = read_slices
    if not 0 <= a < z <= k_sl:
        raise ValueError(f"KNEE_READ_SLICES {a}:{z} outside 0..{k_sl}")
    return (k_sl - z, k_sl - a) if flip == FLIP_SLICES else (a, z)


_WS: dict = {}


def _workspace(device: torch.device, n: int, img: int) -> torch.Tensor:
    """Device workspace for d8s_prep (kept per device and grown on demand)."""
    need = ctypes.c_uint64()
    hip.call("d8s_prep_workspace", n, img, ctypes.byref(need))
    key = str(device)
    ws = _WS.get(key)
    if ws is None or ws.numel() < need.value:
        ws = torch.empty(int(need.value) + 256, dtype=torch.uint8, device=device)
        _WS[key] = ws
    return ws


def _aligned_ptr(ws: torch.Tensor) -> int:
    p = ws.data_ptr()
    return (p + 255) // 256 * 256


_SCRATCH: dict = {}


def _scratch(device: torch.device, nbytes: int) -> torch.Tensor:
    """Device scratch for the resized float32 stacks of a kind-0 d8s_prep call (kept per device and
    grown on demand)."""
    key = str(device)
    sc = _SCRATCH.get(key)
    if sc is None or sc.numel() * 4 < nbytes:
        sc = torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=device)
        _SCRATCH[key] = sc
    return sc


def _run(entry: str, kind: int, img: int, stacks: list[dict], device: torch.device) -> torch.Tensor:
    """Launches `entry` over `stacks` (dicts of D8sPrepStack fields), 16 at a time, on the current
    stream.  Returns the workspace (its head holds the stats of the last chunk).  Calls on one device
    share the workspace and scratch: they are ordered by the stream they are issued on."""
    ws = _workspace(device, hip.PREP_MAX_STACKS, img)
    stream = torch.cuda.current_stream(device).cuda_stream
    for c in range(0, len(stacks), hip.PREP_MAX_STACKS):
        chunk = stacks[c:c + hip.PREP_MAX_STACKS]
        a = hip.PrepArgs()
        a.workspace = _aligned_ptr(ws)
        a.ws_bytes = ws.numel() - (a.workspace - ws.data_ptr())
        if entry == "d8s_prep" and kind == 0:
            need = sum(4 * (s["k1"] - s["k0"]) * img * img for s in chunk)
            sc = _scratch(device, need)
            a.scratch, a.scratch_bytes = sc.data_ptr(), sc.numel() * 4
        a.kind, a.img, a.n_stacks = kind, img, len(chunk)
        for i, s in enumerate(chunk):
            for k, v in s.items():
                setattr(a.s[i], k, v)
        hip.call(entry, ctypes.byref(a), ctypes.c_void_p(stream))
    return ws


def stats(ws: torch.Tensor, n: int) -> list[dict]:
    """The D8sPrepStat records of the last call's first n stacks (synchronises)."""
    off = _aligned_ptr(ws) - ws.data_ptr()
    raw = ws[off: off + n * ctypes.sizeof(hip.PrepStat)].cpu().numpy().tobytes()
    out = []
    for i in range(n):
        r = hip.PrepStat.from_buffer_copy(raw, i * ctypes.sizeof(hip.PrepStat))
        out.append({"lo": r.lo, "hi": r.hi, "scale": r.scale, "bad": bool(r.bad)})
    return out


def _rank_fields(n: int) -> dict:
    k1, k2, g1, g2 = ranks(n)
    return {"r1": k1, "r2": k2, "g1": g1, "g2": g2}


def to_uint8_hist_batch(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """(R, K, H, W) float32 -> uint8: `cache._to_uint8` per stack (bit for bit), H == W a multiple of 8."""
    if x.dtype != torch.float32:
        raise TypeError(f"expected a float32 stack, got {x.dtype}")
    if x.dim() != 4 or x.shape[2] != x.shape[3] or x.shape[3] % 8:
        raise ValueError(f"expected (R, K, img, img) with img a multiple of 8, got {tuple(x.shape)}")
    if not x.is_cuda:
        raise ValueError("to_uint8_hist_batch runs on the GPU only")
    x = x.contiguous()
    R, K, img = x.shape[0], x.shape[1], x.shape[3]
    if out is None:
        out = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    elif out.shape != x.shape or out.dtype != torch.uint8 or not out.is_contiguous():
        raise ValueError("out must be a contiguous uint8 tensor of the input's shape")
    per = K * img * img
    stacks = [dict(src=x.data_ptr() + 4 * r * per, out=out.data_ptr() + r * per, K=K, k0=0, k1=K,
                   flip=FLIP_NONE, **_rank_fields(per)) for r in range(R)]
    _run("d8s_prep", 1, img, stacks, x.device)
    hip.written(out)
    return out


def _region_stack(region: torch.Tensor, resc: torch.Tensor | None, box, k_range) -> dict:
    K, hr, wr = region.shape
    y0, y1, x0, x1 = (int(v) for v in box)
    a, z = k_range if k_range is not None else (0, K)
    return dict(src=region.data_ptr(), resc=0 if resc is None else resc.data_ptr(), K=K, hr=hr, wr=wr,
                y0=y0, y1=y1, x0=x0, x1=x1, k0=a, k1=z)


def resize(region: torch.Tensor, resc: torch.Tensor | None, box, img: int,
           k_range: tuple[int, int] | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """region (K, hr, wr) uint16 values (int16 or uint16 tensor) on the GPU, resc (K, 2) float32 slope
    and intercept or None, box (y0, y1, x0, x1) -> (K, img, img) float32 (slices outside k_range are
    left as they are in `out`, zero when it is allocated here)."""
    if region.dim() != 3 or region.element_size() != 2 or not region.is_cuda:
        raise ValueError("region must be a (K, hr, wr) 16-bit tensor on the GPU")
    region = region.contiguous()
    K = region.shape[0]
    if resc is not None:
        resc = resc.to(device=region.device, dtype=torch.float32).contiguous()
        if tuple(resc.shape) != (K, 2):
            raise ValueError(f"resc must be ({K}, 2), got {tuple(resc.shape)}")
    if out is None:
        out = torch.zeros((K, img, img), dtype=torch.float32, device=region.device)
    elif (tuple(out.shape) != (K, img, img) or out.dtype != torch.float32 or not out.is_contiguous()
          or out.device != region.device):
        raise ValueError(f"out must be a contiguous float32 ({K}, {img}, {img}) tensor on the region's device")
    s = _region_stack(region, resc, box, k_range)
    s["out"] = out.data_ptr()
    _run("d8s_prep_resize", 0, img, [s], region.device)
    hip.written(out)
    return out


def payloads_to_uint8(payloads: list, spec: PrepSpec, device,
                      read_slices: tuple[int, int] | None = None) -> torch.Tensor:
    """The volumes (B, S, K, img, img) uint8 on the device from study payloads (`raw` int16 1-D, `u8`
    uint8 1-D, `resc` float64 (m, 2), `meta` int64 (n, N_META)), as `payloads_to_uint8_torch`."""
    device = torch.device(device)
    img, n_seq = spec.img, spec.n_seq
    # every byte of a slot that has a series is written (the kernels write the read slices and zero
    # the others; CPU series are copied), so only slots without a series are cleared
    vol = torch.empty((len(payloads), *spec.shape), dtype=torch.uint8, device=device)
    filled: set = set()
    stacks: list[dict] = []
    keep: list = []                 # device copies referenced by the launches
    for b, payload in enumerate(payloads):
        meta = payload["meta"]
        meta = meta.cpu().numpy() if isinstance(meta, torch.Tensor) else np.asarray(meta)
        if meta.size == 0:
            continue
        raw = torch.as_tensor(payload["raw"]).to(device, non_blocking=True)
        u8 = torch.as_tensor(payload["u8"]).to(device, non_blocking=True)
        resc_all = torch.as_tensor(payload["resc"])
        resc = resc_all.to(device).float().contiguous() if resc_all.numel() else None
        keep += [raw, u8, resc]
        for row in meta:
            j, k_sl = int(row[M_SLOT]), int(row[M_K])
            if k_sl != spec.slices:
                raise ValueError(f"series with {k_sl} slices in a spec of {spec.slices}")
            filled.update((b, j + k * n_seq) for k in range(spec.n_scales))
            if row[M_MODE] == MODE_GPU:
                hr, wr, off = int(row[M_HR]), int(row[M_WR]), int(row[M_RAW_OFF])
                if off < 0 or off + k_sl * hr * wr > raw.numel():
                    raise ValueError("payload region outside `raw`")
                code = int(row[M_FLIP])
                rr = read_range(k_sl, code, read_slices)
                a, z = rr if rr is not None else (0, k_sl)
                rs = 0
                if row[M_RESC] >= 0:
                    if resc is None or int(row[M_RESC]) + k_sl > resc.shape[0]:
                        raise ValueError("payload Rescale rows outside `resc`")
                    rs = resc.data_ptr() + 8 * int(row[M_RESC])
                for k in range(spec.n_scales):
                    y0, y1, x0, x1 = (int(v) for v in row[M_BOX + 4 * k: M_BOX + 4 * k + 4])
                    stacks.append(dict(src=raw.data_ptr() + 2 * off, resc=rs,
                                       out=vol[b, j + k * n_seq].data_ptr(), K=k_sl, hr=hr, wr=wr,
                                       y0=y0, y1=y1, x0=x0, x1=x1, k0=a, k1=z, flip=code,
                                       **_rank_fields((z - a) * img * img)))
            else:
                off, n = int(row[M_U8_OFF]), k_sl * img * img
                for k in range(spec.n_scales):
                    vol[b, j + k * n_seq] = u8[off + k * n: off + (k + 1) * n].view(k_sl, img, img)
    for b in range(len(payloads)):
        for slot in range(spec.shape[0]):
            if (b, slot) not in filled:
                vol[b, slot].zero_()
    if stacks:
        _run("d8s_prep", 0, img, stacks, device)
        hip.written(vol)
    return vol
