"""Comparisons of the HIP kernels with the oracle, shared by the GPU tests and `__graft_entry__.smoke()`.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Every `run_*` calls one entry point of the C ABI
(`rsna_knee_efficiency_amd.hip`) on device tensors; every `exact_*` recomputes the same output on the
CPU: integer sums by float64 matmul / conv (exact: all partial sums are integers below 2^53) and the
bytes by the C oracle's epilogues (the kernels' fp32 roundings).  The bar is equality, except for the
stem, whose fp32 sums are accumulated in the MFMA's order (tolerance stated where used).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch
import torch.nn.functional as F

from rsna_knee_efficiency_amd import dense8s, hip

from . import cases, lib


def _dev(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def _ptr(t: torch.Tensor) -> int:
    return int(t.data_ptr())


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def bytes_cmp(got: np.ndarray, want: np.ndarray) -> dict:
    d = np.abs(got.astype(np.int64) - want.astype(np.int64))
    return {"n": int(d.size), "mismatch": int((d > 0).sum()),
            "mismatch_frac": float((d > 0).mean()) if d.size else 0.0,
            "max_diff": int(d.max()) if d.size else 0}


def feat_cmp(a: np.ndarray, b: np.ndarray) -> dict:
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    cos = (a * b).sum(1) / np.maximum(np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1), 1e-30)
    return {"max_abs": float(np.abs(a - b).max()),
            "rel_l2": float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)),
            "cos_min": float(cos.min())}


# --- conv1 ------------------------------------------------------------------------------------
def conv1_args(c: cases.GemmCase, device) -> tuple:
    """(d8s_conv1 arguments of case c on the device, the tensors they point into)."""
    HW = c.S * c.width
    M = c.N * HW
    in0, seg, w, abh, gd = (_dev(a, device) for a in (c.in0, c.seg, c.w1, c.abh, c.gd))
    wsum = _dev(c.w1.astype(np.int64).sum(axis=(0, 2)).astype(np.int32), device)
    bott = torch.zeros(4 * M * 32, dtype=torch.uint8, device=device)
    args = hip.GemmArgs(_ptr(in0), _ptr(seg), _ptr(w), _ptr(abh), _ptr(gd), _ptr(wsum), _ptr(bott),
                        c.G0, c.G, c.N, HW, c.width, M, 128, 0)
    return args, (in0, seg, w, abh, gd, wsum, bott)


def run_conv1(c: cases.GemmCase, device, acc32: bool = True,
              variant: int = 0) -> tuple[np.ndarray | None, np.ndarray]:
    """(acc [M, 128] int32 or None, bottleneck [M, 128] uint8) from d8s_conv1(_acc32); `variant` != 0
    (no accumulators): d8s_conv1_as with that kernel variant."""
    if variant:
        args, keep = conv1_args(c, device)
        M = c.N * c.S * c.width
        hip.call("d8s_conv1_as", ctypes.byref(args), variant, _stream(device))
        torch.cuda.synchronize(device)
        return None, keep[-1].cpu().numpy().reshape(4, M, 32).transpose(1, 0, 2).reshape(M, 128)
    HW = c.S * c.width
    M = c.N * HW
    in0, seg, w, abh, gd = (_dev(a, device) for a in (c.in0, c.seg, c.w1, c.abh, c.gd))
    wsum = _dev(c.w1.astype(np.int64).sum(axis=(0, 2)).astype(np.int32), device)
    bott = torch.zeros(4 * M * 32, dtype=torch.uint8, device=device)
    args = hip.GemmArgs(_ptr(in0), _ptr(seg), _ptr(w), _ptr(abh), _ptr(gd), _ptr(wsum), _ptr(bott),
                        c.G0, c.G, c.N, HW, c.width, M, 128, 0)
    acc = None
    if acc32:
        acc = torch.full((M * 128,), -7, dtype=torch.int32, device=device)
        hip.call("d8s_conv1_acc32", ctypes.byref(args), _ptr(acc), _stream(device))
    else:
        hip.call("d8s_conv1", ctypes.byref(args), _stream(device))
    torch.cuda.synchronize(device)
    b = bott.cpu().numpy().reshape(4, M, 32).transpose(1, 0, 2).reshape(M, 128)
    return (None if acc is None else acc.cpu().numpy().reshape(M, 128)), b


def exact_conv1(c: cases.GemmCase) -> tuple[np.ndarray, np.ndarray]:
    """(acc, bytes) of every row: u by the oracle's prologue table, acc by float64 matmul."""
    lut = lib.prologue_lut(c.abh)                               # [C][256]
    C = c.q.shape[1]
    wT = torch.from_numpy(c.w.astype(np.float64).T.copy())      # [C][128]
    accs = []
    for n in range(c.N):
        u = lut[np.arange(C)[:, None], c.q[n].astype(np.int64) + 128]      # [C][HW]
        accs.append((torch.from_numpy(u.T.astype(np.float64)) @ wT).numpy())
    acc = np.concatenate(accs).astype(np.int64)
    assert np.abs(acc).max() < 2**31
    acc = acc.astype(np.int32)
    return acc, lib.conv1_epilogue(acc, c.gd)


# --- conv2 ------------------------------------------------------------------------------------
def run_conv2(c: cases.Conv2Case, device, slots: int = 3, slot: int = 1,
              variant: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """Runs d8s_conv2 (`variant` != 0: d8s_conv2_as with that tile) into slot `slot` of a `slots`-slot
    store filled with a sentinel; returns (the slot [M, 32] int8, the other slots' bytes) so a write
    outside the slot shows."""
    N, _, H, W = c.v.shape
    M = N * H * W
    bott, w2k, sc = (_dev(a, device) for a in (c.bott, c.w2k, c.sc))
    wsum = _dev(c.w2k.astype(np.int64).sum(axis=(0, 1, 3)).astype(np.int32), device)
    store = torch.full((slots * M * 32,), 0x5A, dtype=torch.int8, device=device)
    args = hip.Conv2Args(_ptr(bott), _ptr(w2k), _ptr(sc), _ptr(wsum), _ptr(store) + slot * M * 32,
                         N, H, W, 0)
    if variant:
        hip.call("d8s_conv2_as", ctypes.byref(args), variant, _stream(device))
    else:
        hip.call("d8s_conv2", ctypes.byref(args), _stream(device))
    torch.cuda.synchronize(device)
    s = store.cpu().numpy().reshape(slots, M, 32)
    others = np.concatenate([s[k].reshape(-1) for k in range(slots) if k != slot]) if slots > 1 \
        else np.zeros(0, np.int8)
    return s[slot], others


def exact_conv2(c: cases.Conv2Case) -> tuple[np.ndarray, np.ndarray]:
    """(acc [M, 32], q [M, 32]): zero-padded float64 conv, then the oracle's epilogue."""
    w = torch.from_numpy(c.w2.astype(np.float64))
    accs = []
    for n0 in range(0, c.N, 4):
        v = torch.from_numpy(c.v[n0:n0 + 4].astype(np.float64))
        a = F.conv2d(v, w, padding=1)                          # [n, 32, H, W]
        accs.append(a.permute(0, 2, 3, 1).reshape(-1, 32).numpy())
    acc = np.concatenate(accs).astype(np.int32)
    return acc, lib.conv2_epilogue(acc, c.sc)


# --- fused dense layer ------------------------------------------------------------------------
def run_dense(c: cases.GemmCase, c2: cases.Conv2Case, device, slots: int = 3,
              slot: int = 1) -> tuple[np.ndarray, np.ndarray]:
    """d8s_dense on the store and conv1 tables of `c` and the conv2 tables of `c2`, into slot `slot` of
    a `slots`-slot buffer filled with a sentinel: (the slot [M, 32] int8, the other slots' bytes)."""
    H, W = c.S, c.width
    M = c.N * H * W
    in0, seg, w1, abh, gd, w2k, sc = (_dev(a, device) for a in (c.in0, c.seg, c.w1, c.abh, c.gd, c2.w2k,
                                                                  c2.sc))
    w1sum = _dev(c.w1.astype(np.int64).sum(axis=(0, 2)).astype(np.int32), device)
    w2sum = _dev(c2.w2k.astype(np.int64).sum(axis=(0, 1, 3)).astype(np.int32), device)
    store = torch.full((slots * M * 32,), 0x5A, dtype=torch.int8, device=device)
    args = hip.DenseArgs(_ptr(in0), _ptr(seg), _ptr(w1), _ptr(abh), _ptr(gd), _ptr(w1sum), _ptr(w2k),
                         _ptr(sc), _ptr(w2sum), _ptr(store) + slot * M * 32, c.G0, c.G, c.N, H, W, 0)
    hip.call("d8s_dense", ctypes.byref(args), _stream(device))
    torch.cuda.synchronize(device)
    s = store.cpu().numpy().reshape(slots, M, 32)
    others = np.concatenate([s[k].reshape(-1) for k in range(slots) if k != slot])
    return s[slot], others


def run_chain(c: cases.GemmCase, c2: cases.Conv2Case, device, fused: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """conv2 of `c2` into the store's last slot (group G - 1 of `c`), then conv1 of `c` over all G groups:
    d8s_conv2_conv1 (`fused`) or d8s_conv2 then d8s_conv1.  The last slot starts as a sentinel (its bytes
    in `c` are not used).  Returns (that slot [M, 32] int8, the new bottleneck [M, 128] uint8)."""
    HW = c.S * c.width
    M = c.N * HW
    seg_h = c.seg.copy()
    seg_h[c.G - 1 - c.G0] = 0x5A
    in0, seg, w1, abh, gd, bin_, w2k, sc = (_dev(a, device) for a in (c.in0, seg_h, c.w1, c.abh, c.gd, c2.bott,
                                                                        c2.w2k, c2.sc))
    w1sum = _dev(c.w1.astype(np.int64).sum(axis=(0, 2)).astype(np.int32), device)
    w2sum = _dev(c2.w2k.astype(np.int64).sum(axis=(0, 1, 3)).astype(np.int32), device)
    bout = torch.zeros(4 * M * 32, dtype=torch.uint8, device=device)
    slot = _ptr(seg) + (c.G - 1 - c.G0) * M * 32
    a2 = hip.Conv2Args(_ptr(bin_), _ptr(w2k), _ptr(sc), _ptr(w2sum), slot, c.N, c.S, c.width, 0)
    a1 = hip.GemmArgs(_ptr(in0), _ptr(seg), _ptr(w1), _ptr(abh), _ptr(gd), _ptr(w1sum), _ptr(bout),
                      c.G0, c.G, c.N, HW, c.width, M, 128, 0)
    if fused:
        hip.call("d8s_conv2_conv1", ctypes.byref(a2), ctypes.byref(a1), _stream(device))
    else:
        hip.call("d8s_conv2", ctypes.byref(a2), _stream(device))
        hip.call("d8s_conv1", ctypes.byref(a1), _stream(device))
    torch.cuda.synchronize(device)
    s = seg.cpu().numpy()[c.G - 1 - c.G0].reshape(M, 32)
    b = bout.cpu().numpy().reshape(4, M, 32).transpose(1, 0, 2).reshape(M, 128)
    return s, b


def exact_dense(c: cases.GemmCase, c2: cases.Conv2Case) -> np.ndarray:
    """q [M, 32] of conv1 then conv2: the bottleneck bytes of `exact_conv1`, the 3x3 conv of
    `exact_conv2` on them."""
    _, v = exact_conv1(c)                                        # [M, 128] uint8
    H, W = c.S, c.width
    vv = np.ascontiguousarray(v.reshape(c.N, H, W, 128).transpose(0, 3, 1, 2))
    d = cases.Conv2Case(H, c.N, vv, None, c2.w2, c2.w2k, c2.sc)
    return exact_conv2(d)[1]


# --- transition -------------------------------------------------------------------------------
def trans_args(t: dict, device) -> tuple:
    """(d8s_transition arguments of case t on the device, the tensors they point into)."""
    S, N, cout = t["S"], t["N"], t["cout"]
    HW = S * S
    in0, seg, w, abh, gdf = (_dev(t[k], device) for k in ("in0", "seg", "w", "abh", "gdf"))
    wsum = _dev(t["w"].astype(np.int64).sum(axis=(0, 2)).astype(np.int32), device)
    out = torch.full((N * (cout // 32) * (HW // 4) * 32,), 0x5A, dtype=torch.int8, device=device)
    args = hip.GemmArgs(_ptr(in0), _ptr(seg), _ptr(w), _ptr(abh), _ptr(gdf), _ptr(wsum), _ptr(out),
                        t["G0"], t["G"], N, HW, S, N * HW, cout, cout // 32)
    return args, (in0, seg, w, abh, gdf, wsum, out)


def run_trans(t: dict, device, variant: int = 0) -> np.ndarray:
    """Output [N * HW/4, cout] int8 of d8s_transition (`variant` != 0: d8s_transition_as with that
    variant), from the next block's in0 layout."""
    if variant:
        S, N, cout = t["S"], t["N"], t["cout"]
        args, keep = trans_args(t, device)
        hip.call("d8s_transition_as", ctypes.byref(args), variant, _stream(device))
        torch.cuda.synchronize(device)
        o = keep[-1].cpu().numpy().reshape(N, cout // 32, S * S // 4, 32)
        return o.transpose(0, 2, 1, 3).reshape(N * (S * S // 4), cout)
    S, N, cout = t["S"], t["N"], t["cout"]
    HW = S * S
    in0, seg, w, abh, gdf = (_dev(t[k], device) for k in ("in0", "seg", "w", "abh", "gdf"))
    wsum = _dev(t["w"].astype(np.int64).sum(axis=(0, 2)).astype(np.int32), device)
    out = torch.full((N * (cout // 32) * (HW // 4) * 32,), 0x5A, dtype=torch.int8, device=device)
    args = hip.GemmArgs(_ptr(in0), _ptr(seg), _ptr(w), _ptr(abh), _ptr(gdf), _ptr(wsum), _ptr(out),
                        t["G0"], t["G"], N, HW, S, N * HW, cout, cout // 32)
    hip.call("d8s_transition", ctypes.byref(args), _stream(device))
    torch.cuda.synchronize(device)
    o = out.cpu().numpy().reshape(N, cout // 32, HW // 4, 32)
    return o.transpose(0, 2, 1, 3).reshape(N * (HW // 4), cout)


def exact_trans(t: dict) -> tuple[np.ndarray, np.ndarray]:
    """(S [N * HW/4, cout], q): u by the oracle's prologue, 2x2 sums, float64 matmul, C epilogue."""
    lut = lib.prologue_lut(t["abh"])
    S_, N, C, cout = t["S"], t["N"], t["C"], t["cout"]
    wT = torch.from_numpy(t["tw"].astype(np.float64).T.copy())
    outs = []
    for n in range(N):
        u = lut[np.arange(C)[:, None], t["q"][n].astype(np.int64) + 128].astype(np.int64)
        u = u.reshape(C, S_ // 2, 2, S_ // 2, 2).sum(axis=(2, 4)).reshape(C, -1)   # [C][HW/4]
        outs.append((torch.from_numpy(u.T.astype(np.float64)) @ wT).numpy())
    Sx = np.concatenate(outs).astype(np.int64)
    assert np.abs(Sx).max() < 2**31
    Sx = Sx.astype(np.int32)
    return Sx, lib.trans_epilogue(Sx, t["gdf"])


# --- final ------------------------------------------------------------------------------------
def run_final(in0: np.ndarray, G0: int, seg: np.ndarray, N: int, HW: int, ab: np.ndarray,
              ctot: int, device) -> np.ndarray:
    d_in0, d_seg, d_ab = _dev(in0, device), _dev(seg, device), _dev(ab, device)
    out = torch.full((N, ctot), float("nan"), dtype=torch.float32, device=device)
    hip.call("d8s_final", _ptr(d_in0), G0, _ptr(d_seg), N, HW, _ptr(d_ab), _ptr(out), ctot,
             _stream(device))
    torch.cuda.synchronize(device)
    return out.cpu().numpy()


# --- stem -------------------------------------------------------------------------------------
def run_stem(x: np.ndarray, kind: int, lut: np.ndarray | None, flip: bool, w16: np.ndarray,
             bias: np.ndarray, inv: np.ndarray, device) -> np.ndarray:
    """Block-0 store [N, 64, H/4, W/4] int8 of d8s_stem."""
    N, _, H, W = x.shape
    xd = _dev(x if kind == hip.IN_U8 else np.asarray(x).view(np.int16), device)
    lutd = _dev(lut if lut is not None else np.zeros((3, 256), np.int16), device)
    w, b, iv = _dev(np.asarray(w16).view(np.int16), device), _dev(bias, device), _dev(inv, device)
    Hp, Wp = H // 4, W // 4
    out = torch.full((N * 2 * Hp * Wp * 32,), 0x5A, dtype=torch.int8, device=device)
    args = hip.StemArgs(_ptr(xd), _ptr(lutd), _ptr(w), _ptr(b), _ptr(iv), _ptr(out), N, H, W, kind,
                        int(bool(flip)), 0)
    hip.call("d8s_stem", ctypes.byref(args), _stream(device))
    torch.cuda.synchronize(device)
    o = out.cpu().numpy().reshape(N, 2, Hp * Wp, 32).transpose(0, 1, 3, 2)
    return o.reshape(N, 64, Hp, Wp)


def stem_reference(x: np.ndarray, kind: int, lut, flip: bool, w16, bias, inv) -> np.ndarray:
    """All pooled pixels by float64 conv on the fp16 values: [N, 64, H/4, W/4] int8."""
    if kind == hip.IN_U8:
        xv = np.asarray(lut).view(np.float16).astype(np.float64)[np.arange(3)[None, :, None, None], x]
    else:
        xv = np.asarray(x).view(np.float16).astype(np.float64)
    if flip:
        xv = xv[..., ::-1]
    w = np.asarray(w16).view(np.float16).astype(np.float64).reshape(64, 3, 7, 8)[..., 1:]
    y = F.conv2d(torch.from_numpy(np.ascontiguousarray(xv)), torch.from_numpy(np.ascontiguousarray(w)),
                 stride=2, padding=3)
    y = (y + torch.from_numpy(np.asarray(bias, np.float64)).view(1, -1, 1, 1)).float()   # fp32 sum
    t = torch.clamp_min(y, 0) * torch.from_numpy(np.asarray(inv, np.float32)).view(1, -1, 1, 1)
    q = torch.round(t.clamp(max=127.0))
    return F.max_pool2d(q, 3, 2, 1).numpy().astype(np.int8)


# --- whole encoder ----------------------------------------------------------------------------
def _i8(t) -> np.ndarray:
    """A traced tensor of integer values as int8 numpy (converted on its device first)."""
    return t.to(torch.int8).cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t, np.int8)


def block_store(trace: dict, bi: int, L: int, n: int, g0: int, hw: int) -> tuple[np.ndarray, np.ndarray]:
    """The traced store of block bi in the kernels' layout: in0 [n][g0][hw][32] and seg [L][n][hw][32]
    (at least one slot), each segment converted once."""
    x0 = _i8(trace[(bi, 0)]).reshape(n, g0, 32, hw)
    in0 = np.ascontiguousarray(x0.transpose(0, 1, 3, 2))
    if L == 0:
        return in0, np.zeros((1, n, hw, 32), np.int8)
    seg = np.empty((L, n, hw, 32), np.int8)
    for j in range(L):
        seg[j] = _i8(trace[(bi, j + 1)]).reshape(n, 32, hw).transpose(0, 2, 1)
    return in0, seg


def check_trace(enc, trace: dict, feats: np.ndarray, par: dict, max_rows: int | None = 2048,
                seed: int = 0) -> dict:
    """Every layer of a traced pass against the C oracle, each on the kernels' OWN inputs (so a
    difference cannot propagate; as the reference's `unit_fused`, pack_dense8s.py:323-359).  Rows are
    sampled (`max_rows` per launch, None = all).  Returns the byte comparison of every launch per
    family: "conv1" / "conv2" (two launches per layer, the bottleneck traced), "dense" (a fused layer,
    no bottleneck in memory), "block" (a layer of a whole-block launch, `enc.fused[b] == "img"`),
    "trans", and "final" (features equal or not).  Fused layers are also checked on every pixel of the
    rows where their kernel's bands meet (`band_edges`), besides the sample."""
    rng = np.random.default_rng(seed)
    meta = enc.meta
    n = enc.nb
    kinds = getattr(enc, "fused", {}) or {}
    worst = {"conv1": [], "conv2": [], "dense": [], "block": [], "trans": [], "final": None}

    def pick(m):
        if max_rows is None or m <= max_rows:
            return np.arange(m, dtype=np.int64)
        return np.unique(np.concatenate([rng.choice(m, max_rows, replace=False), [0, m - 1]]))

    for bi, b in enumerate(meta["blocks"]):
        h, w = b["h"], b["w"]
        hw, g0 = h * w, b["c0"] // 32
        in0, seg = block_store(trace, bi, b["L"], n, g0, hw)
        for li in range(b["L"]):
            got_seg = seg[li]                                            # [n][hw][32]
            if ("bott", bi, li) not in trace:
                # fused layer: the oracle's bottleneck on the 3x3 neighbourhoods of sampled pixels,
                # then its conv2 on them
                sel2 = np.union1d(pick(n * hw), band_edges(kinds.get(bi, ""), n, h, w))
                nbr = neighbourhoods(sel2, h, w)
                _, vb = lib.conv1(in0, seg, g0, g0 + li, n, hw, par[f"L{bi}_{li}_abh"],
                                  par[f"L{bi}_{li}_w1"], par[f"L{bi}_{li}_gdu"], nbr)
                rows = np.zeros((n * hw, 128), np.uint8)
                rows[nbr] = vb
                planar = np.ascontiguousarray(rows.reshape(-1, 4, 32).transpose(1, 0, 2))
                _, want2 = lib.conv2(planar, n, h, w, par[f"L{bi}_{li}_w2k"], par[f"L{bi}_{li}_c2u"],
                                     sel2)
                fam = "block" if str(kinds.get(bi, "")).split(":")[0] in ("img", "parts") else "dense"
                worst[fam].append(bytes_cmp(got_seg.reshape(n * hw, 32)[sel2], want2))
                continue
            sel = pick(n * hw)
            _, want = lib.conv1(in0, seg, g0, g0 + li, n, hw, par[f"L{bi}_{li}_abh"],
                                par[f"L{bi}_{li}_w1"], par[f"L{bi}_{li}_gdu"], sel)
            bott = trace[("bott", bi, li)]
            bott = (bott.cpu().numpy() if isinstance(bott, torch.Tensor) else np.asarray(bott))
            bott = bott.astype(np.uint8).reshape(n, 4, 32, hw)                # [n][plane][32][hw]
            got = bott.reshape(n, 128, hw).transpose(0, 2, 1).reshape(n * hw, 128)[sel]
            worst["conv1"].append(bytes_cmp(got, want))
            planar = np.ascontiguousarray(bott.transpose(1, 0, 3, 2))
            sel2 = pick(n * hw)
            _, want2 = lib.conv2(planar.reshape(4, -1, 32), n, h, w, par[f"L{bi}_{li}_w2k"],
                                 par[f"L{bi}_{li}_c2u"], sel2)
            worst["conv2"].append(bytes_cmp(got_seg.reshape(n * hw, 32)[sel2], want2))
        if b["trans"]:
            cout = (b["c0"] + 32 * b["L"]) // 2
            selt = pick(n * hw // 4)
            _, want = lib.trans(in0, seg, g0, g0 + b["L"], n, hw, w, par[f"T{bi}_abh"],
                                par[f"T{bi}_w"], par[f"T{bi}_gdf"], cout, selt)
            nxt = _i8(trace[(bi + 1, 0)])                                 # [n][cout][h/2][w/2]
            got = nxt.reshape(n, cout, hw // 4).transpose(0, 2, 1).reshape(-1, cout)[selt]
            worst["trans"].append(bytes_cmp(got, want))
        else:
            want = lib.final(in0, g0, seg, n, hw, par["F_ab"], b["c0"] + 32 * b["L"])
            worst["final"] = {"max_abs": float(np.abs(feats[:n] - want).max()),
                              "equal": bool(np.array_equal(feats[:n], want))}
    return worst


def band_edges(kind, n: int, h: int, w: int) -> np.ndarray:
    """Rows (n h w + y w + x) where a fused kernel's work split meets itself, for the first and last
    image: "parts:K" (d8s_dense_block_parts) the last row of each band and the first of the next
    (their halo rows cross workgroups), "tile" (d8s_dense's row bands of 8 or 16 rows, or its 2-D
    tiles) every row y with y % 8 in {7, 0}; nothing for the other kinds."""
    kind = str(kind)
    if kind.startswith("parts:"):
        r = h // int(kind.split(":", 1)[1])
        ys = sorted({y for k in range(1, h // r) for y in (k * r - 1, k * r)})
    elif kind == "tile":
        ys = [y for y in range(h) if y % 8 in (7, 0)]
    else:
        return np.zeros(0, np.int64)
    ys = np.asarray(ys, np.int64)
    out = [img * h * w + (ys[:, None] * w + np.arange(w)[None, :]).reshape(-1) for img in sorted({0, n - 1})]
    return np.concatenate(out) if ys.size else np.zeros(0, np.int64)


def neighbourhoods(sel: np.ndarray, h: int, w: int) -> np.ndarray:
    """Rows (n h w + y w + x) of the in-image 3 x 3 neighbourhoods of the rows `sel`, sorted, unique."""
    hw = h * w
    n, p = np.divmod(np.asarray(sel, np.int64), hw)
    y, x = np.divmod(p, w)
    out = []
    for dy in (-1, 0, 1):
        for dx in (-1, 0, 1):
            yy, xx = y + dy, x + dx
            ok = (yy >= 0) & (yy < h) & (xx >= 0) & (xx < w)
            out.append((n * hw + yy * w + xx)[ok])
    return np.unique(np.concatenate(out))


def summarize(worst: dict) -> dict:
    out = {}
    for k in ("conv1", "conv2", "dense", "block", "trans"):
        v = worst[k]
        out[k] = {"launches": len(v), "mismatch": sum(x["mismatch"] for x in v),
                  "max_diff": max((x["max_diff"] for x in v), default=0)}
    out["final"] = worst["final"]
    return out


def smoke_check(device: str = "cuda:0") -> dict:
    """One small pass (a DenseNet with 2 layers per block, 2 images of 64 x 64, uint8 input) on the GPU:
    every launch bit-exact against the C oracle on the kernels' own inputs, the stem within 1 LSB, the
    features close to the float64 emulation.  Block 0 (16 x 16) runs as "chain" (its conv1, one
    chained conv2 + conv1 launch, its last conv2), block 1 (8 x 8) as "parts" (the whole block in one
    launch, images split into row bands), blocks 2-3 as their default "img"."""
    from rsna_knee_efficiency_amd import densenet

    from . import emulate as emu
    torch.manual_seed(0)
    model = densenet.seeded_densenet169(0, blocks=(2, 2, 2, 2))
    rng = np.random.default_rng(5)
    mean, std = 0.5, 0.25
    cal_u8 = rng.integers(0, 256, (4, 3, 64, 64), dtype=np.uint8)
    norm = lambda u: (torch.from_numpy(u).float() / 255 - mean) / std  # noqa: E731
    cal = dense8s.calibrate(model, [norm(cal_u8)])
    plan = dense8s.make_plan(model, cal, 64)
    pack = dense8s.make_pack(plan, 2, input_kind="u8", mean=(mean,) * 3, std=(std,) * 3)
    kinds = dense8s.fused_blocks(pack["meta"])
    kinds.update({0: "chain", 1: "parts"})
    enc = dense8s.Dense8SEncoder(pack, 0, 2, fused=kinds)
    x = rng.integers(0, 256, (2, 3, 64, 64), dtype=np.uint8)
    xd = torch.from_numpy(x).to(device)
    trace, f = enc.trace(xd)
    feats = f.cpu().numpy()
    par = dense8s.kernel_params(plan)
    res = summarize(check_trace(enc, trace, feats, par, max_rows=None))
    lut = dense8s.input_lut([mean] * 3, [std] * 3)
    got0 = trace[(0, 0)].cpu().numpy().astype(np.int8)
    want0 = stem_reference(x, hip.IN_U8, lut, False, par["S_w16"], par["S_bias"], par["S_inv"])
    res["stem"] = bytes_cmp(got0, want0)
    full = enc(xd).cpu().numpy()
    res["call_vs_trace"] = bool(np.array_equal(full, feats))
    xf = torch.from_numpy(np.asarray(lut).view(np.float16).astype(np.float64)[
        np.arange(3)[None, :, None, None], x])
    ref = emu.emulate(plan, xf, par, stem_kind="f16").numpy()
    res["vs_emulate"] = feat_cmp(feats, ref)
    res["wait_errors"] = enc.sync_errors()
    return smoke_gate(res)


def smoke_gate(res: dict) -> dict:
    """The pass/fail rule of `smoke_check`: no byte of any checked launch family differs (conv1,
    conv2, the fused layers, the whole-block layers and the transitions), at least one layer and one
    transition were checked, the final features
    are equal, the stem within 1 LSB on < 1e-3 of its bytes, a plain call equals the trace, the
    features are within rel_l2 1e-2 of the float64 emulation, and no bounded wait of the banded block
    ran out.  Raises AssertionError otherwise."""
    fams = ("conv1", "conv2", "dense", "block", "trans")
    ok = (all(res[k]["mismatch"] == 0 for k in fams)
          and sum(res[k]["launches"] for k in ("conv1", "dense", "block")) > 0
          and res["trans"]["launches"] > 0
          and res["final"]["equal"]
          and res["stem"]["max_diff"] <= 1 and res["stem"]["mismatch_frac"] < 1e-3
          and res["call_vs_trace"] and res["vs_emulate"]["rel_l2"] < 1e-2
          and res.get("wait_errors", 0) == 0)
    res["ok"] = ok
    if not ok:
        raise AssertionError(f"smoke check failed: {res}")
    return res


def oracle_trace(meta: dict, par: dict, stem_q: np.ndarray, n: int) -> tuple[dict, np.ndarray]:
    """A whole pass computed by the C oracle alone, in the format of `Dense8SEncoder.trace` for
    fused layers (no bottleneck entries): {(block, 0): block input, (block, l + 1): layer l's 32
    channels} as float tensors (n, c, h, w) of integers, and the final features (n, C).  `stem_q` is
    block 0's input q [n, c0, h, w] int8.  Every pixel of every layer is computed: tiny maps only."""
    out: dict = {}
    cur = np.asarray(stem_q, np.int8)
    feats = None
    for bi, b in enumerate(meta["blocks"]):
        h, w = b["h"], b["w"]
        hw, g0 = h * w, b["c0"] // 32
        out[(bi, 0)] = torch.from_numpy(cur.astype(np.float32))
        q = cur.reshape(n, -1, hw)
        rows = np.arange(n * hw, dtype=np.int64)
        for li in range(b["L"]):
            in0, seg = cases.store_from_q(q, g0)
            _, v = lib.conv1(in0, seg, g0, g0 + li, n, hw, par[f"L{bi}_{li}_abh"],
                             par[f"L{bi}_{li}_w1"], par[f"L{bi}_{li}_gdu"], rows)
            planar = np.ascontiguousarray(v.reshape(-1, 4, 32).transpose(1, 0, 2))
            _, q2 = lib.conv2(planar, n, h, w, par[f"L{bi}_{li}_w2k"], par[f"L{bi}_{li}_c2u"], rows)
            new = q2.reshape(n, hw, 32).transpose(0, 2, 1)                  # [n][32][hw]
            out[(bi, li + 1)] = torch.from_numpy(new.reshape(n, 32, h, w).astype(np.float32))
            q = np.concatenate([q, new], 1)
        in0, seg = cases.store_from_q(q, g0)
        if b["trans"]:
            cout = (b["c0"] + 32 * b["L"]) // 2
            _, t = lib.trans(in0, seg, g0, g0 + b["L"], n, hw, w, par[f"T{bi}_abh"], par[f"T{bi}_w"],
                             par[f"T{bi}_gdf"], cout, np.arange(n * hw // 4, dtype=np.int64))
            cur = t.reshape(n, hw // 4, cout).transpose(0, 2, 1).reshape(n, cout, h // 2, w // 2)
        else:
            feats = lib.final(in0, g0, seg, n, hw, par["F_ab"], b["c0"] + 32 * b["L"])
    return out, feats
