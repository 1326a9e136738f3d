"""ctypes binding of the C oracle `oracle/d8s_oracle.c` (built by `oracle/Makefile`).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  numpy in, numpy out; rows / pixels are selected by
index so full-size maps can be checked on a sample.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libd8s_oracle.so"
_STATE: dict = {}

vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64


def lib() -> ctypes.CDLL:
    if "lib" not in _STATE:
        if not LIB.is_file():
            subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
        L = ctypes.CDLL(str(LIB))
        L.orc_f16_value.argtypes = [ctypes.c_uint16]
        L.orc_f16_value.restype = ctypes.c_double
        L.orc_f16_bits.argtypes = [ctypes.c_double]
        L.orc_f16_bits.restype = ctypes.c_uint16
        L.orc_prologue.argtypes = [ctypes.c_int8, ctypes.c_uint16, ctypes.c_uint16]
        L.orc_prologue.restype = ctypes.c_uint8
        L.orc_conv1.argtypes = [vp, vp, i32, i32, i32, i32, vp, vp, vp, vp, i64, vp, vp, vp]
        L.orc_conv2.argtypes = [vp, i32, i32, i32, vp, vp, vp, i64, vp, vp]
        L.orc_trans.argtypes = [vp, vp, i32, i32, i32, i32, i32, vp, vp, vp, i32, vp, i64, vp, vp, vp]
        L.orc_final.argtypes = [vp, i32, vp, i32, i32, vp, vp, i32]
        L.orc_stem.argtypes = [vp, i32, vp, i32, i32, i32, i32, vp, vp, vp, vp, i64, vp, vp]
        L.orc_prologue_lut.argtypes = [vp, i32, vp]
        L.orc_conv1_epilogue.argtypes = [vp, i64, i32, vp, vp]
        L.orc_conv2_epilogue.argtypes = [vp, i64, vp, vp]
        L.orc_trans_epilogue.argtypes = [vp, i64, i32, vp, vp]
        for name in ("orc_conv1", "orc_conv2", "orc_trans", "orc_final", "orc_stem",
                     "orc_prologue_lut", "orc_conv1_epilogue", "orc_conv2_epilogue",
                     "orc_trans_epilogue"):
            getattr(L, name).restype = None
        _STATE["lib"] = L
    return _STATE["lib"]


def _p(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=dtype)


def f16_bits(x: float) -> int:
    return int(lib().orc_f16_bits(float(x)))


def f16_value(h: int) -> float:
    return float(lib().orc_f16_value(int(h) & 0xffff))


def prologue(q: int, a16: int, b16: int) -> int:
    return int(lib().orc_prologue(int(q), int(a16) & 0xffff, int(b16) & 0xffff))


def conv1(in0, seg, G0: int, G: int, N: int, HW: int, abh, w1, gd, sel):
    """(acc [n, 128] int32, bottleneck bytes [n, 128] uint8) of the rows `sel`."""
    in0, seg = _c(in0, np.int8), _c(seg if seg is not None else np.zeros(1, np.int8), np.int8)
    abh, w1, gd = _c(abh, np.int16), _c(w1, np.int8), _c(gd, np.float32)
    sel = _c(sel, np.int64)
    acc = np.zeros((len(sel), 128), np.int32)
    out = np.zeros((len(sel), 128), np.uint8)
    scratch = np.zeros(G * 32 * 256, np.uint8)
    lib().orc_conv1(_p(in0), _p(seg), G0, G, N, HW, _p(abh), _p(w1), _p(gd), _p(sel), len(sel),
                    _p(acc), _p(out), _p(scratch))
    return acc, out


def conv2(bott, N: int, H: int, W: int, w2k, sc, sel):
    """(acc [n, 32] int32, q [n, 32] int8) of the pixels `sel` of the planar bottleneck [4][N*H*W][32]."""
    bott, w2k, sc, sel = _c(bott, np.uint8), _c(w2k, np.int8), _c(sc, np.float32), _c(sel, np.int64)
    acc = np.zeros((len(sel), 32), np.int32)
    out = np.zeros((len(sel), 32), np.int8)
    lib().orc_conv2(_p(bott), N, H, W, _p(w2k), _p(sc), _p(sel), len(sel), _p(acc), _p(out))
    return acc, out


def trans(in0, seg, G0: int, G: int, N: int, HW: int, W: int, abh, tw, gdf, cout: int, sel):
    """(S [n, cout] int32, q [n, cout] int8) of the output pixels `sel`."""
    in0, seg = _c(in0, np.int8), _c(seg if seg is not None else np.zeros(1, np.int8), np.int8)
    abh, tw, gdf, sel = _c(abh, np.int16), _c(tw, np.int8), _c(gdf, np.float32), _c(sel, np.int64)
    S = np.zeros((len(sel), cout), np.int32)
    out = np.zeros((len(sel), cout), np.int8)
    scratch = np.zeros(G * 32 * 256, np.uint8)
    lib().orc_trans(_p(in0), _p(seg), G0, G, N, HW, W, _p(abh), _p(tw), _p(gdf), cout, _p(sel),
                    len(sel), _p(S), _p(out), _p(scratch))
    return S, out


def final(in0, G0: int, seg, N: int, HW: int, ab, ctot: int):
    in0, seg = _c(in0, np.int8), _c(seg if seg is not None else np.zeros(1, np.int8), np.int8)
    ab = _c(ab, np.float32)
    out = np.zeros((N, ctot), np.float32)
    lib().orc_final(_p(in0), G0, _p(seg), N, HW, _p(ab), _p(out), ctot)
    return out


def stem(x, kind: int, lut, flip: bool, w16, bias, inv, sel, with_conv: bool = False):
    """int8 [n, 64] of the pooled pixels `sel` (and the [n, 9, 64] conv values if `with_conv`).
    x is uint8 (kind 1) or fp16 bits as uint16 / float16 (kind 0), shape [N, 3, H, W]."""
    N, _, H, W = x.shape
    x = _c(x, np.uint8) if kind == 1 else _c(np.asarray(x).view(np.uint16), np.uint16)
    lut = _c(lut if lut is not None else np.zeros((3, 256), np.int16), np.int16)
    w16 = _c(np.asarray(w16).view(np.uint16), np.uint16)
    bias, inv, sel = _c(bias, np.float32), _c(inv, np.float32), _c(sel, np.int64)
    out = np.zeros((len(sel), 64), np.int8)
    conv = np.zeros((len(sel), 9, 64), np.float32) if with_conv else None
    lib().orc_stem(_p(x), kind, _p(lut), int(bool(flip)), N, H, W, _p(w16), _p(bias), _p(inv),
                   _p(sel), len(sel), _p(out), _p(conv))
    return (out, conv) if with_conv else out


def prologue_lut(abh) -> np.ndarray:
    """[C][256] uint8: u of every channel for q = -128..127 (index q + 128)."""
    abh = _c(abh, np.int16)
    C = abh.shape[0] * 2
    lut = np.zeros((C, 256), np.uint8)
    lib().orc_prologue_lut(_p(abh), C, _p(lut))
    return lut


def conv1_epilogue(acc, gd) -> np.ndarray:
    acc, gd = _c(acc, np.int32), _c(gd, np.float32)
    n, cout = acc.shape
    out = np.zeros((n, cout), np.uint8)
    lib().orc_conv1_epilogue(_p(acc), n, cout, _p(gd), _p(out))
    return out


def conv2_epilogue(acc, sc) -> np.ndarray:
    acc, sc = _c(acc, np.int32), _c(sc, np.float32)
    out = np.zeros(acc.shape, np.int8)
    lib().orc_conv2_epilogue(_p(acc), acc.shape[0], _p(sc), _p(out))
    return out


def trans_epilogue(S, gdf) -> np.ndarray:
    S, gdf = _c(S, np.int32), _c(gdf, np.float32)
    n, cout = S.shape
    out = np.zeros((n, cout), np.int8)
    lib().orc_trans_epilogue(_p(S), n, cout, _p(gdf), _p(out))
    return out
