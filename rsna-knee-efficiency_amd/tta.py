"""The geometric TTA view on the GPU: zoom / shift of the fp16 windows, over the HIP library
(`d8s_grid_sample`, include/d8s_hip.h).

Host side of the reference's `knee.tta.affine_windows` (src/knee/tta.py:131-148) and of the window
preparation of its submission path (src/knee/infer.py:986-1012: `gather_u8_f16` then
`affine_windows`), same names and meaning:
- `affine_windows(w, scale, tx, ty)`: (B, K, D, H, W) fp16 -> same shape; identity = `w` itself;
- `windows_u8(v_u8, slice_idx, out, scale, tx, ty)`: the windows of `slice_idx` gathered from the uint8
  volume (B, S, K, H, W) as fp16 u / 255 (`fused_uint8.gather_u8_f16`, fused_uint8.py:875-905), zoomed
  in the same kernel when the view is geometric.
The sampling grid is the output of `F.affine_grid` on the view's theta in the windows' dtype, computed
once per (shape, view) and shared by every image, as the reference expands one grid.  There is no CPU
path: without the library the calls raise.
"""
from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F

from . import hip

_GRIDS: dict = {}
_LUTS: dict = {}


def lut_u8_f16(device) -> torch.Tensor:
    """fp16 u / 255 for u = 0..255 as the reference builds it (fused_uint8.py:735)."""
    key = str(device)
    if key not in _LUTS:
        _LUTS[key] = torch.arange(256, dtype=torch.uint8, device=device).half().mul_(1.0 / 255.0)
    return _LUTS[key]


def view_grid(h: int, w: int, d: int, scale: float, tx: float, ty: float, dtype, device) -> torch.Tensor:
    """The (H, W, 2) grid of the view: `F.affine_grid` of theta [[1/s, 0, -2 tx], [0, 1/s, -2 ty]]
    (src/knee/tta.py:141-146)."""
    key = (h, w, d, float(scale), float(tx), float(ty), dtype, str(device))
    g = _GRIDS.get(key)
    if g is None:
        theta = torch.tensor([[1.0 / scale, 0.0, -2.0 * tx], [0.0, 1.0 / scale, -2.0 * ty]],
                             device=device, dtype=dtype).unsqueeze(0)
        g = F.affine_grid(theta, (1, d, h, w), align_corners=False)[0].contiguous()
        _GRIDS[key] = g
    return g


def _sample(args: hip.GridArgs, device) -> None:
    stream = torch.cuda.current_stream(device).cuda_stream
    hip.call("d8s_grid_sample", ctypes.byref(args), ctypes.c_void_p(stream))


def affine_windows(w: torch.Tensor, scale: float = 1.0, tx: float = 0.0, ty: float = 0.0) -> torch.Tensor:
    """(B, K, D, H, W) fp16 windows -> the same shape zoomed by `scale` around the centre and shifted by
    (`tx`, `ty`) of the side; the identity returns `w`."""
    if scale == 1.0 and tx == 0.0 and ty == 0.0:
        return w
    if w.dtype != torch.float16 or not w.is_cuda or w.dim() != 5:
        raise ValueError("affine_windows runs on (B, K, D, H, W) fp16 windows on the GPU")
    b, k, d, h, wd = w.shape
    x = w.contiguous()
    out = torch.empty_like(x)
    g = view_grid(h, wd, d, scale, tx, ty, torch.float16, w.device)
    a = hip.GridArgs(src=x.data_ptr(), grid=g.data_ptr(), out=out.data_ptr(), kind=0,
                     N=b * k * d, H=h, W=wd)
    _sample(a, w.device)
    hip.written(out)
    return out


# the last slice-index tensor checked on each device (kept alive, so identity and version name its
# contents) and the bound it was checked against
_SLICES_CHECKED: dict = {}


def _check_slices(idx: torch.Tensor, limit: int) -> None:
    """Raise unless every index lies in 0 .. limit-1.  The check reads the values back (a
    synchronisation), so it runs once per tensor, in-place version and bound: a fixed window layout
    passed as the same tensor on every call is checked once."""
    c = _SLICES_CHECKED.get(idx.device)
    if c is not None and c[0] is idx and c[1] == idx._version and c[2] == limit:
        return
    if bool(((idx < 0) | (idx >= limit)).any()):
        raise ValueError("slice_idx outside the volume")
    _SLICES_CHECKED[idx.device] = (idx, idx._version, limit)


def windows_u8(v_u8: torch.Tensor, slice_idx: torch.Tensor, out: torch.Tensor, scale: float = 1.0,
               tx: float = 0.0, ty: float = 0.0) -> torch.Tensor:
    """`out` (B * nw, depth, H, W) fp16 = the slices `slice_idx` (int64, nw * depth entries) of every
    study of `v_u8` (B, S, K, H, W) as u / 255, zoomed / shifted when the view is geometric."""
    if v_u8.dtype != torch.uint8 or not v_u8.is_cuda or v_u8.dim() != 5 or not v_u8.is_contiguous():
        raise ValueError("v_u8 must be a contiguous (B, S, K, H, W) uint8 tensor on the GPU")
    if slice_idx.dtype != torch.int64 or slice_idx.device != v_u8.device:
        raise ValueError("slice_idx must be int64 on the volume's device")
    b, s, k, h, w = v_u8.shape
    m = int(slice_idx.numel())
    if out.dtype != torch.float16 or not out.is_contiguous() or out.numel() != b * m * h * w:
        raise ValueError("out must be a contiguous fp16 tensor of B * len(slice_idx) images")
    idx = slice_idx.contiguous()
    _check_slices(idx, s * k)
    gp = 0
    if not (scale == 1.0 and tx == 0.0 and ty == 0.0):
        gp = view_grid(h, w, 1, scale, tx, ty, torch.float16, v_u8.device).data_ptr()
    a = hip.GridArgs(src=v_u8.data_ptr(), slice_idx=idx.data_ptr(), lut=lut_u8_f16(v_u8.device).data_ptr(),
                     grid=gp, out=out.data_ptr(), kind=1, N=b * m, H=h, W=w, B=b, SK=s * k, M=m)
    _sample(a, v_u8.device)
    hip.written(out)
    return out
