"""The geometric TTA view (`d8s_grid_sample`): bit for bit against the reference's own operations on
the same GPU (`F.affine_grid` + `F.grid_sample` in fp16, src/knee/tta.py:131-148, and the uint8
gather through the u / 255 table, src/knee/infer.py:986-1012), and within fp16 rounding of a float64
bilinear restatement on the CPU."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from rsna_knee_efficiency_amd import tta

pytestmark = pytest.mark.gpu

VIEWS = [(1.10, 0.0, 0.0), (0.95, 0.0, 0.0), (1.05, 0.0, 0.0), (1.0, 0.03, 0.0), (1.0, 0.0, -0.03),
         (1.10, 0.03, -0.03)]


def _reference(w: torch.Tensor, scale: float, tx: float, ty: float) -> torch.Tensor:
    """src/knee/tta.py:131-148 as torch operations."""
    b, k, d, h, wd = w.shape
    x = w.reshape(b * k, d, h, wd)
    theta = torch.tensor([[1.0 / scale, 0.0, -2.0 * tx], [0.0, 1.0 / scale, -2.0 * ty]],
                         device=x.device, dtype=x.dtype).unsqueeze(0)
    grid = F.affine_grid(theta, (1, d, h, wd), align_corners=False).expand(b * k, h, wd, 2)
    x = F.grid_sample(x, grid, mode="bilinear", padding_mode="zeros", align_corners=False)
    return x.reshape(b, k, d, h, wd)


def _bilinear_f64(img: np.ndarray, grid: np.ndarray) -> np.ndarray:
    """Bilinear sampling with zero padding, align_corners=False, in float64 (grid given)."""
    h, w = img.shape
    ix = ((grid[..., 0].astype(np.float64) + 1) * w - 1) / 2
    iy = ((grid[..., 1].astype(np.float64) + 1) * h - 1) / 2
    x0, y0 = np.floor(ix).astype(int), np.floor(iy).astype(int)
    out = np.zeros(ix.shape)
    for dy in (0, 1):
        for dx in (0, 1):
            xx, yy = x0 + dx, y0 + dy
            wgt = (1 - np.abs(ix - xx)) * (1 - np.abs(iy - yy))
            ok = (xx >= 0) & (xx < w) & (yy >= 0) & (yy < h)
            out += np.where(ok, img[np.clip(yy, 0, h - 1), np.clip(xx, 0, w - 1)], 0.0) * wgt
    return out


@pytest.mark.parametrize("view", VIEWS, ids=[f"s{v[0]}_tx{v[1]}_ty{v[2]}" for v in VIEWS])
def test_affine_windows_is_the_reference_on_the_gpu(dev, view):
    print(f"view {view}", flush=True)
    g = torch.Generator().manual_seed(3)
    w = torch.rand((2, 3, 3, 96, 80), generator=g).half().to(dev)
    got = tta.affine_windows(w, *view)
    ref = _reference(w, *view)
    diff = int((got != ref).sum())
    assert diff == 0, f"{diff} values differ, max {float((got.float() - ref.float()).abs().max())}"
    # and within fp16 rounding of the float64 restatement on the same (fp16) grid
    grid = tta.view_grid(96, 80, 3, *view, torch.float16, dev).float().cpu().numpy()
    want = _bilinear_f64(w[1, 2, 1].float().cpu().numpy(), grid)
    assert np.abs(got[1, 2, 1].float().cpu().numpy() - want).max() <= 2.0 ** -11 + 1e-6


def test_affine_windows_identity_and_full_size(dev):
    w = torch.rand((1, 11, 3, 512, 512), device=dev).half()
    assert tta.affine_windows(w) is w
    got = tta.affine_windows(w, 1.10)
    assert torch.equal(got, _reference(w, 1.10, 0.0, 0.0))


U8_SHAPES = [(64, 48), (40, 46), (512, 512)]


@pytest.mark.parametrize("view", [(1.0, 0.0, 0.0)] + VIEWS, ids=["identity"] + [f"s{v[0]}_tx{v[1]}_ty{v[2]}" for v in VIEWS])
@pytest.mark.parametrize("hw", U8_SHAPES, ids=[f"{h}x{w}" for h, w in U8_SHAPES])
def test_windows_u8_is_the_reference_chain(dev, view, hw):
    """gather_u8_f16 + affine_windows of the submission path (infer.py:986-1012) in one kernel: every
    view, on widths that take the four-pixel kernel (a multiple of 4, both its window path and its
    per-pixel path at the borders) and one that does not."""
    h, w = hw
    b, s, k = (2, 2, 7) if h < 512 else (1, 1, 9)
    print(f"windows_u8 view {view} {h}x{w}", flush=True)
    g = torch.Generator().manual_seed(5)
    v = torch.randint(0, 256, (b, s, k, h, w), generator=g, dtype=torch.uint8).to(dev)
    idx = torch.tensor([0, 1, 2, 2, 3, 4, 8, 9, 13] if s * k > 13 else [0, 1, 2, 2, 3, 4, 6, 7, 8],
                       dtype=torch.int64, device=dev)
    depth = 3
    out = torch.empty((b * idx.numel() // depth, depth, h, w), dtype=torch.float16, device=dev)
    tta.windows_u8(v, idx, out, *view)
    lut = torch.arange(256, dtype=torch.uint8, device=dev).half().mul_(1.0 / 255.0)
    x = lut[v.view(b, s * k, h, w).index_select(1, idx).long()].view(b * idx.numel() // depth, depth, h, w)
    if view != (1.0, 0.0, 0.0):
        x = _reference(x.view(-1, 1, depth, h, w), *view).view(-1, depth, h, w)
    assert torch.equal(out, x)


def test_lut_is_u_over_255():
    lut = tta.lut_u8_f16("cpu").float().numpy()
    u = np.arange(256) / 255.0
    assert np.abs(lut - u).max() <= 2.0 ** -12 and lut[0] == 0 and lut[255] == 1


@pytest.mark.parametrize("view", [(1.0, 0.0, 0.0), (1.10, 0.0, 0.0)])
def test_windows_u8_slice_checks(dev, view):
    """The slice indices are checked once per tensor and in-place version: a valid in-place change is
    seen, an index outside the volume raises; through the C ABI (no host check) such an index is
    clamped into the volume."""
    import ctypes
    from rsna_knee_efficiency_amd import hip
    b, s, k, h, w = 1, 2, 5, 32, 40
    g = torch.Generator().manual_seed(6)
    v = torch.randint(0, 256, (b, s, k, h, w), generator=g, dtype=torch.uint8).to(dev)
    idx = torch.tensor([0, 1, 2, 7, 8, 9], dtype=torch.int64, device=dev)
    out = torch.empty((2, 3, h, w), dtype=torch.float16, device=dev)
    a = tta.windows_u8(v, idx, out, *view).clone()
    idx[0] = 4                                     # in place, still inside the volume
    bb = tta.windows_u8(v, idx, out, *view).clone()
    assert torch.equal(a[1], bb[1]) and not torch.equal(a[0, 0], bb[0, 0])
    idx[0] = 10
    with pytest.raises(ValueError):
        tta.windows_u8(v, idx, out, *view)
    bad = torch.tensor([0, -1, 2, 10, 8, 9], dtype=torch.int64, device=dev)
    gp = 0 if view == (1.0, 0.0, 0.0) else tta.view_grid(h, w, 1, *view, torch.float16, dev).data_ptr()
    out2 = torch.full((2, 3, h, w), 7.0, dtype=torch.float16, device=dev)
    args = hip.GridArgs(src=v.data_ptr(), slice_idx=bad.data_ptr(), lut=tta.lut_u8_f16(dev).data_ptr(),
                        grid=gp, out=out2.data_ptr(), kind=1, N=6, H=h, W=w, B=1, SK=s * k, M=6)
    hip.call("d8s_grid_sample", ctypes.byref(args), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    torch.cuda.synchronize(dev)
    clamped = torch.tensor([0, 0, 2, 9, 8, 9], dtype=torch.int64, device=dev)
    ref = torch.empty_like(out2)
    tta.windows_u8(v, clamped, ref, *view)
    assert torch.equal(out2, ref)
