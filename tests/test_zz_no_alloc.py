"""`d8s_head_noalloc` (the head with its workspace in a static per-GPU device array, no allocation)
against `d8s_head` with a caller workspace, both called through the C ABI: equal logits (the same kernels
in the same order, so bit-identical) on two calls in a row, the second with fewer studies and windows
than the first (the static array keeps the first call's contents); a call beyond the array's size is
rejected on the host."""
from __future__ import annotations

import ctypes

import pytest
import torch

from oracle import head as H
from rsna_knee_efficiency_amd import head, hip

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20        # D8S_HEAD_SCRATCH_BYTES


def _case(b, w, seed):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn((b, w, 1664), generator=g) * 0.5
    slot_of = (torch.arange(w) // 11) % 8
    mask = torch.ones((b, 8), dtype=torch.bool)
    if b > 1:
        mask[1, 3] = mask[1, 7] = False
    return z, slot_of, mask


def _both(hd: head.KneeHead, z, slot_of, mask, dev) -> tuple[torch.Tensor, torch.Tensor, int]:
    """(logits of d8s_head with a fresh workspace, logits of d8s_head_noalloc, workspace bytes)."""
    zd = z.to(dev).contiguous()
    sl = hd._slots(slot_of)
    md = mask.to(dev).view(torch.uint8).contiguous()
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    out_ws = torch.full((z.shape[0], hd.T), float("nan"), dtype=torch.float32, device=dev)
    a = hd._args(zd, sl, md, out_ws)
    need = ctypes.c_uint64()
    hip.call("d8s_head_workspace", ctypes.byref(a), ctypes.byref(need))
    ws = torch.empty(int(need.value) + 256, dtype=torch.uint8, device=dev)
    a.workspace = (ws.data_ptr() + 255) // 256 * 256
    a.ws_bytes = int(need.value)
    hip.call("d8s_head", ctypes.byref(a), stream)
    out_na = torch.full((z.shape[0], hd.T), float("nan"), dtype=torch.float32, device=dev)
    b = hd._args(zd, sl, md, out_na)
    b.workspace, b.ws_bytes = 0, 0                 # ignored by the no-allocation entry point
    hip.call("d8s_head_noalloc", ctypes.byref(b), stream)
    torch.cuda.synchronize(dev)
    return out_ws.cpu(), out_na.cpu(), int(need.value)


def test_noalloc_equals_workspace_entry_twice(dev):
    sd = H.random_state_dict(21)
    hd = head.KneeHead(sd, dev)
    for b, w, seed in ((8, 88, 1), (3, 44, 2)):            # the second call is smaller
        print(f"head noalloc b={b} w={w}", flush=True)
        z, slot_of, mask = _case(b, w, seed)
        want, got, need = _both(hd, z, slot_of, mask, dev)
        assert need <= SCRATCH_BYTES
        assert torch.isfinite(want).all()
        assert torch.equal(got, want), (b, w, (got - want).abs().max().item())
        assert torch.allclose(got, H.head_forward(sd, z, slot_of, mask), rtol=1e-4, atol=1e-4)


def test_noalloc_rejects_sizes_beyond_the_scratch(dev):
    sd = H.random_state_dict(22)
    hd = head.KneeHead(sd, dev)
    z, slot_of, mask = _case(32, 128, 3)                   # about 40 MiB of workspace
    zd = z.to(dev)
    logits = torch.full((32, hd.T), 7.0, dtype=torch.float32, device=dev)
    a = hd._args(zd, hd._slots(slot_of), mask.to(dev).view(torch.uint8).contiguous(), logits)
    need = ctypes.c_uint64()
    hip.call("d8s_head_workspace", ctypes.byref(a), ctypes.byref(need))
    assert need.value > SCRATCH_BYTES
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    with pytest.raises(hip.D8sError, match="exceeds the static scratch"):
        hip.call("d8s_head_noalloc", ctypes.byref(a), stream)
    torch.cuda.synchronize(dev)
    assert torch.equal(logits, torch.full_like(logits, 7.0))   # nothing ran
