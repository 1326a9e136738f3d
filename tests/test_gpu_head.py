"""The head after the encoder (`d8s_head`) against the float32 oracle (`oracle/head.py`), the final
configuration's shapes: 8 slots x 11 windows of 1664-d features, context width 256 with 4 heads."""
from __future__ import annotations

import pytest
import torch

from oracle import head as H
from rsna_knee_efficiency_amd import head

pytestmark = pytest.mark.gpu


def _case(b, w, seed):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn((b, w, 1664), generator=g) * 0.5
    slot_of = (torch.arange(w) // 11) % 8
    mask = torch.ones((b, 8), dtype=torch.bool)
    if b > 1:
        mask[1, 3] = mask[1, 7] = False
    if b > 2:
        mask[2] = False          # a study with no slot present
    return z, slot_of, mask


@pytest.mark.parametrize("b,w", [(3, 88), (1, 88), (4, 44), (2, 128)])
def test_head_matches_the_oracle(dev, b, w):
    print(f"head b={b} w={w}", flush=True)
    sd = H.random_state_dict(7 + w)
    z, slot_of, mask = _case(b, w, b * 100 + w)
    want = H.head_forward(sd, z, slot_of, mask)
    got = head.KneeHead(sd, dev)(z.to(dev), slot_of, mask).cpu()
    err = (got - want).abs().max().item()
    assert torch.allclose(got, want, rtol=1e-4, atol=1e-4), err


def test_head_reference_init_and_repeat(dev):
    """ctx_out zero as the reference initialises it; two calls in a row give the same logits."""
    sd = H.random_state_dict(11)
    sd["ctx_out.weight"].zero_()
    sd["ctx_out.bias"].zero_()
    z, slot_of, mask = _case(3, 88, 5)
    hd = head.KneeHead(sd, dev)
    a = hd(z.to(dev), slot_of, mask)
    b = hd(z.to(dev), slot_of, mask)
    assert torch.equal(a, b)
    assert torch.allclose(a.cpu(), H.head_forward(sd, z, slot_of, mask), rtol=1e-4, atol=1e-4)


def test_head_slot_indices_checked_per_version(dev):
    """The window-to-slot map is checked once per tensor and in-place version: an in-place change to
    another valid map gives that map's logits, one to an index outside 0 .. S-1 raises."""
    sd = H.random_state_dict(12)
    z, slot_of, mask = _case(2, 44, 8)
    hd = head.KneeHead(sd, dev)
    zd = z.to(dev)
    a = hd(zd, slot_of, mask)
    assert torch.allclose(a.cpu(), H.head_forward(sd, z, slot_of, mask), rtol=1e-4, atol=1e-4)
    slot_of[:11] = 7                      # same tensor, new version
    b = hd(zd, slot_of, mask)
    assert torch.allclose(b.cpu(), H.head_forward(sd, z, slot_of, mask), rtol=1e-4, atol=1e-4)
    assert not torch.equal(a, b)
    slot_of[0] = 8
    with pytest.raises(ValueError):
        hd(zd, slot_of, mask)
    dslot = (torch.arange(44) // 11).to(dev)   # a device-resident map
    c = hd(zd, dslot, mask)
    assert torch.allclose(c.cpu(), H.head_forward(sd, z, dslot.cpu(), mask), rtol=1e-4, atol=1e-4)


def test_head_abi_slot_outside_range_reads_nothing(dev):
    """Through the C ABI with a device map holding indices outside 0 .. S-1 (-1 and S): those windows
    take no slot embedding and count as absent, which is the oracle with a zero-embedding slot S that
    no study has."""
    import ctypes
    from rsna_knee_efficiency_amd import hip
    sd = H.random_state_dict(13)
    z, slot_of, mask = _case(2, 44, 9)
    bad = slot_of.clone()
    bad[3], bad[20] = -1, 8
    hd = head.KneeHead(sd, dev)
    zd = z.to(dev).contiguous()
    sl = bad.to(dev, torch.int32)
    md = mask.to(dev).view(torch.uint8).contiguous()
    logits = torch.empty((2, 12), dtype=torch.float32, device=dev)
    a = hd._args(zd, sl, md, logits)
    need = ctypes.c_uint64()
    hip.call("d8s_head_workspace", ctypes.byref(a), ctypes.byref(need))
    ws = torch.empty(int(need.value) + 256, dtype=torch.uint8, device=dev)
    base = (ws.data_ptr() + 255) // 256 * 256
    a.workspace, a.ws_bytes = base, ws.numel() - (base - ws.data_ptr())
    hip.call("d8s_head", ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    torch.cuda.synchronize(dev)
    sd9 = dict(sd)
    sd9["slot_emb"] = torch.cat([sd["slot_emb"], torch.zeros(1, 1664)])
    ref_slot = bad.clone()
    ref_slot[ref_slot < 0] = 8
    ref_mask = torch.cat([mask, torch.zeros((2, 1), dtype=torch.bool)], 1)
    want = H.head_forward(sd9, z, ref_slot, ref_mask)
    assert torch.allclose(logits.cpu(), want, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("d,w,slots,per,cd,targets,b", [
    (602, 37, 5, 7, 128, 5, 3),      # depth not a multiple of 4 (scalar weight staging), odd windows
    (640, 16, 2, 16, 192, 16, 1),    # 3 heads, 16 findings, one query group
    (100, 129 - 1, 8, 11, 64, 1, 2),  # one head, one finding, 128 windows, a partial column tile
])
def test_head_other_shapes(dev, d, w, slots, per, cd, targets, b):
    """Shapes away from the final configuration: partial product tiles in every dimension, the
    scalar weight path, 1-3 heads, 1-16 findings, other slot and position counts."""
    sd = H.random_state_dict(d + w, d=d, slots=slots, per=per, cd=cd, targets=targets)
    g = torch.Generator().manual_seed(w)
    z = torch.randn((b, w, d), generator=g) * 0.5
    slot_of = torch.arange(w) % slots
    mask = torch.rand((b, slots), generator=g) > 0.3
    mask[0, 0] = True
    want = H.head_forward(sd, z, slot_of, mask, heads=cd // 64)
    got = head.KneeHead(sd, dev, context_heads=cd // 64)(z.to(dev), slot_of, mask).cpu()
    assert got.shape == (b, targets)
    assert torch.allclose(got, want, rtol=1e-4, atol=1e-4), float((got - want).abs().max())
