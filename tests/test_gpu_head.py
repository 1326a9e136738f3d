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
