"""Pins of the head oracle (`oracle/head.py`) on the CPU: the transformer layer against a manual
pre-norm attention + feed-forward, and the pooling against closed forms."""
from __future__ import annotations

import numpy as np
import torch

from oracle import head as H

W, D, S = 22, 64, 4


def _inputs(seed=0, b=3):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn((b, W, D), generator=g)
    slot_of = torch.arange(W) // (W // S)
    slot_of[slot_of >= S] = S - 1
    mask = torch.ones((b, S), dtype=torch.bool)
    mask[1, 2] = False
    mask[2] = False
    return z, slot_of, mask


def _sd(seed=1):
    return H.random_state_dict(seed, d=D, slots=S, per=W // S, cd=64)


def _manual_layer(sd, x, pad, heads):
    """Pre-norm encoder layer: x + MHA(LN1 x) with masked keys, then + FF(LN2 .) (ReLU)."""
    p = "ctx.layers.0."
    cd = x.shape[-1]
    dh = cd // heads
    ln = torch.nn.functional.layer_norm
    y = ln(x, (cd,), sd[p + "norm1.weight"], sd[p + "norm1.bias"])
    qkv = y @ sd[p + "self_attn.in_proj_weight"].t() + sd[p + "self_attn.in_proj_bias"]
    q, k, v = qkv.split(cd, dim=-1)
    out = []
    for h in range(heads):
        sl = slice(h * dh, (h + 1) * dh)
        s = q[..., sl] @ k[..., sl].transpose(1, 2) / dh ** 0.5
        s = s.masked_fill(pad.unsqueeze(1), float("-inf"))
        out.append(s.softmax(-1) @ v[..., sl])
    att = torch.cat(out, -1) @ sd[p + "self_attn.out_proj.weight"].t() + sd[p + "self_attn.out_proj.bias"]
    x = x + att
    y = ln(x, (cd,), sd[p + "norm2.weight"], sd[p + "norm2.bias"])
    ff = torch.relu(y @ sd[p + "linear1.weight"].t() + sd[p + "linear1.bias"])
    return x + ff @ sd[p + "linear2.weight"].t() + sd[p + "linear2.bias"]


def test_context_layer_is_prenorm_attention_and_ffn():
    sd, (z, slot_of, mask) = _sd(), _inputs()
    sd["attn.weight"].zero_()
    sd["attn.bias"].zero_()
    got = H.head_forward(sd, z, slot_of, mask)
    f = z + sd["slot_emb"][slot_of]
    valid = mask[:, slot_of]
    pos = torch.arange(W) % sd["ctx_pos"].shape[0]
    h = f @ sd["ctx_in.weight"].t() + sd["ctx_in.bias"] + sd["ctx_pos"][pos]
    pad = ~valid & ~(~valid).all(1, keepdim=True)
    f2 = f + _manual_layer(sd, h, pad, 4) @ sd["ctx_out.weight"].t() + sd["ctx_out.bias"]
    s = f2 @ sd["cls_w"].t()                                   # (B, W, T)
    v = valid.float().unsqueeze(-1)
    v = torch.where(v.sum(1, keepdim=True) > 0, v, torch.ones_like(v))
    want = (s * v).sum(1) / v.sum(1) + sd["cls_b"]             # uniform attention over the valid windows
    assert torch.allclose(got, want, atol=1e-5)


def test_zero_context_output_leaves_the_pooling():
    sd, (z, slot_of, mask) = _sd(2), _inputs(3)
    sd["ctx_out.weight"].zero_()
    sd["ctx_out.bias"].zero_()
    got = H.head_forward(sd, z, slot_of, mask).numpy()
    f = (z + sd["slot_emb"][slot_of]).double().numpy()
    valid = mask[:, slot_of].numpy()
    a = f @ sd["attn.weight"].double().numpy().T + sd["attn.bias"].double().numpy()
    want = np.zeros_like(got, dtype=np.float64)
    for b in range(f.shape[0]):
        keep = valid[b] if valid[b].any() else np.ones(W, bool)
        ab = np.where(keep[:, None], a[b], -np.inf) if valid[b].any() else np.zeros_like(a[b])
        e = np.exp(ab - ab.max(0))
        p = e / e.sum(0)
        pooled = p.T @ f[b]                                     # (T, D)
        want[b] = (pooled * sd["cls_w"].double().numpy()).sum(-1) + sd["cls_b"].double().numpy()
    assert np.allclose(got, want, atol=1e-5)


def test_absent_slots_do_not_change_the_logits():
    sd, (z, slot_of, mask) = _sd(4), _inputs(5)
    base = H.head_forward(sd, z, slot_of, mask)
    z2 = z.clone()
    absent = ~mask[1, slot_of]
    z2[1, absent] += 5.0
    got = H.head_forward(sd, z2, slot_of, mask)
    assert torch.allclose(got[1], base[1], atol=1e-5)
    # a study with no slot at all pools every window uniformly: perturbing its windows changes it
    z3 = z.clone()
    z3[2, 0] += 5.0
    assert not torch.allclose(H.head_forward(sd, z3, slot_of, mask)[2], base[2])
