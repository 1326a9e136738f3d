"""CPU oracle of the head after the encoder -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

`head_forward(sd, encoded, slot_of_window, slot_mask)`: `KneeBaseline.forward(None, slot_of_window,
slot_mask, encoded=encoded)` for the final configuration in float32 torch on the CPU, restated from
src/knee/models/baseline.py: the features with slot identity (`_features_full` :925-931), the context
(`_context` :954-977, the layer built as the reference builds it, :701-713: pre-norm
`nn.TransformerEncoderLayer` of width cd, `heads` heads, feed-forward 2 cd, no dropout, batch first,
wrapped in `nn.TransformerEncoder` with one layer) and the per-finding attention pooling
(`forward` :1122-1168 with `slot_prior_strength` 0 and `slot_prior_mask_at` None).
`random_state_dict` makes seeded weights of that shape (the reference initialises ctx_out to zero;
here every weight is random so that every term is exercised).
"""
from __future__ import annotations

import torch
import torch.nn as nn


def head_forward(sd: dict, encoded: torch.Tensor, slot_of: torch.Tensor, slot_mask: torch.Tensor,
                 heads: int = 4) -> torch.Tensor:
    f = encoded.float() + sd["slot_emb"][slot_of].unsqueeze(0)
    valid = slot_mask[:, slot_of]
    w = f.shape[1]
    per = sd["ctx_pos"].shape[0]
    cd = sd["ctx_in.weight"].shape[0]
    pos = torch.arange(w) % per
    h = f @ sd["ctx_in.weight"].t() + sd["ctx_in.bias"] + sd["ctx_pos"][pos].unsqueeze(0)
    layer = nn.TransformerEncoderLayer(cd, heads, dim_feedforward=2 * cd, dropout=0.0, batch_first=True,
                                       norm_first=True)
    enc = nn.TransformerEncoder(layer, 1, enable_nested_tensor=False)
    enc.load_state_dict({k[len("ctx."):]: v for k, v in sd.items() if k.startswith("ctx.layers.")})
    enc.eval()
    pad = ~valid
    pad = pad & ~pad.all(dim=1, keepdim=True)
    with torch.no_grad():
        h = enc(h, src_key_padding_mask=pad)
    f = f + h @ sd["ctx_out.weight"].t() + sd["ctx_out.bias"]
    a = f @ sd["attn.weight"].t() + sd["attn.bias"]
    v = valid.unsqueeze(-1)
    a = a.masked_fill(~v, float("-inf"))
    dead = ~v.any(dim=1, keepdim=True).expand_as(a)
    a = torch.where(dead, torch.zeros_like(a), a).softmax(dim=1)
    pooled = torch.einsum("bwt,bwd->btd", a, f)
    return (pooled * sd["cls_w"]).sum(-1) + sd["cls_b"]


def random_state_dict(seed: int, d: int = 1664, slots: int = 8, per: int = 11, cd: int = 256,
                      targets: int = 12) -> dict:
    g = torch.Generator().manual_seed(seed)

    def r(*shape, s=0.02):
        return torch.randn(shape, generator=g) * s

    sd = {"slot_emb": r(slots, d), "ctx_in.weight": r(cd, d, s=1 / d ** 0.5), "ctx_in.bias": r(cd),
          "ctx_pos": r(per, cd),
          "ctx.layers.0.self_attn.in_proj_weight": r(3 * cd, cd, s=1 / cd ** 0.5),
          "ctx.layers.0.self_attn.in_proj_bias": r(3 * cd),
          "ctx.layers.0.self_attn.out_proj.weight": r(cd, cd, s=1 / cd ** 0.5),
          "ctx.layers.0.self_attn.out_proj.bias": r(cd),
          "ctx.layers.0.linear1.weight": r(2 * cd, cd, s=1 / cd ** 0.5), "ctx.layers.0.linear1.bias": r(2 * cd),
          "ctx.layers.0.linear2.weight": r(cd, 2 * cd, s=1 / (2 * cd) ** 0.5),
          "ctx.layers.0.linear2.bias": r(cd),
          "ctx.layers.0.norm1.weight": 1 + r(cd, s=0.1), "ctx.layers.0.norm1.bias": r(cd),
          "ctx.layers.0.norm2.weight": 1 + r(cd, s=0.1), "ctx.layers.0.norm2.bias": r(cd),
          "ctx_out.weight": r(d, cd, s=1 / cd ** 0.5), "ctx_out.bias": r(d),
          "attn.weight": r(targets, d, s=1 / d ** 0.5), "attn.bias": r(targets),
          "cls_w": r(targets, d, s=1 / d ** 0.5), "cls_b": r(targets)}
    return sd
